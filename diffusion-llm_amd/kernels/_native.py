"""ctypes binding of libbd3attn.so (the C ABI declared in include/bd3attn.h).

PyTorch only provides device memory and the current HIP stream here; every
computation runs in the library's gfx950 kernels. There is no fallback: if
the library is missing, importing a kernel module still works (so CPU-only
tooling can inspect signatures) but the first call raises RuntimeError.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

_PKG = Path(__file__).resolve().parent.parent
LIB_PATH = Path(os.environ.get("BD3ATTN_LIB", _PKG / "lib" / "libbd3attn.so"))

BD3_OK, BD3_EINVAL, BD3_EHIP = 0, 1, 2

_c_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64p = ctypes.POINTER(ctypes.c_int64)
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# (restype, argtypes) of every exported symbol, mirroring include/bd3attn.h.
SIGNATURES: dict[str, tuple] = {
    "bd3_abi_version": (ctypes.c_int, []),
    "bd3_last_error": (ctypes.c_char_p, []),
    "bd3_attn_fwd": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _i32, _i32, _i32, _i32, _i32,
                                    _i64p, _f32, _c_p]),
    "bd3_attn_bwd_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32]),
    "bd3_attn_bwd": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _sz,
                                    _i32, _i32, _i32, _i32, _i32, _i64p, _f32, _c_p]),
    "bd3_attn_bwd_noalloc": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _i32, _i32,
                                            _i32, _i32, _i32, _i64p, _f32, _c_p]),
    "bd3_attn_bwd_delta": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _i32, _i32, _i32, _i32, _i32, _i64p, _f32, _c_p]),
    "bd3_attn_bwd_main": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _i32, _i32, _i32,
                                         _i32, _i32, _i64p, _f32, _c_p]),
    "bd3_attn_bwd_dq": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _i32, _i32, _i32,
                                       _i32, _i32, _i64p, _f32, _c_p]),
    "bd3_attn_bwd_dkdv": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _i32, _i32, _i32,
                                         _i32, _i32, _i64p, _f32, _c_p]),
    "bd3_decode": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _i32, _i32, _i32, _i32, _i32, _i32,
                                  _i64p, _f32, _c_p, _sz, _c_p]),
    "bd3_decode_auto_splits": (_i32, [_i32, _i32, _i32, _i32]),
    "bd3_decode_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "bd3_decode_splitkv": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _i32, _i32, _i32, _i32, _i32, _i32,
                                          _i32, _i64p, _f32, _c_p, _sz, _c_p]),
    "bd3_qkv_rope": (ctypes.c_int, [_c_p, _i64p, _i32, _i32, _i32, _i32, _c_p, _i32, _c_p, _c_p, _i32,
                                    _c_p, _c_p, _c_p, _i64p, _c_p]),
    "bd3_kv_write": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _i32, _i32, _i32, _i32, _i64p, _c_p]),
    "bd3_subs_sample": (ctypes.c_int, [_c_p, ctypes.c_int64, _i32, _c_p, _c_p, _i32, _i32, _i32, ctypes.c_double,
                                       _c_p, ctypes.c_uint64, ctypes.c_uint64, _c_p]),
    "bd3_ln_modulate": (ctypes.c_int, [_c_p, _i32, _c_p, _i32, _c_p, _c_p, _i32, _c_p, _i32, _i32, _i32, _i32,
                                       _i64p, _f32, _c_p]),
    "bd3_gate_residual": (ctypes.c_int, [_c_p, _i32, _c_p, _i32, _c_p, _i32, _c_p, _i32, _i32, _i32, _i64p, _c_p]),
    "bd3_gate_residual_ln_modulate": (ctypes.c_int, [_c_p, _i32, _c_p, _c_p, _i32, _c_p, _c_p, _i32, _c_p, _c_p,
                                                     _i32, _c_p, _i32, _i32, _i32, _i32, _i64p, _f32,
                                                     _c_p]),
    "bd3_mask_dump": (ctypes.c_int, [_c_p, _i32, _i32, _i32, _i32, _c_p]),
    "bd3_clock_probe": (ctypes.c_int, [_c_p, _i32, _i32, _i64p, _c_p]),
    "bd3_train_tile_census": (ctypes.c_int, [_i32, _i32, _i64p]),
    "bd3_train_classify": (ctypes.c_int, [_i32, _i32, _i32, _i32]),
    "bd3_train_classify_keys": (ctypes.c_int, [_i32, _i32, _i32, _i32]),
    "bd3_train_walk_class": (ctypes.c_int, [_i32, _i32, _i32, _i32, _i32, ctypes.POINTER(ctypes.c_int32)]),
    "bd3_train_intervals": (ctypes.c_int, [_i32, _i32, _i32, _i32, ctypes.POINTER(ctypes.c_int32)]),
}

_lib = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """Load libbd3attn.so once; raise RuntimeError if it was not built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.exists():
                    raise RuntimeError(
                        f"{LIB_PATH} not found: build it with "
                        "`python -c 'import __graft_entry__ as g; g.build()'` "
                        "(or python diffusion-llm_amd/csrc/build.py)")
                handle = ctypes.CDLL(str(LIB_PATH))
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = handle
    return _lib


def last_error() -> str:
    msg = lib().bd3_last_error()
    return msg.decode() if msg else ""


def check(status: int) -> None:
    """Map a C-ABI status to the reference's error behaviour: precondition
    failures are AssertionError (the reference uses `assert`), runtime
    failures RuntimeError."""
    if status == BD3_OK:
        return
    if status == BD3_EINVAL:
        raise AssertionError(last_error())
    raise RuntimeError(f"libbd3attn: {last_error()}")


def strides(*tensors: torch.Tensor):
    """(b, h, s) element strides of each 4-D tensor, as a ctypes int64 array."""
    vals = []
    for t in tensors:
        assert t.dim() == 4 and t.stride(-1) == 1, "tensors must be 4-D with last stride 1"
        vals.extend((t.stride(0), t.stride(1), t.stride(2)))
    return (ctypes.c_int64 * len(vals))(*vals)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def vec_ready(t: torch.Tensor) -> bool:
    """True if the kernels can read t in place: 16-byte aligned base and
    outer strides that are multiples of 8 elements (16-byte rows)."""
    return (t.stride(-1) == 1 and t.data_ptr() % 16 == 0
            and all(s % 8 == 0 for s in t.stride()[:-1]))


def as_kernel_input(t: torch.Tensor) -> torch.Tensor:
    """Return t itself when the kernels can read it in place, otherwise a
    contiguous copy (the reference copies with .contiguous() too,
    kernels/BlockSparseFlashAttention.py:480)."""
    return t if vec_ready(t) else t.contiguous()
