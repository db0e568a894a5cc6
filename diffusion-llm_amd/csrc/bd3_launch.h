// bd3_launch.h - argument blocks and launchers shared between the kernel
// translation units and the C-ABI layer (capi.hip). Internal to the library.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace bd3 {

constexpr int kHeadDim = 64;
constexpr int kBwdOrderMax = 256;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

struct Strides3 {
  int64_t b, h, s;  // element strides; the head_dim stride is 1
};

struct FwdArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse;  // contiguous (B, H, 2n), natural log
  Strides3 sq, sk, sv, so;
  int heads;
  int bh;  // batch * heads
  int n;
  int bs;
  float scale_log2;  // softmax scale * log2(e)
};

struct BwdArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* o;
  const uint16_t* dout;
  const float* lse;  // natural log, contiguous (B, H, 2n)
  uint16_t* dq;
  uint16_t* dk;
  uint16_t* dv;
  float* delta;  // 2 x (B, H, 2n) fp32: Delta, then -L / scale (the Delta pass writes both)
  // Work items of one batch*head, in launch order (host built, longest
  // first): code c < 2n/128 is dQ query tile c, otherwise dK/dV key tile
  // c - 2n/128 (see attn_bwd.hip). With more than kBwdOrderMax items the
  // codes run first_code, first_code + 1, ... instead.
  uint16_t order[256];
  int n_items;
  int first_code;
  // 1: the noisy key tiles' dK/dV (block sizes dividing 32, so only their
  // diagonal blocks are live) are formed at the end of the dQ items of the
  // same rows, and the launch holds no dK/dV item for them.
  int fold_diag;
  Strides3 sq, sk, sv, so, sdo, sdq, sdk, sdv;
  int heads;
  int bh;
  int n;
  int bs;
  float scale;       // softmax scale
  float scale_log2;  // scale * log2(e)
};

struct DecodeArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* part_o;    // (BH, q_tiles, n_splits, QT, 64) fp32, or null
  float* part_lse;  // (BH, q_tiles, n_splits, QT) log2 LSE, or null
  Strides3 sq, sk, sv, so;
  int heads;
  int bh;
  int q_len;
  int kv_len;
  int bs;
  int n_splits;
  int split_len;  // keys per split (multiple of 32)
  int q_tiles;
  // Workgroups per (bh, query tile) along the splits, and the consecutive
  // splits each one computes (groups * splits_per_group >= n_splits). With
  // one split per group the workgroup's waves share the split; with more,
  // each wave computes whole splits and the workgroup merges them.
  int groups;
  int splits_per_group;
  float scale_log2;
};

struct QkvRopeArgs {
  const uint16_t* qkv;  // (batch, seq, 3 * heads * 64), last stride 1
  int64_t sx_b, sx_s;
  const int64_t* positions;  // (seq) absolute positions, or null: pos0 + s
  int pos0;
  const float* sin_t;  // (max_pos, 32) fp32
  const float* cos_t;
  int max_pos;
  uint16_t* q;
  uint16_t* k;
  uint16_t* v;
  Strides3 sq, sk, sv;
  int heads;
  int seq;
  int64_t total;  // batch * seq * 4 * heads work items (< 2^31)
};

struct KvWriteArgs {
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* k_dst;
  uint16_t* v_dst;
  Strides3 sk, sv, skd, svd;
  int batch, heads, seq;
  int64_t total;  // 2 * batch * heads * seq * 8 16-byte parts
};

struct SubsArgs {
  const void* logits;  // (rows, ld) bf16 or fp32
  int64_t ld;          // row stride in elements
  int fp32;            // 1: fp32 logits, 0: bf16
  const int64_t* xt;   // (rows) current tokens
  int64_t* out;        // (rows) next tokens
  int rows, vocab;
  int mask_index;
  double keep;         // s / t
  const double* u;     // (rows, vocab) uniforms, or null: Philox4x32-10(seed, offset)
  uint64_t seed, offset;
};

struct GlueArgs {
  const void* x;       // (batch, seq, d) rows, fp32 or bf16
  const void* weight;  // (d) LayerNorm gain
  const void* shift;   // (batch, d): shift (ln_modulate) or gate (gate_residual)
  const void* scale;   // (batch, d)
  const void* y;       // (batch, seq, d) sublayer output (gate_residual)
  void* out;
  const void* gate;    // (batch, d) gate of the fused residual + LayerNorm (stride sm_b)
  void* out_x;         // (batch, seq, d) updated residual of the fused form
  int x_fp32, w_fp32, m_fp32, y_fp32, out_fp32;
  int rows, seq, d;
  int64_t sx_b, sx_s, sm_b, sy_b, sy_s, so_b, so_s, sxo_b, sxo_s;  // element strides
  float eps;
};

hipError_t launch_attn_fwd(const FwdArgs& a, hipStream_t stream);
// The backward's Delta pass (Delta and -L / scale), then one launch of the
// items in a.order (dQ and / or dK/dV).
hipError_t launch_attn_bwd_delta(const BwdArgs& a, hipStream_t stream);
hipError_t launch_attn_bwd_items(const BwdArgs& a, hipStream_t stream);
hipError_t launch_decode(const DecodeArgs& a, int qt, hipStream_t stream);
hipError_t launch_prefill(const DecodeArgs& a, hipStream_t stream);
hipError_t launch_qkv_rope(const QkvRopeArgs& a, hipStream_t stream);
hipError_t launch_kv_write(const KvWriteArgs& a, hipStream_t stream);
hipError_t launch_subs_sample(const SubsArgs& a, hipStream_t stream);
hipError_t launch_ln_modulate(const GlueArgs& a, hipStream_t stream);
hipError_t launch_gate_residual_ln_modulate(const GlueArgs& a, hipStream_t stream);
hipError_t launch_gate_residual(const GlueArgs& a, hipStream_t stream);
hipError_t launch_mask_dump(uint8_t* out, int mode, int rows, int kv_len,
                            int bs, hipStream_t stream);
hipError_t launch_clock_probe(uint64_t* out, int workgroups, int iters, hipStream_t stream);

}  // namespace bd3
