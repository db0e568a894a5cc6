"""MI355X (gfx950) BD3-LM attention kernels behind the reference's
`kernels/` module interface:

    kernels.BlockSparseFlashAttention.BlockSparseFlashAttention.apply(q, k, v, block_size)
    kernels.BlockSparseDecodeAttention.block_sparse_decode_attention(q, k, v, block_size)
    kernels.SplitKVDecodeAttention.split_kv_decode_attention(q, k, v, block_size)

Each call lands in libbd3attn.so (hand-written HIP for gfx950) through the
C ABI of include/bd3attn.h.
"""
