// capi.hip - the extern "C" boundary of libbd3attn.so (declared in
// include/bd3attn.h): argument validation, workspace sizing, launches and
// host-only census helpers. Validation failures return BD3_EINVAL before any
// HIP call, so they are testable on a machine without a GPU.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <cmath>
#include <mutex>
#include <string>

#include "bd3_launch.h"
#include "bd3_mask.h"
#include "bd3attn.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return BD3_OK;
  return fail(BD3_EHIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Rows of 64 bf16 are read as 16-byte vectors: the base must be 16-byte
// aligned and every outer stride a multiple of 8 elements.
int check_tensor(const void* p, const int64_t* st, const char* name) {
  if (p == nullptr) return fail(BD3_EINVAL, "%s is NULL", name);
  if (!aligned16(p)) return fail(BD3_EINVAL, "%s must be 16-byte aligned", name);
  for (int i = 0; i < 3; ++i)
    if (st[i] % 8 != 0 || st[i] < 0)
      return fail(BD3_EINVAL, "%s stride[%d]=%lld must be a non-negative multiple of 8", name, i,
                  (long long)st[i]);
  return BD3_OK;
}

bd3::Strides3 s3(const int64_t* st) { return bd3::Strides3{st[0], st[1], st[2]}; }

// The training kernels fill LDS tiles of 64 rows with direct loads whose
// per-lane byte offset from the tile's first row, 2 * (row * seq_stride +
// column), is a 32-bit value: row <= 63 and column < 64 keep it below 2^31
// for sequence strides below 2^24 elements.
constexpr int64_t kMaxDmaSeqStride = int64_t(1) << 24;

int check_dma_stride(const int64_t* st, const char* name) {
  if (st[2] >= kMaxDmaSeqStride)
    return fail(BD3_EINVAL, "%s sequence stride %lld must be < 2^24 elements (32-bit tile load offsets)", name,
                (long long)st[2]);
  return BD3_OK;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

constexpr int kDecodeQT = 32;

int decode_q_tiles(int q_len) { return (q_len + kDecodeQT - 1) / kDecodeQT; }

int check_common_decode(const void* q, const void* k, const void* v, void* o, int batch,
                        int heads, int q_len, int kv_len, int head_dim, int block_size,
                        const int64_t* strides) {
  if (batch < 1 || heads < 1) return fail(BD3_EINVAL, "batch and heads must be >= 1");
  if (head_dim != bd3::kHeadDim) return fail(BD3_EINVAL, "head_dim must be 64, got %d", head_dim);
  if (block_size < 1) return fail(BD3_EINVAL, "block_size must be >= 1");
  if (q_len < 1 || q_len > kv_len)
    return fail(BD3_EINVAL, "queries are the last q_len key positions: need 1 <= q_len (%d) <= kv_len (%d)",
                q_len, kv_len);
  if (strides == nullptr) return fail(BD3_EINVAL, "strides is NULL");
  const char* names[4] = {"q", "k", "v", "o"};
  const void* ptrs[4] = {q, k, v, o};
  for (int i = 0; i < 4; ++i) {
    int st = check_tensor(ptrs[i], strides + 3 * i, names[i]);
    if (st) return st;
  }
  return BD3_OK;
}

// The kernels take a row's maximum over the raw scores and scale it
// afterwards, which needs scale > 0 (the reference's is 1 / sqrt(head_dim)).
int check_scale(float scale) {
  if (!(scale > 0.f) || !std::isfinite(scale))
    return fail(BD3_EINVAL, "scale must be finite and > 0, got %g", (double)scale);
  return BD3_OK;
}

int check_bwd_shape(int batch, int heads, int n, int head_dim, int block_size,
                    const int64_t* strides) {
  if (batch < 1 || heads < 1) return fail(BD3_EINVAL, "batch and heads must be >= 1");
  if (head_dim != bd3::kHeadDim) return fail(BD3_EINVAL, "head_dim must be 64, got %d", head_dim);
  if (n < 128 || n % 128 != 0)
    return fail(BD3_EINVAL, "n (half the sequence) must be a positive multiple of 128, got %d", n);
  if (block_size < 1 || n % block_size != 0)
    return fail(BD3_EINVAL, "n (%d) must be a multiple of block_size (%d)", n, block_size);
  if (strides == nullptr) return fail(BD3_EINVAL, "strides is NULL");
  return BD3_OK;
}

bd3::BwdArgs bwd_args(const void* q, const void* k, const void* v, const void* o, const void* dout,
                      const float* lse, void* dq, void* dk, void* dv, float* delta, int batch,
                      int heads, int n, int block_size, float scale) {
  bd3::BwdArgs a = {};
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.o = static_cast<const uint16_t*>(o);
  a.dout = static_cast<const uint16_t*>(dout);
  a.lse = lse;
  a.dq = static_cast<uint16_t*>(dq);
  a.dk = static_cast<uint16_t*>(dk);
  a.dv = static_cast<uint16_t*>(dv);
  a.delta = delta;
  a.heads = heads;
  a.bh = batch * heads;
  a.n = n;
  a.bs = block_size;
  a.scale = scale;
  a.scale_log2 = scale * bd3::kLog2e;
  return a;
}

// The backward's work items of one batch*head in launch order, longest
// first: a stable sort on each item's MFMA work, the tiles it walks times
// the products per tile (a dQ query tile three: S, dP, dQ; a dK/dV key tile
// four: S, dP, dV, dK). Codes as attn_bwd.hip reads them: c < 2n/128 is dQ
// query tile c, otherwise dK/dV key tile c - 2n/128.
void bwd_order(bd3::BwdArgs& a, bool dq, bool dkdv) {
  const int r = 2 * a.n / 128;
  // With both kinds in the launch and a block size dividing 32, the noisy
  // key tiles' diagonal blocks are formed by the dQ items of the same rows
  // (see attn_bwd.hip), so the dK/dV items are the clean key tiles only.
  a.fold_diag = dq && dkdv && 32 % a.bs == 0;
  a.first_code = dq ? 0 : r;
  a.n_items = (dq ? r : 0) + (dkdv ? (a.fold_diag ? r / 2 : r) : 0);
  if (a.n_items > bd3::kBwdOrderMax) return;  // the kernel walks the codes in order
  int cost[2 * bd3::kBwdOrderMax], codes[bd3::kBwdOrderMax];
  for (int i = 0; i < a.n_items; ++i) {
    const int c = a.first_code + i;
    codes[i] = c;
    if (c < r) {
      const int q0 = ((c & 1) ? 0 : a.n) + (r / 2 - 1 - (c >> 1)) * 128;
      const bd3::KeyRanges kr = bd3::train_key_ranges(q0, 128, a.n, a.bs, 64);
      cost[c] = 3 * ((kr.t1 - kr.t0) + (kr.t3 - kr.t2)) + (a.fold_diag && (c & 1) ? 3 : 0);
    } else {
      const int kt = c - r;
      const int k0 = kt < r / 2 ? a.n + kt * 128 : (kt - r / 2) * 128;
      const bd3::KeyRanges qr = bd3::train_query_ranges(k0, 128, a.n, a.bs, 64);
      cost[c] = 4 * ((qr.t1 - qr.t0) + (qr.t3 - qr.t2));
    }
  }
  std::stable_sort(codes, codes + a.n_items, [&](int x, int y) { return cost[x] > cost[y]; });
  for (int i = 0; i < a.n_items; ++i) a.order[i] = (uint16_t)codes[i];
}

// Above this many queries the decode call runs the prefill kernel (128-row
// query tiles sharing each K / V tile; the decode kernels re-read the keys
// once per 32 rows).
constexpr int kPrefillMinQ = 65;

// Splits for the prefill kernel: none when the (row tile, batch*head) items
// alone fill half of the GPU's workgroup slots (4 per CU on 256 CUs);
// otherwise as few as keep the longest item (one split of one 128-row tile)
// under the grid's total work spread over those slots, with kLoneTile = the
// cost of a 64-key tile in a workgroup running alone on its CU relative to
// one of four sharing it. Work is counted in 64-key tiles at block size 1
// (the most keys any block size allows). Fitted to 1-16 splits over ten
// shapes (caches evicted): 482 us in total against 476 for the best split of
// each, e.g. the 3088-token prefill 40.2 us at 4 splits (best 38.5 at 6),
// 32 x 128 queries over 4112 keys 89.3 us at 2.
int32_t prefill_auto_splits(int32_t batch, int32_t heads, int32_t q_len, int32_t kv_len) {
  constexpr double kSlots = 1024.0, kLoneTile = 0.5;
  const int row_tiles = (q_len + 127) / 128;
  if ((int64_t)batch * heads * row_tiles >= (int64_t)kSlots / 2) return 1;
  int64_t tiles = 0;
  for (int t = 0; t < row_tiles; ++t) {
    const int64_t e = (int64_t)kv_len - q_len + (128 * (t + 1) < q_len ? 128 * (t + 1) : q_len);
    tiles += (e + 63) / 64;
  }
  tiles *= (int64_t)batch * heads;
  double longest = (double)tiles / kSlots / kLoneTile;  // tiles one item may take
  if (longest < 4.0) longest = 4.0;
  const int64_t kv_tiles = ((int64_t)kv_len + 63) / 64;
  int64_t s = (int64_t)((double)kv_tiles / longest + 0.999999);
  if (s < 1) s = 1;
  if (s > 64) s = 64;
  return (int32_t)s;
}

int32_t auto_splits(int32_t batch, int32_t heads, int32_t q_len, int32_t kv_len) {
  if (q_len >= kPrefillMinQ) return prefill_auto_splits(batch, heads, q_len, kv_len);
  // A cached step (q_len <= 16, 16-row tiles): at least one workgroup per CU
  // on a 256-CU part; beyond that more splits only add partial traffic and a
  // merge launch. Measured at configs[3] (384 workgroups at one split): 66 us
  // at one split, 68 us at two (including the merge), 71 us at three. Its
  // merge of up to 32 splits is one memory round trip, so it pays for splits
  // down to 128 keys, up to 16 of them: 16 queries over a 3584-token cache,
  // batch 1, 12 heads: 12.7 us at 7 splits, 11.8 at 14 or 16, 12.5-12.9 at
  // 21-28; over 8192 tokens 16.2 / 13.9 / 15.3 / 15.2 us at 8 / 16 / 22 /
  // 32; batch 2, 12 heads, over 1024 tokens 11.6 / 11.1 / 10.5 / 11.0 us at
  // 2 / 4 / 8 / 11.
  // 32-row tiles (16 < q_len <= 64), whose workgroups take 8 waves when there
  // are fewer than 256 of them: about 128 workgroups, and at least 1024 keys
  // per split once there are 64 or more tiles (512 with fewer; the merge
  // launch costs more than a shorter chain saves): at 8 x 12 heads, q_len 32,
  // 2048 keys 16.8 us at 2 splits vs 17.8 at 1 and 19.3 at 3; 1024 keys 12.0
  // at 1 vs 13.7 at 2; batch 1 over 3584 keys 13.3-13.6 at 7-8 splits.
  const int64_t base = (int64_t)batch * heads * decode_q_tiles(q_len);
  const int64_t target = q_len <= 16 ? 256 : 128;
  int64_t s = (target + base - 1) / base;
  if (q_len <= 16 && s > 16) s = 16;
  const int min_keys = q_len <= 16 ? 128 : (base >= 64 ? 1024 : 512);
  const int64_t max_by_len = kv_len / min_keys > 0 ? kv_len / min_keys : 1;
  if (s > max_by_len) s = max_by_len;
  if (s < 1) s = 1;
  return (int32_t)s;
}

int run_decode(const void* q, const void* k, const void* v, void* o, int32_t batch,
               int32_t heads, int32_t q_len, int32_t kv_len, int32_t block_size,
               int32_t n_splits, const int64_t* strides, float scale, void* workspace,
               size_t workspace_bytes, void* stream) {
  if (int st = check_scale(scale)) return st;
  const int q_tiles = decode_q_tiles(q_len);
  const size_t need = bd3_decode_workspace_bytes(batch, heads, q_len, kv_len, bd3::kHeadDim, n_splits);
  if (workspace_bytes < need)
    return fail(BD3_EINVAL, "workspace too small: %zu < %zu bytes", workspace_bytes, need);
  if (need > 0 && (workspace == nullptr || !aligned16(workspace)))
    return fail(BD3_EINVAL, "workspace must be a 16-byte aligned device pointer");
  bd3::DecodeArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.o = static_cast<uint16_t*>(o);
  const size_t po_bytes = (size_t)batch * heads * q_tiles * n_splits * kDecodeQT * bd3::kHeadDim * 4;
  a.part_o = n_splits > 1 ? static_cast<float*>(workspace) : nullptr;
  a.part_lse = n_splits > 1 ? reinterpret_cast<float*>(static_cast<char*>(workspace) + align256(po_bytes))
                            : nullptr;
  a.sq = s3(strides);
  a.sk = s3(strides + 3);
  a.sv = s3(strides + 6);
  a.so = s3(strides + 9);
  a.heads = heads;
  a.bh = batch * heads;
  a.q_len = q_len;
  a.kv_len = kv_len;
  a.bs = block_size;
  a.n_splits = n_splits;
  // Split length: ceil(kv_len / n_splits) rounded up to whole 32-key chunks
  // (the kernels' load and compute unit; a split ending mid-chunk would load
  // the chunk's other half twice).
  int sl = (kv_len + n_splits - 1) / n_splits;
  sl = (sl + 31) / 32 * 32;
  a.split_len = sl;
  a.q_tiles = q_tiles;
  // One workgroup per split, unless that overfills the GPU: then (cached
  // steps, q_len <= 16) a workgroup computes several consecutive splits and
  // merges their partials on chip, so that only enough workgroups for one
  // per CU remain (at configs[3], 384 heads: every split count gives one
  // workgroup per head, no partials in memory, no merge pass).
  a.groups = n_splits;
  a.splits_per_group = 1;
  const int64_t units = (int64_t)batch * heads * q_tiles;
  if (q_len <= 16 && n_splits >= 4 && units * n_splits > 512) {
    const int64_t g = (256 + units - 1) / units;
    const int per = (int)((n_splits + g - 1) / g);
    if (per >= 4) {
      a.splits_per_group = per;
      a.groups = (n_splits + per - 1) / per;
    }
  }
  a.scale_log2 = scale * bd3::kLog2e;
  if (q_len >= kPrefillMinQ) {
    // 128-row tiles, splits of whole 64-key tiles; partials in the same
    // layout (one slot per 32-row tile and split).
    for (int i = 1; i <= 2; ++i) {
      const int st = check_dma_stride(strides + 3 * i, i == 1 ? "k" : "v");
      if (st) return st;
    }
    int pl = (kv_len + n_splits - 1) / n_splits;
    a.split_len = (pl + 63) / 64 * 64;
    a.groups = n_splits;
    a.splits_per_group = 1;
    return hip_status(bd3::launch_prefill(a, static_cast<hipStream_t>(stream)), "prefill launch");
  }
  return hip_status(bd3::launch_decode(a, kDecodeQT, static_cast<hipStream_t>(stream)), "decode launch");
}

}  // namespace

extern "C" {

int bd3_abi_version(void) { return BD3_ABI_VERSION; }

const char* bd3_last_error(void) { return g_err.c_str(); }

int bd3_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse, int32_t batch,
                 int32_t heads, int32_t n, int32_t head_dim, int32_t block_size,
                 const int64_t* strides, float scale, void* stream) {
  if (batch < 1 || heads < 1) return fail(BD3_EINVAL, "batch and heads must be >= 1");
  if (head_dim != bd3::kHeadDim) return fail(BD3_EINVAL, "head_dim must be 64, got %d", head_dim);
  if (n < 128 || n % 128 != 0)
    return fail(BD3_EINVAL, "n (half the sequence) must be a positive multiple of 128, got %d", n);
  if (block_size < 1) return fail(BD3_EINVAL, "block_size must be >= 1");
  if (strides == nullptr) return fail(BD3_EINVAL, "strides is NULL");
  const char* names[4] = {"q", "k", "v", "o"};
  const void* ptrs[4] = {q, k, v, o};
  for (int i = 0; i < 4; ++i) {
    int st = check_tensor(ptrs[i], strides + 3 * i, names[i]);
    if (st) return st;
  }
  for (int i = 1; i < 3; ++i) {
    int st = check_dma_stride(strides + 3 * i, names[i]);
    if (st) return st;
  }
  if (lse == nullptr) return fail(BD3_EINVAL, "lse is NULL");
  if (int st = check_scale(scale)) return st;
  bd3::FwdArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.o = static_cast<uint16_t*>(o);
  a.lse = lse;
  a.sq = s3(strides);
  a.sk = s3(strides + 3);
  a.sv = s3(strides + 6);
  a.so = s3(strides + 9);
  a.heads = heads;
  a.bh = batch * heads;
  a.n = n;
  a.bs = block_size;
  a.scale_log2 = scale * bd3::kLog2e;
  return hip_status(bd3::launch_attn_fwd(a, static_cast<hipStream_t>(stream)), "attn_fwd launch");
}

size_t bd3_attn_bwd_workspace_bytes(int32_t batch, int32_t heads, int32_t n, int32_t head_dim) {
  if (batch < 1 || heads < 1 || n < 1 || head_dim < 1) return 0;
  return align256(2 * (size_t)batch * heads * 2 * n * sizeof(float));  // Delta, -L / scale
}

int bd3_attn_bwd_dq(const void* q, const void* k, const void* v, const void* o, const void* dout,
                    const float* lse, void* dq, float* delta, int32_t batch, int32_t heads, int32_t n,
                    int32_t head_dim, int32_t block_size, const int64_t* strides, float scale,
                    void* stream) {
  int st = check_bwd_shape(batch, heads, n, head_dim, block_size, strides);
  if (st) return st;
  if ((st = check_scale(scale))) return st;
  const char* names[6] = {"q", "k", "v", "o", "dout", "dq"};
  const void* ptrs[6] = {q, k, v, o, dout, dq};
  for (int i = 0; i < 6; ++i)
    if ((st = check_tensor(ptrs[i], strides + 3 * i, names[i]))) return st;
  for (int i = 1; i < 3; ++i)
    if ((st = check_dma_stride(strides + 3 * i, names[i]))) return st;
  if (lse == nullptr || delta == nullptr) return fail(BD3_EINVAL, "lse and delta must be non-NULL");
  bd3::BwdArgs a = bwd_args(q, k, v, o, dout, lse, dq, nullptr, nullptr, delta, batch, heads, n,
                            block_size, scale);
  a.sq = s3(strides);
  a.sk = s3(strides + 3);
  a.sv = s3(strides + 6);
  a.so = s3(strides + 9);
  a.sdo = s3(strides + 12);
  a.sdq = s3(strides + 15);
  bwd_order(a, true, false);
  if ((st = hip_status(bd3::launch_attn_bwd_delta(a, static_cast<hipStream_t>(stream)), "attn_bwd Delta launch")))
    return st;
  return hip_status(bd3::launch_attn_bwd_items(a, static_cast<hipStream_t>(stream)), "attn_bwd_dq launch");
}

int bd3_attn_bwd_dkdv(const void* q, const void* k, const void* v, const void* dout, const float* lse,
                      const float* delta, void* dk, void* dv, int32_t batch, int32_t heads, int32_t n,
                      int32_t head_dim, int32_t block_size, const int64_t* strides, float scale,
                      void* stream) {
  int st = check_bwd_shape(batch, heads, n, head_dim, block_size, strides);
  if (st) return st;
  if ((st = check_scale(scale))) return st;
  const char* names[6] = {"q", "k", "v", "dout", "dk", "dv"};
  const void* ptrs[6] = {q, k, v, dout, dk, dv};
  for (int i = 0; i < 6; ++i)
    if ((st = check_tensor(ptrs[i], strides + 3 * i, names[i]))) return st;
  for (int i : {0, 3})
    if ((st = check_dma_stride(strides + 3 * i, names[i]))) return st;
  if (lse == nullptr || delta == nullptr) return fail(BD3_EINVAL, "lse and delta must be non-NULL");
  bd3::BwdArgs a = bwd_args(q, k, v, nullptr, dout, lse, nullptr, dk, dv, const_cast<float*>(delta),
                            batch, heads, n, block_size, scale);
  a.sq = s3(strides);
  a.sk = s3(strides + 3);
  a.sv = s3(strides + 6);
  a.sdo = s3(strides + 9);
  a.sdk = s3(strides + 12);
  a.sdv = s3(strides + 15);
  bwd_order(a, false, true);
  return hip_status(bd3::launch_attn_bwd_items(a, static_cast<hipStream_t>(stream)), "attn_bwd_dkdv launch");
}

int bd3_attn_bwd_delta(const void* o, const void* dout, const float* lse, float* delta, int32_t batch,
                       int32_t heads, int32_t n, int32_t head_dim, int32_t block_size, const int64_t* strides,
                       float scale, void* stream) {
  int st = check_bwd_shape(batch, heads, n, head_dim, block_size, strides);
  if (st) return st;
  if ((st = check_scale(scale))) return st;
  const char* names[2] = {"o", "dout"};
  const void* ptrs[2] = {o, dout};
  for (int i = 0; i < 2; ++i)
    if ((st = check_tensor(ptrs[i], strides + 3 * i, names[i]))) return st;
  if (lse == nullptr || delta == nullptr) return fail(BD3_EINVAL, "lse and delta must be non-NULL");
  bd3::BwdArgs a = bwd_args(nullptr, nullptr, nullptr, o, dout, lse, nullptr, nullptr, nullptr, delta, batch, heads,
                            n, block_size, scale);
  a.so = s3(strides);
  a.sdo = s3(strides + 3);
  return hip_status(bd3::launch_attn_bwd_delta(a, static_cast<hipStream_t>(stream)), "attn_bwd Delta launch");
}

int bd3_attn_bwd_main(const void* q, const void* k, const void* v, const void* dout, const float* lse,
                      const float* delta, void* dq, void* dk, void* dv, int32_t batch, int32_t heads, int32_t n,
                      int32_t head_dim, int32_t block_size, const int64_t* strides, float scale, void* stream) {
  int st = check_bwd_shape(batch, heads, n, head_dim, block_size, strides);
  if (st) return st;
  if ((st = check_scale(scale))) return st;
  const char* names[7] = {"q", "k", "v", "dout", "dq", "dk", "dv"};
  const void* ptrs[7] = {q, k, v, dout, dq, dk, dv};
  for (int i = 0; i < 7; ++i)
    if ((st = check_tensor(ptrs[i], strides + 3 * i, names[i]))) return st;
  for (int i : {0, 1, 2, 3})
    if ((st = check_dma_stride(strides + 3 * i, names[i]))) return st;
  if (lse == nullptr || delta == nullptr) return fail(BD3_EINVAL, "lse and delta must be non-NULL");
  bd3::BwdArgs a = bwd_args(q, k, v, nullptr, dout, lse, dq, dk, dv, const_cast<float*>(delta), batch, heads, n,
                            block_size, scale);
  a.sq = s3(strides);
  a.sk = s3(strides + 3);
  a.sv = s3(strides + 6);
  a.sdo = s3(strides + 9);
  a.sdq = s3(strides + 12);
  a.sdk = s3(strides + 15);
  a.sdv = s3(strides + 18);
  bwd_order(a, true, true);
  return hip_status(bd3::launch_attn_bwd_items(a, static_cast<hipStream_t>(stream)), "attn_bwd launch");
}

int bd3_attn_bwd(const void* q, const void* k, const void* v, const void* o, const void* dout,
                 const float* lse, void* dq, void* dk, void* dv, void* workspace,
                 size_t workspace_bytes, int32_t batch, int32_t heads, int32_t n,
                 int32_t head_dim, int32_t block_size, const int64_t* strides, float scale,
                 void* stream) {
  int st = check_bwd_shape(batch, heads, n, head_dim, block_size, strides);
  if (st) return st;
  if ((st = check_scale(scale))) return st;
  const char* names[8] = {"q", "k", "v", "o", "dout", "dq", "dk", "dv"};
  const void* ptrs[8] = {q, k, v, o, dout, dq, dk, dv};
  for (int i = 0; i < 8; ++i)
    if ((st = check_tensor(ptrs[i], strides + 3 * i, names[i]))) return st;
  // Both stages' direct-load operands (dQ: k, v; dK/dV: q, dout) are checked
  // before the first launch, so a refused call writes nothing.
  for (int i : {0, 1, 2, 4})
    if ((st = check_dma_stride(strides + 3 * i, names[i]))) return st;
  if (lse == nullptr) return fail(BD3_EINVAL, "lse is NULL");
  const size_t need = bd3_attn_bwd_workspace_bytes(batch, heads, n, head_dim);
  if (workspace == nullptr || !aligned16(workspace) || workspace_bytes < need)
    return fail(BD3_EINVAL, "workspace must be a 16-byte aligned buffer of >= %zu bytes", need);
  // The Delta pass, then every dQ and dK/dV item in one launch.
  float* delta = static_cast<float*>(workspace);
  const int64_t* S = strides;  // q, k, v, o, dout, dq, dk, dv
  const int64_t delta_strides[6] = {S[9], S[10], S[11], S[12], S[13], S[14]};
  const int64_t main_strides[21] = {S[0],  S[1],  S[2],  S[3],  S[4],  S[5],  S[6],  S[7],  S[8],  S[12], S[13],
                                    S[14], S[15], S[16], S[17], S[18], S[19], S[20], S[21], S[22], S[23]};
  if ((st = bd3_attn_bwd_delta(o, dout, lse, delta, batch, heads, n, head_dim, block_size, delta_strides, scale,
                               stream)))
    return st;
  return bd3_attn_bwd_main(q, k, v, dout, lse, delta, dq, dk, dv, batch, heads, n, head_dim, block_size,
                           main_strides, scale, stream);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Backward without a caller workspace (bd3_attn_bwd_noalloc): the Delta and
// -L / scale planes live in `scratch`, a device array of this library that
// each GPU holds from the library's first use on it until the process ends.
// Host code never passes the array's name to a kernel (on the host it is a
// stand-in, not a device address): the address each device gives
// hipGetSymbolAddress is looked up once per device, with that device
// current, and only that address is used.
namespace {

constexpr size_t kScratchBytes = 2 * sizeof(float) * BD3_NOALLOC_MAX_ROWS;  // 8 MiB: 2 planes
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch`, looked up on the device's first
// call (the caller's current device is the device of `stream`, as for every
// entry point).
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_status(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(BD3_EINVAL, "device %d beyond the scratch table", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_status(e, "hipGetSymbolAddress(scratch)");
    if (ptr == nullptr) return fail(BD3_EHIP, "hipGetSymbolAddress(scratch) returned NULL");
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return BD3_OK;
}

}  // namespace

extern "C" {

int bd3_attn_bwd_noalloc(const void* q, const void* k, const void* v, const void* o, const void* dout,
                         const float* lse, void* dq, void* dk, void* dv, int32_t batch, int32_t heads,
                         int32_t n, int32_t head_dim, int32_t block_size, const int64_t* strides, float scale,
                         void* stream) {
  int st = check_bwd_shape(batch, heads, n, head_dim, block_size, strides);
  if (st) return st;
  if ((st = check_scale(scale))) return st;
  const size_t need = bd3_attn_bwd_workspace_bytes(batch, heads, n, head_dim);
  if (need > kScratchBytes)
    return fail(BD3_EINVAL,
                "bd3_attn_bwd_noalloc holds at most %d rows (batch * heads * 2n = %lld): use bd3_attn_bwd with a "
                "workspace", BD3_NOALLOC_MAX_ROWS, (long long)batch * heads * 2 * n);
  void* ws = nullptr;
  if ((st = scratch_address(&ws))) return st;
  // Every element of both planes is written by the dQ stage before the dK/dV
  // stage reads it, so nothing needs clearing between calls.
  return bd3_attn_bwd(q, k, v, o, dout, lse, dq, dk, dv, ws, kScratchBytes, batch, heads, n, head_dim,
                      block_size, strides, scale, stream);
}

int32_t bd3_decode_auto_splits(int32_t batch, int32_t heads, int32_t q_len, int32_t kv_len) {
  if (batch < 1 || heads < 1 || q_len < 1 || kv_len < 1) return 1;
  return auto_splits(batch, heads, q_len, kv_len);
}

size_t bd3_decode_workspace_bytes(int32_t batch, int32_t heads, int32_t q_len, int32_t kv_len,
                                  int32_t head_dim, int32_t n_splits) {
  if (batch < 1 || heads < 1 || q_len < 1 || kv_len < 1 || n_splits < 0) return 0;
  if (n_splits == 0) n_splits = auto_splits(batch, heads, q_len, kv_len);
  if (n_splits <= 1) return 0;
  const size_t slots = (size_t)batch * heads * decode_q_tiles(q_len) * n_splits * kDecodeQT;
  return align256(slots * head_dim * sizeof(float)) + align256(slots * sizeof(float));
}

int bd3_decode(const void* q, const void* k, const void* v, void* o, int32_t batch, int32_t heads,
               int32_t q_len, int32_t kv_len, int32_t head_dim, int32_t block_size,
               const int64_t* strides, float scale, void* workspace, size_t workspace_bytes,
               void* stream) {
  int st = check_common_decode(q, k, v, o, batch, heads, q_len, kv_len, head_dim, block_size, strides);
  if (st) return st;
  const int32_t ns = auto_splits(batch, heads, q_len, kv_len);
  return run_decode(q, k, v, o, batch, heads, q_len, kv_len, block_size, ns, strides, scale,
                    workspace, workspace_bytes, stream);
}

int bd3_decode_splitkv(const void* q, const void* k, const void* v, void* o, int32_t batch,
                       int32_t heads, int32_t q_len, int32_t kv_len, int32_t head_dim,
                       int32_t block_size, int32_t n_splits, const int64_t* strides, float scale,
                       void* workspace, size_t workspace_bytes, void* stream) {
  int st = check_common_decode(q, k, v, o, batch, heads, q_len, kv_len, head_dim, block_size, strides);
  if (st) return st;
  if (n_splits < 1 || n_splits > kv_len)
    return fail(BD3_EINVAL, "n_splits must be in [1, kv_len], got %d", n_splits);
  return run_decode(q, k, v, o, batch, heads, q_len, kv_len, block_size, n_splits, strides, scale,
                    workspace, workspace_bytes, stream);
}

int bd3_qkv_rope(const void* qkv, const int64_t* qkv_strides, int32_t batch, int32_t seq,
                 int32_t heads, int32_t head_dim, const int64_t* positions, int32_t pos0,
                 const float* sin_table, const float* cos_table, int32_t max_pos, void* q_out,
                 void* k_out, void* v_out, const int64_t* out_strides, void* stream) {
  if (batch < 1 || heads < 1 || seq < 0) return fail(BD3_EINVAL, "need batch >= 1, heads >= 1, seq >= 0");
  if (head_dim != bd3::kHeadDim) return fail(BD3_EINVAL, "head_dim must be 64, got %d", head_dim);
  if (qkv == nullptr || !aligned16(qkv)) return fail(BD3_EINVAL, "qkv must be a 16-byte aligned device pointer");
  if (qkv_strides == nullptr || out_strides == nullptr) return fail(BD3_EINVAL, "strides is NULL");
  for (int i = 0; i < 2; ++i)
    if (qkv_strides[i] < 0 || qkv_strides[i] % 8 != 0)
      return fail(BD3_EINVAL, "qkv stride[%d]=%lld must be a non-negative multiple of 8", i,
                  (long long)qkv_strides[i]);
  if (sin_table == nullptr || cos_table == nullptr || !aligned16(sin_table) || !aligned16(cos_table))
    return fail(BD3_EINVAL, "sin_table and cos_table must be 16-byte aligned device pointers");
  if (max_pos < 1) return fail(BD3_EINVAL, "max_pos must be >= 1");
  if (positions == nullptr && (pos0 < 0 || (int64_t)pos0 + seq > max_pos))
    return fail(BD3_EINVAL, "positions %d .. %lld exceed the RoPE table (max_pos %d)", pos0,
                (long long)pos0 + seq - 1, max_pos);
  const char* names[3] = {"q_out", "k_out", "v_out"};
  void* outs[3] = {q_out, k_out, v_out};
  for (int i = 0; i < 3; ++i) {
    int st = check_tensor(outs[i], out_strides + 3 * i, names[i]);
    if (st) return st;
  }
  bd3::QkvRopeArgs a;
  a.qkv = static_cast<const uint16_t*>(qkv);
  a.sx_b = qkv_strides[0];
  a.sx_s = qkv_strides[1];
  a.positions = positions;
  a.pos0 = pos0;
  a.sin_t = sin_table;
  a.cos_t = cos_table;
  a.max_pos = max_pos;
  a.q = static_cast<uint16_t*>(q_out);
  a.k = static_cast<uint16_t*>(k_out);
  a.v = static_cast<uint16_t*>(v_out);
  a.sq = s3(out_strides);
  a.sk = s3(out_strides + 3);
  a.sv = s3(out_strides + 6);
  a.heads = heads;
  a.seq = seq;
  a.total = (int64_t)batch * seq * 4 * heads;
  if (a.total >= ((int64_t)1 << 31))
    return fail(BD3_EINVAL, "batch * seq * heads too large (%lld work items, limit 2^31)", (long long)a.total);
  return hip_status(bd3::launch_qkv_rope(a, static_cast<hipStream_t>(stream)), "qkv_rope launch");
}

int bd3_kv_write(const void* k, const void* v, void* k_dst, void* v_dst, int32_t batch,
                 int32_t heads, int32_t seq, int32_t head_dim, const int64_t* strides,
                 void* stream) {
  if (batch < 1 || heads < 1 || seq < 0) return fail(BD3_EINVAL, "need batch >= 1, heads >= 1, seq >= 0");
  if (head_dim != bd3::kHeadDim) return fail(BD3_EINVAL, "head_dim must be 64, got %d", head_dim);
  if (strides == nullptr) return fail(BD3_EINVAL, "strides is NULL");
  const char* names[4] = {"k", "v", "k_dst", "v_dst"};
  const void* ptrs[4] = {k, v, k_dst, v_dst};
  for (int i = 0; i < 4; ++i) {
    int st = check_tensor(ptrs[i], strides + 3 * i, names[i]);
    if (st) return st;
  }
  bd3::KvWriteArgs a;
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.k_dst = static_cast<uint16_t*>(k_dst);
  a.v_dst = static_cast<uint16_t*>(v_dst);
  a.sk = s3(strides);
  a.sv = s3(strides + 3);
  a.skd = s3(strides + 6);
  a.svd = s3(strides + 9);
  a.batch = batch;
  a.heads = heads;
  a.seq = seq;
  a.total = 2 * (int64_t)batch * heads * seq * 8;
  return hip_status(bd3::launch_kv_write(a, static_cast<hipStream_t>(stream)), "kv_write launch");
}

int bd3_subs_sample(const void* logits, int64_t ld, int32_t logits_fp32, const int64_t* xt,
                    int64_t* out, int32_t rows, int32_t vocab, int32_t mask_index, double keep,
                    const double* u, uint64_t seed, uint64_t offset, void* stream) {
  if (rows < 0) return fail(BD3_EINVAL, "rows must be >= 0");
  if (vocab < 2) return fail(BD3_EINVAL, "vocab must be >= 2, got %d", vocab);
  if (mask_index < 0 || mask_index >= vocab)
    return fail(BD3_EINVAL, "mask_index %d outside [0, vocab = %d)", mask_index, vocab);
  if (ld < vocab) return fail(BD3_EINVAL, "row stride ld (%lld) < vocab (%d)", (long long)ld, vocab);
  if (logits_fp32 != 0 && logits_fp32 != 1) return fail(BD3_EINVAL, "logits_fp32 must be 0 (bf16) or 1 (fp32)");
  if (!(keep >= 0.0 && keep <= 1.0)) return fail(BD3_EINVAL, "keep (s / t) must lie in [0, 1]");
  if (rows > 0 && (logits == nullptr || xt == nullptr || out == nullptr))
    return fail(BD3_EINVAL, "logits, xt and out must be non-NULL");
  bd3::SubsArgs a;
  a.logits = logits;
  a.ld = ld;
  a.fp32 = logits_fp32;
  a.xt = xt;
  a.out = out;
  a.rows = rows;
  a.vocab = vocab;
  a.mask_index = mask_index;
  a.keep = keep;
  a.u = u;
  a.seed = seed;
  a.offset = offset;
  return hip_status(bd3::launch_subs_sample(a, static_cast<hipStream_t>(stream)), "subs_sample launch");
}

namespace {
int check_glue_common(int batch, int seq, int d_model, const int64_t* strides, int n_strides,
                      const int32_t* flags, int n_flags) {
  if (batch < 1 || seq < 0) return fail(BD3_EINVAL, "need batch >= 1 and seq >= 0");
  if (d_model < 8 || d_model % 8 != 0) return fail(BD3_EINVAL, "d_model must be a positive multiple of 8, got %d", d_model);
  if ((int64_t)batch * seq >= ((int64_t)1 << 31)) return fail(BD3_EINVAL, "batch * seq too large");
  if (strides == nullptr) return fail(BD3_EINVAL, "strides is NULL");
  for (int i = 0; i < n_strides; ++i)
    if (strides[i] < 0 || strides[i] % 8 != 0)
      return fail(BD3_EINVAL, "stride[%d]=%lld must be a non-negative multiple of 8", i, (long long)strides[i]);
  for (int i = 0; i < n_flags; ++i)
    if (flags[i] != 0 && flags[i] != 1) return fail(BD3_EINVAL, "dtype flags must be 0 (bf16) or 1 (fp32)");
  return BD3_OK;
}
int check_ptrs(const void* const* p, const char* const* names, int n) {
  for (int i = 0; i < n; ++i) {
    if (p[i] == nullptr) return fail(BD3_EINVAL, "%s is NULL", names[i]);
    if (!aligned16(p[i])) return fail(BD3_EINVAL, "%s must be 16-byte aligned", names[i]);
  }
  return BD3_OK;
}
}  // namespace

int bd3_ln_modulate(const void* x, int32_t x_fp32, const void* weight, int32_t weight_fp32,
                    const void* shift, const void* scale, int32_t mod_fp32, void* out,
                    int32_t out_fp32, int32_t batch, int32_t seq, int32_t d_model,
                    const int64_t* strides, float eps, void* stream) {
  const int32_t flags[4] = {x_fp32, weight_fp32, mod_fp32, out_fp32};
  int st = check_glue_common(batch, seq, d_model, strides, 5, flags, 4);
  if (st) return st;
  const void* ptrs[5] = {x, weight, shift, scale, out};
  const char* names[5] = {"x", "weight", "shift", "scale", "out"};
  if ((st = check_ptrs(ptrs, names, 5))) return st;
  if (!x_fp32 && !mod_fp32 && out_fp32)
    return fail(BD3_EINVAL, "bf16 x with bf16 shift / scale modulates in bf16: out must be bf16");
  if (!(eps >= 0.f)) return fail(BD3_EINVAL, "eps must be >= 0");
  if (d_model > 4096) return fail(BD3_EINVAL, "d_model must be <= 4096, got %d", d_model);
  bd3::GlueArgs a = {};
  a.x = x; a.weight = weight; a.shift = shift; a.scale = scale; a.out = out;
  a.x_fp32 = x_fp32; a.w_fp32 = weight_fp32; a.m_fp32 = mod_fp32; a.out_fp32 = out_fp32;
  a.rows = batch * seq; a.seq = seq > 0 ? seq : 1; a.d = d_model;
  a.sx_b = strides[0]; a.sx_s = strides[1]; a.sm_b = strides[2]; a.so_b = strides[3]; a.so_s = strides[4];
  a.eps = eps;
  return hip_status(bd3::launch_ln_modulate(a, static_cast<hipStream_t>(stream)), "ln_modulate launch");
}

int bd3_gate_residual(const void* x, int32_t x_fp32, const void* gate, int32_t gate_fp32,
                      const void* y, int32_t y_fp32, void* out, int32_t batch, int32_t seq,
                      int32_t d_model, const int64_t* strides, void* stream) {
  const int32_t flags[3] = {x_fp32, gate_fp32, y_fp32};
  int st = check_glue_common(batch, seq, d_model, strides, 7, flags, 3);
  if (st) return st;
  const void* ptrs[4] = {x, gate, y, out};
  const char* names[4] = {"x", "gate", "y", "out"};
  if ((st = check_ptrs(ptrs, names, 4))) return st;
  bd3::GlueArgs a = {};
  a.x = x; a.shift = gate; a.y = y; a.out = out;
  a.x_fp32 = x_fp32; a.m_fp32 = gate_fp32; a.y_fp32 = y_fp32;
  a.rows = batch * seq; a.seq = seq > 0 ? seq : 1; a.d = d_model;
  a.sx_b = strides[0]; a.sx_s = strides[1]; a.sm_b = strides[2]; a.sy_b = strides[3]; a.sy_s = strides[4];
  a.so_b = strides[5]; a.so_s = strides[6];
  return hip_status(bd3::launch_gate_residual(a, static_cast<hipStream_t>(stream)), "gate_residual launch");
}

int bd3_gate_residual_ln_modulate(const void* x, int32_t x_fp32, const void* gate, const void* y,
                                  int32_t y_fp32, void* x_out, const void* weight,
                                  int32_t weight_fp32, const void* shift, const void* scale,
                                  int32_t mod_fp32, void* out, int32_t out_fp32, int32_t batch,
                                  int32_t seq, int32_t d_model, const int64_t* strides, float eps,
                                  void* stream) {
  const int32_t flags[5] = {x_fp32, y_fp32, weight_fp32, mod_fp32, out_fp32};
  int st = check_glue_common(batch, seq, d_model, strides, 9, flags, 5);
  if (st) return st;
  const void* ptrs[8] = {x, gate, y, x_out, weight, shift, scale, out};
  const char* names[8] = {"x", "gate", "y", "x_out", "weight", "shift", "scale", "out"};
  if ((st = check_ptrs(ptrs, names, 8))) return st;
  const bool res_bf16 = !x_fp32 && !mod_fp32 && !y_fp32;
  if (res_bf16 && !mod_fp32 && out_fp32)
    return fail(BD3_EINVAL, "bf16 x_out with bf16 shift / scale modulates in bf16: out must be bf16");
  if (!(eps >= 0.f)) return fail(BD3_EINVAL, "eps must be >= 0");
  if (d_model > 4096) return fail(BD3_EINVAL, "d_model must be <= 4096, got %d", d_model);
  bd3::GlueArgs a = {};
  a.x = x; a.gate = gate; a.y = y; a.out_x = x_out;
  a.weight = weight; a.shift = shift; a.scale = scale; a.out = out;
  a.x_fp32 = x_fp32; a.y_fp32 = y_fp32; a.w_fp32 = weight_fp32; a.m_fp32 = mod_fp32; a.out_fp32 = out_fp32;
  a.rows = batch * seq; a.seq = seq > 0 ? seq : 1; a.d = d_model;
  a.sx_b = strides[0]; a.sx_s = strides[1]; a.sm_b = strides[2]; a.sy_b = strides[3]; a.sy_s = strides[4];
  a.sxo_b = strides[5]; a.sxo_s = strides[6]; a.so_b = strides[7]; a.so_s = strides[8];
  a.eps = eps;
  return hip_status(bd3::launch_gate_residual_ln_modulate(a, static_cast<hipStream_t>(stream)),
                    "gate_residual_ln_modulate launch");
}

int bd3_mask_dump(uint8_t* out, int32_t mode, int32_t rows, int32_t kv_len, int32_t block_size,
                  void* stream) {
  if (out == nullptr) return fail(BD3_EINVAL, "out is NULL");
  if (block_size < 1) return fail(BD3_EINVAL, "block_size must be >= 1");
  if (mode == 0) {
    if (rows < 1) return fail(BD3_EINVAL, "n must be >= 1");
  } else if (mode == 1) {
    if (rows < 1 || rows > kv_len) return fail(BD3_EINVAL, "need 1 <= q_len <= kv_len");
  } else {
    return fail(BD3_EINVAL, "mode must be 0 (training) or 1 (decode)");
  }
  return hip_status(bd3::launch_mask_dump(out, mode, rows, kv_len, block_size,
                                          static_cast<hipStream_t>(stream)),
                    "mask_dump launch");
}

int bd3_clock_probe(uint64_t* out, int32_t workgroups, int32_t iters, int64_t* wall_rate_khz,
                    void* stream) {
  if (out == nullptr || wall_rate_khz == nullptr) return fail(BD3_EINVAL, "out / wall_rate_khz is NULL");
  if (workgroups < 1 || workgroups > 65536) return fail(BD3_EINVAL, "workgroups must be in [1, 65536]");
  if (iters < 1) return fail(BD3_EINVAL, "iters must be >= 1");
  int dev = 0, rate = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&rate, hipDeviceAttributeWallClockRate, dev);
  if (e != hipSuccess) return hip_status(e, "wall clock rate query");
  *wall_rate_khz = rate;
  return hip_status(bd3::launch_clock_probe(out, workgroups, iters, static_cast<hipStream_t>(stream)),
                    "clock_probe launch");
}

int bd3_train_classify(int32_t n, int32_t block_size, int32_t q0, int32_t k0) {
  if (n < 32 || n % 32 != 0 || block_size < 1) return -1;
  if (q0 < 0 || k0 < 0 || q0 + 32 > 2 * n || k0 + 32 > 2 * n || q0 % 32 || k0 % 32) return -1;
  const bd3::RowGroup g = bd3::train_row_group(q0, 32, n, block_size);
  const int c = bd3::row_group_class(g, k0, 32, n);
  // The kernels' threshold form must give the same class.
  return bd3::bounds_class(bd3::row_group_bounds(g, n), k0, 32, n) == c ? c : -2;
}

int bd3_train_classify_keys(int32_t n, int32_t block_size, int32_t q0, int32_t k0) {
  if (n < 32 || n % 32 != 0 || block_size < 1) return -1;
  if (q0 < 0 || k0 < 0 || q0 + 32 > 2 * n || k0 + 32 > 2 * n || q0 % 32 || k0 % 32) return -1;
  const bd3::KeyGroup g = bd3::train_key_group(k0, 32, n, block_size);
  const int c = bd3::key_group_class(g, q0, 32, n);
  return bd3::bounds_class(bd3::key_group_bounds(g, n), q0, 32, n) == c ? c : -2;
}

int bd3_train_walk_class(int32_t n, int32_t block_size, int32_t g0, int32_t i, int32_t mode, int32_t* tile) {
  if (tile == nullptr || n < 128 || n % 128 != 0 || block_size < 1 || (mode != 0 && mode != 1)) return -1;
  if (g0 < 0 || g0 + 32 > 2 * n || g0 % 32 || i < 0) return -1;
  // mode 0: a 32-row group of a 128-row query tile walking key tiles (forward,
  // dQ); mode 1: a 32-key group of a 128-key tile walking query tiles (dK/dV).
  const bd3::KeyRanges kr = mode == 0 ? bd3::train_key_ranges(g0 - g0 % 128, 128, n, block_size, 64)
                                      : bd3::train_query_ranges(g0 - g0 % 128, 128, n, block_size, 64);
  const int n_first = kr.t1 - kr.t0, n_second = kr.t3 - kr.t2;
  if (i >= n_first + n_second) return -3;
  const bd3::ClassBounds b = mode == 0 ? bd3::row_group_bounds(bd3::train_row_group(g0, 32, n, block_size), n)
                                       : bd3::key_group_bounds(bd3::train_key_group(g0, 32, n, block_size), n);
  *tile = i < n_first ? kr.t0 + i : kr.t2 + (i - n_first);
  int out = 0;
  const int parts[3][2] = {{0, 64}, {0, 32}, {32, 32}};  // whole tile, first half, second half
  for (int p = 0; p < 3; ++p) {
    const bd3::WalkClasses w = bd3::walk_classes(b, kr.t0, n_first, kr.t2, n_second, n, 64, parts[p][0], parts[p][1]);
    const int c = bd3::walk_live(w, i, n_first) ? (bd3::walk_full(w, i, n_first) ? bd3::kFull : bd3::kPartial)
                                                : bd3::kNone;
    out |= c << (2 * p);
  }
  return out;
}

int bd3_train_intervals(int32_t n, int32_t block_size, int32_t index, int32_t mode, int32_t* out) {
  if (out == nullptr || n < 1 || block_size < 1 || index < 0 || index >= 2 * n) return -1;
  if (mode != 0 && mode != 1) return -1;
  const bd3::RowIntervals r = mode == 0 ? bd3::train_row_intervals(index, n, block_size)
                                        : bd3::train_col_intervals(index, n, block_size);
  out[0] = r.lo1;
  out[1] = r.hi1;
  out[2] = r.lo2;
  out[3] = r.hi2;
  return 0;
}

int bd3_train_tile_census(int32_t n, int32_t block_size, int64_t* out) {
  if (out == nullptr) return fail(BD3_EINVAL, "out is NULL");
  if (n < 128 || n % 128 != 0 || block_size < 1)
    return fail(BD3_EINVAL, "need n a positive multiple of 128 and block_size >= 1");
  int64_t useful = 0, full = 0, partial = 0, skipped = 0, exec_rows = 0, exec_keys = 0;
  for (int q = 0; q < 2 * n; ++q) useful += bd3::train_row_keys(q, n, block_size);
  // Query-stationary schedule (forward, dQ items): 128-row workgroups
  // visit the 64-key tiles of train_key_ranges; each 32-row wave computes
  // both 32-key halves of a tile when either holds a live pair for its rows
  // (the noisy diagonal aside, below).
  for (int q0 = 0; q0 < 2 * n; q0 += 128) {
    const bd3::KeyRanges kr = bd3::train_key_ranges(q0, 128, n, block_size, 64);
    const int ranges[2][2] = {{kr.t0, kr.t1}, {kr.t2, kr.t3}};
    for (int rg = 0; rg < 2; ++rg)
      for (int t = ranges[rg][0]; t < ranges[rg][1]; ++t)
        for (int w = 0; w < 4; ++w) {
          bool live = false;
          for (int sb = 0; sb < 2; ++sb) {
            const int c = bd3::train_class(q0 + 32 * w, 32, 64 * t + 32 * sb, 32, n, block_size);
            if (c == bd3::kNone) ++skipped;
            else if (c == bd3::kFull) ++full;
            else ++partial;
            live = live || c != bd3::kNone;
          }
          if (live) exec_rows += 32 * 64;
        }
  }
  // Key-stationary schedule (dK/dV items): 128-key workgroups visit the
  // 64-row tiles of train_query_ranges; each 32-key wave computes both 32-row
  // halves of a tile when either holds a live pair for its keys. A noisy key
  // tile with block size dividing 32 computes each wave's diagonal 32 x 32
  // block only.
  for (int k0 = 0; k0 < 2 * n; k0 += 128) {
    if (k0 < n && 32 % block_size == 0) {
      exec_keys += 4 * 32 * 32;
      continue;
    }
    const bd3::KeyRanges qr = bd3::train_query_ranges(k0, 128, n, block_size, 64);
    const int ranges[2][2] = {{qr.t0, qr.t1}, {qr.t2, qr.t3}};
    for (int rg = 0; rg < 2; ++rg)
      for (int t = ranges[rg][0]; t < ranges[rg][1]; ++t)
        for (int w = 0; w < 4; ++w) {
          const bd3::KeyGroup g = bd3::train_key_group(k0 + 32 * w, 32, n, block_size);
          if (bd3::key_group_class(g, 64 * t, 32, n) != bd3::kNone ||
              bd3::key_group_class(g, 64 * t + 32, 32, n) != bd3::kNone)
            exec_keys += 32 * 64;
        }
  }
  // The forward and the main launch's dQ items: with a block size dividing
  // 32 each noisy 32-row wave forms only its diagonal 32 x 32 block of its
  // one live diagonal key tile (a whole 32 x 64 tile in the count above).
  const int64_t exec_fwd = 32 % block_size == 0 ? exec_rows - (int64_t)(n / 32) * (32 * 64 - 32 * 32) : exec_rows;
  // With a block size a multiple of 16 both backward item kinds skip a 32 x
  // 32 block with no live pair, so they compute every live 32 x 32 block
  // once: 1024 pairs per full or partial sub-block counted above.
  const bool blocks32 = block_size % 16 == 0;
  const int64_t exec_dq = blocks32 ? 1024 * (full + partial) : exec_fwd;
  if (blocks32) exec_keys = 1024 * (full + partial);
  const int64_t nn = n, bs = block_size;
  out[0] = useful;
  out[1] = exec_fwd;
  out[2] = full;
  out[3] = partial;
  out[4] = skipped;
  out[5] = nn * nn + nn * bs;
  out[6] = exec_dq;
  out[7] = exec_keys;
  return BD3_OK;
}

}  // extern "C"
