// attn_bwd.hip - BD3-LM training attention backward for gfx950.
//
// Counterpart of BlockSparseFlashAttention.backward
// (kernels/BlockSparseFlashAttention.py:508-562): the Delta torch op (:525),
// block_sparse_attention_bwd_dq_kern (:368-452) and
// block_sparse_attention_dk_dv_bwd_kern (:212-328). Per live pair:
//   P  = exp(S*scale - L)            (S = Q K^T, L the forward's lse)
//   dV = P^T dO,  dP = dO V^T,  dS = P o (dP - Delta),  Delta = rowsum(dO o O)
//   dK = scale * dS^T Q,  dQ = scale * dS K
// Two launches. attn_bwd_delta_kernel forms Delta = rowsum(dO o O) (the
// reference's separate op) and each row's -L / scale. attn_bwd_kernel then
// runs every work item of the reference's two kernels in one launch: dQ
// items own query rows and form dQ, dK/dV items own keys and form dK, dV;
// both recompute S and dP. Neither kind needs atomics or a transposed copy
// of dS, results are deterministic, and as both kinds only read the Delta
// pass's planes the launch orders them freely: longest first (a host-built
// table), so it has one start-up and one tail.
//
// dq_item (query-stationary, the forward's schedule): 4 waves of 32 rows. Q
//   and dO rows live in registers as B operands; K, V key tiles come through
//   LDS. S^T = K Q^T and dP^T = V dO^T put one row per lane, so L and Delta
//   are per-lane scalars; dQ^T += K^T dS^T reads K^T from the LDS tile with
//   ds_read_b64_tr_b16. The two 32-key blocks of a tile run one after the
//   other, each straight into dQ.
// dkdv_item (key-stationary): 4 waves of 32 keys. K and V rows live in
//   registers as B operands of S = Q K^T and dP = dO V^T, which put one key
//   per lane; query tiles (Q, dO, -L / scale, Delta) come through LDS.
//   dV += P^T dO and dK += dS^T Q take P^T / dS^T straight from registers and
//   dO / Q transposed from LDS; the two 32-row blocks of a tile run one after
//   the other, so three waves fit a SIMD next to the dQ items. dK, dV are
//   written through LDS as 16-byte rows.
// With a block size a multiple of 16 (MASK16) a partial block's mask is one
//   test per 16-wide strip, entered as the exponent's addend (-inf for an
//   invisible strip), and a block with no live pair for the wave is skipped.
// Noisy key tiles with a block size dividing 32 (a noisy key is seen only by
//   the noisy rows of its own block, so only the tile's diagonal 32 x 32
//   blocks are live): in a launch with both kinds they get no dK/dV item;
//   the dQ item of the same 128 rows walks its two diagonal key tiles last
//   and stops its loop before them: from their K / V still in the ring and
//   its own Q / dO rows each wave forms its diagonal block once and takes
//   its rows' dQ and those keys' dK and dV from it (diag_block). Alone (the
//   dK/dV stage), each such tile is an item whose waves compute only their
//   diagonal block.
// Every score is the exact fp32 dot product of the bf16 rows; scale and
// log2(e) are applied in fp32 (dQ: one FMA per element; dK/dV: the chain
// starts from -L / scale and the result is scaled by scale * log2(e) in the
// exponent's FMA).
// Both item kinds load their tiles global -> LDS with global_load_lds into
// three-stage rings of swizzled tiles (bd3_swz.h), two tiles ahead, with one
// counted vmcnt wait and barrier per tile, in one LDS buffer of the larger
// ring's size.
#include "bd3_device.h"
#include "bd3_launch.h"
#include "bd3_mask.h"
#include "bd3_swz.h"
#include "bd3_tile.h"

#ifndef BD3_DQ_STAGES
#define BD3_DQ_STAGES 3
#endif

namespace bd3 {
namespace {

// ---------------------------------------------------------------------------
// Key-stationary dK/dV. The query tiles (Q, dO and the rows' L and Delta) go
// global -> LDS with global_load_lds into a three-stage ring of swizzled
// tiles, two tiles ahead. Every live tile runs one code path over both of its
// 32-row blocks, one after the other (a scheduling barrier between them, so
// one block's chains are live at a time); a block that is not fully visible
// to the wave's keys is masked in place (MASK16: block size a multiple of 16,
// two tests per lane).
// Stage layout of the dK/dV ring (bytes): Q tile [0, 8K), dO tile [8K, 16K),
// row scalars [16K, 17K): -L / scale of the 64 rows, then Delta, then both
// again (the load that fetches them writes 1 KB).
constexpr int kDkdvStages = 3;
constexpr int kDkdvStageBytes = 4 * kSwTile + 1024;
constexpr int kDkdvLdsBytes = kDkdvStages * kDkdvStageBytes;
constexpr int kDqStages = BD3_DQ_STAGES;
constexpr int kDqLdsBytes = kDqStages * 2 * kSwTile * 2;  // [stage][K | V] tiles
constexpr int kBwdLdsBytes = kDkdvLdsBytes > kDqLdsBytes ? kDkdvLdsBytes : kDqLdsBytes;

// dK/dV epilogue (every wave is past its last barrier, no load in flight):
// each wave transposes its 32 keys x 64 d of dK, then dV, through its own
// padded LDS slice into row-major bf16, then writes 16-byte row chunks.
__device__ __forceinline__ void dkdv_store(const BwdArgs& a, __bf16* tile, int b, int h, int kw, int lane,
                                           const f32x16 (&dk)[2], const f32x16 (&dv)[2]) {
  const int l32 = lane & 31;
  const int g = lane >> 5;
  uint16_t* outs[2] = {a.dk + b * a.sdk.b + h * a.sdk.h, a.dv + b * a.sdv.b + h * a.sdv.h};
  const int64_t ostr[2] = {a.sdk.s, a.sdv.s};
#pragma unroll
  for (int which = 0; which < 2; ++which) {
    const float mul = which == 0 ? -a.scale : 1.f;  // dK was accumulated from -dS
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int krow = 8 * (r >> 2) + 4 * g + (r & 3);
        const float x = (which == 0 ? dk[db][r] : dv[db][r]) * mul;
        tile[krow * kLdsStride + 32 * db + l32] = (__bf16)x;
      }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = (lane >> 3) + 8 * j;
      const u32x4 v = *reinterpret_cast<const u32x4*>(&tile[row * kLdsStride + 8 * (lane & 7)]);
      st16(outs[which] + (int64_t)(kw + row) * ostr[which] + 8 * (lane & 7), v);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
  }
}

// One dK/dV item: key tile `rank` (clean key tiles 0 .. n/128 - 1 first, the
// heaviest: clean keys are seen by the most rows; then the noisy ones) of
// (batch*head) bh, with the ring in `smem` (kDkdvLdsBytes).
// DIAG: a noisy key tile with a block size dividing 32, whose two query tiles
// are its own 128 rows: wave w's keys are seen only by the rows of 32-row
// block w % 2 of tile w / 2, so each wave computes that one block (exactly
// what the tile loop accumulates; its other blocks contribute zeros).
template <bool MASK16, bool DIAG>
__device__ __forceinline__ void dkdv_item(const BwdArgs& a, __bf16* smem, int bh, int rank) {
  constexpr int kBK = 128;  // keys per workgroup: 4 waves x 32
  constexpr int kStages = kDkdvStages;
  constexpr int kStageBytes = kDkdvStageBytes;

  const int tid = wi_x();
  const int lane = tid & 63;
  const int wave = wave_uniform(tid >> 6);
  const int l32 = lane & 31;
  const int g = lane >> 5;

  const int tiles_half = a.n / kBK;
  const int k0 = rank < tiles_half ? a.n + rank * kBK : (rank - tiles_half) * kBK;
  struct {
    int bh, b, h;
  } bo = {bh, bh / a.heads, bh - (bh / a.heads) * a.heads};

  const uint16_t* qp = uniform_ptr(a.q + bo.b * a.sq.b + bo.h * a.sq.h);
  const uint16_t* dop = uniform_ptr(a.dout + bo.b * a.sdo.b + bo.h * a.sdo.h);
  const uint16_t* kp = a.k + bo.b * a.sk.b + bo.h * a.sk.h;
  const uint16_t* vp = a.v + bo.b * a.sv.b + bo.h * a.sv.h;
  const int64_t rowbase = (int64_t)bo.bh * 2 * a.n;

  const int kw = k0 + 32 * wave;
  const int key = kw + l32;
  bf16x8 kreg[4], vreg[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    kreg[c] = __builtin_bit_cast(bf16x8, ld16(kp + (int64_t)key * a.sk.s + 16 * c + 8 * g));
    vreg[c] = __builtin_bit_cast(bf16x8, ld16(vp + (int64_t)key * a.sv.s + 16 * c + 8 * g));
  }

  const KeyRanges qr = train_query_ranges(k0, kBK, a.n, a.bs, kSwRows);
  const int t0 = wave_uniform(qr.t0), t2 = wave_uniform(qr.t2);
  const int n_first = wave_uniform(qr.t1 - qr.t0);
  const int n_tiles = n_first + wave_uniform(qr.t3 - qr.t2);
  auto tile_of = [&](int i) { return i < n_first ? t0 + i : t2 + (i - n_first); };
  // Wave w fills 1 KB blocks 2w, 2w+1 (rows 16w .. 16w+15) of the Q and dO
  // tiles; wave 0 also fetches the row scalars: lane L reads 16 bytes of L
  // (L % 32 < 16) or Delta, rows 4 (L % 16) .. +3.
  uint32_t qoff[2], dooff[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int r = 16 * wave + 8 * j + (lane >> 3);
    const int ch = 8 * ((lane & 7) ^ swz(r));
    qoff[j] = (uint32_t)(2 * (r * (int)a.sq.s + ch));
    dooff[j] = (uint32_t)(2 * (r * (int)a.sdo.s + ch));
  }
  // L comes as -L / scale, the second plane of the delta buffer (written by the Delta pass).
  const float* scal_src = ((lane & 16) ? a.delta : a.delta + (int64_t)a.bh * 2 * a.n) + rowbase + 4 * (lane & 15);
  const int64_t qstep = (int64_t)kSwRows * a.sq.s, dostep = (int64_t)kSwRows * a.sdo.s;
  const uint32_t lds0 = lds_addr(&smem[0]);
  // Sources of the next tile to request, walked tile by tile (requests are
  // made in order: tile_of(0), tile_of(1), ...).
  TileWalk walk(t0, n_first, t2);
  TilePtr qn(qp, 2 * qstep, t0, n_first, t2), don(dop, 2 * dostep, t0, n_first, t2);
  auto issue = [&](int stage) {
    const uint32_t st = lds0 + (uint32_t)(stage * kStageBytes) + (uint32_t)wave * 2048u;
#pragma unroll
    for (int j = 0; j < 2; ++j) dma16(qn.cur, qoff[j], st + 1024u * j);
#pragma unroll
    for (int j = 0; j < 2; ++j) dma16(don.cur, dooff[j], st + 8192u + 1024u * j);
    if (wave == 0) dma16_va(scal_src + walk.tile * kSwRows, lds0 + (uint32_t)(stage * kStageBytes) + 16384u);
    const bool jumping = walk.left == 1;
    walk.next();
    qn.next(jumping);
    don.next(jumping);
  };
  // Wave 0 has one more load per tile in flight than the others.
  auto wait_barrier = [&](bool in_flight) {
    if (!in_flight)
      vm_wait_barrier<0>();
    else if (wave == 0)
      vm_wait_barrier<5>();
    else
      vm_wait_barrier<4>();
  };

  // Tiles 0 and 1 are requested before the K / V rows are waited for.
  issue(0);
  if (n_tiles > 1) issue(1);
  // V rows are kept negated: the dP products then start from Delta and give
  // Delta - dP directly (no per-element subtraction), so the kernel forms
  // -dS = P o (Delta - dP) and negates dK once at the end.
#pragma unroll
  for (int c = 0; c < 4; ++c)
    vreg[c] = __builtin_bit_cast(bf16x8, __builtin_bit_cast(u32x4, vreg[c]) ^ 0x80008000u);
  // The score chains start from the rows' -L / scale, so they give the
  // exact fp32 S - L / scale; P = exp2 of that times scale * log2(e).
#pragma unroll
  for (int c = 0; c < 4; ++c) asm volatile("" ::"v"(kreg[c]), "v"(vreg[c]));
  const RowIntervals civ = train_col_intervals(key, a.n, a.bs);
  const ClassBounds cb = uniform_bounds(key_group_bounds(train_key_group(kw, 32, a.n, a.bs), a.n));

  f32x16 dk[2] = {}, dv[2] = {};  // [d block]: lane = d column, registers = keys

  // Scores and Delta - dP of 32-row block qb of the current query tile (rows
  // x keys, lane = key column, register r <-> row 32qb + 8(r/4) + 4g + r%4):
  // the chains start from the rows' -L / scale and Delta, read from the
  // tile's row scalars in accumulator order.
  auto block_products = [&](const __bf16* qs, const __bf16* dos, const float* scal, int qb, f32x16& s,
                            f32x16& dp) {
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      const f32x4 dr = *reinterpret_cast<const f32x4*>(&scal[64 + 32 * qb + 8 * rg + 4 * g]);
      const f32x4 lr = *reinterpret_cast<const f32x4*>(&scal[32 * qb + 8 * rg + 4 * g]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        dp[4 * rg + j] = dr[j];
        s[4 * rg + j] = lr[j];
      }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      s = mfma32(sw_row_op(qs, 32 * qb, c, lane), kreg[c], s);
      dp = mfma32(sw_row_op(dos, 32 * qb, c, lane), vreg[c], dp);
    }
  };

  // P^T and -dS^T operands of block qb: P = exp2(s * scale * log2(e)), -dS = P o (Delta -
  // dP). A block that is not fully visible gets P = 0 on its invisible
  // pairs: with MASK16 (block size a multiple of 16) the mask is constant on
  // 16-row x 1-key strips, so one test per lane for rows 0-15 of the block
  // (registers 0-7) and one for rows 16-31 decide it, and it enters the
  // exponent as an addend (0, or -inf for an invisible strip: exp2 gives 0);
  // otherwise every pair is tested, and a dead block is computed and fully
  // masked (with MASK16 the loop skips it).
  auto softmax_ops = [&](const f32x16& s, const f32x16& dp, int q0, int qb, bool masked, bf16x8 (&pop)[2],
                         bf16x8 (&dsop)[2]) {
    float blo = 0.f, bhi = 0.f;  // exponent addends of registers 0-7 and 8-15
    if (MASK16 && masked) {
      blo = iv_has(civ, q0 + 32 * qb) ? 0.f : -INFINITY;
      bhi = iv_has(civ, q0 + 32 * qb + 16) ? 0.f : -INFINITY;
    }
    float p[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = fast_exp2(fmaf(s[r], a.scale_log2, r < 8 ? blo : bhi));
    if (!MASK16 && masked) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        p[r] = iv_has(civ, q0 + 32 * qb + 8 * (r >> 2) + 4 * g + (r & 3)) ? p[r] : 0.f;
    }
    float ds[16];  // -dS
#pragma unroll
    for (int r = 0; r < 16; ++r) ds[r] = p[r] * dp[r];
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      pop[kc] = to_bf16x8(p[8 * kc], p[8 * kc + 1], p[8 * kc + 2], p[8 * kc + 3], p[8 * kc + 4], p[8 * kc + 5],
                          p[8 * kc + 6], p[8 * kc + 7]);
      dsop[kc] = to_bf16x8(ds[8 * kc], ds[8 * kc + 1], ds[8 * kc + 2], ds[8 * kc + 3], ds[8 * kc + 4],
                           ds[8 * kc + 5], ds[8 * kc + 6], ds[8 * kc + 7]);
    }
  };

  // Every key group is seen by its own block, so n_tiles >= 1.
  vm_wait_barrier<0>();
  if constexpr (DIAG) {
    // Both query tiles are in stages 0 and 1 (no further loads); the
    // barrier after the block keeps the epilogue's LDS reuse behind every
    // wave's reads, as the tile loop's last barrier does.
    const int st = wave >> 1, qb = wave & 1;
    const int q0 = wave_uniform((t0 + st) * kSwRows);
    const int cls = bounds_class(cb, q0 + 32 * qb, 32, a.n);
    if (cls != kNone) {
      const __bf16* qs = &smem[st * (kStageBytes / 2)];
      const __bf16* dos = qs + kSwTile;
      const float* scal = reinterpret_cast<const float*>(qs + 2 * kSwTile);
      f32x16 sc, dpc;
      block_products(qs, dos, scal, qb, sc, dpc);
      bf16x8 pop[2], dsop[2];  // [16-row step]
      softmax_ops(sc, dpc, q0, qb, cls != kFull, pop, dsop);
#pragma unroll
      for (int kc = 0; kc < 2; ++kc)
#pragma unroll
        for (int db = 0; db < 2; ++db) {
          dv[db] = mfma32(pop[kc], sw_tr_op(dos, 32 * qb + 16 * kc, 32 * db, lane), dv[db]);
          dk[db] = mfma32(dsop[kc], sw_tr_op(qs, 32 * qb + 16 * kc, 32 * db, lane), dk[db]);
        }
    }
    vm_wait_barrier<0>();
    dkdv_store(a, smem + wave * kTileElems, bo.b, bo.h, kw, lane, dk, dv);
    return;
  }
  int cur = 0;
  for (int it = 0; it < n_tiles; ++it) {
    const bool pf = it + 2 < n_tiles;
    if (pf) issue(cur == 0 ? 2 : cur - 1);
    const int q0 = wave_uniform(tile_of(it) * kSwRows);
    const int c0 = bounds_class(cb, q0, 32, a.n);
    const int c1 = bounds_class(cb, q0 + 32, 32, a.n);
    // One code path for every live tile (the accumulators are updated by one
    // set of instructions, so they keep their registers).
    if ((c0 | c1) != kNone) {
      const __bf16* qs = &smem[cur * (kStageBytes / 2)];
      const __bf16* dos = qs + kSwTile;
      const float* scal = reinterpret_cast<const float*>(qs + 2 * kSwTile);
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        // MASK16: a 32-row block with no live pair is skipped (the first
        // block of a range's first tile for some waves; the per-pair mask
        // instance computes it, which keeps its registers).
        if (!MASK16 || (qb ? c1 : c0) != kNone) {
          f32x16 sc, dpc;
          block_products(qs, dos, scal, qb, sc, dpc);
          bf16x8 pop[2], dsop[2];  // [16-row step]
          softmax_ops(sc, dpc, q0, qb, (qb ? c1 : c0) != kFull, pop, dsop);
          // dV += P^T dO, dK += dS^T Q with dO / Q read transposed.
#pragma unroll
          for (int kc = 0; kc < 2; ++kc)
#pragma unroll
            for (int db = 0; db < 2; ++db) {
              const bf16x8 dot = sw_tr_op(dos, 32 * qb + 16 * kc, 32 * db, lane);
              const bf16x8 qt = sw_tr_op(qs, 32 * qb + 16 * kc, 32 * db, lane);
              dv[db] = mfma32(pop[kc], dot, dv[db]);
              dk[db] = mfma32(dsop[kc], qt, dk[db]);
            }
        }
        if (qb == 0) __builtin_amdgcn_sched_barrier(0);
      }
    }
    wait_barrier(pf);
    cur = cur == 2 ? 0 : cur + 1;
  }

  dkdv_store(a, smem + wave * kTileElems, bo.b, bo.h, kw, lane, dk, dv);
}

// The diagonal 32 x 32 block of a dQ item's wave when the noisy key tiles
// are folded in (fold_diag: block sizes dividing 32). A noisy key is seen
// only by the noisy rows of its own block, all of them in the wave whose
// rows have the key's indices, so this one block gives those 32 keys' whole
// dK and dV and the wave's rows' dQ over their own block: S and dP are formed
// once for dQ, dK and dV (the dQ loop stops before the two diagonal key
// tiles, which it walks last, so their K and V are still in the ring).
// dK/dV take the dK/dV items' arithmetic and layouts (key per lane): S = Q K^T
// and Delta - dP from the wave's own Q / dO operand registers, P and -dS,
// dV += P^T dO, dK += (-dS)^T Q with dO / Q read transposed from a staging
// tile. dQ^T += K^T dS^T takes dS^T through the staging as well (written key
// by row, read transposed, so its key order matches K^T's). Each wave then
// stores its own keys' rows through its own staging region.
template <bool MASK16>
__device__ __forceinline__ void diag_block(const BwdArgs& a, __bf16* smem, int b, int h, int qrow0, int wave, int lane,
                                           const __bf16* ktile, const __bf16* vtile, const bf16x8 (&qreg)[4],
                                           const bf16x8 (&doreg)[4], float lse_row, float drow, f32x16 (&dq)[2]) {
  constexpr int kRegion = 3 * 32 * 64 + 256;  // bf16: Q rows, dO rows, dS^T, 128 row scalars
  static_assert(4 * kRegion * 2 <= kBwdLdsBytes, "four staging regions fit the LDS buffer");
  static_assert(32 * kLdsStride <= kRegion, "the store's 32 rows fit a region");
  const int l32 = lane & 31;
  const int g = lane >> 5;
  const int key = qrow0 + l32;
  const int kr0 = 32 * (wave & 1);  // the wave's keys: rows kr0 .. kr0 + 31 of its diagonal tile
  // From the ring, before any wave reuses it: K rows and negated V rows (B
  // operands of S and dP) and K^T (A operands of dQ^T += K^T dS^T).
  bf16x8 kreg[4], vreg[4], kt[2][2];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    kreg[c] = sw_row_op(ktile, kr0, c, lane);
    vreg[c] = __builtin_bit_cast(bf16x8, __builtin_bit_cast(u32x4, sw_row_op(vtile, kr0, c, lane)) ^ 0x80008000u);
  }
#pragma unroll
  for (int kc = 0; kc < 2; ++kc)
#pragma unroll
    for (int db = 0; db < 2; ++db) kt[kc][db] = sw_tr_op(ktile, kr0 + 16 * kc, 32 * db, lane);
#pragma unroll
  for (int c = 0; c < 4; ++c) asm volatile("" ::"v"(kreg[c]), "v"(vreg[c]));
#pragma unroll
  for (int kc = 0; kc < 2; ++kc) asm volatile("" ::"v"(kt[kc][0]), "v"(kt[kc][1]));
  __syncthreads();

  __bf16* qs = smem + wave * kRegion;
  __bf16* dos = qs + 32 * 64;
  __bf16* dst = dos + 32 * 64;                           // dS^T: row = key, column = query row
  float* scal = reinterpret_cast<float*>(dst + 32 * 64);  // [0, 32): -L / scale, [64, 96): Delta
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int off = l32 * 64 + (((2 * c + g) ^ swz(l32)) << 3);
    *reinterpret_cast<bf16x8*>(&qs[off]) = qreg[c];
    *reinterpret_cast<bf16x8*>(&dos[off]) = doreg[c];
  }
  if (g == 0) {
    scal[l32] = -lse_row / a.scale;
    scal[64 + l32] = drow;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();

  const RowIntervals civ = train_col_intervals(key, a.n, a.bs);
  const ClassBounds cb = uniform_bounds(key_group_bounds(train_key_group(qrow0, 32, a.n, a.bs), a.n));
  const int cls = bounds_class(cb, qrow0, 32, a.n);
  f32x16 dk[2] = {}, dv[2] = {};
  if (cls != kNone) {
    // S - L / scale and Delta - dP (rows x keys, lane = key), seeded from the row scalars.
    f32x16 s, dp;
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      const f32x4 dr = *reinterpret_cast<const f32x4*>(&scal[64 + 8 * rg + 4 * g]);
      const f32x4 lr = *reinterpret_cast<const f32x4*>(&scal[8 * rg + 4 * g]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        dp[4 * rg + j] = dr[j];
        s[4 * rg + j] = lr[j];
      }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      s = mfma32(qreg[c], kreg[c], s);
      dp = mfma32(doreg[c], vreg[c], dp);
    }
    // Mask as in the dK/dV items: MASK16 strips through the exponent's addend.
    float blo = 0.f, bhi = 0.f;
    if (MASK16 && cls != kFull) {
      blo = iv_has(civ, qrow0) ? 0.f : -INFINITY;
      bhi = iv_has(civ, qrow0 + 16) ? 0.f : -INFINITY;
    }
    float p[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = fast_exp2(fmaf(s[r], a.scale_log2, r < 8 ? blo : bhi));
    if (!MASK16 && cls != kFull) {
#pragma unroll
      for (int r = 0; r < 16; ++r) p[r] = iv_has(civ, qrow0 + 8 * (r >> 2) + 4 * g + (r & 3)) ? p[r] : 0.f;
    }
    bf16x8 pop[2], dsop[2];  // P^T, -dS^T = (P o (Delta - dP))^T [16-row step]
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      pop[kc] = to_bf16x8(p[8 * kc], p[8 * kc + 1], p[8 * kc + 2], p[8 * kc + 3], p[8 * kc + 4], p[8 * kc + 5],
                          p[8 * kc + 6], p[8 * kc + 7]);
      dsop[kc] = to_bf16x8(p[8 * kc] * dp[8 * kc], p[8 * kc + 1] * dp[8 * kc + 1], p[8 * kc + 2] * dp[8 * kc + 2],
                           p[8 * kc + 3] * dp[8 * kc + 3], p[8 * kc + 4] * dp[8 * kc + 4],
                           p[8 * kc + 5] * dp[8 * kc + 5], p[8 * kc + 6] * dp[8 * kc + 6],
                           p[8 * kc + 7] * dp[8 * kc + 7]);
      // dS^T row `key`, columns (query rows) 16kc + 4g .. +3 and 16kc + 8 + 4g .. +3:
      // +dS (the sign bit flipped, exact), 8 bytes each.
      const u32x4 ds4 = __builtin_bit_cast(u32x4, dsop[kc]) ^ 0x80008000u;
      const int c0 = 16 * kc + 4 * g, c1 = c0 + 8;
      *reinterpret_cast<u32x2*>(&dst[l32 * 64 + (((c0 >> 3) ^ swz(l32)) << 3) + (c0 & 7)]) = u32x2{ds4[0], ds4[1]};
      *reinterpret_cast<u32x2*>(&dst[l32 * 64 + (((c1 >> 3) ^ swz(l32)) << 3) + (c1 & 7)]) = u32x2{ds4[2], ds4[3]};
    }
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        dv[db] = mfma32(pop[kc], sw_tr_op(dos, 16 * kc, 32 * db, lane), dv[db]);
        dk[db] = mfma32(dsop[kc], sw_tr_op(qs, 16 * kc, 32 * db, lane), dk[db]);
      }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
#pragma unroll
      for (int db = 0; db < 2; ++db) dq[db] = mfma32(kt[kc][db], sw_tr_op(dst, 16 * kc, 0, lane), dq[db]);
  }
  // The store reuses this wave's region after its operand reads (in order).
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  dkdv_store(a, qs, b, h, qrow0, lane, dk, dv);
}

// ---------------------------------------------------------------------------
// Query-stationary dQ (and Delta). K / V key tiles go global -> LDS with
// global_load_lds into a three-stage ring of swizzled tiles, two tiles ahead.
// Every live tile runs one code path over both of its 32-key blocks; a block
// that is not fully visible to the wave's rows is masked in place (MASK16:
// block size a multiple of 16, two tests per lane).
// One dQ item: 128-row query tile `rank` (heaviest first: rank r is tile
// n/128 - 1 - r/2 of the clean half for even r, of the noisy half for odd r)
// of (batch*head) bh, with the ring in `smem` (kDqLdsBytes). Delta and the
// rows' L come from the Delta pass.
template <bool MASK16>
__device__ __forceinline__ void dq_item(const BwdArgs& a, __bf16* smem, int bh, int rank) {
  constexpr int kBM = 128;  // query rows per workgroup: 4 waves x 32
  constexpr int kStages = kDqStages;
  constexpr int kAhead = kStages - 1;  // tiles requested ahead of the one being computed
  auto stage_k = [&](int st) { return smem + st * (2 * kSwTile); };
  auto stage_v = [&](int st) { return smem + st * (2 * kSwTile) + kSwTile; };

  // threadIdx here, unlike the other kernels: with the id builtin the
  // allocator spills one more VGPR in this tile loop (2 us slower at
  // configs[1], outputs identical).
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = wave_uniform(tid >> 6);
  const int l32 = lane & 31;
  const int g = lane >> 5;

  struct {
    int bh, b, h;
  } bo = {bh, bh / a.heads, bh - (bh / a.heads) * a.heads};
  const int tiles_half = a.n / kBM;
  const int t = tiles_half - 1 - (rank >> 1);
  const int q0 = ((rank & 1) ? 0 : a.n) + t * kBM;

  const uint16_t* qp = a.q + bo.b * a.sq.b + bo.h * a.sq.h;
  const uint16_t* kp = uniform_ptr(a.k + bo.b * a.sk.b + bo.h * a.sk.h);
  const uint16_t* vp = uniform_ptr(a.v + bo.b * a.sv.b + bo.h * a.sv.h);
  const uint16_t* dop = a.dout + bo.b * a.sdo.b + bo.h * a.sdo.h;
  const int64_t rowbase = (int64_t)bo.bh * 2 * a.n;

  const int qrow0 = q0 + 32 * wave;
  const int myq = qrow0 + l32;
  bf16x8 qreg[4], doreg[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int col = 16 * c + 8 * g;
    qreg[c] = __builtin_bit_cast(bf16x8, ld16(qp + (int64_t)myq * a.sq.s + col));
    doreg[c] = __builtin_bit_cast(bf16x8, ld16(dop + (int64_t)myq * a.sdo.s + col));
  }
  const float lse_row = a.lse[rowbase + myq];
  const float drow = a.delta[rowbase + myq];

  const KeyRanges kr = train_key_ranges(q0, kBM, a.n, a.bs, kSwRows);
  // With the noisy key tiles folded in (odd ranks are noisy row tiles), the
  // walk takes the clean-key range first and the two diagonal tiles (the
  // first range) last, so that the epilogue finds their K and V in the ring.
  const bool fold = a.fold_diag && (rank & 1);
  const int t0 = wave_uniform(fold ? kr.t2 : kr.t0), t2 = wave_uniform(fold ? kr.t0 : kr.t2);
  const int n_first = wave_uniform(fold ? kr.t3 - kr.t2 : kr.t1 - kr.t0);
  const int n_tiles = wave_uniform(kr.t1 - kr.t0 + kr.t3 - kr.t2);
  auto tile_of = [&](int i) { return i < n_first ? t0 + i : t2 + (i - n_first); };

  // Wave w fills 1 KB blocks 2w, 2w+1 (rows 16w .. 16w+15) of the K and V tiles.
  uint32_t koff[2], voff[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int r = 16 * wave + 8 * j + (lane >> 3);
    const int ch = 8 * ((lane & 7) ^ swz(r));
    koff[j] = (uint32_t)(2 * (r * (int)a.sk.s + ch));
    voff[j] = (uint32_t)(2 * (r * (int)a.sv.s + ch));
  }
  const int64_t kstep = (int64_t)kSwRows * a.sk.s, vstep = (int64_t)kSwRows * a.sv.s;
  const uint32_t lds_w = lds_addr(smem) + (uint32_t)wave * 2048u;
  // Sources of the next tile to request, walked tile by tile.
  TileWalk walk(t0, n_first, t2);
  TilePtr kn(kp, 2 * kstep, t0, n_first, t2), vn(vp, 2 * vstep, t0, n_first, t2);
  auto issue = [&](int stage) {
    const uint32_t dst = lds_w + (uint32_t)stage * 16384u;
#pragma unroll
    for (int j = 0; j < 2; ++j) dma16(kn.cur, koff[j], dst + 1024u * j);
#pragma unroll
    for (int j = 0; j < 2; ++j) dma16(vn.cur, voff[j], dst + 8192u + 1024u * j);
    const bool jumping = walk.left == 1;
    walk.next();
    kn.next(jumping);
    vn.next(jumping);
  };

  // The first kAhead tiles are requested before the row loads are waited for.
#pragma unroll
  for (int i = 0; i < kAhead; ++i)
    if (i < n_tiles) issue(i);
  const float lrow = lse_row * kLog2e;
#pragma unroll
  for (int c = 0; c < 4; ++c) asm volatile("" ::"v"(qreg[c]), "v"(doreg[c]));
  const RowIntervals riv = train_row_intervals(myq, a.n, a.bs);
  const ClassBounds cb = uniform_bounds(row_group_bounds(train_row_group(qrow0, 32, a.n, a.bs), a.n));

  f32x16 dq[2] = {};  // dQ^T [d block]

  // dS^T operands of one 32-key block sb of the current tile: S^T, dP^T
  // (keys x rows, lane = row, register r <-> key k0 + 32sb + 8(r/4) + 4g +
  // r%4), P, dS. A block that is not fully visible gets P = 0 on its
  // invisible pairs: with MASK16 (block size a multiple of 16) the mask is
  // constant on 1-row x 16-key strips, so one test per lane for keys 0-15 of
  // the block (registers 0-7) and one for keys 16-31 decide it, and it
  // enters the exponent as its addend (-L, or -inf for an invisible strip);
  // otherwise every pair is tested, and a dead block is computed and fully
  // masked (with MASK16 the loop skips it).
  auto block_ops = [&](const __bf16* ks, const __bf16* vs, int k0, int sb, bool masked, bf16x8 (&dsop)[2]) {
    bf16x8 kop[4], vop[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      kop[c] = sw_row_op(ks, 32 * sb, c, lane);
      vop[c] = sw_row_op(vs, 32 * sb, c, lane);
    }
    f32x16 s = {}, dp = {};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      s = mfma32(kop[c], qreg[c], s);
      dp = mfma32(vop[c], doreg[c], dp);
    }
    float blo = -lrow, bhi = -lrow;  // exponent addends of registers 0-7 and 8-15
    if (MASK16 && masked) {
      blo = iv_has(riv, k0 + 32 * sb) ? -lrow : -INFINITY;
      bhi = iv_has(riv, k0 + 32 * sb + 16) ? -lrow : -INFINITY;
    }
    float p[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] = fast_exp2(fmaf(s[r], a.scale_log2, r < 8 ? blo : bhi));
    if (!MASK16 && masked) {
#pragma unroll
      for (int r = 0; r < 16; ++r)
        p[r] = iv_has(riv, k0 + 32 * sb + 8 * (r >> 2) + 4 * g + (r & 3)) ? p[r] : 0.f;
    }
    float ds[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) ds[r] = p[r] * (dp[r] - drow);
#pragma unroll
    for (int kc = 0; kc < 2; ++kc)
      dsop[kc] = to_bf16x8(ds[8 * kc], ds[8 * kc + 1], ds[8 * kc + 2], ds[8 * kc + 3], ds[8 * kc + 4],
                           ds[8 * kc + 5], ds[8 * kc + 6], ds[8 * kc + 7]);
  };

  // Every row group sees at least its own block, so n_tiles >= 1. Folded:
  // the two diagonal tiles (the walk's last) are left to diag_block; a noisy
  // row tile also sees clean keys, so the loop keeps at least one tile.
  vm_wait_barrier<0>();
  const int n_loop = fold ? n_tiles - 2 : n_tiles;
  int cur = 0;
  for (int it = 0; it < n_loop; ++it) {
    const bool pf = it + kAhead < n_tiles;
    if (pf) issue(cur + kAhead < kStages ? cur + kAhead : cur + kAhead - kStages);
    const int k0 = wave_uniform(tile_of(it) * kSwRows);
    const int c0 = bounds_class(cb, k0, 32, a.n);
    const int c1 = bounds_class(cb, k0 + 32, 32, a.n);
    // One code path for every live tile (the accumulators keep their registers):
    // its two 32-key blocks one after the other, each straight into dQ.
    if ((c0 | c1) != kNone) {
      const __bf16* ks = stage_k(cur);
      const __bf16* vs = stage_v(cur);
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        // MASK16: a block with no live pair for the wave's rows is skipped
        // (the second block of a range's last tile for some waves).
        if (!MASK16 || (sb ? c1 : c0) != kNone) {
          bf16x8 dsop[2];  // [16-key step]
          block_ops(ks, vs, k0, sb, (sb ? c1 : c0) != kFull, dsop);
          // dQ^T += K^T dS^T with K^T read transposed.
#pragma unroll
          for (int kc = 0; kc < 2; ++kc)
#pragma unroll
            for (int db = 0; db < 2; ++db)
              dq[db] = mfma32(sw_tr_op(ks, 32 * sb + 16 * kc, 32 * db, lane), dsop[kc], dq[db]);
        }
      }
    }
    if (pf)
      vm_wait_barrier<4 * (kAhead - 1)>();
    else
      vm_wait_barrier<0>();
    cur = cur + 1 == kStages ? 0 : cur + 1;
  }

  if (fold) {
    // Both diagonal tiles resident (the loop's last wait left the second in
    // flight) and no wave still in the loop: waves 0, 1 take their keys from
    // the first diagonal tile, waves 2, 3 from the second.
    vm_wait_barrier<0>();
    const int sd = (n_tiles - 2 + (wave >> 1)) % kStages;
    diag_block<MASK16>(a, smem, bo.b, bo.h, qrow0, wave, lane, stage_k(sd), stage_v(sd), qreg, doreg, lse_row, drow,
                       dq);
  }
  uint16_t* dqp = a.dq + bo.b * a.sdq.b + bo.h * a.sdq.h + (int64_t)myq * a.sdq.s;
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int rg = 0; rg < 4; ++rg)
      *reinterpret_cast<bf16x4*>(dqp + 32 * db + 8 * rg + 4 * g) =
          to_bf16x4(dq[db][4 * rg] * a.scale, dq[db][4 * rg + 1] * a.scale, dq[db][4 * rg + 2] * a.scale,
                    dq[db][4 * rg + 3] * a.scale);
}

// Delta = rowsum(dO o O) (the reference's separate torch op,
// kernels/BlockSparseFlashAttention.py:525) and -L / scale (the dK/dV score
// chains' seed) of every row, into the two workspace planes: 8 lanes per row
// (16 bytes each), 32 rows per pass of a 256-thread workgroup, kPasses
// passes with every load issued before the first use. Bound by reading O
// and dO once.
__global__ __launch_bounds__(256) void attn_bwd_delta_kernel(BwdArgs a) {
  constexpr int kPasses = 4;
  const int tid = wi_x();
  const int grp = tid >> 3, part = tid & 7;
  const int rows_bh = 2 * a.n;
  u32x4 ov[kPasses], dv[kPasses];
  int64_t row[kPasses];
#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
    const int64_t r = (int64_t)wg_x() * (32 * kPasses) + 32 * p + grp;
    const int bh = (int)(r / rows_bh), s = (int)(r - (int64_t)bh * rows_bh);
    const int b = bh / a.heads, h = bh - b * a.heads;
    row[p] = r;
    ov[p] = ld16(a.o + b * a.so.b + h * a.so.h + (int64_t)s * a.so.s + 8 * part);
    dv[p] = ld16(a.dout + b * a.sdo.b + h * a.sdo.h + (int64_t)s * a.sdo.s + 8 * part);
  }
  float lse[kPasses];
#pragma unroll
  for (int p = 0; p < kPasses; ++p) lse[p] = part == 0 ? a.lse[row[p]] : 0.f;
#pragma unroll
  for (int p = 0; p < kPasses; ++p) {
    const bf16x8 o8 = __builtin_bit_cast(bf16x8, ov[p]), d8 = __builtin_bit_cast(bf16x8, dv[p]);
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) sum = fmaf((float)d8[j], (float)o8[j], sum);
    sum += shfl_xor(sum, 1);
    sum += shfl_xor(sum, 2);
    sum += shfl_xor(sum, 4);
    if (part == 0) {
      a.delta[row[p]] = sum;
      a.delta[(int64_t)a.bh * rows_bh + row[p]] = -lse[p] / a.scale;
    }
  }
}

// The backward's work items in one launch: dQ query tiles and dK/dV key
// tiles of every batch*head, in the host's order (a.order, longest first,
// the two kinds interleaved), batch*head the fastest grid axis so that a
// head's items share one XCD and its L2. Both kinds only read the Delta
// pass's planes, so they need no ordering between them, and one launch has
// one start-up and one tail instead of two. One LDS buffer serves either
// kind's ring.
template <int OCC, bool MASK16>
__global__ __launch_bounds__(256, OCC) void attn_bwd_kernel(BwdArgs a) {
  __shared__ __attribute__((aligned(1024))) __bf16 smem[kBwdLdsBytes / 2];
  const int id = wg_x();
  const int slot = id / a.bh, bh = id - slot * a.bh;
  const int code = a.n_items <= kBwdOrderMax ? (int)a.order[slot] : a.first_code + slot;
  const int dq_items = 2 * a.n / 128;
  const int dk_rank = code - dq_items;
  if (code < dq_items)
    dq_item<MASK16>(a, smem, bh, code);
  else if (dk_rank >= a.n / 128 && 32 % a.bs == 0)  // a noisy key tile, blocks within 32 keys
    dkdv_item<MASK16, true>(a, smem, bh, dk_rank);
  else
    dkdv_item<MASK16, false>(a, smem, bh, dk_rank);
}

}  // namespace

hipError_t launch_attn_bwd_delta(const BwdArgs& a, hipStream_t stream) {
  // 128 rows per workgroup; batch * heads * 2n is a multiple of 256.
  const int64_t rows = (int64_t)a.bh * 2 * a.n;
  hipLaunchKernelGGL(attn_bwd_delta_kernel, dim3((unsigned)(rows / 128)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_attn_bwd_items(const BwdArgs& a, hipStream_t stream) {
  // One 4-wave workgroup per (item, batch*head); three per CU (168 VGPRs,
  // 51 KB of LDS). Measured against two waves per SIMD with the dK/dV
  // items' four product chains interleaved (230 VGPRs): 258 vs 276 us at
  // B=4, H=16, n=2048, 348 vs 380 at B=2, H=12, n=4096, 689 vs 746 at n=8192.
  const dim3 grid(a.bh * a.n_items), block(256);
  if (a.bs % 16 == 0)
    hipLaunchKernelGGL((attn_bwd_kernel<3, true>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((attn_bwd_kernel<3, false>), grid, block, 0, stream, a);
  return hipGetLastError();
}

}  // namespace bd3
