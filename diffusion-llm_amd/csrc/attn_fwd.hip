// attn_fwd.hip - BD3-LM training attention forward for gfx950.
//
// O = softmax(Q K^T * scale + M) V over cat(x_t, x_0) (length 2n), M the
// block-diffusion mask (bd3_mask.h); lse = logsumexp per row, natural log.
// Counterpart of block_sparse_attention_fwd_kern
// (kernels/BlockSparseFlashAttention.py:75-172).
//
// Work split: one workgroup per (batch*head, 128-row query tile), 4 waves of
// 32 rows; a query tile lies in one half. Only key tiles (64 keys) where the
// mask has live pairs for the workgroup are visited (train_key_ranges); each
// wave skips tiles that are dead for its rows and masks only partial ones.
// Noisy rows with a block size dividing 32 start with their own two noisy
// key tiles loaded at once: each wave forms only its 32 x 32 diagonal block,
// all four waves in one half-tile step.
//
// Loads: K/V tiles go global -> LDS with global_load_lds_dwordx4 into a
// ring of swizzled tiles (bd3_swz.h): no VGPR staging and no LDS store pass;
// each tile ends with one counted vmcnt wait and a plain s_barrier. Built
// with two stages (the next tile loads during the current one) and 4
// workgroups per CU (4 waves per SIMD, 128 VGPRs, 32 KB of LDS each); with
// three stages (two tiles ahead) only 3 workgroups' rings fit the LDS.
//
// Per wave and key tile:
//   S^T (keys x rows) = K Q^T on v_mfma_f32_32x32x16_bf16: a lane holds one
//   query row (lane % 32) and 16 of its keys per 32x32 block, so the softmax
//   statistics are lane-local up to one permlane32 exchange. The K operands
//   come from LDS two at a time, each pair just ahead of its two products
//   (the other waves on the SIMD cover that latency).
//   O^T (64 x rows) += V^T P^T, V^T read from the LDS tile by
//   ds_read_b64_tr_b16 (requested right after the S^T products, so the reads
//   hide behind the softmax), P^T taken from the S^T registers (key order in
//   the reduction permuted identically on both sides).
// Softmax in base 2 with scale*log2(e) folded into one FMA. The running max
// is updated lazily: O and l are rescaled only when some row's max grew by
// more than kRescale (log2 units); otherwise the stale max is kept, which
// bounds P by 2^kRescale and leaves O / l exact.
//
// Prefill mode (prefill_attn_kernel, DecodeArgs): the same body over the
// decode mask when many queries attend to the cache at once (the uncached
// block-causal prefill of kernels/BlockSparseDecodeAttention.py:40-110 with
// q_len = kv_len, or a long query block over a cached prefix). Row i of the
// q_len queries sees keys [0, e(i)), e(i) = min(kv_len, (p / bs + 1) * bs),
// p = kv_len - q_len + i: one interval per row, so a wave's tile classes
// come from e at its first and last row. Work items are (128-row query
// tile, split of the keys, batch*head), longest rows first; a query tile
// whose keys all lie in the first split writes O, the others write
// normalised fp32 partials and base-2 LSEs in the decode kernels' layout for
// prefill_combine. Rows past q_len re-read the last query row and are not
// stored; key rows past kv_len re-read the last key row and are masked.
#include <type_traits>

#include "bd3_device.h"
#include "bd3_launch.h"
#include "bd3_mask.h"
#include "bd3_swz.h"
#include "bd3_tile.h"

namespace bd3 {
namespace {

constexpr float kRescale = 8.0f;

#ifndef BD3_FWD_OCC
#define BD3_FWD_OCC 4
#endif
#ifndef BD3_FWD_STAGES
#define BD3_FWD_STAGES 2
#endif

// One class per 64-key tile for the wave (dead / full / partial, as walk
// index intervals of its row group): a full tile runs straight-line code with
// no mask arithmetic. MASK16: every row's key intervals start and end on
// multiples of 16 (training: the block size is a multiple of 16; prefill:
// the block size and kv_len are).
template <bool MASK16, bool PREFILL, class Args>
__device__ __forceinline__ void fwd_body(Args a) {
  constexpr int kBM = 128;  // query rows per workgroup: 4 waves x 32
  constexpr int kStages = BD3_FWD_STAGES;
  constexpr int kAhead = kStages - 1;  // tiles requested ahead of the one being computed
  __shared__ __attribute__((aligned(1024))) __bf16 smem[kStages][2][kSwTile];  // [stage][K|V]

  const int tid = wi_x();
  const int lane = tid & 63;
  const int wave = wave_uniform(tid >> 6);
  const int l32 = lane & 31;
  const int g = lane >> 5;

  int bh, b, h, q0;
  int split = 0, e_wg = 0;  // prefill: the item's split and the tile's key end
  if constexpr (PREFILL) {
    bh = wg_x();
    split = wg_y();
    q0 = kBM * ((a.q_len + kBM - 1) / kBM - 1 - wg_z());
    e_wg = decode_key_end(q0, kBM, a.q_len, a.kv_len, a.bs);
    if (split * a.split_len >= e_wg) return;  // no key of this split is visible to the tile
    b = bh / a.heads;
    h = bh - b * a.heads;
  } else {
    const BlockOrder bo(a.bh, a.heads);
    const int tiles_half = a.n / kBM;
    const int t = tiles_half - 1 - (bo.rank >> 1);
    q0 = ((bo.rank & 1) ? 0 : a.n) + t * kBM;
    bh = bo.bh;
    b = bo.b;
    h = bo.h;
  }

  const uint16_t* qp = a.q + b * a.sq.b + h * a.sq.h;
  const uint16_t* kp = uniform_ptr(a.k + b * a.sk.b + h * a.sk.h);
  const uint16_t* vp = uniform_ptr(a.v + b * a.sv.b + h * a.sv.h);

  const int qrow0 = q0 + 32 * wave;
  const int myq = qrow0 + l32;
  int qsrc = myq;  // the row whose Q the lane holds
  if constexpr (PREFILL) qsrc = imin(myq, a.q_len - 1);
  bf16x8 qreg[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
    qreg[c] = __builtin_bit_cast(bf16x8, ld16(qp + (int64_t)qsrc * a.sq.s + 16 * c + 8 * g));

  int t0, t2, n_first, n_tiles;
  if constexpr (PREFILL) {
    // One range: the split's tiles up to the tile's key end.
    t0 = wave_uniform(split * (a.split_len / kSwRows));
    const int kend = imin(e_wg, (split + 1) * a.split_len);
    n_first = wave_uniform((kend + kSwRows - 1) / kSwRows - t0);
    t2 = t0 + n_first;
    n_tiles = n_first;
  } else {
    const KeyRanges kr = train_key_ranges(q0, kBM, a.n, a.bs, kSwRows);
    t0 = wave_uniform(kr.t0);
    t2 = wave_uniform(kr.t2);
    n_first = wave_uniform(kr.t1 - kr.t0);
    n_tiles = n_first + wave_uniform(kr.t3 - kr.t2);
  }
  auto tile_of = [&](int i) { return i < n_first ? t0 + i : t2 + (i - n_first); };

  // Wave w fills the 1 KB blocks 2w and 2w+1 (rows 16w .. 16w+15) of each K
  // and V tile: lane L fetches logical chunk (L%8) ^ swz(row) of row
  // 16w + 8j + L/8 (byte offsets from the tile's row 0).
  uint32_t koff[2], voff[2];
  int lrow[2], lch[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int r = 16 * wave + 8 * j + (lane >> 3);
    const int ch = 8 * ((lane & 7) ^ swz(r));
    koff[j] = (uint32_t)(2 * (r * (int)a.sk.s + ch));
    voff[j] = (uint32_t)(2 * (r * (int)a.sv.s + ch));
    lrow[j] = r;
    lch[j] = ch;
  }
  const int64_t kstep = (int64_t)kSwRows * a.sk.s, vstep = (int64_t)kSwRows * a.sv.s;
  // LDS byte address of this wave's first K block in stage 0; a stage is
  // 2 * 8 KB (K then V).
  const uint32_t lds_w = lds_addr(&smem[0][0][0]) + (uint32_t)wave * 2048u;
  // Source of the next tile to request, walked tile by tile (requests are
  // made in order: tile_of(0), tile_of(1), ...).
  TileWalk walk(t0, n_first, t2);
  TilePtr kn(kp, 2 * kstep, t0, n_first, t2), vn(vp, 2 * vstep, t0, n_first, t2);
  auto issue = [&](int stage) {
    const uint32_t dst = lds_w + (uint32_t)stage * 16384u;
    uint32_t ko[2] = {koff[0], koff[1]}, vo[2] = {voff[0], voff[1]};
    if constexpr (PREFILL) {
      // Rows past the last key re-read the last key row (masked out).
      const int lim = a.kv_len - 1 - walk.tile * kSwRows;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int r = imin(lrow[j], lim);
        ko[j] = (uint32_t)(2 * (r * (int)a.sk.s + lch[j]));
        vo[j] = (uint32_t)(2 * (r * (int)a.sv.s + lch[j]));
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) dma16(kn.cur, ko[j], dst + 1024u * j);
#pragma unroll
    for (int j = 0; j < 2; ++j) dma16(vn.cur, vo[j], dst + 8192u + 1024u * j);
    const bool jumping = walk.left == 1;
    walk.next();
    kn.next(jumping);
    vn.next(jumping);
  };

  // Noisy rows with a block size dividing 32 (training, two-stage ring): the
  // walk's first two tiles are the workgroup's own noisy blocks, where each
  // wave's live pairs form the 32 x 32 block of its own rows (keys qrow0 ..
  // qrow0 + 31). Both tiles are loaded at once and every wave forms its block
  // in one half-tile step, instead of a whole-tile step on one of the two
  // tiles while the other two waves wait at its barrier.
  // The first tiles are requested before waiting for Q, so the latencies
  // overlap. Consuming Q here (an empty asm reading it) makes the compiler
  // place its own wait for the Q loads at this point; that wait also covers
  // the direct loads issued after them, which is harmless.
  bool diag_first = false;
  if constexpr (!PREFILL && kStages == 2) diag_first = q0 < a.n && 32 % a.bs == 0;
  if (diag_first) {
    issue(0);
    issue(1);
  } else {
#pragma unroll
    for (int i = 0; i < kAhead; ++i)
      if (i < n_tiles) issue(i);
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) asm volatile("" ::"v"(qreg[c]));
  RowIntervals riv;
  WalkClasses wc;
  if constexpr (PREFILL) {
    const int ql = a.q_len;
    auto key_end = [&](int i) { return imin(((a.kv_len - ql + i) / a.bs + 1) * a.bs, a.kv_len); };
    riv = RowIntervals{0, key_end(qsrc), 0, 0};
    // Tiles below the first row's key end are full, those from the last
    // row's key end on are dead; a wave with no row below q_len has none live.
    ClassBounds cb;
    const int emax = qrow0 < ql ? key_end(imin(qrow0 + 31, ql - 1)) : 0;
    const int emin = key_end(imin(qrow0, ql - 1));
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      cb.lo[hh] = 0;
      cb.hi[hh] = emax;
      cb.flo[hh] = 0;
      cb.fhi[hh] = emin;
    }
    wc = uniform_walk(walk_classes(cb, t0, n_first, t2, 0, kBoundBig, kSwRows, 0, kSwRows));
  } else {
    riv = train_row_intervals(myq, a.n, a.bs);
    wc = uniform_walk(walk_classes(row_group_bounds(train_row_group(qrow0, 32, a.n, a.bs), a.n), t0, n_first, t2,
                                   n_tiles - n_first, a.n, kSwRows, 0, kSwRows));
  }

  f32x16 o[2] = {};  // O^T [d block]
  // mref: the row's reference maximum (log2 units); `valid` once the row
  // has met a live key. Scores are exact fp32 dot products of the bf16 rows;
  // scale * log2(e) is applied to each one in the exponent's FMA.
  float mref = 0.f, lsum = 0.f;
  bool valid = false;
  const float c2 = a.scale_log2;

  // One tile step over NSB 32-key halves of the current 64-key tile,
  // starting at half sb0 (NSB = 1: the other half is dead for this wave).
  // EARLY: the V^T operands are read together with the K operands, and once
  // both are in registers `reads_done` runs (the tile's LDS may then be
  // refilled while the step computes).
  auto step = [&](auto nsb_c, auto early_c, int sb0, int k0, int cls, const __bf16* ks, const __bf16* vs,
                  auto&& reads_done) {
    constexpr int NSB = decltype(nsb_c)::value;
    constexpr bool EARLY = decltype(early_c)::value;
    bf16x8 kop[NSB][4];
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
      for (int c = 0; c < 4; ++c) kop[sb][c] = sw_row_op(ks, 32 * (sb0 + sb), c, lane);
    bf16x8 vpre[EARLY ? NSB : 1][2][2];
    if constexpr (EARLY) {
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
        for (int kc = 0; kc < 2; ++kc)
#pragma unroll
          for (int db = 0; db < 2; ++db) vpre[sb][kc][db] = sw_tr_op(vs, 32 * (sb0 + sb) + 16 * kc, 32 * db, lane);
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
        for (int c = 0; c < 4; ++c) asm volatile("" ::"v"(kop[sb][c]));
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
        for (int kc = 0; kc < 2; ++kc)
#pragma unroll
          for (int db = 0; db < 2; ++db) asm volatile("" ::"v"(vpre[sb][kc][db]));
      reads_done();
    }
    f32x16 s[NSB];
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) s[sb] = mfma32(kop[sb][0], qreg[0], f32x16{});
#pragma unroll
    for (int c = 1; c < 4; ++c)
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb) s[sb] = mfma32(kop[sb][c], qreg[c], s[sb]);

    // Partial tile. With MASK16 (block size a multiple of 16) the mask is
    // constant on 1-row x 16-key strips: registers 0-7 of a key block hold
    // its keys 0-15, registers 8-15 keys 16-31, so one test per strip decides
    // them; an invisible strip is left out of the row max and enters the
    // exponent with a -inf addend (P = 0). Otherwise invisible pairs are set
    // to -inf one by one.
    bool live[NSB][2];  // MASK16 partial tile: strip h of key block sb visible to the lane's row
    if (cls == kPartial) {
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb) {
        const int kb = k0 + 32 * (sb0 + sb);
        if (MASK16) {
          live[sb][0] = iv_has(riv, kb);
          live[sb][1] = iv_has(riv, kb + 16);
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kb + 8 * (r >> 2) + 4 * g + (r & 3);
            s[sb][r] = iv_has(riv, key) ? s[sb][r] : -INFINITY;
          }
        }
      }
    }
    // Row max of the scores: one v_max3 chain per strip, then scaled to the
    // base-2 exponent relative to the current reference.
    float mst[NSB][2];
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int r0 = 8 * hh;
        float m = fmaxf(fmaxf(s[sb][r0], s[sb][r0 + 1]), s[sb][r0 + 2]);
        m = fmaxf(fmaxf(m, s[sb][r0 + 3]), s[sb][r0 + 4]);
        m = fmaxf(fmaxf(m, s[sb][r0 + 5]), s[sb][r0 + 6]);
        mst[sb][hh] = fmaxf(m, s[sb][r0 + 7]);
      }
    if (MASK16 && cls == kPartial) {
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) mst[sb][hh] = live[sb][hh] ? mst[sb][hh] : -INFINITY;
    }
    float mrow = fmaxf(mst[0][0], mst[0][1]);
#pragma unroll
    for (int sb = 1; sb < NSB; ++sb) mrow = fmaxf(fmaxf(mrow, mst[sb][0]), mst[sb][1]);
    const float mt = fmaf(max_xor32(mrow), c2, -mref);
    // A new reference when the row had none (and this tile has a live key)
    // or its maximum grew by more than kRescale: the reference rises by
    // delta, O and l scale by 2^-delta.
    if (__ballot(!valid || mt > kRescale) != 0) {
      const float delta = valid ? fmaxf(mt, 0.f) : (mt == -INFINITY ? 0.f : mt);
      const float alpha = valid ? fast_exp2(-delta) : 1.f;
      valid = valid || mt != -INFINITY;
      mref += delta;
      lsum *= alpha;
      o[0] *= alpha;
      o[1] *= alpha;
    }
    // Exponent addends per strip: -mref, or -inf for an invisible strip.
    float nm[NSB][2];
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) nm[sb][0] = nm[sb][1] = -mref;
    if (MASK16 && cls == kPartial) {
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) nm[sb][hh] = live[sb][hh] ? -mref : -INFINITY;
    }
    bf16x8 pop[NSB][2];  // P^T operands [key block][16-key step]
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) {
      float p[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) p[r] = fast_exp2(fmaf(s[sb][r], c2, nm[sb][r >> 3]));
      // The row sum in fp32 from the unrounded P, as the reference's l.
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        pop[sb][kc] = to_bf16x8(p[8 * kc], p[8 * kc + 1], p[8 * kc + 2], p[8 * kc + 3], p[8 * kc + 4],
                                p[8 * kc + 5], p[8 * kc + 6], p[8 * kc + 7]);
        lsum += ((p[8 * kc] + p[8 * kc + 1]) + (p[8 * kc + 2] + p[8 * kc + 3])) +
                ((p[8 * kc + 4] + p[8 * kc + 5]) + (p[8 * kc + 6] + p[8 * kc + 7]));
      }
    }
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) {
      bf16x8 vop[2][2];  // V^T operands of key block sb [16-key step][d block], read just before use
#pragma unroll
      for (int kc = 0; kc < 2; ++kc)
#pragma unroll
        for (int db = 0; db < 2; ++db) {
          if constexpr (EARLY)
            vop[kc][db] = vpre[sb][kc][db];
          else
            vop[kc][db] = sw_tr_op(vs, 32 * (sb0 + sb) + 16 * kc, 32 * db, lane);
        }
#pragma unroll
      for (int kc = 0; kc < 2; ++kc)
#pragma unroll
        for (int db = 0; db < 2; ++db) o[db] = mfma32(vop[kc][db], pop[sb][kc], o[db]);
    }
  };

  // Every row group sees at least its own block, so n_tiles >= 1.
  vm_wait_barrier<0>();

  int it = 0, cur = 0;
  if (diag_first) {
    // Wave w's block lies in half w % 2 of tile w / 2 (stage w / 2). Once
    // every wave holds its operands, stage 0 takes the first tile of the
    // loop, which loads while the blocks are formed.
    const int st = wave >> 1;
    step(std::integral_constant<int, 1>(), std::true_type(), wave & 1, wave_uniform(tile_of(st) * kSwRows),
         a.bs == 32 ? kFull : kPartial, smem[st][0], smem[st][1], [&] {
           vm_wait_barrier<0>();
           if (n_tiles > 2) issue(0);
         });
    it = 2;
    vm_wait_barrier<0>();
  }
  for (; it < n_tiles; ++it) {
    const bool pf = it + kAhead < n_tiles;
    if (pf) issue(cur + kAhead < kStages ? cur + kAhead : cur + kAhead - kStages);
    const int k0 = wave_uniform(tile_of(it) * kSwRows);
    // The tile's class for this wave's rows.
    if (walk_live(wc, it, n_first))
      step(std::integral_constant<int, 2>(), std::false_type(), 0, k0,
           walk_full(wc, it, n_first) ? kFull : kPartial, smem[cur][0], smem[cur][1], [] {});
    // Tile it+1 complete (the loads of later tiles may stay in flight), and
    // every wave is done reading stage `cur` before it is refilled.
    if (pf)
      vm_wait_barrier<4 * (kAhead - 1)>();
    else
      vm_wait_barrier<0>();
    cur = cur + 1 == kStages ? 0 : cur + 1;
  }

  const float ltot = sum_xor32(lsum);
  if constexpr (PREFILL) {
    if (myq >= a.q_len) return;
    // A row may see no key of a later split: O = 0, LSE = -inf.
    const bool seen = ltot > 0.f;
    const float inv = seen ? 1.f / ltot : 0.f;
    if (e_wg <= a.split_len) {  // the tile's keys all lie in the first split
      uint16_t* op = a.o + b * a.so.b + h * a.so.h + (int64_t)myq * a.so.s;
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int rg4 = 0; rg4 < 4; ++rg4)
          *reinterpret_cast<bf16x4*>(op + 32 * db + 8 * rg4 + 4 * g) =
              to_bf16x4(o[db][4 * rg4] * inv, o[db][4 * rg4 + 1] * inv, o[db][4 * rg4 + 2] * inv,
                        o[db][4 * rg4 + 3] * inv);
    } else {
      const int64_t slot = ((int64_t)bh * a.q_tiles + (qrow0 >> 5)) * a.n_splits + split;
      float* po = a.part_o + (slot * 32 + l32) * kHeadDim;
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int rg4 = 0; rg4 < 4; ++rg4)
          *reinterpret_cast<f32x4*>(po + 32 * db + 8 * rg4 + 4 * g) =
              f32x4{o[db][4 * rg4] * inv, o[db][4 * rg4 + 1] * inv, o[db][4 * rg4 + 2] * inv,
                    o[db][4 * rg4 + 3] * inv};
      if (g == 0) a.part_lse[slot * 32 + l32] = seen ? mref + fast_log2(ltot) : -INFINITY;
    }
  } else {
    const float inv = 1.f / ltot;
    uint16_t* op = a.o + b * a.so.b + h * a.so.h + (int64_t)myq * a.so.s;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int rg4 = 0; rg4 < 4; ++rg4)
        *reinterpret_cast<bf16x4*>(op + 32 * db + 8 * rg4 + 4 * g) =
            to_bf16x4(o[db][4 * rg4] * inv, o[db][4 * rg4 + 1] * inv, o[db][4 * rg4 + 2] * inv,
                      o[db][4 * rg4 + 3] * inv);
    if (g == 0) a.lse[(int64_t)bh * 2 * a.n + myq] = (mref + fast_log2(ltot)) * kLn2;
  }
}

template <int OCC, bool MASK16>
__global__ __launch_bounds__(256, OCC) void attn_fwd_dma_kernel(FwdArgs a) {
  fwd_body<MASK16, false>(a);
}

template <int OCC, bool MASK16>
__global__ __launch_bounds__(256, OCC) void prefill_attn_kernel(DecodeArgs a) {
  fwd_body<MASK16, true>(a);
}

// Merges the split partials of the rows whose 128-row tile spans several
// splits (the kernel wrote the other rows' O): weights exp2(lse_s - max lse)
// as in decode_combine; 16 threads per row, 4 outputs each, all 32 rows of a
// tile in one workgroup. Up to 8 splits (the common case) take one memory
// round trip: every load is issued before the first use; more splits go 8
// per round trip. Grid: (32-row tiles, batch*head).
__global__ __launch_bounds__(512) void prefill_combine(DecodeArgs a) {
  const int qt = wg_x();
  const int bh = wg_y();
  const int i0 = qt * 32;
  const int e = decode_key_end(i0 & ~127, 128, a.q_len, a.kv_len, a.bs);
  const int ns = (e + a.split_len - 1) / a.split_len;
  const int tid = wi_x();
  const int row = tid >> 4;
  if (ns <= 1 || i0 + row >= a.q_len) return;
  const int b = bh / a.heads, h = bh - b * a.heads;
  uint16_t* op = a.o + b * a.so.b + h * a.so.h;
  const int64_t slot0 = ((int64_t)bh * a.q_tiles + qt) * a.n_splits;
  const int d0 = 4 * (tid & 15);
  constexpr int kG = 8;
  const float* lp = a.part_lse + slot0 * 32 + row;                  // split s: lp[32 s]
  const float* pp = a.part_o + (slot0 * 32 + row) * kHeadDim + d0;  // split s: pp[32 * 64 s]
  float mm = -INFINITY, wt = 0.f;
  f32x4 acc = {};
  if (ns <= kG) {
    float l[kG];
    f32x4 po[kG];
#pragma unroll
    for (int k = 0; k < kG; ++k) {
      l[k] = k < ns ? lp[k * 32] : -INFINITY;
      po[k] = k < ns ? *reinterpret_cast<const f32x4*>(pp + k * 32 * kHeadDim) : f32x4{};
    }
#pragma unroll
    for (int k = 0; k < kG; ++k) mm = fmaxf(mm, l[k]);
#pragma unroll
    for (int k = 0; k < kG; ++k) {
      const float w = k < ns ? fast_exp2(l[k] - mm) : 0.f;  // a split the row does not see: 0
      wt += w;
      acc += w * po[k];
    }
  } else {
    for (int s0 = 0; s0 < ns; s0 += kG) {
      float l[kG];
#pragma unroll
      for (int k = 0; k < kG; ++k) l[k] = s0 + k < ns ? lp[(s0 + k) * 32] : -INFINITY;
#pragma unroll
      for (int k = 0; k < kG; ++k) mm = fmaxf(mm, l[k]);
    }
    for (int s0 = 0; s0 < ns; s0 += kG) {
      float l[kG];
      f32x4 po[kG];
#pragma unroll
      for (int k = 0; k < kG; ++k) {
        if (s0 + k < ns) {
          l[k] = lp[(s0 + k) * 32];
          po[k] = *reinterpret_cast<const f32x4*>(pp + (s0 + k) * 32 * kHeadDim);
        }
      }
#pragma unroll
      for (int k = 0; k < kG; ++k) {
        if (s0 + k < ns) {
          const float w = fast_exp2(l[k] - mm);
          wt += w;
          acc += w * po[k];
        }
      }
    }
  }
  const float inv = 1.f / wt;
  *reinterpret_cast<bf16x4*>(op + (int64_t)(i0 + row) * a.so.s + d0) =
      to_bf16x4(acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv);
}

}  // namespace



hipError_t launch_attn_fwd(const FwdArgs& a, hipStream_t stream) {
  // n % 128 == 0 always holds (validated): 128-row query tiles of 4 waves.
  const dim3 grid(a.bh * (2 * a.n / 128)), block(256);
  if (a.bs % 16 == 0)
    hipLaunchKernelGGL((attn_fwd_dma_kernel<BD3_FWD_OCC, true>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((attn_fwd_dma_kernel<BD3_FWD_OCC, false>), grid, block, 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_prefill(const DecodeArgs& a, hipStream_t stream) {
  // Items (batch*head, split, 128-row tile), longest rows first; splits past
  // the last key and those a tile does not reach exit at once.
  const int row_tiles = (a.q_len + 127) / 128;
  const int splits = (a.kv_len + a.split_len - 1) / a.split_len;
  const dim3 grid(a.bh, splits, row_tiles), block(256);
  if (a.bs % 16 == 0 && a.kv_len % 16 == 0)
    hipLaunchKernelGGL((prefill_attn_kernel<BD3_FWD_OCC, true>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((prefill_attn_kernel<BD3_FWD_OCC, false>), grid, block, 0, stream, a);
  hipError_t e = hipGetLastError();
  // The last tile sees the most keys: if they fit one split, no partials.
  if (e != hipSuccess || decode_key_end(128 * (row_tiles - 1), 128, a.q_len, a.kv_len, a.bs) <= a.split_len)
    return e;
  hipLaunchKernelGGL(prefill_combine, dim3(a.q_tiles, a.bh), dim3(512), 0, stream, a);
  return hipGetLastError();
}

}  // namespace bd3
