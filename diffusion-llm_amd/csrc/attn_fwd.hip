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
//
// Loads: K/V tiles go global -> LDS with global_load_lds_dwordx4 into a
// three-stage ring of swizzled tiles (bd3_swz.h), two tiles ahead: no VGPR
// staging and no LDS store pass; each tile ends with one counted vmcnt wait
// and a plain s_barrier (the loads of the tile after next stay in flight).
//
// Per wave and key tile:
//   S^T (keys x rows) = K Q^T on v_mfma_f32_32x32x16_bf16: a lane holds one
//   query row (lane % 32) and 16 of its keys per 32x32 block, so the softmax
//   statistics are lane-local up to one permlane32 exchange. All K operands
//   of the tile are read from LDS in one batch.
//   O^T (64 x rows) += V^T P^T, V^T read from the LDS tile by
//   ds_read_b64_tr_b16 (requested right after the S^T products, so the reads
//   hide behind the softmax), P^T taken from the S^T registers (key order in
//   the reduction permuted identically on both sides).
// Softmax in base 2 with scale*log2(e) folded into one FMA. The running max
// is updated lazily: O and l are rescaled only when some row's max grew by
// more than kRescale (log2 units); otherwise the stale max is kept, which
// bounds P by 2^kRescale and leaves O / l exact.
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
#define BD3_FWD_OCC 3
#endif
#ifndef BD3_FWD_STAGES
#define BD3_FWD_STAGES 3
#endif

// One class per 64-key tile for the wave (dead / full / partial, as walk
// index intervals of its row group): a full tile runs straight-line code with
// no mask arithmetic. MASK16: the block size is a multiple of 16.
template <int OCC, bool MASK16>
__global__ __launch_bounds__(256, OCC) void attn_fwd_dma_kernel(FwdArgs a) {
  constexpr int kBM = 128;  // query rows per workgroup: 4 waves x 32
  constexpr int kStages = BD3_FWD_STAGES;
  constexpr int kAhead = kStages - 1;  // tiles requested ahead of the one being computed
  __shared__ __attribute__((aligned(1024))) __bf16 smem[kStages][2][kSwTile];  // [stage][K|V]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = wave_uniform(tid >> 6);
  const int l32 = lane & 31;
  const int g = lane >> 5;

  const BlockOrder bo(a.bh, a.heads);
  const int tiles_half = a.n / kBM;
  const int t = tiles_half - 1 - (bo.rank >> 1);
  const int q0 = ((bo.rank & 1) ? 0 : a.n) + t * kBM;

  const uint16_t* qp = a.q + bo.b * a.sq.b + bo.h * a.sq.h;
  const uint16_t* kp = uniform_ptr(a.k + bo.b * a.sk.b + bo.h * a.sk.h);
  const uint16_t* vp = uniform_ptr(a.v + bo.b * a.sv.b + bo.h * a.sv.h);

  const int qrow0 = q0 + 32 * wave;
  const int myq = qrow0 + l32;
  bf16x8 qreg[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
    qreg[c] = __builtin_bit_cast(bf16x8, ld16(qp + (int64_t)myq * a.sq.s + 16 * c + 8 * g));

  const KeyRanges kr = train_key_ranges(q0, kBM, a.n, a.bs, kSwRows);
  const int t0 = wave_uniform(kr.t0), t2 = wave_uniform(kr.t2);
  const int n_first = wave_uniform(kr.t1 - kr.t0);
  const int n_tiles = n_first + wave_uniform(kr.t3 - kr.t2);
  auto tile_of = [&](int i) { return i < n_first ? t0 + i : t2 + (i - n_first); };

  // Wave w fills the 1 KB blocks 2w and 2w+1 (rows 16w .. 16w+15) of each K
  // and V tile: lane L fetches logical chunk (L%8) ^ swz(row) of row
  // 16w + 8j + L/8 (byte offsets from the tile's row 0).
  uint32_t koff[2], voff[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int r = 16 * wave + 8 * j + (lane >> 3);
    const int ch = 8 * ((lane & 7) ^ swz(r));
    koff[j] = (uint32_t)(2 * (r * (int)a.sk.s + ch));
    voff[j] = (uint32_t)(2 * (r * (int)a.sv.s + ch));
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
#pragma unroll
    for (int j = 0; j < 2; ++j) dma16(kn.cur, koff[j], dst + 1024u * j);
#pragma unroll
    for (int j = 0; j < 2; ++j) dma16(vn.cur, voff[j], dst + 8192u + 1024u * j);
    const bool jumping = walk.left == 1;
    walk.next();
    kn.next(jumping);
    vn.next(jumping);
  };

  // The first two tiles are requested before waiting for Q, so the two
  // latencies overlap. Consuming Q here (an empty asm reading it) makes the
  // compiler place its own wait for the Q loads at this point; that wait
  // also covers the direct loads issued after them, which is harmless.
#pragma unroll
  for (int i = 0; i < kAhead; ++i)
    if (i < n_tiles) issue(i);
  // Q times scale * log2(e), rounded to bf16: K Q'^T is then the base-2
  // exponent, and a chain started from -m gives S * scale * log2(e) - m.
#pragma unroll
  for (int c = 0; c < 4; ++c) qreg[c] = scale_bf16x8(qreg[c], a.scale_log2);
  const RowIntervals riv = train_row_intervals(myq, a.n, a.bs);
  const WalkClasses wc = uniform_walk(walk_classes(row_group_bounds(train_row_group(qrow0, 32, a.n, a.bs), a.n),
                                                   t0, n_first, t2, n_tiles - n_first, a.n, kSwRows, 0, kSwRows));

  f32x16 o[2] = {};  // O^T [d block]
  // mref: the row's reference maximum (log2 units); the score chains start
  // from negm = -mref. `valid` once the row has met a live key.
  float mref = 0.f, lsum = 0.f;
  bool valid = false;
  f32x16 negm = {};

  // One tile step over NSB 32-key halves of the current 64-key tile,
  // starting at half sb0 (NSB = 1: the other half is dead for this wave).
  auto step = [&](auto nsb_c, int sb0, int k0, int cls, const __bf16* ks, const __bf16* vs) {
    constexpr int NSB = decltype(nsb_c)::value;
    bf16x8 kop[NSB][4];
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
      for (int c = 0; c < 4; ++c) kop[sb][c] = sw_row_op(ks, 32 * (sb0 + sb), c, lane);
    f32x16 s[NSB];
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) s[sb] = mfma32(kop[sb][0], qreg[0], negm);
#pragma unroll
    for (int c = 1; c < 4; ++c)
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb) s[sb] = mfma32(kop[sb][c], qreg[c], s[sb]);

    // Partial tile: invisible pairs to -inf. With MASK16 (block size a
    // multiple of 16) the mask is constant on 1-row x 16-key strips:
    // registers 0-7 of a key block hold its keys 0-15, registers 8-15 keys
    // 16-31, so one test per strip decides them.
    if (cls == kPartial) {
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb) {
        const int kb = k0 + 32 * (sb0 + sb);
        if (MASK16) {
          const bool lo = iv_has(riv, kb), hi = iv_has(riv, kb + 16);
#pragma unroll
          for (int r = 0; r < 16; ++r) s[sb][r] = (r < 8 ? lo : hi) ? s[sb][r] : -INFINITY;
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kb + 8 * (r >> 2) + 4 * g + (r & 3);
            s[sb][r] = iv_has(riv, key) ? s[sb][r] : -INFINITY;
          }
        }
      }
    }
    // Row max of the shifted scores: four independent v_max3 chains.
    float mq[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      mq[q] = fmaxf(fmaxf(s[0][4 * q], s[0][4 * q + 1]), s[0][4 * q + 2]);
      mq[q] = fmaxf(mq[q], s[0][4 * q + 3]);
#pragma unroll
      for (int sb = 1; sb < NSB; ++sb) {
        mq[q] = fmaxf(fmaxf(mq[q], s[sb][4 * q]), s[sb][4 * q + 1]);
        mq[q] = fmaxf(fmaxf(mq[q], s[sb][4 * q + 2]), s[sb][4 * q + 3]);
      }
    }
    const float mt = max_xor32(fmaxf(fmaxf(mq[0], mq[1]), fmaxf(mq[2], mq[3])));
    // A new reference when the row had none (and this tile has a live key)
    // or its maximum grew by more than kRescale: the scores shift by delta,
    // O and l scale by 2^-delta.
    if (__ballot(!valid || mt > kRescale) != 0) {
      const float delta = valid ? fmaxf(mt, 0.f) : (mt == -INFINITY ? 0.f : mt);
      const float alpha = valid ? fast_exp2(-delta) : 1.f;
      valid = valid || mt != -INFINITY;
      mref += delta;
      negm = splat16(-mref);
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[sb][r] -= delta;
      lsum *= alpha;
      o[0] *= alpha;
      o[1] *= alpha;
    }
    bf16x8 pop[NSB][2];  // P^T operands [key block][16-key step]
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) {
      float p[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) p[r] = fast_exp2(s[sb][r]);
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        pop[sb][kc] = to_bf16x8(p[8 * kc], p[8 * kc + 1], p[8 * kc + 2], p[8 * kc + 3], p[8 * kc + 4],
                                p[8 * kc + 5], p[8 * kc + 6], p[8 * kc + 7]);
        lsum = sum_bf16x8(pop[sb][kc], lsum);
      }
    }
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) {
      bf16x8 vop[2][2];  // V^T operands of key block sb [16-key step][d block], read just before use
#pragma unroll
      for (int kc = 0; kc < 2; ++kc)
#pragma unroll
        for (int db = 0; db < 2; ++db) vop[kc][db] = sw_tr_op(vs, 32 * (sb0 + sb) + 16 * kc, 32 * db, lane);
#pragma unroll
      for (int kc = 0; kc < 2; ++kc)
#pragma unroll
        for (int db = 0; db < 2; ++db) o[db] = mfma32(vop[kc][db], pop[sb][kc], o[db]);
    }
  };

  // Every row group sees at least its own block, so n_tiles >= 1.
  vm_wait_barrier<0>();

  int cur = 0;
  for (int it = 0; it < n_tiles; ++it) {
    const bool pf = it + kAhead < n_tiles;
    if (pf) issue(cur + kAhead < kStages ? cur + kAhead : cur + kAhead - kStages);
    const int k0 = wave_uniform(tile_of(it) * kSwRows);
    // The tile's class for this wave's rows.
    if (walk_live(wc, it, n_first))
      step(std::integral_constant<int, 2>(), 0, k0, walk_full(wc, it, n_first) ? kFull : kPartial, smem[cur][0],
           smem[cur][1]);
    // Tile it+1 complete (the loads of later tiles may stay in flight), and
    // every wave is done reading stage `cur` before it is refilled.
    if (pf)
      vm_wait_barrier<4 * (kAhead - 1)>();
    else
      vm_wait_barrier<0>();
    cur = cur + 1 == kStages ? 0 : cur + 1;
  }

  const float ltot = sum_xor32(lsum);
  const float inv = 1.f / ltot;
  uint16_t* op = a.o + bo.b * a.so.b + bo.h * a.so.h + (int64_t)myq * a.so.s;
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int rg4 = 0; rg4 < 4; ++rg4)
      *reinterpret_cast<bf16x4*>(op + 32 * db + 8 * rg4 + 4 * g) =
          to_bf16x4(o[db][4 * rg4] * inv, o[db][4 * rg4 + 1] * inv, o[db][4 * rg4 + 2] * inv,
                    o[db][4 * rg4 + 3] * inv);
  if (g == 0) a.lse[(int64_t)bo.bh * 2 * a.n + myq] = (mref + fast_log2(ltot)) * kLn2;
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

}  // namespace bd3
