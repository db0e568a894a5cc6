// attn_bwd.hip - BD3-LM training attention backward for gfx950.
//
// Counterpart of BlockSparseFlashAttention.backward
// (kernels/BlockSparseFlashAttention.py:508-562): the Delta torch op (:525),
// block_sparse_attention_bwd_dq_kern (:368-452) and
// block_sparse_attention_dk_dv_bwd_kern (:212-328). Per live pair:
//   P  = exp(S*scale - L)            (S = Q K^T, L the forward's lse)
//   dV = P^T dO,  dP = dO V^T,  dS = P o (dP - Delta),  Delta = rowsum(dO o O)
//   dK = scale * dS^T Q,  dQ = scale * dS K
// Like the reference, two kernels: one owns query rows and forms dQ, the
// other owns keys and forms dK, dV; both recompute S and dP. Neither needs
// atomics or a transposed copy of dS, and results are deterministic.
//
// attn_bwd_dq_kernel (query-stationary, the forward's schedule): NW waves of
//   64 rows. Q and dO rows live in registers as B operands; K, V key tiles are
//   staged through LDS. S^T = K Q^T and dP^T = V dO^T put one row per lane,
//   so L and Delta are per-lane scalars; dQ^T += K^T dS^T reads K^T from the
//   row-major LDS tile with ds_read_b64_tr_b16. Delta = rowsum(dO o O) is
//   formed here from the row registers and stored for the second kernel
//   (this fuses the reference's separate Delta op).
// attn_bwd_dkdv_kernel (key-stationary): NW waves of 64 keys. K and V rows
//   live in registers as B operands of S = Q K^T and dP = dO V^T, which put
//   one key per lane; query tiles (Q, dO, L, Delta) are staged through LDS.
//   dV += P^T dO and dK += dS^T Q take P^T / dS^T straight from registers and
//   dO / Q transposed from LDS. dK, dV are written through LDS as 16-byte rows.
#include "bd3_device.h"
#include "bd3_launch.h"
#include "bd3_mask.h"
#include "bd3_tile.h"

namespace bd3 {
namespace {

// ---------------------------------------------------------------------------
template <int NW, int RB, int OCC>
__global__ __launch_bounds__(NW * 64, OCC) void attn_bwd_dq_kernel(BwdArgs a) {
  constexpr int kThreads = NW * 64;
  constexpr int kBM = 32 * RB * NW;
  __shared__ __attribute__((aligned(16))) __bf16 smem[2][2][kTileElems];  // [stage][K|V]

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
  const uint16_t* kp = a.k + bo.b * a.sk.b + bo.h * a.sk.h;
  const uint16_t* vp = a.v + bo.b * a.sv.b + bo.h * a.sv.h;
  const uint16_t* opp = a.o + bo.b * a.so.b + bo.h * a.so.h;
  const uint16_t* dop = a.dout + bo.b * a.sdo.b + bo.h * a.sdo.h;
  const int64_t rowbase = (int64_t)bo.bh * 2 * a.n;

  const int qrow0 = q0 + 32 * RB * wave;
  bf16x8 qreg[RB][4], doreg[RB][4];
  RowIntervals riv[RB];
  RowGroup rgs[RB];
  float lrow[RB], drow[RB];
#pragma unroll
  for (int qb = 0; qb < RB; ++qb) {
    const int myq = qrow0 + 32 * qb + l32;
    riv[qb] = train_row_intervals(myq, a.n, a.bs);
    rgs[qb] = uniform_row_group(qrow0 + 32 * qb, 32, a.n, a.bs);
    float dsum = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int col = 16 * c + 8 * g;
      qreg[qb][c] = __builtin_bit_cast(bf16x8, ld16(qp + (int64_t)myq * a.sq.s + col));
      doreg[qb][c] = __builtin_bit_cast(bf16x8, ld16(dop + (int64_t)myq * a.sdo.s + col));
      const bf16x8 ov = __builtin_bit_cast(bf16x8, ld16(opp + (int64_t)myq * a.so.s + col));
#pragma unroll
      for (int j = 0; j < 8; ++j) dsum = fmaf((float)doreg[qb][c][j], (float)ov[j], dsum);
    }
    drow[qb] = sum_xor32(dsum);
    lrow[qb] = a.lse[rowbase + myq] * kLog2e;
    if (g == 0) a.delta[rowbase + myq] = drow[qb];
  }

  const KeyRanges kr = train_key_ranges(q0, kBM, a.n, a.bs, kTileRows);
  const int t0 = wave_uniform(kr.t0), t2 = wave_uniform(kr.t2);
  const int n_first = wave_uniform(kr.t1 - kr.t0);
  const int n_tiles = n_first + wave_uniform(kr.t3 - kr.t2);
  auto tile_of = [&](int i) { return i < n_first ? t0 + i : t2 + (i - n_first); };

  TileStager<kThreads, 2> st;
  {
    const int64_t rs[2] = {a.sk.s, a.sv.s};
    st.init(tid, rs);
  }
  auto stage_load = [&](int i) {
    const int64_t k0 = (int64_t)tile_of(i) * kTileRows;
    const uint16_t* base[2] = {kp + k0 * a.sk.s, vp + k0 * a.sv.s};
    st.load(base);
  };

  f32x16 dq[RB][2];  // dQ^T [row block][d block]
#pragma unroll
  for (int qb = 0; qb < RB; ++qb) dq[qb][0] = dq[qb][1] = f32x16{};

  // n_tiles >= 1 (every row group sees its own block): unconditional prologue.
  {
    stage_load(0);
    __bf16* dst[2] = {smem[0][0], smem[0][1]};
    st.store(dst);
  }
  __syncthreads();

  for (int it = 0; it < n_tiles; ++it) {
    const int stage = it & 1;
    if (it + 1 < n_tiles) stage_load(it + 1);
    const int k0 = wave_uniform(tile_of(it) * kTileRows);
    const __bf16* ks = smem[stage][0];
    const __bf16* vs = smem[stage][1];

    int cls[RB][2];
    int live[2] = {kNone, kNone};
#pragma unroll
    for (int qb = 0; qb < RB; ++qb)
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        cls[qb][sb] = row_group_class(rgs[qb], k0 + 32 * sb, 32, a.n);
        live[sb] |= cls[qb][sb];
      }

    bf16x8 dsop[RB][2][2];  // dS^T operands [row block][key block][16-key step]
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      if (live[sb] == kNone) continue;
      f32x16 s[RB], dp[RB];
#pragma unroll
      for (int qb = 0; qb < RB; ++qb) s[qb] = dp[qb] = f32x16{};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const bf16x8 kop = lds_row_op(ks, 32 * sb, c, lane);
        const bf16x8 vop = lds_row_op(vs, 32 * sb, c, lane);
#pragma unroll
        for (int qb = 0; qb < RB; ++qb)
          if (cls[qb][sb] != kNone) {
            s[qb] = mfma32(kop, qreg[qb][c], s[qb]);
            dp[qb] = mfma32(vop, doreg[qb][c], dp[qb]);
          }
      }
#pragma unroll
      for (int qb = 0; qb < RB; ++qb) {
        if (cls[qb][sb] == kNone) continue;
        float ds[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float p = fast_exp2(fmaf(s[qb][r], a.scale_log2, -lrow[qb]));
          if (cls[qb][sb] == kPartial) {
            const int key = k0 + 32 * sb + 8 * (r >> 2) + 4 * g + (r & 3);
            p = iv_has(riv[qb], key) ? p : 0.f;
          }
          ds[r] = p * (dp[qb][r] - drow[qb]);
        }
#pragma unroll
        for (int kc = 0; kc < 2; ++kc)
          dsop[qb][sb][kc] = to_bf16x8(ds[8 * kc], ds[8 * kc + 1], ds[8 * kc + 2], ds[8 * kc + 3],
                                       ds[8 * kc + 4], ds[8 * kc + 5], ds[8 * kc + 6], ds[8 * kc + 7]);
      }
    }
    // dQ^T += K^T dS^T, K^T operands shared by both row blocks.
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      if (live[sb] == kNone) continue;
#pragma unroll
      for (int kc = 0; kc < 2; ++kc)
#pragma unroll
        for (int db = 0; db < 2; ++db) {
          const bf16x8 kt = lds_tr_op(ks, 32 * sb + 16 * kc, 32 * db, lane);
#pragma unroll
          for (int qb = 0; qb < RB; ++qb)
            if (cls[qb][sb] != kNone) dq[qb][db] = mfma32(kt, dsop[qb][sb][kc], dq[qb][db]);
        }
    }

    if (it + 1 < n_tiles) {
      __bf16* dst[2] = {smem[stage ^ 1][0], smem[stage ^ 1][1]};
      st.store(dst);
    }
    __syncthreads();
  }

  uint16_t* dqp = a.dq + bo.b * a.sdq.b + bo.h * a.sdq.h;
#pragma unroll
  for (int qb = 0; qb < RB; ++qb) {
    const int myq = qrow0 + 32 * qb + l32;
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int d = 32 * db + 8 * rg + 4 * g;
        *reinterpret_cast<bf16x4*>(dqp + (int64_t)myq * a.sdq.s + d) =
            to_bf16x4(dq[qb][db][4 * rg] * a.scale, dq[qb][db][4 * rg + 1] * a.scale,
                      dq[qb][db][4 * rg + 2] * a.scale, dq[qb][db][4 * rg + 3] * a.scale);
      }
  }
}

// ---------------------------------------------------------------------------
template <int NW, int KB, int OCC>
__global__ __launch_bounds__(NW * 64, OCC) void attn_bwd_dkdv_kernel(BwdArgs a) {
  constexpr int kThreads = NW * 64;
  constexpr int kBK = 32 * KB * NW;
  static_assert(NW <= 4, "the epilogue gives each wave one of the four staging tiles");
  __shared__ __attribute__((aligned(16))) __bf16 smem[2][2][kTileElems];  // [stage][Q|dO]
  __shared__ __attribute__((aligned(16))) float s_ld[2][2][kTileRows];    // [stage][L|Delta]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = wave_uniform(tid >> 6);
  const int l32 = lane & 31;
  const int g = lane >> 5;

  // Heaviest key tiles first: clean tiles are seen by the most rows.
  const BlockOrder bo(a.bh, a.heads);
  const int tiles_half = a.n / kBK;
  const int k0 = bo.rank < tiles_half ? a.n + bo.rank * kBK : (bo.rank - tiles_half) * kBK;

  const uint16_t* qp = a.q + bo.b * a.sq.b + bo.h * a.sq.h;
  const uint16_t* kp = a.k + bo.b * a.sk.b + bo.h * a.sk.h;
  const uint16_t* vp = a.v + bo.b * a.sv.b + bo.h * a.sv.h;
  const uint16_t* dop = a.dout + bo.b * a.sdo.b + bo.h * a.sdo.h;
  const int64_t rowbase = (int64_t)bo.bh * 2 * a.n;

  const int kw = k0 + 32 * KB * wave;
  bf16x8 kreg[KB][4], vreg[KB][4];
  RowIntervals civ[KB];
  KeyGroup kgs[KB];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    const int key = kw + 32 * kb + l32;
    civ[kb] = train_col_intervals(key, a.n, a.bs);
    kgs[kb] = uniform_key_group(kw + 32 * kb, 32, a.n, a.bs);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      kreg[kb][c] = __builtin_bit_cast(bf16x8, ld16(kp + (int64_t)key * a.sk.s + 16 * c + 8 * g));
      vreg[kb][c] = __builtin_bit_cast(bf16x8, ld16(vp + (int64_t)key * a.sv.s + 16 * c + 8 * g));
    }
  }

  const KeyRanges qr = train_query_ranges(k0, kBK, a.n, a.bs, kTileRows);
  const int t0 = wave_uniform(qr.t0), t2 = wave_uniform(qr.t2);
  const int n_first = wave_uniform(qr.t1 - qr.t0);
  const int n_tiles = n_first + wave_uniform(qr.t3 - qr.t2);
  auto tile_of = [&](int i) { return i < n_first ? t0 + i : t2 + (i - n_first); };

  TileStager<kThreads, 2> st;
  {
    const int64_t rs[2] = {a.sq.s, a.sdo.s};
    st.init(tid, rs);
  }
  float lbuf = 0.f, dbuf = 0.f;
  auto stage_load = [&](int i) {
    const int64_t q0 = (int64_t)tile_of(i) * kTileRows;
    const uint16_t* base[2] = {qp + q0 * a.sq.s, dop + q0 * a.sdo.s};
    st.load(base);
    if (tid < kTileRows) {
      lbuf = a.lse[rowbase + q0 + tid] * kLog2e;
      dbuf = a.delta[rowbase + q0 + tid];
    }
  };
  auto stage_store = [&](int stage) {
    __bf16* dst[2] = {smem[stage][0], smem[stage][1]};
    st.store(dst);
    if (tid < kTileRows) {
      s_ld[stage][0][tid] = lbuf;
      s_ld[stage][1][tid] = dbuf;
    }
  };

  f32x16 dk[KB][2], dv[KB][2];  // [key block][d block]: lane = d column
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) dk[kb][0] = dk[kb][1] = dv[kb][0] = dv[kb][1] = f32x16{};

  // n_tiles >= 1 (every key group is seen by its own block): unconditional prologue.
  stage_load(0);
  stage_store(0);
  __syncthreads();

  for (int it = 0; it < n_tiles; ++it) {
    const int stage = it & 1;
    if (it + 1 < n_tiles) stage_load(it + 1);
    const int q0 = wave_uniform(tile_of(it) * kTileRows);
    const __bf16* qs = smem[stage][0];
    const __bf16* dos = smem[stage][1];

    int cls[2][KB];  // [row block][key block]
    int live[2] = {kNone, kNone};  // per row block: live for any key block
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        cls[qb][kb] = key_group_class(kgs[kb], q0 + 32 * qb, 32, a.n);
        live[qb] |= cls[qb][kb];
      }

#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      if (live[qb] == kNone) continue;
      // Q and dO rows of this block as A operands, read once for both key blocks.
      bf16x8 qa[4], da[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        qa[c] = lds_row_op(qs, 32 * qb, c, lane);
        da[c] = lds_row_op(dos, 32 * qb, c, lane);
      }
      bf16x8 pop[KB][2], dsop[KB][2];  // [key block][16-row step]
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        if (cls[qb][kb] == kNone) continue;
        // S, dP (rows x keys): lane = key column, register r <-> row
        // 32qb + 8(r/4) + 4g + r%4.
        f32x16 s = {}, dp = {};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          s = mfma32(qa[c], kreg[kb][c], s);
          dp = mfma32(da[c], vreg[kb][c], dp);
        }
        float p[16], ds[16];
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) {
          const f32x4 lr = *reinterpret_cast<const f32x4*>(&s_ld[stage][0][32 * qb + 8 * rg + 4 * g]);
          const f32x4 dr = *reinterpret_cast<const f32x4*>(&s_ld[stage][1][32 * qb + 8 * rg + 4 * g]);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int r = 4 * rg + j;
            float pv = fast_exp2(fmaf(s[r], a.scale_log2, -lr[j]));
            if (cls[qb][kb] == kPartial) {
              const int row = q0 + 32 * qb + 8 * rg + 4 * g + j;
              pv = iv_has(civ[kb], row) ? pv : 0.f;
            }
            p[r] = pv;
            ds[r] = pv * (dp[r] - dr[j]);
          }
        }
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
          pop[kb][kc] = to_bf16x8(p[8 * kc], p[8 * kc + 1], p[8 * kc + 2], p[8 * kc + 3],
                                  p[8 * kc + 4], p[8 * kc + 5], p[8 * kc + 6], p[8 * kc + 7]);
          dsop[kb][kc] = to_bf16x8(ds[8 * kc], ds[8 * kc + 1], ds[8 * kc + 2], ds[8 * kc + 3],
                                   ds[8 * kc + 4], ds[8 * kc + 5], ds[8 * kc + 6], ds[8 * kc + 7]);
        }
      }
      // dV += P^T dO, dK += dS^T Q over this row block; the transposed dO / Q
      // operands are shared by both key blocks.
#pragma unroll
      for (int kc = 0; kc < 2; ++kc)
#pragma unroll
        for (int db = 0; db < 2; ++db) {
          const bf16x8 dot = lds_tr_op(dos, 32 * qb + 16 * kc, 32 * db, lane);
          const bf16x8 qt = lds_tr_op(qs, 32 * qb + 16 * kc, 32 * db, lane);
#pragma unroll
          for (int kb = 0; kb < KB; ++kb)
            if (cls[qb][kb] != kNone) {
              dv[kb][db] = mfma32(pop[kb][kc], dot, dv[kb][db]);
              dk[kb][db] = mfma32(dsop[kb][kc], qt, dk[kb][db]);
            }
        }
    }

    if (it + 1 < n_tiles) stage_store(stage ^ 1);
    __syncthreads();
  }

  // Epilogue: each wave transposes its 32*KB keys x 64 d of dK, then dV, through
  // its own LDS slice into row-major bf16, then writes 16-byte row chunks.
  __bf16* tile = &smem[0][0][0] + wave * kTileElems;
  uint16_t* outs[2] = {a.dk + bo.b * a.sdk.b + bo.h * a.sdk.h, a.dv + bo.b * a.sdv.b + bo.h * a.sdv.h};
  const int64_t ostr[2] = {a.sdk.s, a.sdv.s};
#pragma unroll
  for (int which = 0; which < 2; ++which) {
    const float mul = which == 0 ? a.scale : 1.f;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int krow = 32 * kb + 8 * (r >> 2) + 4 * g + (r & 3);
          const float x = (which == 0 ? dk[kb][db][r] : dv[kb][db][r]) * mul;
          tile[krow * kLdsStride + 32 * db + l32] = (__bf16)x;
        }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int j = 0; j < 4 * KB; ++j) {
      const int row = (lane >> 3) + 8 * j;
      const u32x4 v = *reinterpret_cast<const u32x4*>(&tile[row * kLdsStride + 8 * (lane & 7)]);
      st16(outs[which] + (int64_t)(kw + row) * ostr[which] + 8 * (lane & 7), v);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
  }
}

#ifndef BD3_DQ_NW
#define BD3_DQ_NW 4
#endif
#ifndef BD3_DQ_RB
#define BD3_DQ_RB 1
#endif
#ifndef BD3_KV_NW
#define BD3_KV_NW 4
#endif
#ifndef BD3_KV_KB
#define BD3_KV_KB 1
#endif
#ifndef BD3_DQ_OCC
#define BD3_DQ_OCC 3
#endif
#ifndef BD3_KV_OCC
#define BD3_KV_OCC 2
#endif

}  // namespace

hipError_t launch_attn_bwd_dq(const BwdArgs& a, hipStream_t stream) {
  constexpr int kNW = BD3_DQ_NW, kRB = BD3_DQ_RB, kOcc = BD3_DQ_OCC, kBM = 32 * kNW * kRB;
  if (a.n % kBM == 0)
    hipLaunchKernelGGL((attn_bwd_dq_kernel<kNW, kRB, kOcc>), dim3(a.bh * (2 * a.n / kBM)), dim3(kNW * 64), 0,
                       stream, a);
  else  // n % 128 == 0 always holds (validated)
    hipLaunchKernelGGL((attn_bwd_dq_kernel<4, 1, 2>), dim3(a.bh * (2 * a.n / 128)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_attn_bwd_dkdv(const BwdArgs& a, hipStream_t stream) {
  constexpr int kNW = BD3_KV_NW, kKB = BD3_KV_KB, kOcc = BD3_KV_OCC, kBK = 32 * kNW * kKB;
  if (a.n % kBK == 0)
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<kNW, kKB, kOcc>), dim3(a.bh * (2 * a.n / kBK)), dim3(kNW * 64), 0,
                       stream, a);
  else
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<4, 1, 2>), dim3(a.bh * (2 * a.n / 128)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace bd3
