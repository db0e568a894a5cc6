// attn_bwd.hip - BD3-LM training attention backward for gfx950.
//
// Counterpart of BlockSparseFlashAttention.backward
// (kernels/BlockSparseFlashAttention.py:508-562): the Delta torch op (:525),
// block_sparse_attention_bwd_dq_kern (:368-452) and
// block_sparse_attention_dk_dv_bwd_kern (:212-328). Math per live pair:
//   P  = exp(S*scale - L)            (S = Q K^T, L the forward's lse)
//   dV = P^T dO,  dP = dO V^T,  dS = P o (dP - Delta),  Delta = rowsum(dO o O)
//   dK = scale * dS^T Q,  dQ = scale * dS K
//
// The reference splits this into a dQ kernel (S, dP, dQ) and a dK/dV kernel
// (S, dP, dV, dK): seven matrix products per live tile. Here one kernel does
// the five products once:
//   bwd_preprocess: Delta = rowsum(dO o O) (fp32), zeroes the fp32 dQ sum.
//   bwd_main: one workgroup per (batch*head, 128-key tile), four waves of 32
//     keys. Each wave keeps its K and V rows in registers (B operands of S
//     and dP) and its dK, dV sums in registers. It walks the 64-row query
//     tiles that see its keys (train_query_ranges), staging Q, dO, L, Delta
//     through LDS (double-buffered). dS goes through LDS once so that
//     dQ = dS K can be formed per 32x32 output block with a 128-key reduction
//     and added to the fp32 dQ sum with hardware float atomics.
//   bwd_finalize: dQ = bf16(scale * dQ sum).
//
// Operand layouts (see bd3_device.h):
//   S, dP (32 rows x 32 keys): A = Q / dO rows (b128 LDS reads), B = K / V
//     rows from registers; a lane then holds one key column and 16 rows.
//   dV, dK (32 keys x 32 d): A = P^T / dS^T straight from those registers,
//     B = dO / Q read transposed from row-major LDS (ds_read_b64_tr_b16).
//   dQ (32 rows x 32 d): A = dS read transposed from the [key][row] LDS copy,
//     B = K read transposed from the row-major LDS key tile.
#include "bd3_device.h"
#include "bd3_launch.h"
#include "bd3_mask.h"

namespace bd3 {
namespace {

constexpr int kNW = 4;
constexpr int kThreads = kNW * 64;
constexpr int kBK = 32 * kNW;  // keys per workgroup
constexpr int kBQ = 64;        // query rows per iteration
constexpr int kStride = 72;    // padded LDS row (bf16)
constexpr int kQChunks = (kBQ * kHeadDim / 8) / kThreads;  // 16-B chunks per thread

// ---------------------------------------------------------------------------
// Delta = rowsum(dO o O), zero dQ sum. One 8-lane group per row.
__global__ __launch_bounds__(256) void bwd_preprocess(BwdArgs a) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t rows = (int64_t)a.bh * 2 * a.n;
  const int64_t row = gid >> 3;
  const int part = gid & 7;
  if (row >= rows) return;
  const int bh = (int)(row / (2 * a.n));
  const int q = (int)(row - (int64_t)bh * 2 * a.n);
  const int b = bh / a.heads, h = bh - b * a.heads;
  const u32x4 dov = ld16(a.dout + b * a.sdo.b + h * a.sdo.h + (int64_t)q * a.sdo.s + 8 * part);
  const u32x4 ov = ld16(a.o + b * a.so.b + h * a.so.h + (int64_t)q * a.so.s + 8 * part);
  const bf16x8 d8 = __builtin_bit_cast(bf16x8, dov);
  const bf16x8 o8 = __builtin_bit_cast(bf16x8, ov);
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) acc += (float)d8[j] * (float)o8[j];
  acc += __shfl_xor(acc, 1, 64);
  acc += __shfl_xor(acc, 2, 64);
  acc += __shfl_xor(acc, 4, 64);
  if (part == 0) a.delta[row] = acc;
  float* zq = a.dq_acc + row * kHeadDim + 8 * part;
  reinterpret_cast<f32x4*>(zq)[0] = f32x4{};
  reinterpret_cast<f32x4*>(zq)[1] = f32x4{};
}

// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void bwd_main(BwdArgs a) {
  __shared__ __attribute__((aligned(16))) __bf16 s_qdo[2][2][kBQ * kStride];  // [stage][Q|dO]
  __shared__ __attribute__((aligned(16))) __bf16 s_k[kBK * kStride];          // key tile
  __shared__ __attribute__((aligned(16))) __bf16 s_ds[kBK * kStride];         // dS^T [key][row]
  __shared__ float s_l[2][kBQ], s_delta[2][kBQ];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int g = lane >> 5;

  // Heaviest key tiles first: clean tiles see the most query rows (tile 0 is
  // seen by every later row), noisy tiles only by their own blocks.
  const int tiles_half = a.n / kBK;
  const int rank = blockIdx.x / a.bh;
  const int bh = blockIdx.x - rank * a.bh;
  const int k0 = rank < tiles_half ? a.n + rank * kBK : (rank - tiles_half) * kBK;
  const int b = bh / a.heads, h = bh - b * a.heads;

  const uint16_t* qp = a.q + b * a.sq.b + h * a.sq.h;
  const uint16_t* kp = a.k + b * a.sk.b + h * a.sk.h;
  const uint16_t* vp = a.v + b * a.sv.b + h * a.sv.h;
  const uint16_t* dop = a.dout + b * a.sdo.b + h * a.sdo.h;
  const float* lp = a.lse + (int64_t)bh * 2 * a.n;
  const float* dp = a.delta + (int64_t)bh * 2 * a.n;
  float* dqp = a.dq_acc + (int64_t)bh * 2 * a.n * kHeadDim;

  // This wave's keys as B operands: lane holds key kw + l32, d = 16c + 8g.
  const int kw = k0 + 32 * wave;
  bf16x8 kreg[4], vreg[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    kreg[c] = __builtin_bit_cast(bf16x8, ld16(kp + (int64_t)(kw + l32) * a.sk.s + 16 * c + 8 * g));
    vreg[c] = __builtin_bit_cast(bf16x8, ld16(vp + (int64_t)(kw + l32) * a.sv.s + 16 * c + 8 * g));
  }
  // Whole key tile row-major in LDS for dQ = dS K.
#pragma unroll
  for (int j = 0; j < (kBK * kHeadDim / 8) / kThreads; ++j) {
    const int c = tid + j * kThreads;
    *reinterpret_cast<u32x4*>(&s_k[(c >> 3) * kStride + (c & 7) * 8]) =
        ld16(kp + (int64_t)(k0 + (c >> 3)) * a.sk.s + (c & 7) * 8);
  }

  const KeyRanges qr = train_query_ranges(k0, kBK, a.n, a.bs, kBQ);
  const int n_first = qr.t1 - qr.t0;
  const int n_tiles = n_first + (qr.t3 - qr.t2);
  auto tile_of = [&](int i) { return i < n_first ? qr.t0 + i : qr.t2 + (i - n_first); };

  u32x4 qbuf[kQChunks], dobuf[kQChunks];
  float lbuf = 0.f, dbuf = 0.f;
  auto load_q = [&](int i) {
    const int q0 = tile_of(i) * kBQ;
#pragma unroll
    for (int j = 0; j < kQChunks; ++j) {
      const int c = tid + j * kThreads;
      const int row = q0 + (c >> 3);
      qbuf[j] = ld16(qp + (int64_t)row * a.sq.s + (c & 7) * 8);
      dobuf[j] = ld16(dop + (int64_t)row * a.sdo.s + (c & 7) * 8);
    }
    if (tid < kBQ) {
      lbuf = lp[q0 + tid] * kLog2e;  // natural -> log2 units
      dbuf = dp[q0 + tid];
    }
  };
  auto store_q = [&](int stage) {
#pragma unroll
    for (int j = 0; j < kQChunks; ++j) {
      const int c = tid + j * kThreads;
      const int off = (c >> 3) * kStride + (c & 7) * 8;
      *reinterpret_cast<u32x4*>(&s_qdo[stage][0][off]) = qbuf[j];
      *reinterpret_cast<u32x4*>(&s_qdo[stage][1][off]) = dobuf[j];
    }
    if (tid < kBQ) {
      s_l[stage][tid] = lbuf;
      s_delta[stage][tid] = dbuf;
    }
  };

  f32x16 dk[2] = {}, dv[2] = {};  // [db]: lane = d column 32db + l32, key rows

  if (n_tiles > 0) {
    load_q(0);
    store_q(0);
  }
  __syncthreads();

  // Transposed-read addressing inside a 16-lane group (bd3_device.h):
  const int tr_row = (lane & 15) >> 2;                       // + r0
  const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);  // + c0

  for (int it = 0; it < n_tiles; ++it) {
    const int stage = it & 1;
    if (it + 1 < n_tiles) load_q(it + 1);
    const int q0 = tile_of(it) * kBQ;
    const __bf16* qs = s_qdo[stage][0];
    const __bf16* dos = s_qdo[stage][1];

    // Live classes of every (wave, row block) of this tile, uniform across
    // the workgroup so dQ can skip dead key chunks.
    int cls[kNW][2];
#pragma unroll
    for (int w = 0; w < kNW; ++w)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
        cls[w][qb] = train_class(q0 + 32 * qb, 32, k0 + 32 * w, 32, a.n, a.bs);

#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const int c = cls[wave][qb];
      if (c == kNone) continue;
      // S and dP: 32 rows x 32 keys; lane = key kw + l32, rows via registers.
      f32x16 s = {}, dpm = {};
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) {
        const int off = (32 * qb + l32) * kStride + 16 * cc + 8 * g;
        const bf16x8 qa = *reinterpret_cast<const bf16x8*>(&qs[off]);
        const bf16x8 da = *reinterpret_cast<const bf16x8*>(&dos[off]);
        s = mfma32(qa, kreg[cc], s);
        dpm = mfma32(da, vreg[cc], dpm);
      }
      // P and dS. Register r <-> row 32qb + 8(r/4) + 4g + r%4.
      float p[16], ds[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int rl = 32 * qb + 8 * (r >> 2) + 4 * g + (r & 3);
        const float lrow = s_l[stage][rl];
        const float drow = s_delta[stage][rl];
        float pv = fast_exp2(fmaf(s[r], a.scale_log2, -lrow));
        if (c == kPartial && !train_visible(q0 + rl, kw + l32, a.n, a.bs)) pv = 0.f;
        p[r] = pv;
        ds[r] = pv * (dpm[r] - drow);
      }
      // dS^T into LDS as [key][row] (4 consecutive rows per 8-byte store).
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int rl = 32 * qb + 8 * rg + 4 * g;
        *reinterpret_cast<bf16x4*>(&s_ds[(32 * wave + l32) * kStride + rl]) =
            to_bf16x4(ds[4 * rg], ds[4 * rg + 1], ds[4 * rg + 2], ds[4 * rg + 3]);
      }
      // dV += P^T dO, dK += dS^T Q over this block's 32 rows (two K=16 steps).
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const bf16x8 pa = to_bf16x8(p[8 * kc], p[8 * kc + 1], p[8 * kc + 2], p[8 * kc + 3],
                                    p[8 * kc + 4], p[8 * kc + 5], p[8 * kc + 6], p[8 * kc + 7]);
        const bf16x8 sa = to_bf16x8(ds[8 * kc], ds[8 * kc + 1], ds[8 * kc + 2], ds[8 * kc + 3],
                                    ds[8 * kc + 4], ds[8 * kc + 5], ds[8 * kc + 6], ds[8 * kc + 7]);
        const int row = 32 * qb + 16 * kc + 4 * g + tr_row;
#pragma unroll
        for (int db = 0; db < 2; ++db) {
          const int col = 32 * db + tr_col;
          const bf16x8 dob = cat8(lds_read_tr(&dos[row * kStride + col]),
                                  lds_read_tr(&dos[(row + 8) * kStride + col]));
          const bf16x8 qbv = cat8(lds_read_tr(&qs[row * kStride + col]),
                                  lds_read_tr(&qs[(row + 8) * kStride + col]));
          dv[db] = mfma32(pa, dob, dv[db]);
          dk[db] = mfma32(sa, qbv, dk[db]);
        }
      }
    }
    __syncthreads();  // dS^T complete

    // dQ block (rows 32*qbo .. +32, d 32*dbo .. +32) over the live key chunks.
    {
      const int qbo = wave >> 1, dbo = wave & 1;
      f32x16 dq = {};
      bool any = false;
#pragma unroll
      for (int w = 0; w < kNW; ++w) {
        if (cls[w][qbo] == kNone) continue;
        any = true;
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
          // natural key order: rows 32w + 16kc + 8g + tr_row (+4)
          const int krow = 32 * w + 16 * kc + 8 * g + tr_row;
          const bf16x8 dsa = cat8(lds_read_tr(&s_ds[krow * kStride + 32 * qbo + tr_col]),
                                  lds_read_tr(&s_ds[(krow + 4) * kStride + 32 * qbo + tr_col]));
          const bf16x8 kb = cat8(lds_read_tr(&s_k[krow * kStride + 32 * dbo + tr_col]),
                                 lds_read_tr(&s_k[(krow + 4) * kStride + 32 * dbo + tr_col]));
          dq = mfma32(dsa, kb, dq);
        }
      }
      if (any) {
        // lane = d column 32dbo + l32; register r <-> row 8(r/4) + 4g + r%4
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = q0 + 32 * qbo + 8 * (r >> 2) + 4 * g + (r & 3);
          unsafeAtomicAdd(dqp + (int64_t)row * kHeadDim + 32 * dbo + l32, dq[r]);
        }
      }
    }

    if (it + 1 < n_tiles) store_q(stage ^ 1);
    __syncthreads();
  }

  // dK = scale * sum dS^T Q, dV = sum P^T dO. Lane = d column; key rows.
  uint16_t* dkp = a.dk + b * a.sdk.b + h * a.sdk.h;
  uint16_t* dvp = a.dv + b * a.sdv.b + h * a.sdv.h;
#pragma unroll
  for (int db = 0; db < 2; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = kw + 8 * (r >> 2) + 4 * g + (r & 3);
      const int d = 32 * db + l32;
      const __bf16 kv = (__bf16)(dk[db][r] * a.scale);
      const __bf16 vv = (__bf16)dv[db][r];
      dkp[(int64_t)key * a.sdk.s + d] = __builtin_bit_cast(uint16_t, kv);
      dvp[(int64_t)key * a.sdv.s + d] = __builtin_bit_cast(uint16_t, vv);
    }
}

// ---------------------------------------------------------------------------
// dQ = bf16(scale * dQ sum). One thread per 8 elements.
__global__ __launch_bounds__(256) void bwd_finalize(BwdArgs a) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t rows = (int64_t)a.bh * 2 * a.n;
  const int64_t row = gid >> 3;
  const int part = gid & 7;
  if (row >= rows) return;
  const int bh = (int)(row / (2 * a.n));
  const int q = (int)(row - (int64_t)bh * 2 * a.n);
  const int b = bh / a.heads, h = bh - b * a.heads;
  const float* src = a.dq_acc + row * kHeadDim + 8 * part;
  const f32x4 x0 = reinterpret_cast<const f32x4*>(src)[0];
  const f32x4 x1 = reinterpret_cast<const f32x4*>(src)[1];
  const bf16x8 y = to_bf16x8(x0[0] * a.scale, x0[1] * a.scale, x0[2] * a.scale, x0[3] * a.scale,
                             x1[0] * a.scale, x1[1] * a.scale, x1[2] * a.scale, x1[3] * a.scale);
  *reinterpret_cast<bf16x8*>(a.dq + b * a.sdq.b + h * a.sdq.h + (int64_t)q * a.sdq.s + 8 * part) = y;
}

}  // namespace

hipError_t launch_attn_bwd(const BwdArgs& a, hipStream_t stream) {
  const int64_t rows = (int64_t)a.bh * 2 * a.n;
  const int eblocks = (int)((rows * 8 + 255) / 256);
  hipLaunchKernelGGL(bwd_preprocess, dim3(eblocks), dim3(256), 0, stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(bwd_main, dim3(a.bh * (2 * a.n / kBK)), dim3(kThreads), 0, stream, a);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(bwd_finalize, dim3(eblocks), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace bd3
