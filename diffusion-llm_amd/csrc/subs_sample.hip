// subs_sample.hip - one ancestral denoising step of BD3-LM sampling, fused:
// SUBS parameterization + categorical draw + carry-over of unmasked tokens.
//
// Counterpart of subs_parameterization (model/subs.py:11-43) followed by the
// sampler's update (sample/sampler.py:110-122) and sample_categorical
// (sample/sampler.py:11-34), for rows whose token is [MASK] (the others keep
// their token, which is what torch.where(block != mask, block, new) does):
//   x_i   = logits_i + bias_i            (bias = NEG_INF = -1e6 at [MASK], in the logits dtype)
//   lp_i  = (x_i - max x) - log(sum_j exp(x_j - max x))   (model/modules.py:791-799)
//   q_i   = double(exp(lp_i)) * (1 - s/t),  q_mask = s/t
//   new   = argmax_i q_i / (EPS - log(u_i + EPS)),  u_i ~ U[0, 1) in float64, EPS = 1e-10
// in the dtypes the reference runs under bf16 autocast: for bf16 logits the
// bias add and the shift x - max are bf16 ops (rounded), exp / sum / log and
// the final subtraction are fp32; for fp32 logits everything up to q is
// fp32. q, the noise and the ratio are float64, as in the reference.
// The uniforms come either from the caller (u, float64 per element: the
// reference's torch.rand_like draw, for exact reproduction) or from the
// counter-based Philox4x32-10 generator (Salmon, Moraes, Dror, Shaw,
// "Parallel random numbers: as easy as 1, 2, 3", SC'11), keyed by a 64-bit
// seed with the 64-bit element-pair index and a 64-bit offset as counter, so
// no noise tensor is materialised.
//
// One workgroup per row (1024 threads; a row is long and rows are few, so
// the parallelism is inside the row): pass 1 the max, pass 2 the sum of
// exponentials, pass 3 the noisy ratio and its argmax (first index on ties,
// as torch.argmax). bf16 rows up to 65528 elements are staged in LDS with
// 16-byte loads (one HBM read); others are re-read from L2 / MALL.
// Logits must be finite (the token drawn for a row with NaN / inf logits is
// unspecified).
#include "bd3_device.h"
#include "bd3_launch.h"

namespace bd3 {
namespace {

constexpr int kSubsThreads = 1024;
constexpr float kNegInf = -1e6f;   // model/subs.py:8
constexpr double kEps = 1e-10;     // sample/sampler.py:8

__device__ __forceinline__ float bf16_round(float f) {
  return (float)(__bf16)f;  // round to nearest even
}

// Philox4x32-10 block: counter c, key k (Random123's philox4x32, 10 rounds).
__device__ __forceinline__ void philox4x32_10(uint32_t c[4], uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = (uint64_t)0xD2511F53u * c[0];
    const uint64_t p1 = (uint64_t)0xCD9E8D57u * c[2];
    const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0;
    const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1;
    c[0] = n0;
    c[1] = (uint32_t)p1;
    c[2] = n2;
    c[3] = (uint32_t)p0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
}

// 53-bit uniform in [0, 1) from 64 random bits.
__device__ __forceinline__ double u53(uint32_t lo, uint32_t hi) {
  const uint64_t v = ((uint64_t)hi << 32) | lo;
  return (double)(v >> 11) * 0x1.0p-53;
}

template <typename T>
__device__ __forceinline__ float load_logit(const T* p, int i);
template <>
__device__ __forceinline__ float load_logit<uint16_t>(const uint16_t* p, int i) {
  return __builtin_bit_cast(float, (uint32_t)p[i] << 16);
}
template <>
__device__ __forceinline__ float load_logit<float>(const float* p, int i) {
  return p[i];
}

// x_i: the logit l of element i plus the [MASK] bias, rounded to the logits dtype.
template <typename T>
__device__ __forceinline__ float biased(float l, int i, int mask_index) {
  if (i != mask_index) return l;
  if constexpr (sizeof(T) == 2) {
    return bf16_round(l + bf16_round(kNegInf));
  } else {
    return l + kNegInf;
  }
}

template <typename T>
__device__ __forceinline__ float shifted(float x, float m) {
  if constexpr (sizeof(T) == 2) {
    return bf16_round(x - m);
  } else {
    return x - m;
  }
}

__device__ __forceinline__ float block_max(float v, float* red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < kSubsThreads / 64; ++i) r = fmaxf(r, red[i]);
  __syncthreads();
  return r;
}

__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < kSubsThreads / 64; ++i) r += red[i];
  __syncthreads();
  return r;
}

// (value, index) argmax, first index on ties (torch.argmax). The ratios are
// finite and non-negative for finite logits: q >= 0 and the noise term
// EPS - log(u + EPS) > 0 for every u in [0, 1).
__device__ __forceinline__ bool better(double v, int i, double bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

// bf16 rows of up to kMaxStaged elements are copied to LDS once (16-byte
// loads) and the three passes read them there; fp32 rows and longer bf16
// rows are read from global memory in every pass.
constexpr int kMaxStaged = 65536 - 8;

template <typename T, bool STAGED>
__global__ __launch_bounds__(kSubsThreads) void subs_sample_kernel(SubsArgs a) {
  __shared__ float red[kSubsThreads / 64];
  __shared__ double bval[kSubsThreads / 64];
  __shared__ int bidx[kSubsThreads / 64];
  __shared__ __attribute__((aligned(16))) uint16_t srow[STAGED ? kMaxStaged + 8 : 8];
  constexpr int NT = kSubsThreads;
  const int row = blockIdx.x;
  const int64_t xt = a.xt[row];
  if (xt != a.mask_index) {  // carry-over: an unmasked token stays (uniform per workgroup)
    if (threadIdx.x == 0) a.out[row] = xt;
    return;
  }
  const T* lp = static_cast<const T*>(a.logits) + (int64_t)row * a.ld;
  const int V = a.vocab;

  // Element i sits at LDS slot i + sh, with sh chosen so that the first
  // element on a 16-byte boundary of the row lands on a 16-byte slot.
  int sh = 0;
  if constexpr (STAGED) {
    const uint16_t* p = reinterpret_cast<const uint16_t*>(lp);
    const int mis = (int)(reinterpret_cast<uintptr_t>(p) & 15);  // even: bf16 rows are 2-byte aligned
    int head = ((16 - mis) & 15) >> 1;                            // elements before that boundary
    head = head < V ? head : V;
    sh = (8 - head) & 7;
    const int nb = (V - head) >> 3;
    const int tail0 = head + 8 * nb;
    if ((int)threadIdx.x < head) srow[threadIdx.x + sh] = p[threadIdx.x];
    for (int k = threadIdx.x; k < nb; k += NT)
      *reinterpret_cast<u32x4*>(&srow[head + sh + 8 * k]) = ld16(p + head + 8 * k);
    if ((int)threadIdx.x < V - tail0) srow[tail0 + threadIdx.x + sh] = p[tail0 + threadIdx.x];
    __syncthreads();
  }
  auto val = [&](int i) -> float {
    if constexpr (STAGED) {
      return __builtin_bit_cast(float, (uint32_t)srow[i + sh] << 16);
    } else {
      return load_logit<T>(lp, i);
    }
  };
  float m = -INFINITY;
  for (int i = threadIdx.x; i < V; i += 4 * NT) {
    float x[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) x[k] = i + k * NT < V ? biased<T>(val(i + k * NT), i + k * NT, a.mask_index) : -INFINITY;
    m = fmaxf(m, fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])));
  }
  m = block_max(m, red);

  float sum = 0.f;
  for (int i = threadIdx.x; i < V; i += 4 * NT) {
    float x[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) x[k] = i + k * NT < V ? biased<T>(val(i + k * NT), i + k * NT, a.mask_index) : 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) sum += i + k * NT < V ? expf(shifted<T>(x[k], m)) : 0.f;
  }
  const float lse = logf(block_sum(sum, red));

  const double keep = a.keep;         // s / t
  const double move = 1.0 - a.keep;   // 1 - s / t
  double best = -INFINITY;
  int besti = 0x7fffffff;
  const int64_t base = (int64_t)row * V;
  // uniforms of elements i0 and i0 + 1 (i0 + 1 < V or ignored)
  auto uniforms = [&](int i0, double& u0, double& u1) {
    if (a.u != nullptr) {
      u0 = a.u[base + i0];
      u1 = i0 + 1 < V ? a.u[base + i0 + 1] : 0.0;
      return;
    }
    const uint64_t e = (uint64_t)(base + i0);
    const uint64_t pair = e >> 1;
    uint32_t c[4] = {(uint32_t)pair, (uint32_t)(pair >> 32), (uint32_t)a.offset, (uint32_t)(a.offset >> 32)};
    philox4x32_10(c, (uint32_t)a.seed, (uint32_t)(a.seed >> 32));
    if ((e & 1) == 0) {  // element e uses words (0, 1), e + 1 words (2, 3)
      u0 = u53(c[0], c[1]);
      u1 = u53(c[2], c[3]);
    } else {  // V odd, odd row: e + 1 starts the next pair
      u0 = u53(c[2], c[3]);
      const uint64_t p2 = pair + 1;
      uint32_t d[4] = {(uint32_t)p2, (uint32_t)(p2 >> 32), (uint32_t)a.offset, (uint32_t)(a.offset >> 32)};
      philox4x32_10(d, (uint32_t)a.seed, (uint32_t)(a.seed >> 32));
      u1 = u53(d[0], d[1]);
    }
  };
  // Pruning: an element whose ratio clearly cannot reach the running best
  // skips the float64 log and division (the chosen token is unchanged).
  //  - u < 0.999: g = EPS - log(u + EPS) is estimated in fp32 (relative error
  //    below 1e-4 there: log's absolute error ~1e-7 against g >= 1e-3), and
  //    the element is skipped when q < best * g_est * (1 - 2e-4) in fp32;
  //  - otherwise -log(x) >= 1 - x gives g >= 1 - u, tight as u -> 1, and the
  //    element is skipped when q < best * (1 - u) * (1 - 1e-6) in float64
  //    (the margin covers the rounding of u + EPS, 1.1e-16 absolute, while
  //    1 - u > 1e-6; closer to 1 the element always takes the full path).
  // The fp32 test compares against the wave's best (any lane's best bounds
  // the row's winner from below), refreshed after every loop iteration, so
  // after the first iterations almost no lane of a wave needs the float64
  // path (a lane-local best would leave some lane on it at nearly every
  // element position: each lane sees a new record every few elements).
  float bestf = -INFINITY;  // this lane's best rounded to fp32 (ratios are at most 1e10)
  float thr = -INFINITY;    // the wave's best at the last refresh
  auto consider = [&](int i, double u) {
    double q;
    if (i == a.mask_index) {
      q = keep;
    } else {
      const float l = shifted<T>(biased<T>(val(i), i, a.mask_index), m) - lse;
      q = (double)expf(l) * move;
    }
    const float uf = (float)u;
    if (uf < 0.999f) {
      const float gf = 1e-10f - __builtin_amdgcn_logf(uf + 1e-10f) * 0.69314718f;
      if ((float)q < thr * gf * 0.9998f) return;
    } else {
      const double om = 1.0 - u;
      if (om > 1e-6 && q < best * om * (1.0 - 1e-6)) return;
    }
    const double r = q / (kEps - log(u + kEps));
    if (better(r, i, best, besti)) {
      best = r;
      besti = i;
      bestf = (float)r;
    }
  };
  // two independent element pairs per iteration
  for (int i0 = 2 * threadIdx.x; i0 < V; i0 += 4 * NT) {
    const int j0 = i0 + 2 * NT;
    double u[4];
    uniforms(i0, u[0], u[1]);
    if (j0 < V) uniforms(j0, u[2], u[3]);
    const int idx[4] = {i0, i0 + 1, j0, j0 + 1};
#pragma unroll
    for (int h = 0; h < 4; ++h)
      if (idx[h] < V) consider(idx[h], u[h]);
    float w = bestf;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) w = fmaxf(w, __shfl_xor(w, o, 64));
    thr = w;
  }
  // argmax across the workgroup
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const double ov = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(besti, o, 64);
    if (better(ov, oi, best, besti)) {
      best = ov;
      besti = oi;
    }
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    bval[w] = best;
    bidx[w] = besti;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double bv = bval[0];
    int bi = bidx[0];
    for (int k = 1; k < kSubsThreads / 64; ++k)
      if (better(bval[k], bidx[k], bv, bi)) {
        bv = bval[k];
        bi = bidx[k];
      }
    a.out[row] = bi;
  }
}

}  // namespace

hipError_t launch_subs_sample(const SubsArgs& a, hipStream_t stream) {
  if (a.rows == 0) return hipSuccess;
  if (a.fp32)
    hipLaunchKernelGGL((subs_sample_kernel<float, false>), dim3(a.rows), dim3(kSubsThreads), 0, stream, a);
  else if (a.vocab <= kMaxStaged)
    hipLaunchKernelGGL((subs_sample_kernel<uint16_t, true>), dim3(a.rows), dim3(kSubsThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((subs_sample_kernel<uint16_t, false>), dim3(a.rows), dim3(kSubsThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace bd3
