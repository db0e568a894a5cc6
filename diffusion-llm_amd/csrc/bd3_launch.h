// bd3_launch.h - argument blocks and launchers shared between the kernel
// translation units and the C-ABI layer (capi.hip). Internal to the library.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace bd3 {

constexpr int kHeadDim = 64;
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
  float* delta;  // (B, H, 2n) fp32: written by the dQ kernel, read by dK/dV
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
  float* part_lse;  // (BH, q_tiles, n_splits, QT) natural log, or null
  Strides3 sq, sk, sv, so;
  int heads;
  int bh;
  int q_len;
  int kv_len;
  int bs;
  int n_splits;
  int split_len;  // keys per split (multiple of 64)
  int q_tiles;
  float scale_log2;
};

hipError_t launch_attn_fwd(const FwdArgs& a, hipStream_t stream);
hipError_t launch_attn_bwd_dq(const BwdArgs& a, hipStream_t stream);
hipError_t launch_attn_bwd_dkdv(const BwdArgs& a, hipStream_t stream);
hipError_t launch_decode(const DecodeArgs& a, int qt, hipStream_t stream);
hipError_t launch_mask_dump(uint8_t* out, int mode, int rows, int kv_len,
                            int bs, hipStream_t stream);

}  // namespace bd3
