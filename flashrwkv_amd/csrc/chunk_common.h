// Device helpers shared by the chunked WKV7 kernels (forward and backward).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wkv7_device.h"
#include "wkv7_mfma.h"

namespace frwkv {

constexpr int kChunk = 64;
constexpr int kHead = 64;
constexpr int kChunkThreads = 256;
constexpr float kSpanLimit = 80.0f;   // log2 units
constexpr float kSpanFloor = 0x1p-80f; // 2^-kSpanLimit: the same limit as a decay product
constexpr float kLog2Min = -20.0f;    // per-token clamp of log2 retention
// A buffer offset past every resource's range (resources here are under
// 2 GiB): a store there is dropped and a load returns zero. Masked lanes use
// it instead of a branch around the access, so every pass issues the same
// number of memory instructions and the compiler's in-order wait counts stay
// exact.
constexpr uint32_t kDropOffset = 0x80000000u;
// Head count limit of the chunked kernels: a chunk's row offsets (at most
// 2 x 64 rows of H x 64 x 2 bytes) then stay below 2^30, so neither an
// in-range offset nor kDropOffset plus a row offset wraps in 32 bits.
constexpr int32_t kMaxChunkHeads = 65536;

// Operand tiles: 64 rows x 64 bf16, row stride 68 elements (136 B = 34
// dwords): the 16 rows of an 8-byte operand read hit 16 distinct dword pairs.
constexpr int kOpStride = 68;
constexpr int kOpTile = 64 * kOpStride;
// Lower-triangular C x C matrices: the 10 blocks (p, q <= p) of 16 x 16,
// packed, row stride 20 (40 B = 10 dwords, conflict-free the same way).
constexpr int kTriStride = 20;
constexpr int kTriBlock = 16 * kTriStride;
constexpr int kTriBlocks = 10;

enum TriMatrix { kLab = 0, kLak = 1, kArb = 2, kArk = 3 };

__device__ __forceinline__ int tri_index(int p, int q) { return (p * (p + 1)) / 2 + q; }

__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// threadIdx.x through an empty volatile asm: values derived from it (per-lane
// LDS and buffer offsets) are then recomputed in each phase of a chunk loop
// instead of being hoisted out of it, where dozens of them would stay live
// in registers across every phase.
__device__ __forceinline__ int lane_tid() {
  int t = static_cast<int>(threadIdx.x);
  asm volatile("" : "+v"(t));
  return t;
}

// A kernel's by-value argument block read through an opaque kernarg pointer:
// fields are fetched with scalar loads where used. Read through the argument
// itself, the compiler hoists every pointer and buffer descriptor out of the
// chunk loop into SGPRs, which then spill.
template <typename P>
__device__ __forceinline__ const __attribute__((address_space(4))) P& kernel_args() {
  auto ptr = (const __attribute__((address_space(4))) P*)(__builtin_amdgcn_kernarg_segment_ptr());
  asm volatile("" : "+s"(ptr));
  return *ptr;
}

// 2^x on the hardware exponential (v_exp_f32). Every exponent here lies in
// [-80, 80] (the decay span limit), inside fp32's normal range, so the
// denormal-range handling of exp2f is not needed.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

template <typename T>
__device__ __forceinline__ void unpack8(uint4 q, float (&out)[8]) {
  const typename IoTraits<T>::storage* p =
      reinterpret_cast<const typename IoTraits<T>::storage*>(&q);
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = to_f32<T>(p[e]);
}

template <typename T>
__device__ __forceinline__ uint4 load_row8(const void* base, int64_t offset) {
  return *reinterpret_cast<const uint4*>(
      static_cast<const typename IoTraits<T>::storage*>(base) + offset);
}

// log2 of the retention, clamped to [kLog2Min, 0]. Logits mode:
// log2 w = -e^{-1/2} log2(e) sigmoid(x); raw mode: log2 w (v_log_f32).
template <DecayMode M>
__device__ __forceinline__ float log2_retention(float x) {
  float lg;
  if constexpr (M == DecayMode::kLogits) {
    const float sig = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-kLog2E * x));
    lg = -(kExpNegHalf * kLog2E) * sig;
  } else {
    lg = __builtin_amdgcn_logf(x);
  }
  return __builtin_amdgcn_fmed3f(lg, kLog2Min, 0.0f);
}

// The retention itself, clamped to [2^kLog2Min, 1] as log2_retention is:
// raw mode clamps the input, logits mode is 2^(log2 w).
template <DecayMode M>
__device__ __forceinline__ float clamped_retention(float x) {
  if constexpr (M == DecayMode::kLogits) {
    return __builtin_amdgcn_exp2f(log2_retention<M>(x));
  } else {
    return __builtin_amdgcn_fmed3f(x, 0x1p-20f, 1.0f);
  }
}

// 8 floats -> 8 bf16 at an 8-byte aligned LDS address (two 8-byte writes).
__device__ __forceinline__ void store8_bf16(uint16_t* dst, const float (&x)[8]) {
  uint2 lo, hi;
  lo.x = pack_bf16x2(x[0], x[1]);
  lo.y = pack_bf16x2(x[2], x[3]);
  hi.x = pack_bf16x2(x[4], x[5]);
  hi.y = pack_bf16x2(x[6], x[7]);
  reinterpret_cast<uint2*>(dst)[0] = lo;
  reinterpret_cast<uint2*>(dst)[1] = hi;
}

// store8_bf16 of the split pairs x = hi + lo: hi to dst_hi, lo to dst_lo.
__device__ __forceinline__ void store8_bf16_split(uint16_t* dst_hi, uint16_t* dst_lo,
                                                  const float (&x)[8]) {
  const uint2 p0 = split_bf16x2(x[0], x[1]);
  const uint2 p1 = split_bf16x2(x[2], x[3]);
  const uint2 p2 = split_bf16x2(x[4], x[5]);
  const uint2 p3 = split_bf16x2(x[6], x[7]);
  reinterpret_cast<uint2*>(dst_hi)[0] = make_uint2(p0.x, p1.x);
  reinterpret_cast<uint2*>(dst_hi)[1] = make_uint2(p2.x, p3.x);
  reinterpret_cast<uint2*>(dst_lo)[0] = make_uint2(p0.y, p1.y);
  reinterpret_cast<uint2*>(dst_lo)[1] = make_uint2(p2.y, p3.y);
}

// Inclusive-scan step over groups of 8 lanes: lane l adds lane l - N when
// l % 8 >= N (DPP row shift; the groups never straddle a 16-lane row).
template <int N>
__device__ __forceinline__ float scan8_step(float x, int tp) {
  const float y = __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x110 + N, 0xf, 0xf, true));
  return tp >= N ? x + y : x;
}

// The same scan with products (lanes l % 8 < N keep x).
template <int N>
__device__ __forceinline__ float scan8_mul(float x, int tp) {
  const float y = __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x110 + N, 0xf, 0xf, true));
  return tp >= N ? x * y : x;
}

// Exclusive product scan from an inclusive one: lane l takes lane l - 1's
// value, and the first lane of each 8-lane group the empty product 1.
__device__ __forceinline__ float scan8_exclusive(float incl, int tp) {
  const float y = __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(incl), 0x111, 0xf, 0xf, true));
  return tp >= 1 ? y : 1.0f;
}

}  // namespace frwkv
