// Device-side helpers shared by the WKV7 HIP kernels (gfx950, wave64).
//
// Decay transform: the reference's public boundary is raw decay logits x,
// turned into the retention w = exp(-e^{-1/2} * sigmoid(x + bias))
// (reference csrc/sm120/tmix/wkv7/recurrent_decay.cuh:10-22). This build also
// accepts the retention w itself (DecayMode::kRawW), which is what the
// measurement harness feeds (w = exp(-exp(u)) covers values below the
// logits mode's floor of exp(-e^{-1/2}) = 0.5453).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace frwkv {

enum class DecayMode : int { kLogits = 0, kRawW = 1 };

// e^{-1/2}: the clampw scale of the retention transform.
constexpr float kExpNegHalf = 0.60653065971263342f;
constexpr float kLog2E = 1.4426950408889634f;

// Retention and its natural log from a pre-transform decay input.
// Logits: log w = -e^{-1/2} * sigmoid(x); computing log w directly keeps full
// precision for w close to 1, which the chunked kernels need.
// The sigmoid and the exponential use the hardware reciprocal and exp2
// (v_rcp_f32, v_exp_f32, about 1 ulp): exp2 of a large positive argument is
// +inf and its reciprocal 0, so sigmoid(x) -> 0 for x -> -inf without a
// special case, and log w lies in [-e^{-1/2}, 0], far from exp2's denormal
// range.
template <DecayMode M>
__device__ __forceinline__ float decay_log(float x) {
  if constexpr (M == DecayMode::kLogits) {
    const float sig = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-kLog2E * x));
    return -kExpNegHalf * sig;
  } else {
    return __logf(x);
  }
}

template <DecayMode M>
__device__ __forceinline__ float decay_retention(float x) {
  if constexpr (M == DecayMode::kLogits) {
    return __builtin_amdgcn_exp2f(kLog2E * decay_log<M>(x));
  } else {
    return x;
  }
}

// ------------------------------------------------------------ io types ----

typedef uint16_t bf16_bits;
typedef uint16_t f16_bits;

struct Bf16 {};
struct F16 {};

template <typename T> struct IoTraits;
template <> struct IoTraits<float> {
  using storage = float;
  static constexpr int kBytes = 4;
};
template <> struct IoTraits<Bf16> {
  using storage = uint16_t;
  static constexpr int kBytes = 2;
};
template <> struct IoTraits<F16> {
  using storage = uint16_t;
  static constexpr int kBytes = 2;
};

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t bits16) {
  _Float16 h;
  __builtin_memcpy(&h, &bits16, 2);
  return static_cast<float>(h);
}

template <typename T>
__device__ __forceinline__ float to_f32(typename IoTraits<T>::storage x) {
  if constexpr (__is_same(T, float)) {
    return x;
  } else if constexpr (__is_same(T, Bf16)) {
    return bf16_to_f32(x);
  } else {
    return f16_to_f32(x);
  }
}

template <typename T>
__device__ __forceinline__ typename IoTraits<T>::storage from_f32(float x) {
  if constexpr (__is_same(T, float)) {
    return x;
  } else if constexpr (__is_same(T, Bf16)) {
    __bf16 h = static_cast<__bf16>(x);  // v_cvt_pk_bf16_f32: round to nearest even
    uint16_t bits;
    __builtin_memcpy(&bits, &h, 2);
    return bits;
  } else {
    _Float16 h = static_cast<_Float16>(x);
    uint16_t bits;
    __builtin_memcpy(&bits, &h, 2);
    return bits;
  }
}

// Two floats -> two 16-bit io values packed in one dword (lo in bits 0..15),
// rounded to nearest even. The vector conversion lets the compiler select one
// packed conversion (v_cvt_pk_bf16_f32 for bf16) instead of a conversion per
// value followed by shift/mask/or packing.
template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  typedef float v2f __attribute__((ext_vector_type(2)));
  const v2f v = {lo, hi};
  if constexpr (__is_same(T, Bf16)) {
    typedef __bf16 v2h __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, v2h));
  } else {
    static_assert(__is_same(T, F16), "pack2 packs 16-bit io types");
    typedef _Float16 v2h __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, v2h));
  }
}

// Loads N contiguous elements (16-byte aligned when N*bytes >= 16) as floats.
template <typename T, int N>
__device__ __forceinline__ void load_vec(const typename IoTraits<T>::storage* p,
                                         float (&out)[N]) {
  if constexpr (__is_same(T, float)) {
    static_assert(N % 4 == 0, "fp32 rows load in float4 pieces");
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      const float4 q = reinterpret_cast<const float4*>(p)[i];
      out[4 * i + 0] = q.x;
      out[4 * i + 1] = q.y;
      out[4 * i + 2] = q.z;
      out[4 * i + 3] = q.w;
    }
  } else if constexpr (N % 8 == 0) {
#pragma unroll
    for (int i = 0; i < N / 8; ++i) {
      const uint4 q = reinterpret_cast<const uint4*>(p)[i];
      const uint32_t words[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        out[8 * i + 2 * j + 0] = to_f32<T>(static_cast<uint16_t>(words[j] & 0xffffu));
        out[8 * i + 2 * j + 1] = to_f32<T>(static_cast<uint16_t>(words[j] >> 16));
      }
    }
  } else {
    static_assert(N % 4 == 0, "16-bit rows load in 8-byte pieces");
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      const uint2 q = reinterpret_cast<const uint2*>(p)[i];
      out[4 * i + 0] = to_f32<T>(static_cast<uint16_t>(q.x & 0xffffu));
      out[4 * i + 1] = to_f32<T>(static_cast<uint16_t>(q.x >> 16));
      out[4 * i + 2] = to_f32<T>(static_cast<uint16_t>(q.y & 0xffffu));
      out[4 * i + 3] = to_f32<T>(static_cast<uint16_t>(q.y >> 16));
    }
  }
}

// Raw (undecoded) storage of N contiguous elements, loaded with 16-, 8- or
// (two 16-bit elements) 4-byte loads. Decoding is split from loading so that
// a kernel can issue the loads of later tokens long before it decodes them.
template <typename T, int N>
struct RawRow {
  static constexpr int kWords = N * IoTraits<T>::kBytes / 4;
  static_assert(kWords % 2 == 0 || kWords == 1, "rows load in 4-, 8- or 16-byte pieces");
  uint32_t w[kWords];
};

template <typename T, int N>
__device__ __forceinline__ void load_raw(const typename IoTraits<T>::storage* p,
                                         RawRow<T, N>& out) {
  constexpr int kWords = RawRow<T, N>::kWords;
  if constexpr (kWords == 1) {
    out.w[0] = *reinterpret_cast<const uint32_t*>(p);
  } else if constexpr (kWords % 4 == 0) {
#pragma unroll
    for (int i = 0; i < kWords / 4; ++i) {
      const uint4 q = reinterpret_cast<const uint4*>(p)[i];
      out.w[4 * i + 0] = q.x;
      out.w[4 * i + 1] = q.y;
      out.w[4 * i + 2] = q.z;
      out.w[4 * i + 3] = q.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < kWords / 2; ++i) {
      const uint2 q = reinterpret_cast<const uint2*>(p)[i];
      out.w[2 * i + 0] = q.x;
      out.w[2 * i + 1] = q.y;
    }
  }
}

// load_raw through a buffer resource: byte offsets voffset (per lane) and
// soffset (uniform) into the resource.
template <typename T, int N>
__device__ __forceinline__ void load_raw_buf(__amdgpu_buffer_rsrc_t rs, uint32_t voffset,
                                             int soffset, RawRow<T, N>& out) {
  constexpr int kWords = RawRow<T, N>::kWords;
  if constexpr (kWords == 1) {
    out.w[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, voffset, soffset, 0);
  } else if constexpr (kWords % 4 == 0) {
#pragma unroll
    for (int i = 0; i < kWords / 4; ++i) {
      typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
      const u32x4_t q = __builtin_amdgcn_raw_buffer_load_b128(rs, voffset + 16 * i, soffset, 0);
      out.w[4 * i + 0] = q.x;
      out.w[4 * i + 1] = q.y;
      out.w[4 * i + 2] = q.z;
      out.w[4 * i + 3] = q.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < kWords / 2; ++i) {
      typedef uint32_t u32x2_t2 __attribute__((ext_vector_type(2)));
      const u32x2_t2 q = __builtin_amdgcn_raw_buffer_load_b64(rs, voffset + 8 * i, soffset, 0);
      out.w[2 * i + 0] = q.x;
      out.w[2 * i + 1] = q.y;
    }
  }
}

template <typename T, int N>
__device__ __forceinline__ void decode_raw(const RawRow<T, N>& in, float (&out)[N]) {
  if constexpr (__is_same(T, float)) {
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = __uint_as_float(in.w[i]);
  } else {
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      out[2 * i + 0] = to_f32<T>(static_cast<uint16_t>(in.w[i] & 0xffffu));
      out[2 * i + 1] = to_f32<T>(static_cast<uint16_t>(in.w[i] >> 16));
    }
  }
}

// Stores 4 contiguous values.
template <typename T>
__device__ __forceinline__ void store4(typename IoTraits<T>::storage* p, float x0,
                                       float x1, float x2, float x3) {
  if constexpr (__is_same(T, float)) {
    *reinterpret_cast<float4*>(p) = make_float4(x0, x1, x2, x3);
  } else {
    uint2 q;
    q.x = pack2<T>(x0, x1);
    q.y = pack2<T>(x2, x3);
    *reinterpret_cast<uint2*>(p) = q;
  }
}

// store4 through a buffer resource (byte offsets voffset per lane, soffset
// uniform).
template <typename T>
__device__ __forceinline__ void store4_buf(__amdgpu_buffer_rsrc_t rs, uint32_t voffset,
                                           int soffset, float x0, float x1, float x2, float x3) {
  if constexpr (__is_same(T, float)) {
    typedef float f32x4_b __attribute__((ext_vector_type(4)));
    const f32x4_b q = {x0, x1, x2, x3};
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(
                                               uint32_t __attribute__((ext_vector_type(4))), q),
                                           rs, voffset, soffset, 0);
  } else {
    typedef uint32_t u32x2_b __attribute__((ext_vector_type(2)));
    const u32x2_b q = {pack2<T>(x0, x1), pack2<T>(x2, x3)};
    __builtin_amdgcn_raw_buffer_store_b64(q, rs, voffset, soffset, 0);
  }
}

// Streaming (nontemporal) 16-byte state traffic: each state slab is read and
// written once per launch, so it should not displace reusable lines.
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 load_f4_stream(const float* p) {
  const f32x4_t x = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(p));
  return make_float4(x.x, x.y, x.z, x.w);
}

__device__ __forceinline__ void store_f4_stream(float* p, float4 v) {
  const f32x4_t x = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(x, reinterpret_cast<f32x4_t*>(p));
}

template <typename T>
__device__ __forceinline__ typename IoTraits<T>::storage nan_value() {
  return from_f32<T>(__int_as_float(0x7fc00000));
}

// x + x[lane ^ 16] and x + x[lane ^ 32] through the gfx950 lane swaps
// (v_permlane16_swap / v_permlane32_swap: VALU exchanges between the 16-lane
// rows, or the 32-lane halves, of two registers; no LDS-crossbar round trip).
// Swapping a register with itself leaves x[lo] in one result and x[hi] in the
// other at both lanes of a pair, so both lanes add the same two values and
// end with the same bits, as x + __shfl_xor(x, 16 or 32) does.
__device__ __forceinline__ float add_xor16(float x) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

__device__ __forceinline__ float add_xor32(float x) {
  const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}

// Grid-stride NaN fill used when the metadata status word reports an error:
// outputs become NaN and no state is written (fail closed).
template <typename T>
__device__ __forceinline__ void fill_nan(typename IoTraits<T>::storage* out,
                                         int64_t elements) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const auto nan = nan_value<T>();
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       i < elements; i += stride) {
    out[i] = nan;
  }
}

}  // namespace frwkv
