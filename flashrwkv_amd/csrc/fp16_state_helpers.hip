// Side helpers of the fp16-state recurrent family.
//
// Replaces the reference's advance_i32_kernel, advance_i32_varlen_kernel and
// recurrent_add_vec(_2d)_kernel with their launchers
// (csrc/sm120/tmix/wkv7/infer_recurrent_fp16_forward_varlen.cu:57-122,
// 1217-1281). Contract:
//   * advance: elapsed[i] += amount for every slot (int32, wrapping);
//   * varlen advance: elapsed[state_indices[s]] += sequence length s, and
//     nothing at all when the metadata status word is non-zero (fail closed);
//   * add_vec: out[n, c] = fp16(float(x[n, c]) + float(vec[c])), round to
//     nearest even.
// All three are HBM-bound streams; add_vec moves 16 bytes per lane when the
// row length allows it.
#include "capi_internal.h"
#include "wkv7_device.h"

namespace frwkv {
namespace {

constexpr int kThreads = 256;

__global__ __launch_bounds__(kThreads) void advance_kernel(int32_t* __restrict__ x,
                                                           int32_t amount, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += stride) {
    x[i] = static_cast<int32_t>(static_cast<uint32_t>(x[i]) + static_cast<uint32_t>(amount));
  }
}

// Validated metadata has unique slots, so no two threads touch one entry.
__global__ __launch_bounds__(kThreads) void advance_varlen_kernel(
    const int32_t* __restrict__ cu_seqlens, const int32_t* __restrict__ slots,
    const int32_t* __restrict__ status, int32_t* __restrict__ elapsed,
    int32_t num_sequences, int32_t state_pool_size) {
  const int s = blockIdx.x * kThreads + threadIdx.x;
  if (s >= num_sequences || status[0] != 0) return;
  const int32_t slot = slots[s];
  if (slot < 0 || slot >= state_pool_size) return;
  const uint32_t length = static_cast<uint32_t>(cu_seqlens[s + 1] - cu_seqlens[s]);
  elapsed[slot] = static_cast<int32_t>(static_cast<uint32_t>(elapsed[slot]) + length);
}

__device__ __forceinline__ uint32_t add_pair(uint32_t x, uint32_t v) {
  const float lo = f16_to_f32(static_cast<uint16_t>(x & 0xffffu)) +
                   f16_to_f32(static_cast<uint16_t>(v & 0xffffu));
  const float hi = f16_to_f32(static_cast<uint16_t>(x >> 16)) +
                   f16_to_f32(static_cast<uint16_t>(v >> 16));
  return pack2<F16>(lo, hi);
}

// Each lane adds W consecutive elements of one row (W = 8: 16-byte loads,
// needs C % 8 == 0; W = 2 otherwise, C is even).
template <int W>
__global__ __launch_bounds__(kThreads) void add_vec_kernel(const uint16_t* __restrict__ x,
                                                           const uint16_t* __restrict__ vec,
                                                           uint16_t* __restrict__ out,
                                                           int32_t channels, int64_t pieces) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  const int32_t per_row = channels / W;
  for (int64_t q = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; q < pieces;
       q += stride) {
    const int32_t c = static_cast<int32_t>(q % per_row) * W;
    if constexpr (W == 8) {
      const uint4 xv = reinterpret_cast<const uint4*>(x)[q];
      const uint4 vv = *reinterpret_cast<const uint4*>(vec + c);
      uint4 o;
      o.x = add_pair(xv.x, vv.x);
      o.y = add_pair(xv.y, vv.y);
      o.z = add_pair(xv.z, vv.z);
      o.w = add_pair(xv.w, vv.w);
      reinterpret_cast<uint4*>(out)[q] = o;
    } else {
      const uint32_t xv = reinterpret_cast<const uint32_t*>(x)[q];
      const uint32_t vv = *reinterpret_cast<const uint32_t*>(vec + c);
      reinterpret_cast<uint32_t*>(out)[q] = add_pair(xv, vv);
    }
  }
}

int grid_for(int64_t work) {
  // Enough workgroups to cover 256 CUs several times; the loops stride.
  const int64_t blocks = (work + kThreads - 1) / kThreads;
  return static_cast<int>(blocks < 8192 ? (blocks < 1 ? 1 : blocks) : 8192);
}

}  // namespace
}  // namespace frwkv

extern "C" int frwkv_advance_i32(int32_t* elapsed_state, int64_t count, int32_t amount,
                                 void* stream) {
  using namespace frwkv;
  if (!elapsed_state || count <= 0) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_advance_i32: elapsed state must be non-empty");
  }
  hipLaunchKernelGGL(advance_kernel, dim3(grid_for(count)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), elapsed_state, amount, count);
  return check_launch("advance_kernel");
}

extern "C" int frwkv_advance_i32_varlen(int32_t num_sequences, int32_t state_pool_size,
                                        const int32_t* cu_seqlens,
                                        const int32_t* state_indices,
                                        const int32_t* metadata_status,
                                        int32_t* elapsed_state_pool, void* stream) {
  using namespace frwkv;
  if (!cu_seqlens || !state_indices || !metadata_status || !elapsed_state_pool) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_advance_i32_varlen: null pointer argument");
  }
  if (num_sequences <= 0 || num_sequences > 65535 || state_pool_size <= 0) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_advance_i32_varlen: B=%d must be in 1..65535 and slots=%d positive",
                     num_sequences, state_pool_size);
  }
  const int blocks = (num_sequences + kThreads - 1) / kThreads;
  hipLaunchKernelGGL(advance_varlen_kernel, dim3(blocks), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), cu_seqlens, state_indices,
                     metadata_status, elapsed_state_pool, num_sequences, state_pool_size);
  return check_launch("advance_varlen_kernel");
}

extern "C" int frwkv_add_vec(int64_t rows, int32_t channels, const void* x, const void* vec,
                             void* output, void* stream) {
  using namespace frwkv;
  if (!x || !vec || !output) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT, "frwkv_add_vec: null pointer argument");
  }
  if (rows <= 0 || channels <= 0 || channels % 2 != 0) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_add_vec: x must have packed shape [rows,C] with even C "
                     "(rows=%lld, C=%d)",
                     static_cast<long long>(rows), channels);
  }
  if (reinterpret_cast<uintptr_t>(x) % 4 != 0 || reinterpret_cast<uintptr_t>(vec) % 4 != 0 ||
      reinterpret_cast<uintptr_t>(output) % 4 != 0) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_add_vec: x, vec and output must be 4-byte aligned");
  }
  const auto* xs = static_cast<const uint16_t*>(x);
  const auto* vs = static_cast<const uint16_t*>(vec);
  auto* os = static_cast<uint16_t*>(output);
  const bool wide = channels % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(vec) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(output) % 16 == 0;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (wide) {
    const int64_t pieces = rows * (channels / 8);
    hipLaunchKernelGGL(add_vec_kernel<8>, dim3(grid_for(pieces)), dim3(kThreads), 0, s, xs,
                       vs, os, channels, pieces);
  } else {
    const int64_t pieces = rows * (channels / 2);
    hipLaunchKernelGGL(add_vec_kernel<2>, dim3(grid_for(pieces)), dim3(kThreads), 0, s, xs,
                       vs, os, channels, pieces);
  }
  return check_launch("add_vec_kernel");
}
