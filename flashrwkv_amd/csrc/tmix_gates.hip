// TMix producer and consumer of the WKV7 operator, as standalone kernels.
//
// kk_a_gate (reference csrc/sm120/tmix/kk_a_gate/infer_fp16_forward_varlen.cu,
// contract docs/kernel_api.md:159-165) turns the key and the a-gate input
// into the three WKV7 inputs, per (token, head) row of D features:
//   u = k * k_k,  kk = u / max(|u|, 1e-12),  gate = sigmoid(a0 + a12),
//   new_k = k * (gate * k_a + 1 - k_a),  neg_kk = -kk,  kka = kk * gate.
// lnx_rkvres_xg (reference csrc/sm120/tmix/lnx_rkvres_xg/infer_fp16_forward_varlen.cu,
// contract docs/kernel_api.md:167-173) consumes the WKV7 output x:
//   mean, var over the row's D features (biased), rstd = 1 / sqrt(var + 64e-5),
//   rkv = sum_d r k r_k,  out = ((x - mean) rstd weight + bias + rkv v) g.
//
// Both are HBM-bound elementwise passes with one or three per-row
// reductions. A row of D 16-bit values is D/8 lanes of 16-byte loads; a wave
// covers 64/(D/8) rows and reduces with xor shuffles inside each row's lane
// group; the grid strides over rows. Arithmetic is fp32; outputs are rounded
// to the io type (nearest even).
#include "capi_internal.h"
#include "wkv7_device.h"

namespace frwkv {
namespace {

constexpr int kGateThreads = 256;
constexpr float kNormEps = 1.0e-12f;
constexpr float kLnEps = 64.0e-5f;

__device__ __forceinline__ float sigmoid(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-kLog2E * x));
}

// Sum over the L consecutive lanes of a row group (L a power of two <= 64).
template <int L>
__device__ __forceinline__ float row_sum(float x) {
#pragma unroll
  for (int off = 1; off < L; off <<= 1) x += __shfl_xor(x, off, 64);
  return x;
}

template <typename T>
__device__ __forceinline__ void unpack8(uint4 q, float (&out)[8]) {
  const typename IoTraits<T>::storage* s =
      reinterpret_cast<const typename IoTraits<T>::storage*>(&q);
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = to_f32<T>(s[e]);
}

template <typename T>
__device__ __forceinline__ void load8(const typename IoTraits<T>::storage* p, float (&out)[8]) {
  unpack8<T>(*reinterpret_cast<const uint4*>(p), out);
}

template <typename T>
__device__ __forceinline__ void store8(typename IoTraits<T>::storage* p, const float (&x)[8]) {
  uint4 q;
  q.x = pack2<T>(x[0], x[1]);
  q.y = pack2<T>(x[2], x[3]);
  q.z = pack2<T>(x[4], x[5]);
  q.w = pack2<T>(x[6], x[7]);
  *reinterpret_cast<uint4*>(p) = q;
}

// One row per L = D/8 lanes; rows = tokens * heads, row index = token * H + head.
template <typename T, int D>
__global__ __launch_bounds__(kGateThreads) void kk_a_gate_kernel(
    const typename IoTraits<T>::storage* __restrict__ k,
    const typename IoTraits<T>::storage* __restrict__ k_k,
    const typename IoTraits<T>::storage* __restrict__ a0,
    const typename IoTraits<T>::storage* __restrict__ a12,
    const typename IoTraits<T>::storage* __restrict__ k_a,
    typename IoTraits<T>::storage* __restrict__ new_k,
    typename IoTraits<T>::storage* __restrict__ neg_kk,
    typename IoTraits<T>::storage* __restrict__ kka, int64_t rows, int32_t heads) {
  constexpr int L = D / 8;
  constexpr int kRowsPerBlock = kGateThreads / L;
  const int sub = threadIdx.x % L;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kRowsPerBlock;
  for (int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / L;
       row < rows; row += stride) {
    // The L lanes of a row always take the loop together, and the shuffles
    // stay inside those L lanes, so a row group that has run out of rows
    // never feeds another group's sums.
    const int64_t idx = row * D + 8 * sub;
    const int c = static_cast<int>(row % heads) * D + 8 * sub;
    float kv[8], kkp[8], a0v[8], a12v[8], kav[8];
    load8<T>(k + idx, kv);
    load8<T>(a12 + idx, a12v);
    load8<T>(k_k + c, kkp);
    load8<T>(a0 + c, a0v);
    load8<T>(k_a + c, kav);
    float u[8], ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      u[e] = kv[e] * kkp[e];
      ss = fmaf(u[e], u[e], ss);
    }
    ss = row_sum<L>(ss);
    const float inv = __builtin_amdgcn_rcpf(fmaxf(__builtin_sqrtf(ss), kNormEps));
    float o_k[8], o_neg[8], o_kka[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float kkn = u[e] * inv;
      const float gate = sigmoid(a0v[e] + a12v[e]);
      o_k[e] = kv[e] * fmaf(gate, kav[e], 1.0f - kav[e]);
      o_neg[e] = -kkn;
      o_kka[e] = kkn * gate;
    }
    store8<T>(new_k + idx, o_k);
    store8<T>(neg_kk + idx, o_neg);
    store8<T>(kka + idx, o_kka);
  }
}

template <typename T, int D>
__global__ __launch_bounds__(kGateThreads) void lnx_rkvres_xg_kernel(
    const typename IoTraits<T>::storage* __restrict__ x,
    const typename IoTraits<T>::storage* __restrict__ r,
    const typename IoTraits<T>::storage* __restrict__ k,
    const typename IoTraits<T>::storage* __restrict__ v,
    const typename IoTraits<T>::storage* __restrict__ r_k,
    const typename IoTraits<T>::storage* __restrict__ weight,
    const typename IoTraits<T>::storage* __restrict__ bias,
    const typename IoTraits<T>::storage* __restrict__ g,
    typename IoTraits<T>::storage* __restrict__ out, int64_t rows, int32_t heads) {
  constexpr int L = D / 8;
  constexpr int kRowsPerBlock = kGateThreads / L;
  const int sub = threadIdx.x % L;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kRowsPerBlock;
  for (int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / L;
       row < rows; row += stride) {
    const int64_t idx = row * D + 8 * sub;
    const int c = static_cast<int>(row % heads) * D + 8 * sub;
    float xv[8], rv[8], kv[8], vv[8], gv[8], rkp[8], wv[8], bv[8];
    load8<T>(x + idx, xv);
    load8<T>(r + idx, rv);
    load8<T>(k + idx, kv);
    load8<T>(v + idx, vv);
    load8<T>(g + idx, gv);
    load8<T>(r_k + c, rkp);
    load8<T>(weight + c, wv);
    load8<T>(bias + c, bv);
    float sum = 0.0f, dot = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      sum += xv[e];
      dot = fmaf(rv[e] * kv[e], rkp[e], dot);
    }
    const float mean = row_sum<L>(sum) * (1.0f / D);
    const float rkv = row_sum<L>(dot);
    float sq = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float d = xv[e] - mean;
      sq = fmaf(d, d, sq);
    }
    const float var = row_sum<L>(sq) * (1.0f / D);
    const float rstd = __builtin_amdgcn_rsqf(var + kLnEps);
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      o[e] = fmaf((xv[e] - mean) * rstd, wv[e], fmaf(rkv, vv[e], bv[e])) * gv[e];
    }
    store8<T>(out + idx, o);
  }
}

int gate_grid(int64_t rows, int row_lanes) {
  const int64_t rows_per_block = kGateThreads / row_lanes;
  const int64_t blocks = (rows + rows_per_block - 1) / rows_per_block;
  return static_cast<int>(blocks < 8192 ? (blocks < 1 ? 1 : blocks) : 8192);
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

int check_gate_shapes(const char* what, int io_dtype, int64_t tokens, int32_t heads,
                      int32_t head_size) {
  if (io_dtype != FRWKV_DTYPE_F16 && io_dtype != FRWKV_DTYPE_BF16) {
    return set_error(FRWKV_ERR_UNSUPPORTED, "%s: io dtype must be float16 or bfloat16", what);
  }
  if (head_size != 64 && head_size != 128 && head_size != 256) {
    return set_error(FRWKV_ERR_UNSUPPORTED, "%s: head_size must be 64, 128, or 256, got %d",
                     what, head_size);
  }
  if (tokens <= 0 || heads <= 0) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "%s: tokens and heads must be positive (N=%lld, H=%d)", what,
                     static_cast<long long>(tokens), heads);
  }
  return FRWKV_OK;
}

template <typename T, int D>
void launch_kk_a_gate(const void* k, const void* k_k, const void* a0, const void* a12,
                      const void* k_a, void* new_k, void* neg_kk, void* kka, int64_t rows,
                      int32_t heads, hipStream_t s) {
  using S = typename IoTraits<T>::storage;
  hipLaunchKernelGGL((kk_a_gate_kernel<T, D>), dim3(gate_grid(rows, D / 8)),
                     dim3(kGateThreads), 0, s, static_cast<const S*>(k),
                     static_cast<const S*>(k_k), static_cast<const S*>(a0),
                     static_cast<const S*>(a12), static_cast<const S*>(k_a),
                     static_cast<S*>(new_k), static_cast<S*>(neg_kk), static_cast<S*>(kka),
                     rows, heads);
}

template <typename T, int D>
void launch_lnx(const void* x, const void* r, const void* k, const void* v, const void* r_k,
                const void* weight, const void* bias, const void* g, void* out, int64_t rows,
                int32_t heads, hipStream_t s) {
  using S = typename IoTraits<T>::storage;
  hipLaunchKernelGGL((lnx_rkvres_xg_kernel<T, D>), dim3(gate_grid(rows, D / 8)),
                     dim3(kGateThreads), 0, s, static_cast<const S*>(x),
                     static_cast<const S*>(r), static_cast<const S*>(k),
                     static_cast<const S*>(v), static_cast<const S*>(r_k),
                     static_cast<const S*>(weight), static_cast<const S*>(bias),
                     static_cast<const S*>(g), static_cast<S*>(out), rows, heads);
}

template <typename T>
void dispatch_kk_a_gate(int32_t d, const void* k, const void* k_k, const void* a0,
                        const void* a12, const void* k_a, void* new_k, void* neg_kk, void* kka,
                        int64_t rows, int32_t heads, hipStream_t s) {
  if (d == 64) launch_kk_a_gate<T, 64>(k, k_k, a0, a12, k_a, new_k, neg_kk, kka, rows, heads, s);
  if (d == 128) launch_kk_a_gate<T, 128>(k, k_k, a0, a12, k_a, new_k, neg_kk, kka, rows, heads, s);
  if (d == 256) launch_kk_a_gate<T, 256>(k, k_k, a0, a12, k_a, new_k, neg_kk, kka, rows, heads, s);
}

template <typename T>
void dispatch_lnx(int32_t d, const void* x, const void* r, const void* k, const void* v,
                  const void* r_k, const void* weight, const void* bias, const void* g,
                  void* out, int64_t rows, int32_t heads, hipStream_t s) {
  if (d == 64) launch_lnx<T, 64>(x, r, k, v, r_k, weight, bias, g, out, rows, heads, s);
  if (d == 128) launch_lnx<T, 128>(x, r, k, v, r_k, weight, bias, g, out, rows, heads, s);
  if (d == 256) launch_lnx<T, 256>(x, r, k, v, r_k, weight, bias, g, out, rows, heads, s);
}

}  // namespace
}  // namespace frwkv

extern "C" int frwkv_kk_a_gate(int io_dtype, int64_t total_tokens, int32_t num_heads,
                               int32_t head_size, const void* k, const void* k_k,
                               const void* a0, const void* a12, const void* k_a, void* new_k,
                               void* neg_kk, void* kka, void* stream) {
  using namespace frwkv;
  if (!k || !k_k || !a0 || !a12 || !k_a || !new_k || !neg_kk || !kka) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT, "frwkv_kk_a_gate: null pointer argument");
  }
  int rc = check_gate_shapes("frwkv_kk_a_gate", io_dtype, total_tokens, num_heads, head_size);
  if (rc != FRWKV_OK) return rc;
  const void* all[] = {k, k_k, a0, a12, k_a, new_k, neg_kk, kka};
  for (const void* p : all) {
    if (!aligned16(p)) {
      return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                       "frwkv_kk_a_gate: every buffer must be 16-byte aligned");
    }
  }
  const int64_t rows = total_tokens * num_heads;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (io_dtype == FRWKV_DTYPE_F16) {
    dispatch_kk_a_gate<F16>(head_size, k, k_k, a0, a12, k_a, new_k, neg_kk, kka, rows,
                            num_heads, s);
  } else {
    dispatch_kk_a_gate<Bf16>(head_size, k, k_k, a0, a12, k_a, new_k, neg_kk, kka, rows,
                             num_heads, s);
  }
  return check_launch("kk_a_gate_kernel");
}

extern "C" int frwkv_lnx_rkvres_xg(int io_dtype, int64_t total_tokens, int32_t num_heads,
                                   int32_t head_size, const void* x, const void* r,
                                   const void* k, const void* v, const void* r_k,
                                   const void* weight, const void* bias, const void* g,
                                   void* output, void* stream) {
  using namespace frwkv;
  if (!x || !r || !k || !v || !r_k || !weight || !bias || !g || !output) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT, "frwkv_lnx_rkvres_xg: null pointer argument");
  }
  int rc =
      check_gate_shapes("frwkv_lnx_rkvres_xg", io_dtype, total_tokens, num_heads, head_size);
  if (rc != FRWKV_OK) return rc;
  const void* all[] = {x, r, k, v, r_k, weight, bias, g, output};
  for (const void* p : all) {
    if (!aligned16(p)) {
      return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                       "frwkv_lnx_rkvres_xg: every buffer must be 16-byte aligned");
    }
  }
  const int64_t rows = total_tokens * num_heads;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (io_dtype == FRWKV_DTYPE_F16) {
    dispatch_lnx<F16>(head_size, x, r, k, v, r_k, weight, bias, g, output, rows, num_heads, s);
  } else {
    dispatch_lnx<Bf16>(head_size, x, r, k, v, r_k, weight, bias, g, output, rows, num_heads, s);
  }
  return check_launch("lnx_rkvres_xg_kernel");
}
