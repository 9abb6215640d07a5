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
// The training form of lnx_rkvres_xg (reference
// flashrwkv2/tmix/lnx_rkvres_xg/pretrain.py:33-77, kernels
// csrc/sm90/tmix/lnx_rkvres_xg/pretrain_bf16_forward.cu:63-126 and
// pretrain_bf16_backward.cu:125-275) runs the
// same forward and also writes each row's mean and rstd (fp32); its backward
// gives, per row with gy = dout g, xhat = (x - mean) rstd, dxhat = gy weight,
// q = sum_d gy v:
//   dx = (dxhat - mean_d(dxhat) - xhat mean_d(dxhat xhat)) rstd,
//   dv = gy rkv,  dr = q k r_k,  dk = q r r_k,
//   dg = dout (xhat weight + bias + rkv v),
// and the parameter gradients summed over all rows: dweight = sum gy xhat,
// dbias = sum gy, dr_k = sum q r k. Those sums are formed per block of tokens
// in registers and LDS, then added over the blocks in a fixed order by a
// second kernel, so they are deterministic (the reference adds them with
// floating-point atomics).
//
// All of these are HBM-bound elementwise passes with one or three per-row
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

// mean / rstd (rows of fp32, or null): the row statistics the training
// backward reads.
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
    typename IoTraits<T>::storage* __restrict__ out, float* __restrict__ mean_out,
    float* __restrict__ rstd_out, int64_t rows, int32_t heads) {
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
    if (mean_out != nullptr && sub == 0) {
      mean_out[row] = mean;
      rstd_out[row] = rstd;
    }
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      o[e] = fmaf((xv[e] - mean) * rstd, wv[e], fmaf(rkv, vv[e], bv[e])) * gv[e];
    }
    store8<T>(out + idx, o);
  }
}

// Training backward of lnx_rkvres_xg. Workgroup (bx, by) covers tokens
// 64 bx .. 64 bx + 63 and columns 512 by .. 512 by + 511 (8 per lane, so a
// wave holds whole heads: 512 is a multiple of D); wave w takes the block's
// tokens w, w + 4, .... A lane keeps its columns for the whole loop and sums
// its parameter-gradient terms in registers; the four waves are then added in
// order through LDS, and partial[bx][j][c] (j: weight, bias, r_k) receives
// the block's sums.
constexpr int kLnxTokensPerBlock = 64;
constexpr int kLnxColsPerBlock = 512;

template <typename T, int D>
__global__ __launch_bounds__(kGateThreads) void lnx_train_backward_kernel(
    const typename IoTraits<T>::storage* __restrict__ dout,
    const typename IoTraits<T>::storage* __restrict__ x,
    const typename IoTraits<T>::storage* __restrict__ r,
    const typename IoTraits<T>::storage* __restrict__ k,
    const typename IoTraits<T>::storage* __restrict__ v,
    const typename IoTraits<T>::storage* __restrict__ r_k,
    const typename IoTraits<T>::storage* __restrict__ weight,
    const typename IoTraits<T>::storage* __restrict__ bias,
    const typename IoTraits<T>::storage* __restrict__ g,
    const float* __restrict__ mean, const float* __restrict__ rstd,
    typename IoTraits<T>::storage* __restrict__ dx, typename IoTraits<T>::storage* __restrict__ dr,
    typename IoTraits<T>::storage* __restrict__ dk, typename IoTraits<T>::storage* __restrict__ dv,
    typename IoTraits<T>::storage* __restrict__ dg, float* __restrict__ partial,
    int64_t tokens, int32_t heads) {
  constexpr int L = D / 8;
  __shared__ float red[4][3][8][64];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t channels = static_cast<int64_t>(heads) * D;
  const int col = static_cast<int>(blockIdx.y) * kLnxColsPerBlock + 8 * lane;
  // A head's L lanes are all inside or all outside [0, channels), since
  // channels and the block's first column are multiples of D.
  const bool active = col < channels;
  const int head = col / D;
  float wv[8], bv[8], rkp[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) wv[e] = bv[e] = rkp[e] = 0.0f;
  if (active) {
    load8<T>(weight + col, wv);
    load8<T>(bias + col, bv);
    load8<T>(r_k + col, rkp);
  }
  float pw[8], pb[8], prk[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) pw[e] = pb[e] = prk[e] = 0.0f;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kLnxTokensPerBlock;
  for (int i = wave; i < kLnxTokensPerBlock; i += 4) {
    const int64_t t = t0 + i;
    if (t >= tokens) break;  // wave-uniform
    const int64_t row = t * heads + head;
    const int64_t idx = t * channels + col;
    float go[8], xv[8], gv[8], vv[8], rv[8], kv[8];
    float m = 0.0f, rs = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) go[e] = xv[e] = gv[e] = vv[e] = rv[e] = kv[e] = 0.0f;
    if (active) {
      load8<T>(dout + idx, go);
      load8<T>(x + idx, xv);
      load8<T>(g + idx, gv);
      load8<T>(v + idx, vv);
      load8<T>(r + idx, rv);
      load8<T>(k + idx, kv);
      m = mean[row];
      rs = rstd[row];
    }
    float gy[8], xh[8], s_dx = 0.0f, s_dxx = 0.0f, s_q = 0.0f, s_rk = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      gy[e] = go[e] * gv[e];
      xh[e] = (xv[e] - m) * rs;
      const float dxh = gy[e] * wv[e];
      s_dx += dxh;
      s_dxx = fmaf(dxh, xh[e], s_dxx);
      s_q = fmaf(gy[e], vv[e], s_q);
      s_rk = fmaf(rv[e] * kv[e], rkp[e], s_rk);
    }
    const float mdx = row_sum<L>(s_dx) * (1.0f / D);
    const float mdxx = row_sum<L>(s_dxx) * (1.0f / D);
    const float q = row_sum<L>(s_q);
    const float rkv = row_sum<L>(s_rk);
    if (active) {
      float o_x[8], o_r[8], o_k[8], o_v[8], o_g[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        o_x[e] = (gy[e] * wv[e] - mdx - xh[e] * mdxx) * rs;
        o_v[e] = gy[e] * rkv;
        o_r[e] = q * kv[e] * rkp[e];
        o_k[e] = q * rv[e] * rkp[e];
        o_g[e] = go[e] * fmaf(xh[e], wv[e], fmaf(rkv, vv[e], bv[e]));
        pw[e] = fmaf(gy[e], xh[e], pw[e]);
        pb[e] += gy[e];
        prk[e] = fmaf(q * rv[e], kv[e], prk[e]);
      }
      store8<T>(dx + idx, o_x);
      store8<T>(dv + idx, o_v);
      store8<T>(dr + idx, o_r);
      store8<T>(dk + idx, o_k);
      store8<T>(dg + idx, o_g);
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    red[wave][0][e][lane] = pw[e];
    red[wave][1][e][lane] = pb[e];
    red[wave][2][e][lane] = prk[e];
  }
  __syncthreads();
  // Wave j of the block adds parameter j's four wave partials in order.
  if (wave < 3 && active) {
    float sum[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      sum[e] = ((red[0][wave][e][lane] + red[1][wave][e][lane]) + red[2][wave][e][lane]) +
               red[3][wave][e][lane];
    }
    float* dst = partial + (static_cast<int64_t>(blockIdx.x) * 3 + wave) * channels + col;
#pragma unroll
    for (int e = 0; e < 8; e += 4) {
      *reinterpret_cast<float4*>(dst + e) = make_float4(sum[e], sum[e + 1], sum[e + 2], sum[e + 3]);
    }
  }
}

// out_j[c] = io(sum over token blocks b, in order, of partial[b][j][c]), for
// j = weight, bias, r_k.
template <typename T>
__global__ __launch_bounds__(kGateThreads) void lnx_param_reduce_kernel(
    const float* __restrict__ partial, int32_t blocks, int32_t channels,
    typename IoTraits<T>::storage* __restrict__ dweight,
    typename IoTraits<T>::storage* __restrict__ dbias,
    typename IoTraits<T>::storage* __restrict__ dr_k) {
  const int c = static_cast<int>(blockIdx.x) * kGateThreads + static_cast<int>(threadIdx.x);
  const int j = static_cast<int>(blockIdx.y);
  if (c >= channels) return;
  float sum = 0.0f;
  for (int b = 0; b < blocks; ++b) sum += partial[(static_cast<int64_t>(b) * 3 + j) * channels + c];
  typename IoTraits<T>::storage* dst = j == 0 ? dweight : j == 1 ? dbias : dr_k;
  dst[c] = from_f32<T>(sum);
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
                const void* weight, const void* bias, const void* g, void* out, float* mean,
                float* rstd, int64_t rows, int32_t heads, hipStream_t s) {
  using S = typename IoTraits<T>::storage;
  hipLaunchKernelGGL((lnx_rkvres_xg_kernel<T, D>), dim3(gate_grid(rows, D / 8)),
                     dim3(kGateThreads), 0, s, static_cast<const S*>(x),
                     static_cast<const S*>(r), static_cast<const S*>(k),
                     static_cast<const S*>(v), static_cast<const S*>(r_k),
                     static_cast<const S*>(weight), static_cast<const S*>(bias),
                     static_cast<const S*>(g), static_cast<S*>(out), mean, rstd, rows, heads);
}

struct LnxGrads {
  const void* dout;
  const void *x, *r, *k, *v, *r_k, *weight, *bias, *g;
  const float *mean, *rstd;
  void *dx, *dr, *dk, *dv, *dr_k, *dweight, *dbias, *dg;
  float* partial;
};

template <typename T, int D>
void launch_lnx_backward(const LnxGrads& a, int64_t tokens, int32_t heads, hipStream_t s) {
  using S = typename IoTraits<T>::storage;
  const int64_t channels = static_cast<int64_t>(heads) * D;
  const int blocks_t =
      static_cast<int>((tokens + kLnxTokensPerBlock - 1) / kLnxTokensPerBlock);
  const int blocks_c = static_cast<int>((channels + kLnxColsPerBlock - 1) / kLnxColsPerBlock);
  hipLaunchKernelGGL((lnx_train_backward_kernel<T, D>), dim3(blocks_t, blocks_c),
                     dim3(kGateThreads), 0, s, static_cast<const S*>(a.dout),
                     static_cast<const S*>(a.x), static_cast<const S*>(a.r),
                     static_cast<const S*>(a.k), static_cast<const S*>(a.v),
                     static_cast<const S*>(a.r_k), static_cast<const S*>(a.weight),
                     static_cast<const S*>(a.bias), static_cast<const S*>(a.g), a.mean, a.rstd,
                     static_cast<S*>(a.dx), static_cast<S*>(a.dr), static_cast<S*>(a.dk),
                     static_cast<S*>(a.dv), static_cast<S*>(a.dg), a.partial, tokens, heads);
  hipLaunchKernelGGL((lnx_param_reduce_kernel<T>),
                     dim3(static_cast<unsigned>((channels + kGateThreads - 1) / kGateThreads), 3),
                     dim3(kGateThreads), 0, s, a.partial, blocks_t,
                     static_cast<int32_t>(channels), static_cast<S*>(a.dweight),
                     static_cast<S*>(a.dbias), static_cast<S*>(a.dr_k));
}

template <typename T>
void dispatch_lnx_backward(int32_t d, const LnxGrads& a, int64_t tokens, int32_t heads,
                           hipStream_t s) {
  if (d == 64) launch_lnx_backward<T, 64>(a, tokens, heads, s);
  if (d == 128) launch_lnx_backward<T, 128>(a, tokens, heads, s);
  if (d == 256) launch_lnx_backward<T, 256>(a, tokens, heads, s);
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
                  void* out, float* mean, float* rstd, int64_t rows, int32_t heads,
                  hipStream_t s) {
  if (d == 64) launch_lnx<T, 64>(x, r, k, v, r_k, weight, bias, g, out, mean, rstd, rows, heads, s);
  if (d == 128) launch_lnx<T, 128>(x, r, k, v, r_k, weight, bias, g, out, mean, rstd, rows, heads, s);
  if (d == 256) launch_lnx<T, 256>(x, r, k, v, r_k, weight, bias, g, out, mean, rstd, rows, heads, s);
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
    dispatch_lnx<F16>(head_size, x, r, k, v, r_k, weight, bias, g, output, nullptr, nullptr,
                      rows, num_heads, s);
  } else {
    dispatch_lnx<Bf16>(head_size, x, r, k, v, r_k, weight, bias, g, output, nullptr, nullptr,
                       rows, num_heads, s);
  }
  return check_launch("lnx_rkvres_xg_kernel");
}

extern "C" int frwkv_lnx_pretrain_forward(int io_dtype, int64_t total_tokens, int32_t num_heads,
                                          int32_t head_size, const void* x, const void* r,
                                          const void* k, const void* v,
                                          const void* residual_scale, const void* weight,
                                          const void* bias, const void* g, void* output,
                                          float* mean, float* rstd, void* stream) {
  using namespace frwkv;
  if (!x || !r || !k || !v || !residual_scale || !weight || !bias || !g || !output || !mean ||
      !rstd) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_lnx_pretrain_forward: null pointer argument");
  }
  int rc = check_gate_shapes("frwkv_lnx_pretrain_forward", io_dtype, total_tokens, num_heads,
                             head_size);
  if (rc != FRWKV_OK) return rc;
  const void* all[] = {x, r, k, v, residual_scale, weight, bias, g, output};
  for (const void* p : all) {
    if (!aligned16(p)) {
      return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                       "frwkv_lnx_pretrain_forward: every token and parameter buffer must be "
                       "16-byte aligned");
    }
  }
  const int64_t rows = total_tokens * num_heads;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (io_dtype == FRWKV_DTYPE_F16) {
    dispatch_lnx<F16>(head_size, x, r, k, v, residual_scale, weight, bias, g, output, mean,
                      rstd, rows, num_heads, s);
  } else {
    dispatch_lnx<Bf16>(head_size, x, r, k, v, residual_scale, weight, bias, g, output, mean,
                       rstd, rows, num_heads, s);
  }
  return check_launch("lnx_rkvres_xg_kernel");
}

extern "C" size_t frwkv_lnx_pretrain_backward_workspace_bytes(int64_t total_tokens,
                                                             int32_t num_heads,
                                                             int32_t head_size) {
  using namespace frwkv;
  if (total_tokens <= 0 || num_heads <= 0 || head_size <= 0) return 0;
  const int64_t blocks = (total_tokens + kLnxTokensPerBlock - 1) / kLnxTokensPerBlock;
  return static_cast<size_t>(blocks) * 3 * static_cast<size_t>(num_heads) * head_size *
         sizeof(float);
}

extern "C" int frwkv_lnx_pretrain_backward(
    int io_dtype, int64_t total_tokens, int32_t num_heads, int32_t head_size,
    const void* grad_output, const void* x, const void* r, const void* k, const void* v,
    const void* residual_scale, const void* weight, const void* bias, const void* g,
    const float* mean, const float* rstd, void* grad_x, void* grad_r, void* grad_k,
    void* grad_v, void* grad_residual_scale, void* grad_weight, void* grad_bias, void* grad_g,
    void* workspace, size_t workspace_bytes, void* stream) {
  using namespace frwkv;
  if (!grad_output || !x || !r || !k || !v || !residual_scale || !weight || !bias || !g ||
      !mean || !rstd || !grad_x || !grad_r || !grad_k || !grad_v || !grad_residual_scale ||
      !grad_weight || !grad_bias || !grad_g || !workspace) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_lnx_pretrain_backward: null pointer argument");
  }
  int rc = check_gate_shapes("frwkv_lnx_pretrain_backward", io_dtype, total_tokens, num_heads,
                             head_size);
  if (rc != FRWKV_OK) return rc;
  if (total_tokens > INT32_MAX / 2) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_lnx_pretrain_backward: too many tokens (%lld)",
                     static_cast<long long>(total_tokens));
  }
  const size_t need =
      frwkv_lnx_pretrain_backward_workspace_bytes(total_tokens, num_heads, head_size);
  if (workspace_bytes < need) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_lnx_pretrain_backward: workspace of %zu bytes given, %zu needed",
                     workspace_bytes, need);
  }
  const void* all[] = {grad_output, x, r, k, v, residual_scale, weight, bias, g,
                       grad_x, grad_r, grad_k, grad_v, grad_g, workspace};
  for (const void* p : all) {
    if (!aligned16(p)) {
      return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                       "frwkv_lnx_pretrain_backward: every token, parameter and workspace "
                       "buffer must be 16-byte aligned");
    }
  }
  LnxGrads a{grad_output, x, r, k, v, residual_scale, weight, bias, g, mean, rstd,
             grad_x, grad_r, grad_k, grad_v, grad_residual_scale, grad_weight, grad_bias,
             grad_g, static_cast<float*>(workspace)};
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (io_dtype == FRWKV_DTYPE_F16) {
    dispatch_lnx_backward<F16>(head_size, a, total_tokens, num_heads, s);
  } else {
    dispatch_lnx_backward<Bf16>(head_size, a, total_tokens, num_heads, s);
  }
  return check_launch("lnx_train_backward_kernel");
}
