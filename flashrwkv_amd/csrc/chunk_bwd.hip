// Chunked WKV7 backward on bf16 MFMA (training, StateTune gradients).
//
// Replaces the reference's StateTune backward
// (csrc/sm90/tmix/wkv7/statetune_recurrent_fp32io16_backward.cu:49-676),
// which rebuilds S_{t-1} = (S_t - k v^T - b sa^T) / w token by token; that
// division loses all precision over a 64-token chunk. This kernel never
// divides by the decay: the forward writes the state at every chunk start
// (the StateTune boundary output) and the backward recomputes each chunk's
// forward quantities from it.
//
// One workgroup per (sequence, head) walks the chunks in reverse, carrying
// the state adjoint dS (dL/dS at the current chunk end) in registers. With
// the chunk notation of the forward kernel (At, Rt, Bh, Kh, Bt = Bh g,
// Kt = Kh g, g = 2^GC, Lab, Lak, Arb, Ark, T = (I - Lab)^{-1}, SA) and
// dYs = scale dY, per chunk:
//   dSA = Arb^T dYs + Bh (g o dS)            dZ  = T^T dSA
//   dV  = Ark^T dYs + Lak^T dZ + Kh (g o dS)
//   dS0 = g o dS + Rt^T dYs + At^T dZ        (becomes dS for the chunk before)
//   dArb = lower(dYs SA^T)   dArk = lower(dYs V^T)
//   dLab = strict(dZ SA^T)   dLak = strict(dZ V^T)
//   dRt = dYs S0^T + dArb Bh + dArk Kh       dAt = dZ S0^T + dLab Bh + dLak Kh
//   dBh = dLab^T At + dArb^T Rt              dKh = dLak^T At + dArk^T Rt
//   dBt = SA dS^T                            dKt = V dS^T
//   dg  = rowsum(S0 o dS)
// and the raw gradients follow elementwise: dr = dRt 2^G, da = dAt 2^Gp,
// db = 2^-G (dBh + g dBt), dk = 2^-G (dKh + g dKt). The decay enters through
// every 2^(+-G) factor; with e1_t = dRt Rt - (dBh + g dBt) Bh - (dKh + g dKt) Kh,
// e2_t = dAt At and e3_t = g (dBt Bh + dKt Kh) (per feature), the gradient of
// the log2 retention is
//   dlg_j = sum_{t>=j} (e1_t + e2_t) - e2_j + sum_t e3_t + dg g,
// a reverse scan over the chunk's tokens; the natural-log factors cancel
// against d(log2 w)/dw = 1 / (w ln 2), so dw = dlg / w and, for logits,
// dx = dlg * (-e^{-1/2} sigmoid(x) (1 - sigmoid(x))).
//
// Phases per chunk (barrier between phases):
//   prepare     operand tiles as in the forward, plus At^T, Rt^T and G;
//   intra       Lab, Lak (forward layout), Arb^T, Ark^T, Lab^T, Lak^T, T, T^T;
//   columns     wave w owns value columns 16w..16w+15: SA (forward
//               substitution), dSA, dZ (backward substitution), dV, dS0 and
//               the partial dg, all chained through registers;
//   matrices    the four C x C gradient matrices in both layouts, spread over
//               the waves, from LDS operand tiles (SA, dZ, dY, V);
//   tokens      wave p owns tokens 16p..16p+15: the [token][feature]
//               gradients, the decay scan, and the stores.
// Every HBM input of a chunk (token rows, dY and V tiles, the checkpoint
// slice) is loaded while the chunk after it computes, so no phase waits on
// HBM; the tokens phase loads its raw inputs one feature block ahead.
// Chunks must be at most 64 tokens (segments); the training wrapper splits
// longer caller chunks. A chunk whose decay span exceeds the forward's
// single-reference limit is not supported here: its sequence's gradients are
// NaN (fail closed).
#include "capi_internal.h"
#include "chunk_common.h"

namespace frwkv {
namespace {

enum BwdTri { kBLab = 0, kBLak = 1, kBArbT = 2, kBArkT = 3, kBLabT = 4, kBLakT = 5 };
enum GradTri {
  kGArb = 0, kGArbT = 1, kGArk = 2, kGArkT = 3, kGLab = 4, kGLabT = 5, kGLak = 6, kGLakT = 7
};

struct BwdSmem {
  uint16_t btT[kOpTile];  // [k][t]
  uint16_t ktT[kOpTile];  // [k][t]
  uint16_t atT[kOpTile];  // [k][t]
  uint16_t rtT[kOpTile];  // [k][t]
  uint16_t dy_x[kOpTile];       // scale * dY [t][v]
  uint16_t v_x[kOpTile];        // V  [t][v]
  float gc[kHead];              // 2^GC
  float inv_gc[kHead];          // 2^-GC
  float wave_tot[4][kHead];     // per-block sums of log2 w (prepare; read by tokens)
  float carry[4][kHead];        // token scan carries
  float carry3[4][kHead];
  float dgamma[4][kHead];       // per-wave partial of rowsum(S0 o dS)
  uint16_t sa_x[kOpTile];       // SA  [t][v]
  uint16_t dz_x[kOpTile];       // dZ  [t][v]
  union {
    struct {
      uint16_t at[kOpTile], rt[kOpTile], bh[kOpTile], kh[kOpTile];  // [t][k]
      uint16_t tri[6][kTriBlocks * kTriBlock];
      uint16_t t_r[4][kTriBlock];  // T   row-major
      uint16_t t_c[4][kTriBlock];  // T^T row-major
    } f;
    struct {
      uint16_t s0_x[kOpTile];  // S0 [k][v]
      uint16_t ds_x[kOpTile];  // dS [k][v] (adjoint at the chunk end)
      uint16_t tri[8][kTriBlocks * kTriBlock];
    } g;
  } u;
};
static_assert(sizeof(BwdSmem) <= 160 * 1024, "backward LDS budget");

struct ChunkBwdParams {
  int32_t num_heads;
  int32_t total_tokens;
  int32_t num_segments;
  const int32_t* seg_offsets;
  const int32_t* seg_starts;
  const int32_t* seg_ends;
  const float* checkpoint;      // [num_segments, H, 64, 64] state at each segment start
  const void* r;
  const void* decay;
  const void* bias;
  const void* k;
  const void* v;
  const void* a;
  const void* b;
  const void* dy;               // or null (zero)
  const float* dstate_final;    // or null (zero)
  void* dr;
  void* ddecay;
  void* dk;
  void* dv;
  void* da;
  void* db;
  float* dstate0;               // or null (not needed)
  float scale;
  // Dense layout: > 0 means every sequence has dense_t tokens and is walked
  // in 64-token chunks, with no segment arrays.
  int32_t dense_t;
  // 1: checkpoint is [B, H, dense_t / 16, D, D] (the state every 16
  // tokens); chunk c of a sequence starts at entry 4c.
  int32_t ckpt16;
};

__device__ __forceinline__ const uint16_t* ftri(const BwdSmem& sm, int m, int p, int q) {
  return sm.u.f.tri[m] + tri_index(p, q) * kTriBlock;
}
__device__ __forceinline__ const uint16_t* gtri(const BwdSmem& sm, int m, int p, int q) {
  return sm.u.g.tri[m] + tri_index(p, q) * kTriBlock;
}

// Suffix-scan step over the 16 lanes of a row: lane n adds lane n + N.
template <int N>
__device__ __forceinline__ float suffix16_step(float x) {
  const float y = __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x100 + N, 0xf, 0xf, true));
  return x + y;
}

// Prefix-scan step over the 16 lanes of a row: lane n adds lane n - N (zero
// for n < N).
template <int N>
__device__ __forceinline__ float prefix16_step(float x) {
  const float y = __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x110 + N, 0xf, 0xf, true));
  return x + y;
}

__device__ __forceinline__ float prefix16(float x) {
  x = prefix16_step<1>(x);
  x = prefix16_step<2>(x);
  x = prefix16_step<4>(x);
  return prefix16_step<8>(x);
}

__device__ __forceinline__ float suffix16(float x) {
  x = suffix16_step<1>(x);
  x = suffix16_step<2>(x);
  x = suffix16_step<4>(x);
  return suffix16_step<8>(x);
}

// HBM inputs of one chunk, loaded one chunk ahead of use: r, w, k, a, b in
// the prepare layout (thread: tokens 16w + 2tp, +1, features 8kg .. +7), dY
// and V as 16-byte pieces of [t][v] tiles (piece tid + 256 s: row
// (tid + 256 s) / 8, columns 8 ((tid + 256 s) % 8) .. +7), and this lane's
// slice of the chunk-start state.
struct BwdRows {
  uint4 r[2], w[2], k[2], a[2], b[2];
  uint4 dy[2], v[2];
  f32x4 s0[4];
};

// 8 io-dtype values -> 8 bf16 at an 8-byte aligned LDS address.
template <typename T>
__device__ __forceinline__ void store_piece_bf16(uint16_t* dst, uint4 q) {
  if constexpr (__is_same(T, Bf16)) {
    reinterpret_cast<uint2*>(dst)[0] = make_uint2(q.x, q.y);
    reinterpret_cast<uint2*>(dst)[1] = make_uint2(q.z, q.w);
  } else {
    float x[8];
    unpack8<T>(q, x);
    store8_bf16(dst, x);
  }
}

// 8 io-dtype values times `scale` -> 8 bf16 at an 8-byte aligned LDS address.
template <typename T>
__device__ __forceinline__ void store_piece_scaled_bf16(uint16_t* dst, uint4 q, float scale) {
  float x[8];
  unpack8<T>(q, x);
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] *= scale;
  store8_bf16(dst, x);
}

// Prepare: the forward's operand tiles restricted to the chunk, plus At^T,
// Rt^T (token-contiguous), the per-block decay sums and the dY / V tiles.
// Returns whether the decay span is within the single-reference limit. Ends
// with a barrier.
template <typename T, DecayMode M>
__device__ bool prepare_bwd(BwdSmem& sm, const BwdRows& rows, const float (&bias)[8],
                            int ntok, float scale) {
  const int tid = threadIdx.x;
  const int wave = uniform(tid >> 6);
  const int lane = tid & 63;
  const int tp = lane & 7;
  const int kg = lane >> 3;
  const int t0 = 16 * wave + 2 * tp;
  const float on0 = t0 < ntok ? 1.0f : 0.0f;
  const float on1 = t0 + 1 < ntok ? 1.0f : 0.0f;

  __syncthreads();

  float lg0[8], lg1[8];
  {
    float w0[8], w1[8];
    unpack8<T>(rows.w[0], w0);
    unpack8<T>(rows.w[1], w1);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      lg0[e] = on0 * log2_retention<M>(w0[e] + bias[e]);
      lg1[e] = on1 * log2_retention<M>(w1[e] + bias[e]);
    }
  }
  float incl[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float x = lg0[e] + lg1[e];
    x = scan8_step<1>(x, tp);
    x = scan8_step<2>(x, tp);
    incl[e] = scan8_step<4>(x, tp);
  }
  if (tp == 7) {
#pragma unroll
    for (int e = 0; e < 8; ++e) sm.wave_tot[wave][8 * kg + e] = incl[e];
  }
  __syncthreads();

  float g0[8], g1[8], gp0[8], total[8];
  bool over = false;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float base = 0.0f, tot = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float x = sm.wave_tot[q][8 * kg + e];
      base += (q < wave) ? x : 0.0f;
      tot += x;
    }
    total[e] = tot;
    over |= -tot > kSpanLimit;
    gp0[e] = base + incl[e] - lg0[e] - lg1[e];
    g0[e] = gp0[e] + lg0[e];
    g1[e] = g0[e] + lg1[e];
  }
  const bool whole = __builtin_amdgcn_ballot_w64(over) == 0;

#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int piece = tid + 256 * s;
    const int off = (piece >> 3) * kOpStride + 8 * (piece & 7);
    store_piece_scaled_bf16<T>(sm.dy_x + off, rows.dy[s], scale);
    store_piece_bf16<T>(sm.v_x + off, rows.v[s]);
  }
  float up0[8], up1[8], dn0[8], dn1[8], gcv[8], upp[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    upp[e] = fast_exp2(gp0[e]);
    up0[e] = fast_exp2(g0[e]);
    up1[e] = fast_exp2(g1[e]);
    dn0[e] = fast_exp2(-g0[e]);
    dn1[e] = fast_exp2(-g1[e]);
    gcv[e] = fast_exp2(total[e]);
  }
  auto row_tile = [&](uint16_t* dst, const float (&x0)[8], const float (&x1)[8],
                      const float (&f0)[8], const float (&f1)[8]) {
    float t[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) t[e] = on0 * x0[e] * f0[e];
    store8_bf16(dst + t0 * kOpStride + 8 * kg, t);
#pragma unroll
    for (int e = 0; e < 8; ++e) t[e] = on1 * x1[e] * f1[e];
    store8_bf16(dst + (t0 + 1) * kOpStride + 8 * kg, t);
  };
  auto col_tile = [&](uint16_t* dst, const float (&x0)[8], const float (&x1)[8],
                      const float (&f0)[8], const float (&f1)[8], const float (&s)[8]) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      *reinterpret_cast<uint32_t*>(dst + (8 * kg + e) * kOpStride + t0) =
          pack_bf16x2(on0 * x0[e] * (s[e] * f0[e]), on1 * x1[e] * (s[e] * f1[e]));
    }
  };
  const float ones[8] = {1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f};
  float x0[8], x1[8];
  unpack8<T>(rows.a[0], x0);
  unpack8<T>(rows.a[1], x1);
  row_tile(sm.u.f.at, x0, x1, upp, up0);
  col_tile(sm.atT, x0, x1, upp, up0, ones);
  unpack8<T>(rows.r[0], x0);
  unpack8<T>(rows.r[1], x1);
  row_tile(sm.u.f.rt, x0, x1, up0, up1);
  col_tile(sm.rtT, x0, x1, up0, up1, ones);
  unpack8<T>(rows.b[0], x0);
  unpack8<T>(rows.b[1], x1);
  row_tile(sm.u.f.bh, x0, x1, dn0, dn1);
  col_tile(sm.btT, x0, x1, dn0, dn1, gcv);
  unpack8<T>(rows.k[0], x0);
  unpack8<T>(rows.k[1], x1);
  row_tile(sm.u.f.kh, x0, x1, dn0, dn1);
  col_tile(sm.ktT, x0, x1, dn0, dn1, gcv);
  if (wave == 0 && tp == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      sm.gc[8 * kg + e] = gcv[e];
      sm.inv_gc[8 * kg + e] = __builtin_amdgcn_rcpf(gcv[e]);
    }
  }
  __syncthreads();
  return whole;
}

// Intra-chunk matrices of the backward: Lab, Lak in the forward layout
// ([t][i]), Arb, Ark, Lab, Lak transposed ([i][t]), and T, T^T. Ends with a
// barrier. A product with A = source rows, B = target rows stores [t][i];
// with A = target rows, B = source rows it stores [i][t].
// issue(i), i = 0..4, is called between the product groups: the caller
// issues a fifth of the earlier chunk's loads there, so they enter the
// memory system while the products run instead of stalling the wave on one
// burst of 30 outstanding loads.
template <typename Issue>
__device__ __forceinline__ void intra_bwd(BwdSmem& sm, Issue&& issue) {
  const int tid = threadIdx.x;
  const int wave = uniform(tid >> 6);
  const int lane = tid & 63;
  const int g = lane >> 4;
  const int n = lane & 15;

  auto mask_store = [&](int m, int p, int q, f32x4 acc, bool strict, bool transposed) {
    if (p == q) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // [t][i] storage: lane holds M[n][4g + j]; [i][t]: M[4g + j][n].
        const int t = transposed ? 4 * g + j : n;
        const int i = transposed ? n : 4 * g + j;
        const bool keep = strict ? (i < t) : (i <= t);
        acc[j] = keep ? acc[j] : 0.0f;
      }
    }
    lds_store_transposed(sm.u.f.tri[m] + tri_index(p, q) * kTriBlock, kTriStride, g, n, acc);
    return acc;
  };

  // group with_b: Lab, Lab^T, Arb^T (share Bh_q); with_k: Lak, Lak^T, Ark^T.
  auto group = [&](int p, int q, bool with_b, bool with_k, f32x4* l_r, f32x4* l_c) {
    f32x4 m0 = zero4(), m1 = zero4(), m2 = zero4();
    f32x4 n0 = zero4(), n1 = zero4(), n2 = zero4();
#pragma unroll
    for (int c = 0; c < 64; c += 32) {
      const i16x8 xa = lds_operand32<kOpStride>(sm.u.f.at, 16 * p + n, c, g);
      const i16x8 xr = lds_operand32<kOpStride>(sm.u.f.rt, 16 * p + n, c, g);
      if (with_b) {
        const i16x8 yb = lds_operand32<kOpStride>(sm.u.f.bh, 16 * q + n, c, g);
        m0 = mfma32(yb, xa, m0);  // Lab   -> [t][i]
        m1 = mfma32(xa, yb, m1);  // Lab^T -> [i][t]
        m2 = mfma32(xr, yb, m2);  // Arb^T -> [i][t]
      }
      if (with_k) {
        const i16x8 yk = lds_operand32<kOpStride>(sm.u.f.kh, 16 * q + n, c, g);
        n0 = mfma32(yk, xa, n0);  // Lak
        n1 = mfma32(xa, yk, n1);  // Lak^T
        n2 = mfma32(xr, yk, n2);  // Ark^T
      }
    }
    if (with_b) {
      const f32x4 lr = mask_store(kBLab, p, q, m0, true, false);
      const f32x4 lc = mask_store(kBLabT, p, q, m1, true, true);
      mask_store(kBArbT, p, q, m2, false, true);
      if (l_r != nullptr) {
        *l_r = lr;  // lane (g, n): L[n][4g + j]
        *l_c = lc;  // lane (g, n): L[4g + j][n]
      }
    }
    if (with_k) {
      mask_store(kBLak, p, q, n0, true, false);
      mask_store(kBLakT, p, q, n1, true, true);
      mask_store(kBArkT, p, q, n2, false, true);
    }
  };

  f32x4 l_r, l_c;
  issue(0);
  group(wave, wave, true, true, &l_r, &l_c);
  issue(1);
  // T = (I - L)^{-1} = (I + L)(I + L^2)(I + L^4)(I + L^8) in both layouts
  // (see the forward kernel): Z = X Y gives Z_C = mfma(X_R, Y_C) and
  // Z_R = mfma(Y_C, X_R).
  {
    const i16x4 lr = to_operand(l_r), lc = to_operand(l_c);
    const i16x4 p2c = to_operand(mfma16(lr, lc, zero4()));
    const i16x4 p2r = to_operand(mfma16(lc, lr, zero4()));
    const i16x4 p4c = to_operand(mfma16(p2r, p2c, zero4()));
    const i16x4 p4r = to_operand(mfma16(p2c, p2r, zero4()));
    const i16x4 p8c = to_operand(mfma16(p4r, p4c, zero4()));
    f32x4 tr = l_r, tc = l_c;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float d = (4 * g + j == n) ? 1.0f : 0.0f;
      tr[j] += d;
      tc[j] += d;
    }
    const i16x4 pc[3] = {p2c, p4c, p8c};
#pragma unroll
    for (int s = 0; s < 3; ++s) {
      const i16x4 tro = to_operand(tr);
      tc = mfma16(tro, pc[s], tc);  // (T P)_C
      tr = mfma16(pc[s], tro, tr);  // (T P)_R
    }
    lds_store_transposed(sm.u.f.t_r[wave], kTriStride, g, n, tr);  // T   [t][i]
    lds_store_transposed(sm.u.f.t_c[wave], kTriStride, g, n, tc);  // T^T [i][t]
  }
#pragma unroll
  for (int r = 0; r < 3; ++r) {
    const int item = wave + 4 * r;
    const int pair = item >> 1;
    const int p = pair < 1 ? 1 : (pair < 3 ? 2 : 3);
    const int q = pair - (p * (p - 1)) / 2;
    issue(2 + r);
    group(p, q, (item & 1) == 0, (item & 1) == 1, nullptr, nullptr);
  }
  __syncthreads();
}

template <typename T, DecayMode M>
__global__ __launch_bounds__(kChunkThreads, 1) void chunk_bwd_kernel(ChunkBwdParams p) {
  __shared__ BwdSmem sm;
  using S16 = typename IoTraits<T>::storage;

  const int tid = threadIdx.x;
  const int wave = uniform(tid >> 6);
  const int lane = tid & 63;
  const int g = lane >> 4;
  const int n = lane & 15;
  const int tp = lane & 7;
  const int kg = lane >> 3;
  const int heads = p.num_heads;
  const int seq = blockIdx.x / heads;
  const int head = blockIdx.x % heads;
  const int seg_lo = p.dense_t > 0 ? 0 : uniform(max(p.seg_offsets[seq], 0));
  const int seg_hi = p.dense_t > 0 ? (p.dense_t + kChunk - 1) / kChunk
                                   : uniform(min(p.seg_offsets[seq + 1], p.num_segments));

  float bias[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) bias[e] = 0.0f;
  if constexpr (M == DecayMode::kLogits) {
    if (p.bias != nullptr) {
      unpack8<T>(load_row8<T>(p.bias, static_cast<int64_t>(head) * kHead + 8 * kg), bias);
    }
  }

  const uint32_t row_bytes = static_cast<uint32_t>(heads) * kHead * 2;
  const uint32_t prep_off = static_cast<uint32_t>(16 * wave + 2 * tp) * row_bytes + 16 * kg;
  const uint32_t v_off = static_cast<uint32_t>(4 * g) * row_bytes + 2 * (16 * wave + n);
  // State slices: element (row, col) of a 64 x 64 fp32 state at byte
  // 4 * (64 row + col); lane (g, n) of wave w holds rows 16kb + 4g + j, col 16w + n.
  const uint32_t s_off = static_cast<uint32_t>((4 * g) * kHead + 16 * wave + n) * 4;
  const int64_t unit_state = (static_cast<int64_t>(seq) * heads + head) * kHead * kHead;

  f32x4 dS[4];
  {
    const auto rs = buffer_rsrc(p.dstate_final != nullptr ? p.dstate_final + unit_state : nullptr,
                                p.dstate_final != nullptr ? kHead * kHead * 4 : 0);
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        dS[kb][j] = __uint_as_float(
            __builtin_amdgcn_raw_buffer_load_b32(rs, s_off, (16 * kb + j) * kHead * 4, 0));
      }
    }
  }
  bool failed = false;
  const float kNaN = __int_as_float(0x7fc00000);

  // Segment bounds, 64 segments at a time in VGPR lanes (lane i: segment
  // cache_base + i), read back with readlane. A per-segment memory read would
  // need a vmcnt wait, which on gfx9's in-order counter also waits for every
  // gradient store still in flight.
  int cache_base = seg_hi;
  int starts_v = 0, ends_v = 0;
  auto seg_bounds = [&](int seg, int& tb, int& te) {
    if (p.dense_t > 0) {
      tb = seq * p.dense_t + kChunk * seg;
      te = min(tb + kChunk, (seq + 1) * p.dense_t);
      return;
    }
    if (seg < cache_base) {
      cache_base = uniform(max(seg - 63, seg_lo));
      const int idx = cache_base + lane;
      starts_v = idx <= seg ? p.seg_starts[idx] : 0;
      ends_v = idx <= seg ? p.seg_ends[idx] : 0;
      __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt(0): nothing pending at the join
    }
    tb = uniform(max(__builtin_amdgcn_readlane(starts_v, seg - cache_base), 0));
    te = uniform(min(__builtin_amdgcn_readlane(ends_v, seg - cache_base), p.total_tokens));
  };

  // Inputs of a chunk (see BwdRows), in five pieces (0: w, r; 1: k, a;
  // 2: b, dY; 3: V and the first half of the checkpoint slice; 4: the rest).
  // Rows past the chunk's tokens read as zero through the buffer bounds; an
  // invalid segment (seg < seg_lo) has empty ranges and loads zeros.
  struct ChunkSrc {
    int64_t b0;
    uint32_t nbytes;
    int64_t ck_index;
    bool valid;
  };
  auto chunk_src = [&](int seg) {
    ChunkSrc c{0, 0u, 0, false};
    if (seg < seg_lo) return c;
    int tb, te;
    seg_bounds(seg, tb, te);
    const int nt = uniform(max(min(te - tb, kChunk), 0));
    c.b0 = (static_cast<int64_t>(tb) * heads + head) * kHead;
    c.nbytes = static_cast<uint32_t>(nt) * row_bytes;
    c.ck_index = p.ckpt16 ? (static_cast<int64_t>(seq) * heads + head) * (p.dense_t / 16) + 4 * seg
                          : static_cast<int64_t>(seg) * heads + head;
    c.valid = true;
    return c;
  };
  auto load_piece = [&](const ChunkSrc& c, BwdRows& rows, int piece) {
    auto brs = [&](const void* x) {
      return buffer_rsrc(x != nullptr ? static_cast<const S16*>(x) + c.b0 : nullptr,
                         x != nullptr ? c.nbytes : 0u);
    };
    auto ld = [&](__amdgpu_buffer_rsrc_t r, uint32_t off, int so) {
      const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(r, off, so, 0);
      return make_uint4(x.x, x.y, x.z, x.w);
    };
    auto rows2 = [&](const void* x, uint4 (&dst)[2]) {
      const auto r = brs(x);
#pragma unroll
      for (int s = 0; s < 2; ++s) dst[s] = ld(r, prep_off, s * static_cast<int>(row_bytes));
    };
    auto tile2 = [&](const void* x, uint4 (&dst)[2]) {
      const auto r = brs(x);
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int tp_piece = tid + 256 * s;
        dst[s] = ld(r, static_cast<uint32_t>(tp_piece >> 3) * row_bytes + 16 * (tp_piece & 7), 0);
      }
    };
    auto ckpt = [&](int kb0) {
      const auto ck = buffer_rsrc(c.valid ? p.checkpoint + c.ck_index * kHead * kHead : nullptr,
                                  c.valid ? kHead * kHead * 4 : 0);
#pragma unroll
      for (int kb = kb0; kb < kb0 + 2; ++kb) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          rows.s0[kb][j] = __uint_as_float(
              __builtin_amdgcn_raw_buffer_load_b32(ck, s_off, (16 * kb + j) * kHead * 4, 0));
        }
      }
    };
    if (piece == 0) {
      rows2(p.decay, rows.w);
      rows2(p.r, rows.r);
    } else if (piece == 1) {
      rows2(p.k, rows.k);
      rows2(p.a, rows.a);
    } else if (piece == 2) {
      rows2(p.b, rows.b);
      tile2(p.dy, rows.dy);
    } else if (piece == 3) {
      tile2(p.v, rows.v);
      ckpt(0);
    } else {
      ckpt(2);
    }
  };
  auto load_chunk = [&](int seg, BwdRows& rows) {
    const ChunkSrc c = chunk_src(seg);
#pragma unroll
    for (int piece = 0; piece < 5; ++piece) load_piece(c, rows, piece);
  };

  BwdRows rows;
  int loaded = seg_hi;

  for (int seg = seg_hi - 1; seg >= seg_lo; --seg) {
    if (loaded != seg) {
      // First chunk, or the one after an empty segment: load in place and
      // drain (vmcnt(0)), so that only the prefetched rows are pending where
      // the paths join.
      load_chunk(seg, rows);
      loaded = seg;
      __builtin_amdgcn_s_waitcnt(0xF70);
    }
    int t_begin, t_end;
    seg_bounds(seg, t_begin, t_end);
    const int ntok = uniform(min(t_end - t_begin, kChunk));
    if (ntok <= 0) continue;
    // Chunks longer than 64 tokens have no checkpoint inside: fail closed.
    failed = failed || (t_end - t_begin > kChunk);
    const int64_t base = (static_cast<int64_t>(t_begin) * heads + head) * kHead;
    const uint32_t bytes = static_cast<uint32_t>(ntok) * row_bytes;
    auto rs = [&](const void* x) {
      return buffer_rsrc(x != nullptr ? static_cast<const S16*>(x) + base : nullptr,
                         x != nullptr ? bytes : 0u);
    };
    const auto r_rs = rs(p.r), w_rs = rs(p.decay), k_rs = rs(p.k), a_rs = rs(p.a),
               b_rs = rs(p.b);

    const bool whole = prepare_bwd<T, M>(sm, rows, bias, ntok, p.scale);
    failed = failed || !whole;
    f32x4 S0[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) S0[kb] = rows.s0[kb];
    // The rows are in LDS now: the chunk before this one is loaded during
    // the intra-chunk products (below, or here on the fail-closed path).
    // Unconditional: before the first segment the ranges are empty (a
    // skipped load would make the compiler's in-order wait counts too
    // strict).
    const ChunkSrc prev = chunk_src(seg - 1);
    if (prev.valid) loaded = seg - 1;
    if (failed) {
#pragma unroll
      for (int piece = 0; piece < 5; ++piece) load_piece(prev, rows, piece);
      // Fail closed: NaN gradients for this chunk, and for every earlier one
      // (the adjoint would be wrong from here on).
      // Rows past the chunk's tokens fall outside the buffer range and are
      // dropped (as for every gradient store below).
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const u32x4 nan4 = {0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u};
        const int so = s * static_cast<int>(row_bytes);
        __builtin_amdgcn_raw_buffer_store_b128(nan4, rs(p.dr), prep_off, so, 0);
        __builtin_amdgcn_raw_buffer_store_b128(nan4, rs(p.ddecay), prep_off, so, 0);
        __builtin_amdgcn_raw_buffer_store_b128(nan4, rs(p.dk), prep_off, so, 0);
        __builtin_amdgcn_raw_buffer_store_b128(nan4, rs(p.dv), prep_off, so, 0);
        __builtin_amdgcn_raw_buffer_store_b128(nan4, rs(p.da), prep_off, so, 0);
        __builtin_amdgcn_raw_buffer_store_b128(nan4, rs(p.db), prep_off, so, 0);
      }
      continue;
    }
    intra_bwd(sm, [&](int piece) { load_piece(prev, rows, piece); });

    // ---------------------------------------------------------- columns --
    // V and scale * dY in operand layout: lane (g, n) holds X[16q + 4g + e][16w + n].
    i16x4 vs[4], dys[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      vs[q] = lds_operand_tr<kOpStride>(sm.v_x, 16 * q, 16 * wave, g, n);
      dys[q] = lds_operand_tr<kOpStride>(sm.dy_x, 16 * q, 16 * wave, g, n);
    }
    const i16x4 z4 = {0, 0, 0, 0};
    auto lo32 = [&](i16x4 x) { return cat(x, z4); };
    auto ft16 = [&](int m, int pp, int q) {
      return lds_operand<kTriStride>(ftri(sm, m, pp, q), n, 4 * g);
    };
    const i16x8 s01 = cat(to_operand(S0[0]), to_operand(S0[1]));
    const i16x8 s23 = cat(to_operand(S0[2]), to_operand(S0[3]));
    const i16x8 v01 = cat(vs[0], vs[1]), v23 = cat(vs[2], vs[3]);

    // SA = T (At S0 + Lak V), as in the forward.
    f32x4 rhs[4];
#pragma unroll
    for (int pb = 0; pb < 4; ++pb) {
      rhs[pb] = mfma32(lds_operand32<kOpStride>(sm.u.f.at, 16 * pb + n, 0, g), s01, zero4());
    }
#pragma unroll
    for (int pb = 0; pb < 4; ++pb) {
      rhs[pb] = mfma32(lds_operand32<kOpStride>(sm.u.f.at, 16 * pb + n, 32, g), s23, rhs[pb]);
    }
    rhs[0] = mfma32(lo32(ft16(kBLak, 0, 0)), lo32(vs[0]), rhs[0]);
    rhs[1] = mfma32(cat(ft16(kBLak, 1, 0), ft16(kBLak, 1, 1)), v01, rhs[1]);
    rhs[2] = mfma32(cat(ft16(kBLak, 2, 0), ft16(kBLak, 2, 1)), v01, rhs[2]);
    rhs[3] = mfma32(cat(ft16(kBLak, 3, 0), ft16(kBLak, 3, 1)), v01, rhs[3]);
    rhs[2] = mfma32(lo32(ft16(kBLak, 2, 2)), lo32(vs[2]), rhs[2]);
    rhs[3] = mfma32(cat(ft16(kBLak, 3, 2), ft16(kBLak, 3, 3)), v23, rhs[3]);
    auto tr16 = [&](int pb) { return lds_operand<kTriStride>(sm.u.f.t_r[pb], n, 4 * g); };
    auto tc16 = [&](int pb) { return lds_operand<kTriStride>(sm.u.f.t_c[pb], n, 4 * g); };
    f32x4 sa[4];
    i16x4 sab[4];
    sa[0] = mfma32(lo32(tr16(0)), lo32(to_operand(rhs[0])), zero4());
    sab[0] = to_operand(sa[0]);
    rhs[1] = mfma32(lo32(ft16(kBLab, 1, 0)), lo32(sab[0]), rhs[1]);
    sa[1] = mfma32(lo32(tr16(1)), lo32(to_operand(rhs[1])), zero4());
    sab[1] = to_operand(sa[1]);
    const i16x8 sa01 = cat(sab[0], sab[1]);
    rhs[2] = mfma32(cat(ft16(kBLab, 2, 0), ft16(kBLab, 2, 1)), sa01, rhs[2]);
    rhs[3] = mfma32(cat(ft16(kBLab, 3, 0), ft16(kBLab, 3, 1)), sa01, rhs[3]);
    sa[2] = mfma32(lo32(tr16(2)), lo32(to_operand(rhs[2])), zero4());
    sab[2] = to_operand(sa[2]);
    rhs[3] = mfma32(lo32(ft16(kBLab, 3, 2)), lo32(sab[2]), rhs[3]);
    sa[3] = mfma32(lo32(tr16(3)), lo32(to_operand(rhs[3])), zero4());

    // g o dS and the partial row sums of S0 o dS.
    i16x4 gds[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      f32x4 x;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int kf = 16 * kb + 4 * g + j;
        x[j] = sm.gc[kf] * dS[kb][j];
        float s = S0[kb][j] * dS[kb][j];
        s = suffix16(s);  // lane n = 0 holds the row sum
        if (n == 0) sm.dgamma[wave][kf] = s;
      }
      gds[kb] = to_operand(x);
    }
    const i16x8 gds01 = cat(gds[0], gds[1]), gds23 = cat(gds[2], gds[3]);
    const i16x8 dy01 = cat(dys[0], dys[1]), dy23 = cat(dys[2], dys[3]);

    // dSA_p = sum_{q>=p} Arb^T(q,p) dYs_q + Bh_p (g o dS). Arb^T block (q, p)
    // (stored at tri index (q, p)) has rows i of block p, columns t of q.
    f32x4 dsa[4];
#pragma unroll
    for (int pb = 0; pb < 4; ++pb) {
      dsa[pb] = mfma32(lds_operand32<kOpStride>(sm.u.f.bh, 16 * pb + n, 0, g), gds01, zero4());
    }
#pragma unroll
    for (int pb = 0; pb < 4; ++pb) {
      dsa[pb] = mfma32(lds_operand32<kOpStride>(sm.u.f.bh, 16 * pb + n, 32, g), gds23, dsa[pb]);
    }
    dsa[0] = mfma32(cat(ft16(kBArbT, 0, 0), ft16(kBArbT, 1, 0)), dy01, dsa[0]);
    dsa[0] = mfma32(cat(ft16(kBArbT, 2, 0), ft16(kBArbT, 3, 0)), dy23, dsa[0]);
    dsa[1] = mfma32(lo32(ft16(kBArbT, 1, 1)), lo32(dys[1]), dsa[1]);
    dsa[1] = mfma32(cat(ft16(kBArbT, 2, 1), ft16(kBArbT, 3, 1)), dy23, dsa[1]);
    dsa[2] = mfma32(cat(ft16(kBArbT, 2, 2), ft16(kBArbT, 3, 2)), dy23, dsa[2]);
    dsa[3] = mfma32(lo32(ft16(kBArbT, 3, 3)), lo32(dys[3]), dsa[3]);

    // dZ = T^T dSA: dZ_p = T_pp^T (dSA_p + sum_{q>p} Lab^T(q,p) dZ_q).
    f32x4 dz[4];
    i16x4 dzb[4];
    dz[3] = mfma32(lo32(tc16(3)), lo32(to_operand(dsa[3])), zero4());
    dzb[3] = to_operand(dz[3]);
    dsa[2] = mfma32(lo32(ft16(kBLabT, 3, 2)), lo32(dzb[3]), dsa[2]);
    dz[2] = mfma32(lo32(tc16(2)), lo32(to_operand(dsa[2])), zero4());
    dzb[2] = to_operand(dz[2]);
    const i16x8 dz23 = cat(dzb[2], dzb[3]);
    dsa[1] = mfma32(cat(ft16(kBLabT, 2, 1), ft16(kBLabT, 3, 1)), dz23, dsa[1]);
    dsa[0] = mfma32(cat(ft16(kBLabT, 2, 0), ft16(kBLabT, 3, 0)), dz23, dsa[0]);
    dz[1] = mfma32(lo32(tc16(1)), lo32(to_operand(dsa[1])), zero4());
    dzb[1] = to_operand(dz[1]);
    dsa[0] = mfma32(lo32(ft16(kBLabT, 1, 0)), lo32(dzb[1]), dsa[0]);
    dz[0] = mfma32(lo32(tc16(0)), lo32(to_operand(dsa[0])), zero4());
    dzb[0] = to_operand(dz[0]);
    const i16x8 dz01 = cat(dzb[0], dzb[1]);

    // dV_p = sum_{q>=p} (Ark^T(q,p) dYs_q + Lak^T(q,p) dZ_q) + Kh_p (g o dS).
    {
      f32x4 dvv[4];
#pragma unroll
      for (int pb = 0; pb < 4; ++pb) {
        dvv[pb] = mfma32(lds_operand32<kOpStride>(sm.u.f.kh, 16 * pb + n, 0, g), gds01, zero4());
      }
#pragma unroll
      for (int pb = 0; pb < 4; ++pb) {
        dvv[pb] = mfma32(lds_operand32<kOpStride>(sm.u.f.kh, 16 * pb + n, 32, g), gds23, dvv[pb]);
      }
      dvv[0] = mfma32(cat(ft16(kBArkT, 0, 0), ft16(kBArkT, 1, 0)), dy01, dvv[0]);
      dvv[0] = mfma32(cat(ft16(kBArkT, 2, 0), ft16(kBArkT, 3, 0)), dy23, dvv[0]);
      dvv[0] = mfma32(cat(ft16(kBLakT, 0, 0), ft16(kBLakT, 1, 0)), dz01, dvv[0]);
      dvv[0] = mfma32(cat(ft16(kBLakT, 2, 0), ft16(kBLakT, 3, 0)), dz23, dvv[0]);
      dvv[1] = mfma32(lo32(ft16(kBArkT, 1, 1)), lo32(dys[1]), dvv[1]);
      dvv[1] = mfma32(cat(ft16(kBArkT, 2, 1), ft16(kBArkT, 3, 1)), dy23, dvv[1]);
      dvv[1] = mfma32(lo32(ft16(kBLakT, 1, 1)), lo32(dzb[1]), dvv[1]);
      dvv[1] = mfma32(cat(ft16(kBLakT, 2, 1), ft16(kBLakT, 3, 1)), dz23, dvv[1]);
      dvv[2] = mfma32(cat(ft16(kBArkT, 2, 2), ft16(kBArkT, 3, 2)), dy23, dvv[2]);
      dvv[2] = mfma32(cat(ft16(kBLakT, 2, 2), ft16(kBLakT, 3, 2)), dz23, dvv[2]);
      dvv[3] = mfma32(lo32(ft16(kBArkT, 3, 3)), lo32(dys[3]), dvv[3]);
      dvv[3] = mfma32(lo32(ft16(kBLakT, 3, 3)), lo32(dzb[3]), dvv[3]);
      const auto dv_rs = rs(p.dv);
#pragma unroll
      for (int pb = 0; pb < 4; ++pb) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int t = 16 * pb + 4 * g + j;
          __builtin_amdgcn_raw_buffer_store_b16(
              from_f32<T>(dvv[pb][j]), dv_rs,
              static_cast<uint32_t>(t) * row_bytes + 2 * (16 * wave + n), 0, 0);
        }
      }
    }

    // dS0 = g o dS + Rt^T dYs + At^T dZ (new adjoint for the chunk before).
    f32x4 dS_end[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      dS_end[kb] = dS[kb];
      f32x4 acc;
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = sm.gc[16 * kb + 4 * g + j] * dS[kb][j];
      acc = mfma32(lds_operand32<kOpStride>(sm.rtT, 16 * kb + n, 0, g), dy01, acc);
      acc = mfma32(lds_operand32<kOpStride>(sm.rtT, 16 * kb + n, 32, g), dy23, acc);
      acc = mfma32(lds_operand32<kOpStride>(sm.atT, 16 * kb + n, 0, g), dz01, acc);
      acc = mfma32(lds_operand32<kOpStride>(sm.atT, 16 * kb + n, 32, g), dz23, acc);
      dS[kb] = acc;
    }

    // Exchange SA and dZ ([t][v]) for the matrix and token phases.
#pragma unroll
    for (int pb = 0; pb < 4; ++pb) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = 16 * pb + 4 * g + j;
        sm.sa_x[t * kOpStride + 16 * wave + n] = to_bf16_bits(sa[pb][j]);
        sm.dz_x[t * kOpStride + 16 * wave + n] = to_bf16_bits(dz[pb][j]);
      }
    }
    __syncthreads();

    // --------------------------------------------------------- matrices --
    // S0 and dS (adjoint at the chunk end) as [k][v] operand tiles.
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int kf = 16 * kb + 4 * g + j;
        sm.u.g.s0_x[kf * kOpStride + 16 * wave + n] = to_bf16_bits(S0[kb][j]);
        sm.u.g.ds_x[kf * kOpStride + 16 * wave + n] = to_bf16_bits(dS_end[kb][j]);
      }
    }
    // The tokens phase's raw inputs: (token 16w + n, features 16kb + 4g .. +3).
    const uint32_t tok_off = static_cast<uint32_t>(16 * wave + n) * row_bytes + 8 * g;
    // Loaded one feature block ahead of use (block 0 here, block kb + 1
    // while block kb computes).
    u32x2 raw_next[5];
    auto load_raw = [&](int kb) {
      const int so = 2 * 16 * kb;
      raw_next[0] = __builtin_amdgcn_raw_buffer_load_b64(a_rs, tok_off, so, 0);
      raw_next[1] = __builtin_amdgcn_raw_buffer_load_b64(r_rs, tok_off, so, 0);
      raw_next[2] = __builtin_amdgcn_raw_buffer_load_b64(b_rs, tok_off, so, 0);
      raw_next[3] = __builtin_amdgcn_raw_buffer_load_b64(k_rs, tok_off, so, 0);
      raw_next[4] = __builtin_amdgcn_raw_buffer_load_b64(w_rs, tok_off, so, 0);
    };
    load_raw(0);
    // 40 (matrix, block pair) items, 10 per wave; both layouts each.
#pragma unroll 1
    for (int item = wave; item < 40; item += 4) {
      const int m = item / 10;      // 0 dArb, 1 dArk, 2 dLab, 3 dLak
      const int pair = item % 10;
      const int pb = pair < 1 ? 0 : pair < 3 ? 1 : pair < 6 ? 2 : 3;
      const int q = pair - (pb * (pb + 1)) / 2;
      const bool strict = m >= 2;
      f32x4 mt = zero4(), mc = zero4();  // M^T in C layout (stores [t][i]), M (stores [i][t])
#pragma unroll
      for (int c = 0; c < 64; c += 32) {
        const i16x8 x = lds_operand32<kOpStride>(m < 2 ? sm.dy_x : sm.dz_x, 16 * pb + n, c, g);
        const i16x8 y = lds_operand32<kOpStride>((m & 1) ? sm.v_x : sm.sa_x, 16 * q + n, c, g);
        mt = mfma32(y, x, mt);
        mc = mfma32(x, y, mc);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (pb == q) {
          // mt: lane holds M[t = n][i = 4g + j]; mc: M[t = 4g + j][i = n].
          const int it = 4 * g + j;
          const bool keep_t = strict ? (it < n) : (it <= n);
          const bool keep_c = strict ? (n < it) : (n <= it);
          mt[j] = keep_t ? mt[j] : 0.0f;
          mc[j] = keep_c ? mc[j] : 0.0f;
        }
      }
      lds_store_transposed(sm.u.g.tri[2 * m] + tri_index(pb, q) * kTriBlock, kTriStride, g, n, mt);
      lds_store_transposed(sm.u.g.tri[2 * m + 1] + tri_index(pb, q) * kTriBlock, kTriStride, g,
                           n, mc);
    }
    __syncthreads();

    // ----------------------------------------------------------- tokens --
    // Wave p owns tokens 16p..16p+15. Output blocks X^T (rows = features
    // 16kb + 4g + j, cols = tokens): lane (g, n) holds X[t = 16p + n][k].
    const int pb = wave;
    auto gt16 = [&](int mm, int pp, int q) {
      return lds_operand<kTriStride>(gtri(sm, mm, pp, q), n, 4 * g);
    };
    // Kept for the decay gradient after the barrier: the in-block suffix sums
    // of e1 + e2, e2 itself and the decay input.
    float suf[4][4], e2v[4][4], dec_in[4][4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      u32x2 raw_cur[5];
#pragma unroll
      for (int i = 0; i < 5; ++i) raw_cur[i] = raw_next[i];
      if (kb < 3) load_raw(kb + 1);
      f32x4 acc_s = zero4(), acc_z = zero4(), acc_bt = zero4(), acc_kt = zero4();
#pragma unroll
      for (int c = 0; c < 64; c += 32) {
        const i16x8 s0r = lds_operand32<kOpStride>(sm.u.g.s0_x, 16 * kb + n, c, g);
        const i16x8 dsr = lds_operand32<kOpStride>(sm.u.g.ds_x, 16 * kb + n, c, g);
        acc_s = mfma32(s0r, lds_operand32<kOpStride>(sm.dy_x, 16 * pb + n, c, g), acc_s);  // S0 dY^T
        acc_z = mfma32(s0r, lds_operand32<kOpStride>(sm.dz_x, 16 * pb + n, c, g), acc_z);  // S0 dZ^T
        acc_bt = mfma32(dsr, lds_operand32<kOpStride>(sm.sa_x, 16 * pb + n, c, g), acc_bt);  // dS SA^T
        acc_kt = mfma32(dsr, lds_operand32<kOpStride>(sm.v_x, 16 * pb + n, c, g), acc_kt);  // dS V^T
      }
      // Bt^T dArb^T + Kt^T dArk^T and Bt^T dLab^T + Kt^T dLak^T over source
      // blocks q <= p (K = tokens i).
      f32x4 acc_r = zero4(), acc_a = zero4();
      auto bt16 = [&](const uint16_t* tile, int q) {
        return lds_operand<kOpStride>(tile, 16 * kb + n, 16 * q + 4 * g);
      };
      if (pb == 0) {
        acc_r = mfma32(lo32(bt16(sm.btT, 0)), lo32(gt16(kGArb, 0, 0)), acc_r);
        acc_r = mfma32(lo32(bt16(sm.ktT, 0)), lo32(gt16(kGArk, 0, 0)), acc_r);
        acc_a = mfma32(lo32(bt16(sm.btT, 0)), lo32(gt16(kGLab, 0, 0)), acc_a);
        acc_a = mfma32(lo32(bt16(sm.ktT, 0)), lo32(gt16(kGLak, 0, 0)), acc_a);
      } else {
        const i16x8 b01 = cat(bt16(sm.btT, 0), bt16(sm.btT, 1));
        const i16x8 k01 = cat(bt16(sm.ktT, 0), bt16(sm.ktT, 1));
        acc_r = mfma32(b01, cat(gt16(kGArb, pb, 0), gt16(kGArb, pb, 1)), acc_r);
        acc_r = mfma32(k01, cat(gt16(kGArk, pb, 0), gt16(kGArk, pb, 1)), acc_r);
        acc_a = mfma32(b01, cat(gt16(kGLab, pb, 0), gt16(kGLab, pb, 1)), acc_a);
        acc_a = mfma32(k01, cat(gt16(kGLak, pb, 0), gt16(kGLak, pb, 1)), acc_a);
        if (pb == 2) {
          acc_r = mfma32(lo32(bt16(sm.btT, 2)), lo32(gt16(kGArb, 2, 2)), acc_r);
          acc_r = mfma32(lo32(bt16(sm.ktT, 2)), lo32(gt16(kGArk, 2, 2)), acc_r);
          acc_a = mfma32(lo32(bt16(sm.btT, 2)), lo32(gt16(kGLab, 2, 2)), acc_a);
          acc_a = mfma32(lo32(bt16(sm.ktT, 2)), lo32(gt16(kGLak, 2, 2)), acc_a);
        } else if (pb == 3) {
          const i16x8 b23 = cat(bt16(sm.btT, 2), bt16(sm.btT, 3));
          const i16x8 k23 = cat(bt16(sm.ktT, 2), bt16(sm.ktT, 3));
          acc_r = mfma32(b23, cat(gt16(kGArb, 3, 2), gt16(kGArb, 3, 3)), acc_r);
          acc_r = mfma32(k23, cat(gt16(kGArk, 3, 2), gt16(kGArk, 3, 3)), acc_r);
          acc_a = mfma32(b23, cat(gt16(kGLab, 3, 2), gt16(kGLab, 3, 3)), acc_a);
          acc_a = mfma32(k23, cat(gt16(kGLak, 3, 2), gt16(kGLak, 3, 3)), acc_a);
        }
      }
      // dBh^T, dKh^T for source tokens i in block p: K = target tokens t in
      // blocks qt >= p; B = dLab^T / dArb^T rows i (stored at (qt, p)).
      f32x4 acc_bh = zero4(), acc_kh = zero4();
      auto at16 = [&](const uint16_t* tile, int qt) {
        return lds_operand<kOpStride>(tile, 16 * kb + n, 16 * qt + 4 * g);
      };
      auto tr_pair = [&](int qa, int qb2) {
        acc_bh = mfma32(cat(at16(sm.atT, qa), at16(sm.atT, qb2)),
                        cat(gt16(kGLabT, qa, pb), gt16(kGLabT, qb2, pb)), acc_bh);
        acc_bh = mfma32(cat(at16(sm.rtT, qa), at16(sm.rtT, qb2)),
                        cat(gt16(kGArbT, qa, pb), gt16(kGArbT, qb2, pb)), acc_bh);
        acc_kh = mfma32(cat(at16(sm.atT, qa), at16(sm.atT, qb2)),
                        cat(gt16(kGLakT, qa, pb), gt16(kGLakT, qb2, pb)), acc_kh);
        acc_kh = mfma32(cat(at16(sm.rtT, qa), at16(sm.rtT, qb2)),
                        cat(gt16(kGArkT, qa, pb), gt16(kGArkT, qb2, pb)), acc_kh);
      };
      auto tr_single = [&](int qa) {
        acc_bh = mfma32(lo32(at16(sm.atT, qa)), lo32(gt16(kGLabT, qa, pb)), acc_bh);
        acc_bh = mfma32(lo32(at16(sm.rtT, qa)), lo32(gt16(kGArbT, qa, pb)), acc_bh);
        acc_kh = mfma32(lo32(at16(sm.atT, qa)), lo32(gt16(kGLakT, qa, pb)), acc_kh);
        acc_kh = mfma32(lo32(at16(sm.rtT, qa)), lo32(gt16(kGArkT, qa, pb)), acc_kh);
      };
      if (pb == 0) {
        tr_pair(0, 1);
        tr_pair(2, 3);
      } else if (pb == 1) {
        tr_single(1);
        tr_pair(2, 3);
      } else if (pb == 2) {
        tr_pair(2, 3);
      } else {
        tr_single(3);
      }

      // Elementwise chain rule for (token t = 16p + n, feature 16kb + 4g + j).
      const int so = static_cast<int>(2 * 16 * kb);
      auto raw4 = [&](const u32x2 x, float (&out)[4]) {
        out[0] = to_f32<T>(static_cast<uint16_t>(x.x & 0xffffu));
        out[1] = to_f32<T>(static_cast<uint16_t>(x.x >> 16));
        out[2] = to_f32<T>(static_cast<uint16_t>(x.y & 0xffffu));
        out[3] = to_f32<T>(static_cast<uint16_t>(x.y >> 16));
      };
      float ra[4], rr[4], rb[4], rk[4], rw[4];
      raw4(raw_cur[0], ra);
      raw4(raw_cur[1], rr);
      raw4(raw_cur[2], rb);
      raw4(raw_cur[3], rk);
      raw4(raw_cur[4], rw);
      float grad_r[4], grad_a[4], grad_b[4], grad_k[4];
      const int t = 16 * pb + n;
      // Per-feature chunk factors of the lane's 4 consecutive features, and
      // the block sums of the earlier token blocks, as 16-byte LDS reads.
      const int kf0 = 16 * kb + 4 * g;
      const float4 gam4 = *reinterpret_cast<const float4*>(&sm.gc[kf0]);
      const float4 inv4 = *reinterpret_cast<const float4*>(&sm.inv_gc[kf0]);
      float4 carry4 = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        if (q < pb) {
          const float4 c = *reinterpret_cast<const float4*>(&sm.wave_tot[q][kf0]);
          carry4.x += c.x; carry4.y += c.y; carry4.z += c.z; carry4.w += c.w;
        }
      }
      const float gam_v[4] = {gam4.x, gam4.y, gam4.z, gam4.w};
      const float inv_v[4] = {inv4.x, inv4.y, inv4.z, inv4.w};
      const float carry_v[4] = {carry4.x, carry4.y, carry4.z, carry4.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int kf = kf0 + j;
        float xin = rw[j];
        if constexpr (M == DecayMode::kLogits) {
          if (p.bias != nullptr) {
            xin += to_f32<T>(static_cast<const S16*>(p.bias)[static_cast<int64_t>(head) * kHead + kf]);
          }
        }
        const bool on = t < ntok;
        const float lg = on ? log2_retention<M>(xin) : 0.0f;
        const float gam = gam_v[j];
        const float inv_g = inv_v[j];
        // Inclusive cumulative log2 decay G_t: the block sums of earlier
        // token blocks plus a scan over this block's 16 tokens (lane n).
        const float G = prefix16(lg) + carry_v[j];
        const float upp = fast_exp2(G - lg);
        // 2^G = 2^(G - lg) w: in raw-retention mode w is the (clamped) input,
        // which saves an exponential; the logits mode evaluates 2^G directly.
        float upg;
        if constexpr (M == DecayMode::kRawW) {
          upg = upp * (on ? __builtin_amdgcn_fmed3f(xin, 0x1p-20f, 1.0f) : 1.0f);
        } else {
          upg = fast_exp2(G);
        }
        const float dng = fast_exp2(-G);
        const float dRt = acc_s[j] + inv_g * acc_r[j];
        const float dAt = acc_z[j] + inv_g * acc_a[j];
        const float dBc = acc_bh[j] + gam * acc_bt[j];  // dBh + g dBt
        const float dKc = acc_kh[j] + gam * acc_kt[j];  // dKh + g dKt
        grad_r[j] = dRt * upg;
        grad_a[j] = dAt * upp;
        grad_b[j] = dng * dBc;
        grad_k[j] = dng * dKc;
        const float rt_v = rr[j] * upg, at_v = ra[j] * upp;
        const float bh_v = rb[j] * dng, kh_v = rk[j] * dng;
        e2v[kb][j] = dAt * at_v;
        // Decay gradient pieces: suffix sum of e1 + e2 over the block's
        // tokens and the block total of e3 (lane n = 0 holds the totals).
        suf[kb][j] = suffix16(dRt * rt_v - dBc * bh_v - dKc * kh_v + e2v[kb][j]);
        const float tot3 = suffix16(gam * (acc_bt[j] * bh_v + acc_kt[j] * kh_v));
        if (n == 0) {
          sm.carry[pb][kf] = suf[kb][j];
          sm.carry3[pb][kf] = tot3;
        }
        dec_in[kb][j] = xin;
      }
      {
        auto st4 = [&](void* dst, const float (&x)[4]) {
          u32x2 q;
          q.x = pack2<T>(x[0], x[1]);
          q.y = pack2<T>(x[2], x[3]);
          __builtin_amdgcn_raw_buffer_store_b64(q, rs(dst), tok_off, so, 0);
        };
        st4(p.dr, grad_r);
        st4(p.da, grad_a);
        st4(p.db, grad_b);
        st4(p.dk, grad_k);
      }
    }

    // Decay gradient: combine the blocks' suffix sums and e3 totals.
    __syncthreads();
    {
      const int t = 16 * pb + n;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        float dwv[4];
        // Block carries of the lane's 4 consecutive features, 16-byte reads.
        const int kf0 = 16 * kb + 4 * g;
        float4 later4 = make_float4(0.f, 0.f, 0.f, 0.f), all3_4 = later4, dgam4 = later4;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float4 c1 = *reinterpret_cast<const float4*>(&sm.carry[q][kf0]);
          const float4 c3 = *reinterpret_cast<const float4*>(&sm.carry3[q][kf0]);
          const float4 dg = *reinterpret_cast<const float4*>(&sm.dgamma[q][kf0]);
          if (q > pb) {
            later4.x += c1.x; later4.y += c1.y; later4.z += c1.z; later4.w += c1.w;
          }
          all3_4.x += c3.x; all3_4.y += c3.y; all3_4.z += c3.z; all3_4.w += c3.w;
          dgam4.x += dg.x; dgam4.y += dg.y; dgam4.z += dg.z; dgam4.w += dg.w;
        }
        const float4 gc4 = *reinterpret_cast<const float4*>(&sm.gc[kf0]);
        const float later_v[4] = {later4.x, later4.y, later4.z, later4.w};
        const float all3_v[4] = {all3_4.x, all3_4.y, all3_4.z, all3_4.w};
        const float dgam_v[4] = {dgam4.x, dgam4.y, dgam4.z, dgam4.w};
        const float gc_v[4] = {gc4.x, gc4.y, gc4.z, gc4.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float dlg =
              suf[kb][j] + later_v[j] - e2v[kb][j] + all3_v[j] + dgam_v[j] * gc_v[j];
          const float xin = dec_in[kb][j];
          float d;
          if constexpr (M == DecayMode::kLogits) {
            const float sig = __builtin_amdgcn_rcpf(1.0f + fast_exp2(-kLog2E * xin));
            d = dlg * (-kExpNegHalf) * sig * (1.0f - sig);
          } else {
            // log2 w is clamped to [-20, 0]: zero derivative outside, i.e.
            // for w outside [2^-20, 1].
            d = (xin < 0x1p-20f || xin > 1.0f) ? 0.0f : dlg * __builtin_amdgcn_rcpf(xin);
          }
          dwv[j] = d;
        }
        {
          u32x2 q;
          q.x = pack2<T>(dwv[0], dwv[1]);
          q.y = pack2<T>(dwv[2], dwv[3]);
          __builtin_amdgcn_raw_buffer_store_b64(q, rs(p.ddecay), tok_off,
                                                static_cast<int>(2 * 16 * kb), 0);
        }
      }
    }
  }

  // Gradient of the initial state.
  if (p.dstate0 != nullptr) {
    const auto rs0 = buffer_rsrc(p.dstate0 + unit_state, kHead * kHead * 4);
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float x = failed ? kNaN : dS[kb][j];
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x), rs0, s_off,
                                              (16 * kb + j) * kHead * 4, 0);
      }
    }
  }
}

template <typename T, DecayMode M>
int launch_bwd(const ChunkBwdParams& p, int units, hipStream_t stream) {
  hipLaunchKernelGGL((chunk_bwd_kernel<T, M>), dim3(units), dim3(kChunkThreads), 0, stream, p);
  return check_launch("chunk_bwd_kernel");
}

template <typename T>
int dispatch_bwd_decay(const ChunkBwdParams& p, int decay_mode, int units, hipStream_t s) {
  if (decay_mode == FRWKV_DECAY_LOGITS) return launch_bwd<T, DecayMode::kLogits>(p, units, s);
  if (decay_mode == FRWKV_DECAY_RAW_W) {
    if (p.bias != nullptr) {
      return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                       "decay_bias is only defined for the logits decay mode");
    }
    return launch_bwd<T, DecayMode::kRawW>(p, units, s);
  }
  return set_error(FRWKV_ERR_INVALID_ARGUMENT, "unknown decay mode %d", decay_mode);
}

}  // namespace
}  // namespace frwkv

extern "C" int frwkv_statetune_backward(
    int io_dtype, int decay_mode, int32_t num_sequences, int32_t num_heads, int32_t head_size,
    int32_t total_tokens, int32_t num_chunks, const int32_t* sequence_chunk_offsets,
    const int32_t* chunk_token_starts, const int32_t* chunk_token_ends, const float* boundary,
    const void* r, const void* decay, const void* decay_bias, const void* k, const void* v,
    const void* a, const void* b, const void* grad_output, const float* grad_final_state,
    void* grad_r, void* grad_decay, void* grad_k, void* grad_v, void* grad_a, void* grad_b,
    float* grad_initial_state, float scale, void* stream) {
  using namespace frwkv;
  if (!sequence_chunk_offsets || !chunk_token_starts || !chunk_token_ends || !boundary || !r ||
      !decay || !k || !v || !a || !b || !grad_r || !grad_decay || !grad_k || !grad_v ||
      !grad_a || !grad_b || !grad_initial_state) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_statetune_backward: null pointer argument");
  }
  if (num_sequences <= 0 || num_heads <= 0 || total_tokens <= 0 || num_chunks <= 0) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_statetune_backward: sizes must be positive");
  }
  if (!__builtin_isfinite(scale)) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT, "scale must be finite");
  }
  if (head_size == 128 || head_size == 256) {
    return frwkv_train_recurrent_backward(
        io_dtype, decay_mode, num_sequences, num_heads, head_size, total_tokens,
        sequence_chunk_offsets, chunk_token_starts, chunk_token_ends, num_chunks, /*dense_t=*/0,
        boundary,
        r, decay, decay_bias, k, v, a, b, grad_output, grad_final_state, grad_r, grad_decay,
        grad_k, grad_v, grad_a, grad_b, grad_initial_state, scale, stream);
  }
  if (head_size != 64) {
    return set_error(FRWKV_ERR_UNSUPPORTED, "head size must be 64, 128, or 256, got %d",
                     head_size);
  }
  ChunkBwdParams p{};
  p.num_heads = num_heads;
  p.total_tokens = total_tokens;
  p.num_segments = num_chunks;
  p.seg_offsets = sequence_chunk_offsets;
  p.seg_starts = chunk_token_starts;
  p.seg_ends = chunk_token_ends;
  p.checkpoint = boundary;
  p.r = r;
  p.decay = decay;
  p.bias = decay_bias;
  p.k = k;
  p.v = v;
  p.a = a;
  p.b = b;
  p.dy = grad_output;
  p.dstate_final = grad_final_state;
  p.dr = grad_r;
  p.ddecay = grad_decay;
  p.dk = grad_k;
  p.dv = grad_v;
  p.da = grad_a;
  p.db = grad_b;
  p.dstate0 = grad_initial_state;
  p.scale = scale;
  const int units = num_sequences * num_heads;
  auto s = static_cast<hipStream_t>(stream);
  switch (io_dtype) {
    case FRWKV_DTYPE_BF16:
      return dispatch_bwd_decay<Bf16>(p, decay_mode, units, s);
    case FRWKV_DTYPE_F16:
      return dispatch_bwd_decay<F16>(p, decay_mode, units, s);
    default:
      return set_error(FRWKV_ERR_UNSUPPORTED,
                       "chunked kernels take float16 or bfloat16 tokens (io dtype %d)", io_dtype);
  }
}

extern "C" int frwkv_pretrain_backward(int io_dtype, int decay_mode, int32_t batch,
                                       int32_t tokens, int32_t num_heads, int32_t head_size,
                                       const void* r, const void* decay, const void* k,
                                       const void* v, const void* a, const void* b,
                                       const void* grad_output, const float* boundary,
                                       void* grad_r, void* grad_decay, void* grad_k,
                                       void* grad_v, void* grad_a, void* grad_b, void* stream) {
  using namespace frwkv;
  if (!boundary || !r || !decay || !k || !v || !a || !b || !grad_output || !grad_r ||
      !grad_decay || !grad_k || !grad_v || !grad_a || !grad_b) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_pretrain_backward: null pointer argument");
  }
  if (batch <= 0 || tokens <= 0 || num_heads <= 0 || tokens % 16 != 0) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_pretrain_backward: B, H > 0 and T a positive multiple of 16 "
                     "(B=%d, T=%d, H=%d)", batch, tokens, num_heads);
  }
  if (static_cast<int64_t>(batch) * tokens > INT32_MAX) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT, "frwkv_pretrain_backward: B * T too large");
  }
  if (head_size == 128 || head_size == 256) {
    return frwkv_train_recurrent_backward(
        io_dtype, decay_mode, batch, num_heads, head_size, batch * tokens, nullptr, nullptr,
        nullptr, 0, tokens, boundary, r, decay, /*decay_bias=*/nullptr, k, v, a, b, grad_output,
        /*grad_final_state=*/nullptr, grad_r, grad_decay, grad_k, grad_v, grad_a, grad_b,
        /*grad_initial_state=*/nullptr, 1.0f, stream);
  }
  if (head_size != 64) {
    return set_error(FRWKV_ERR_UNSUPPORTED, "head size must be 64, 128, or 256, got %d",
                     head_size);
  }
  ChunkBwdParams p{};
  p.num_heads = num_heads;
  p.total_tokens = batch * tokens;
  p.dense_t = tokens;
  p.ckpt16 = 1;
  p.checkpoint = boundary;
  p.r = r;
  p.decay = decay;
  p.k = k;
  p.v = v;
  p.a = a;
  p.b = b;
  p.dy = grad_output;
  p.dr = grad_r;
  p.ddecay = grad_decay;
  p.dk = grad_k;
  p.dv = grad_v;
  p.da = grad_a;
  p.db = grad_b;
  p.scale = 1.0f;
  const int units = batch * num_heads;
  auto s = static_cast<hipStream_t>(stream);
  switch (io_dtype) {
    case FRWKV_DTYPE_BF16:
      return dispatch_bwd_decay<Bf16>(p, decay_mode, units, s);
    case FRWKV_DTYPE_F16:
      return dispatch_bwd_decay<F16>(p, decay_mode, units, s);
    default:
      return set_error(FRWKV_ERR_UNSUPPORTED,
                       "chunked kernels take float16 or bfloat16 tokens (io dtype %d)", io_dtype);
  }
}
