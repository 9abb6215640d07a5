// Training forward and backward for head size 128 on bf16 MFMA, over
// 16-token pieces.
//
// Replaces the reference's StateTune / pretraining kernels at head size 128
// (csrc/sm90/tmix/wkv7/statetune_recurrent_fp32io16_{forward,backward}.cu,
// backward :317-502; pretrain_recurrent_bf16_{forward,backward}.cu). The
// reference's backward rebuilds S_{t-1} by dividing by the decay token by
// token. Here, as in chunk_bwd.hip, every piece is recomputed from a stored
// state: the forward stores the state at every chunk start (fp32) and at
// every further 16-token piece start (the interior slots, bf16), and the backward walks
// each sequence's pieces in reverse, carrying the state adjoint dS (dL/dS at
// the current piece end) in registers.
//
// A 16-token piece is one 16 x 16 block of the chunk algebra of chunk_fwd.hip
// (tokens t, i in 0..15, keys k and values v in 0..127, G the cumulative log2
// retention from the piece start, Gp = G - log2 w, g = 2^G at the last token):
//   At = a 2^Gp, Rt = r 2^G, Bh = b 2^-G, Kh = k 2^-G;
//   Lab = strict(At Bh^T), Lak = strict(At Kh^T), Arb = lower(Rt Bh^T),
//   Ark = lower(Rt Kh^T), T = (I - Lab)^{-1}, SA = T (At S0 + Lak V);
//   Y = scale (Rt S0 + Arb SA + Ark V), S' = diag(g) (S0 + Bh^T SA + Kh^T V).
// Its adjoint, with dYs = scale dY and dU = g o dS:
//   dSA = Arb^T dYs + Bh dU                    dZ = T^T dSA
//   dV  = Ark^T dYs + Lak^T dZ + Kh dU
//   dS0 = dU + Rt^T dYs + At^T dZ              (the adjoint of the piece before)
//   dArb = lower(dYs SA^T)   dArk = lower(dYs V^T)
//   dLab = strict(dZ SA^T)   dLak = strict(dZ V^T)
//   dRt = dYs S0^T + dArb Bh + dArk Kh         dAt = dZ S0^T + dLab Bh + dLak Kh
//   dBh = dLab^T At + dArb^T Rt                dKh = dLak^T At + dArk^T Rt
//   dBt = SA dS^T    dKt = V dS^T              dg = rowsum(S0 o dS)
// and elementwise dr = dRt 2^G, da = dAt 2^Gp, db = 2^-G (dBh + g dBt),
// dk = 2^-G (dKh + g dKt). With e1 = dr r - db b - dk k, e2 = da a and
// e3 = g 2^-G (dBt b + dKt k), the gradient of the log2 retention of token j
// is dlg_j = sum_{t>=j} (e1_t + e2_t) - e2_j + sum_t e3_t + g dg; the decay
// input's gradient is dlg / w for raw retention (clamped to [2^-20, 1], zero
// outside) and dlg (-e^{-1/2}) sigmoid(x) (1 - sigmoid(x)) for logits. The
// products with r, a, b, k use the bf16 tile values the MFMA products used,
// so their cancellations match.
//
// Work decomposition: one 512-thread workgroup (8 waves, lane (g, n) with
// g = lane / 16, n = lane % 16) per (sequence, head), its fp32 state slab in
// MFMA accumulators (wave w: value columns 16w .. 16w+15, all 128 keys). Per
// piece, phases separated by barriers:
//   stage    thread (wave w, lane (g, n)) decodes token n, features
//            16w + 4g .. +3: the retention, a product scan over the 16
//            tokens of its DPP row, the scaled tiles At, Rt, Bh, Kh, V (and
//            dYs in the backward; [t][k], bf16); it keeps the decay factors
//            in registers for the tokens phase, whose lane layout is the same;
//   intra    waves 0-3: Lab, Lak, Arb, Ark ([t][i] blocks), wave 0 also T;
//   forward  (forward kernel) every wave, its columns: SA, y, state_dot_a and
//            the state update;
//   columns  (backward) wave w, its columns: S0 and dS tiles ([v][k]), SA,
//            dSA, dZ (tiles SA and dZ, [t][v]), dV (stored), dS0;
//   matrices (backward) waves 0-3: dArb, dArk, dLab, dLak; every wave
//            meanwhile forms the products over values of the tokens phase;
//   tokens   (backward) wave w, keys 16w .. 16w+15, lane (g, n) = keys
//            16w + 4g + j of token n: dRt, dAt, dBh, dKh, dBt, dKt and dg
//            (transposed products), the chain rules, the decay gradient's
//            suffix sums over the row's 16 tokens, and 8-byte gradient stores.
// The next piece's rows are loaded while a piece computes: into registers in
// the forward, into an LDS staging area (direct buffer-to-LDS loads) in the
// backward, whose registers are full.
// Strong decay: the factorisation needs the piece's decay span (-log2 of its
// retention product) within 80; a piece above it runs as 4-token sub-pieces
// (a 4-token span is at most 80 under the [2^-20, 1] clamp), sub-piece s
// starting from the state recomputed by forward passes over sub-pieces
// 0 .. s-1 from the piece start.
#include "capi_internal.h"
#include "chunk_common.h"
#include "train_common.h"

namespace frwkv {
namespace {

constexpr int kPD = 128;            // head size
constexpr int kPS = kPD + 8;        // LDS row stride (bf16 elements) of the 128-wide tiles
constexpr int kPThreads = 512;
constexpr int kPWaves = 8;

struct PieceSmem {
  uint16_t at[kPiece * kPS], rt[kPiece * kPS], bh[kPiece * kPS], kh[kPiece * kPS];  // [t][k]
  uint16_t vt[kPiece * kPS], dy[kPiece * kPS], sa[kPiece * kPS], dz[kPiece * kPS];  // [t][v]
  uint16_t s0[kPD * kPS], ds[kPD * kPS];                                            // [v][k]
  uint16_t tri[5][kTriBlock];   // Lab, Lak, Arb, Ark, T: [t][i]
  uint16_t grad[4][kTriBlock];  // dArb, dArk, dLab, dLak: [t][i]
  float gc[kPD];                // 2^G at the piece's last token, per key
  float dg[kPD];                // rowsum(S0 o dS), per key
  int span_ok[kPWaves];
};
static_assert(sizeof(PieceSmem) <= 160 * 1024, "one workgroup per CU");

enum PieceTri { kTLab = 0, kTLak = 1, kTArb = 2, kTArk = 3, kTT = 4 };
enum PieceGrad { kGArb = 0, kGArk = 1, kGLab = 2, kGLak = 3 };

// 4 io-dtype values of an 8-byte row piece, as fp32.
template <typename T>
__device__ __forceinline__ void unpack4(uint2 q, float (&x)[4]) {
  using S = typename IoTraits<T>::storage;
  x[0] = to_f32<T>(static_cast<S>(q.x & 0xffffu));
  x[1] = to_f32<T>(static_cast<S>(q.x >> 16));
  x[2] = to_f32<T>(static_cast<S>(q.y & 0xffffu));
  x[3] = to_f32<T>(static_cast<S>(q.y >> 16));
}

__device__ __forceinline__ uint2 bf16x4(float x0, float x1, float x2, float x3) {
  return make_uint2(pack_bf16x2(x0, x1), pack_bf16x2(x2, x3));
}

// Inclusive product scan over the 16 lanes of a DPP row (lane n = token n).
template <int N>
__device__ __forceinline__ float scan16_mul_step(float x, int n) {
  const float y = __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x110 + N, 0xf, 0xf, true));
  return n >= N ? x * y : x;
}
__device__ __forceinline__ float scan16_mul(float x, int n) {
  x = scan16_mul_step<1>(x, n);
  x = scan16_mul_step<2>(x, n);
  x = scan16_mul_step<4>(x, n);
  return scan16_mul_step<8>(x, n);
}
// Lane n - 1's value (row_shr:1), 1 for the row's first lane.
__device__ __forceinline__ float shift16_one(float x, int n) {
  const float y = __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x111, 0xf, 0xf, true));
  return n >= 1 ? y : 1.0f;
}
// Suffix sum over the row: lane n gets sum_{m >= n} x_m (row_shl shifts
// read zero past the row end).
template <int N>
__device__ __forceinline__ float suffix16_step(float x) {
  return x + __int_as_float(
                 __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x100 + N, 0xf, 0xf, true));
}
__device__ __forceinline__ float suffix16_sum(float x) {
  x = suffix16_step<1>(x);
  x = suffix16_step<2>(x);
  x = suffix16_step<4>(x);
  return suffix16_step<8>(x);
}
// Sum over the row, in every lane (row_ror rotations).
template <int N>
__device__ __forceinline__ float rowsum16_step(float x) {
  return x + __int_as_float(
                 __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x120 + N, 0xf, 0xf, false));
}
__device__ __forceinline__ float rowsum16(float x) {
  x = rowsum16_step<8>(x);
  x = rowsum16_step<4>(x);
  x = rowsum16_step<2>(x);
  return rowsum16_step<1>(x);
}

// The thread's share of a piece, kept from the stage to the tokens phase:
// the decay factors 2^G, 2^Gp, 2^-G of token n, features 16w + 4g .. +3, and
// the derivative of the decay input's gradient with respect to dlg.
struct PieceRows {
  float fg[4], fgp[4], fgn[4], dwf[4];
  bool on;     // token n is inside the pass's range
  int lo, hi;  // the pass's range (wave-uniform)
};

// The rows of token n, features 16w + 4g .. +3, of the piece at token t0
// with ntok tokens (zeros past ntok; dy only for the backward).
struct PieceLoad {
  uint2 r, k, a, b, x, v, y;
};

template <typename T, bool kGrad>
__device__ __forceinline__ void piece_load(PieceLoad& L, const TrainParams& p, int head,
                                           int32_t t0, int ntok) {
  using S = typename IoTraits<T>::storage;
  const int tid = lane_tid();
  const int w = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, n = lane & 15;
  const uint32_t row_bytes = static_cast<uint32_t>(p.num_heads) * kPD * 2;
  const int64_t base = (static_cast<int64_t>(t0) * p.num_heads + head) * kPD;
  const uint32_t range = static_cast<uint32_t>(ntok) * row_bytes;
  const uint32_t off = static_cast<uint32_t>(n) * row_bytes + 2 * (16 * w + 4 * g);
  auto load = [&](const void* src) {
    const auto rs = buffer_rsrc(src != nullptr ? static_cast<const S*>(src) + base : nullptr,
                                src != nullptr ? range : 0u);
    const u32x2 q = __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 0);
    return make_uint2(q.x, q.y);
  };
  L.r = load(p.r);
  L.k = load(p.k);
  L.a = load(p.a);
  L.b = load(p.b);
  L.x = load(p.decay);
  L.v = load(p.v);
  L.y = kGrad ? load(p.dy) : make_uint2(0u, 0u);
}

// One (sub-)piece pass over tokens [lo, hi) of the loaded piece: masks the
// tokens outside [lo, hi) (retention 1, zero operands), writes the scaled
// tiles, 2^g and the wave's span verdict. Ends with a barrier.
template <typename T, DecayMode M, bool kGrad>
__device__ __forceinline__ void piece_stage(PieceSmem& sm, PieceRows& rows, const PieceLoad& L,
                                            const TrainParams& p, const float (&bias)[4], int lo,
                                            int hi) {
  const int tid = lane_tid();
  const int w = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, n = lane & 15;
  const int f0 = 16 * w + 4 * g;
  const uint2 rq = L.r, kq = L.k, aq = L.a, bq = L.b, xq = L.x, vq = L.v, yq = L.y;
  rows.on = n >= lo && n < hi;
  rows.lo = lo;
  rows.hi = hi;

  float x[4];
  unpack4<T>(xq, x);
  float mn = 1.0f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float xb = x[e] + bias[e];
    const float ret = clamped_retention<M>(xb);
    const float wv = rows.on ? ret : 1.0f;
    const float incl = scan16_mul(wv, n);
    rows.fg[e] = incl;
    rows.fgp[e] = shift16_one(incl, n);
    rows.fgn[e] = __builtin_amdgcn_rcpf(incl);
    mn = fminf(mn, incl);
    if constexpr (kGrad) {
      float dwf;
      if constexpr (M == DecayMode::kLogits) {
        const float sig = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-kLog2E * xb));
        dwf = -kExpNegHalf * sig * (1.0f - sig);
      } else {
        dwf = (xb >= 0x1p-20f && xb <= 1.0f) ? __builtin_amdgcn_rcpf(xb) : 0.0f;
      }
      rows.dwf[e] = rows.on ? dwf : 0.0f;
    }
  }
  float a4[4], r4[4], b4[4], k4[4], v4[4], y4[4];
  unpack4<T>(aq, a4);
  unpack4<T>(rq, r4);
  unpack4<T>(bq, b4);
  unpack4<T>(kq, k4);
  unpack4<T>(vq, v4);
  unpack4<T>(yq, y4);
  const float on = rows.on ? 1.0f : 0.0f;
  const int o = n * kPS + f0;
  auto put = [&](uint16_t* tile, float x0, float x1, float x2, float x3) {
    *reinterpret_cast<uint2*>(tile + o) = bf16x4(x0, x1, x2, x3);
  };
  put(sm.at, on * a4[0] * rows.fgp[0], on * a4[1] * rows.fgp[1], on * a4[2] * rows.fgp[2],
      on * a4[3] * rows.fgp[3]);
  put(sm.rt, on * r4[0] * rows.fg[0], on * r4[1] * rows.fg[1], on * r4[2] * rows.fg[2],
      on * r4[3] * rows.fg[3]);
  put(sm.bh, on * b4[0] * rows.fgn[0], on * b4[1] * rows.fgn[1], on * b4[2] * rows.fgn[2],
      on * b4[3] * rows.fgn[3]);
  put(sm.kh, on * k4[0] * rows.fgn[0], on * k4[1] * rows.fgn[1], on * k4[2] * rows.fgn[2],
      on * k4[3] * rows.fgn[3]);
  put(sm.vt, on * v4[0], on * v4[1], on * v4[2], on * v4[3]);
  if constexpr (kGrad) {
    const float ys = on * p.scale;
    put(sm.dy, ys * y4[0], ys * y4[1], ys * y4[2], ys * y4[3]);
  }
  if (n == 15) {
    *reinterpret_cast<float4*>(&sm.gc[f0]) =
        make_float4(rows.fg[0], rows.fg[1], rows.fg[2], rows.fg[3]);
  }
  // The product at the last token is each feature's smallest.
  const bool ok = __builtin_amdgcn_ballot_w64(!(mn >= kSpanFloor)) == 0;
  if (lane == 0) sm.span_ok[w] = ok ? 1 : 0;
  __syncthreads();
}

// Load and stage in one (the backward's prepare).
template <typename T, DecayMode M>
__device__ __forceinline__ void piece_prepare(PieceSmem& sm, PieceRows& rows,
                                              const TrainParams& p, const float (&bias)[4],
                                              int head, int32_t t0, int ntok, int lo, int hi) {
  PieceLoad L;
  piece_load<T, true>(L, p, head, t0, ntok);
  piece_stage<T, M, true>(sm, rows, L, p, bias, lo, hi);
}

// The rows of the backward's next piece, loaded straight into LDS (buffer ->
// LDS loads, 16 bytes per lane) while the current piece computes: r, k, a, b,
// decay, v and dy, 16 tokens x 256 bytes each. A 1 KiB block holds 4 tokens;
// token n's 16-byte chunk c (features 8c .. 8c + 7) sits at position
// (n % 4) * 16 + ((c + n) & 15) of its block, so that the stage's 8-byte reads
// (16 tokens x 2 chunks per wave) fall on distinct bank pairs. Tokens past
// the piece read as zeros (out of the buffer range).
constexpr int kStageTensors = 7;
struct RowStage {
  uint16_t x[kStageTensors][kPiece * kPD];
};

template <typename T>
__device__ __forceinline__ void piece_rows_to_lds(RowStage& st, const TrainParams& p, int head,
                                                  int32_t t0, int ntok) {
  using S = typename IoTraits<T>::storage;
  const int tid = lane_tid();
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const uint32_t row_bytes = static_cast<uint32_t>(p.num_heads) * kPD * 2;
  const int64_t base = (static_cast<int64_t>(t0) * p.num_heads + head) * kPD;
  const uint32_t range = static_cast<uint32_t>(ntok) * row_bytes;
  // 28 wave loads of 1 KiB (tensor ti, block b): waves 0-3 take four, 4-7 three.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int slot = w + 8 * i;
    if (slot < kStageTensors * 4) {
      const int ti = slot >> 2, b = slot & 3;
      const void* src = ti == 0   ? p.r
                        : ti == 1 ? p.k
                        : ti == 2 ? p.a
                        : ti == 3 ? p.b
                        : ti == 4 ? p.decay
                        : ti == 5 ? p.v
                                  : p.dy;
      const uint64_t addr =
          src != nullptr ? reinterpret_cast<uint64_t>(static_cast<const S*>(src) + base) : 0;
      const u32x4 rs = {static_cast<uint32_t>(addr), static_cast<uint32_t>(addr >> 32),
                        src != nullptr ? range : 0u, 0x00020000u};
      const uint32_t lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
          (__attribute__((address_space(3))) void*)&st.x[ti][4 * b * kPD]));
      const int n = 4 * b + (lane >> 4);
      const int c = ((lane & 15) - n) & 15;
      const uint32_t off = static_cast<uint32_t>(n) * row_bytes + 16 * c;
      // Written as assembly so that the compiler does not order every later
      // LDS access after these loads: the staging area is only read after
      // the column phase's explicit vmcnt(0) wait and the barriers after it.
      // M0 holds the load's LDS base; the block saves and restores it, so a
      // value the compiler keeps in M0 survives.
      uint32_t m0_saved;
      asm volatile(
          "s_mov_b32 %0, m0\n\t"
          "s_mov_b32 m0, %3\n\t"
          "buffer_load_dwordx4 %1, %2, 0 offen lds\n\t"
          "s_mov_b32 m0, %0"
          : "=&s"(m0_saved)
          : "v"(off), "s"(rs), "s"(lds)
          : "memory");
    }
  }
}

// The thread's rows (token n, features 16w + 4g .. +3) from the staged piece.
__device__ __forceinline__ void piece_load_staged(PieceLoad& L, const RowStage& st) {
  const int tid = lane_tid();
  const int w = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, n = lane & 15;
  const int c = 2 * w + (g >> 1);
  const int off = (n >> 2) * 4 * kPD + 8 * ((n & 3) * 16 + ((c + n) & 15)) + 4 * (g & 1);
  auto rd = [&](int ti) { return *reinterpret_cast<const uint2*>(&st.x[ti][off]); };
  L.r = rd(0);
  L.k = rd(1);
  L.a = rd(2);
  L.b = rd(3);
  L.x = rd(4);
  L.v = rd(5);
  L.y = rd(6);
}

// Lab, Lak, Arb, Ark (waves 0-3) and T = (I - Lab)^{-1} (wave 0). Ends with a
// barrier.
__device__ __forceinline__ void piece_intra(PieceSmem& sm) {
  const int tid = lane_tid();
  const int w = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, n = lane & 15;
  if (w < 4) {
    __builtin_amdgcn_s_setprio(1);
    const uint16_t* X = w < 2 ? sm.at : sm.rt;          // token side t
    const uint16_t* Y = (w & 1) == 0 ? sm.bh : sm.kh;   // token side i
    f32x4 acc = zero4();
#pragma unroll
    for (int c = 0; c < kPD; c += 32) {
      acc = mfma32(lds_operand32<kPS>(Y, n, c, g), lds_operand32<kPS>(X, n, c, g), acc);
    }
    // lane (g, n): M[t = n][i = 4g + j]; Lab and Lak strictly lower.
    const bool strict = w < 2;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = 4 * g + j;
      acc[j] = (strict ? i < n : i <= n) ? acc[j] : 0.0f;
    }
    lds_store_transposed(sm.tri[w], kTriStride, g, n, acc);
    if (w == 0) {
      // The Neumann product of chunk_fwd.hip's diagonal blocks:
      // (I - L)^{-1} = (I + L)(I + L^2)(I + L^4)(I + L^8). l_r: lane (g, n)
      // holds L[n][4g + j]; lc, the B operand of L, is a transpose read of
      // the block just stored (same wave, in order).
      const f32x4 l_r = acc;
      const i16x4 lr = to_operand(l_r);
      const i16x4 lc = lds_operand_tr<kTriStride>(sm.tri[kTLab], 0, 0, g, n);
      const i16x4 p2c = to_operand(mfma16(lr, lc, zero4()));
      const i16x4 p2r = to_operand(mfma16(lc, lr, zero4()));
      const i16x4 p4c = to_operand(mfma16(p2r, p2c, zero4()));
      const i16x4 p4r = to_operand(mfma16(p2c, p2r, zero4()));
      const i16x4 p8c = to_operand(mfma16(p4r, p4c, zero4()));
      f32x4 t = l_r;
#pragma unroll
      for (int j = 0; j < 4; ++j) t[j] += (4 * g + j == n) ? 1.0f : 0.0f;
      t = mfma16(p2c, to_operand(t), t);
      t = mfma16(p4c, to_operand(t), t);
      t = mfma16(p8c, to_operand(t), t);
      lds_store_transposed(sm.tri[kTT], kTriStride, g, n, t);
    }
    __builtin_amdgcn_s_setprio(0);
  }
  __syncthreads();
}

// State slab of wave w: value columns 16w .. 16w+15, key rows in C layout,
// S[kb][j] = S[16kb + 4g + j][16w + n].
struct Slab {
  f32x4 x[kPD / 16];
};

__device__ __forceinline__ void load_slab16(Slab& s, const float* base) {
  const int tid = lane_tid();
  const int w = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, n = lane & 15;
  const auto rs = buffer_rsrc(base, kPD * kPD * 4);
  const uint32_t off = static_cast<uint32_t>((4 * g) * kPD + 16 * w + n) * 4;
#pragma unroll
  for (int kb = 0; kb < kPD / 16; ++kb) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      s.x[kb][j] = __uint_as_float(
          __builtin_amdgcn_raw_buffer_load_b32(rs, off, (16 * kb + j) * kPD * 4, 0));
    }
  }
}

__device__ __forceinline__ void store_slab16(float* base, const Slab& s) {
  const int tid = lane_tid();
  const int w = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, n = lane & 15;
  const auto rs = buffer_rsrc(base, kPD * kPD * 4);
  const uint32_t off = static_cast<uint32_t>((4 * g) * kPD + 16 * w + n) * 4;
#pragma unroll
  for (int kb = 0; kb < kPD / 16; ++kb) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(s.x[kb][j]), rs, off,
                                            (16 * kb + j) * kPD * 4, 0);
    }
  }
}

// Interior piece-start states (slot = piece start / 16) are kept in bf16 in
// the slab's lane order: thread i = 64w + lane holds S[kb][j] for kb < 8,
// j < 4; kb pair (2q, 2q + 1) goes to the 16 bytes at (q * 512 + i) * 16 of
// the (slot, head) block as the bf16 pairs (j0 j1)(j2 j3) of 2q, then of
// 2q + 1. Every wave store and load is one contiguous KiB. The backward uses
// a piece's start state only as bf16 MFMA operands (rounded to nearest even,
// as here), so the rounding changes none of its results; a strong-decay
// piece, whose sub-piece states are recomputed in fp32, starts from the
// rounded state.
constexpr int64_t kInteriorBlock = static_cast<int64_t>(kPD) * kPD;  // bf16 per (slot, head)

__device__ __forceinline__ uint16_t* interior_block(const TrainParams& p, int head, int32_t t0) {
  return reinterpret_cast<uint16_t*>(p.interior) +
         (static_cast<int64_t>(t0 / kPiece) * p.num_heads + head) * kInteriorBlock;
}

__device__ __forceinline__ void store_slab_bf16(uint16_t* base, const Slab& s) {
  const uint32_t off = static_cast<uint32_t>(lane_tid()) * 16;
  const auto rs = buffer_rsrc(base, kPD * kPD * 2);
#pragma unroll
  for (int q = 0; q < kPD / 32; ++q) {
    const f32x4 a = s.x[2 * q], b = s.x[2 * q + 1];
    const u32x4 v = {pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3]), pack_bf16x2(b[0], b[1]),
                     pack_bf16x2(b[2], b[3])};
    __builtin_amdgcn_raw_buffer_store_b128(v, rs, off, q * kPThreads * 16, 0);
  }
}

__device__ __forceinline__ void load_slab_bf16(Slab& s, const uint16_t* base) {
  const uint32_t off = static_cast<uint32_t>(lane_tid()) * 16;
  const auto rs = buffer_rsrc(base, kPD * kPD * 2);
#pragma unroll
  for (int q = 0; q < kPD / 32; ++q) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, off, q * kPThreads * 16, 0);
    s.x[2 * q] = f32x4{__uint_as_float(v[0] << 16), __uint_as_float(v[0] & 0xffff0000u),
                       __uint_as_float(v[1] << 16), __uint_as_float(v[1] & 0xffff0000u)};
    s.x[2 * q + 1] = f32x4{__uint_as_float(v[2] << 16), __uint_as_float(v[2] & 0xffff0000u),
                           __uint_as_float(v[3] << 16), __uint_as_float(v[3] & 0xffff0000u)};
  }
}

__device__ __forceinline__ i16x8 lo32(i16x4 x) {
  const i16x4 z = {0, 0, 0, 0};
  return cat(x, z);
}

// The outputs of a forward pass, held until they are stored: lane (g, n)
// has y[t = n][16w + 4g .. +3] (scaled, packed) and state_dot_a[t][16w + n]
// for the pass's tokens t = 4g + j.
struct PieceOut {
  u32x2 y;
  f32x4 sa;
  int32_t t0;
  int ntok, lo, hi;
  bool on;  // token n is inside [lo, hi)
};

// Stores the held outputs; tokens outside the pass's range go to
// kDropOffset (dropped), so every lane issues the same stores.
template <typename T>
__device__ __forceinline__ void store_piece_out(const PieceOut& o, const TrainParams& p,
                                                int head) {
  using St = typename IoTraits<T>::storage;
  const int tid = lane_tid();
  const int w = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, n = lane & 15;
  const uint32_t row_bytes = static_cast<uint32_t>(p.num_heads) * kPD * 2;
  const int64_t base = (static_cast<int64_t>(o.t0) * p.num_heads + head) * kPD;
  const auto out_rs =
      buffer_rsrc(static_cast<St*>(p.out) + base, static_cast<uint32_t>(o.ntok) * row_bytes);
  __builtin_amdgcn_raw_buffer_store_b64(
      o.y, out_rs, o.on ? static_cast<uint32_t>(n) * row_bytes + 2 * (16 * w + 4 * g) : kDropOffset,
      0, 0);
  const auto sda_rs =
      buffer_rsrc(p.state_dot_a + base, static_cast<uint32_t>(o.ntok) * row_bytes * 2);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int t = 4 * g + j;
    const bool on = t >= o.lo && t < o.hi;
    __builtin_amdgcn_raw_buffer_store_b32(
        __float_as_uint(o.sa[j]), sda_rs,
        on ? static_cast<uint32_t>(t) * row_bytes * 2 + 4 * (16 * w + n) : kDropOffset, 0, 0);
  }
}

// A forward pass of the prepared (sub-)piece on the wave's slab:
// S <- diag(g) (S + Bh^T SA + Kh^T V). kOut: also the outputs of its tokens,
// y = scale (Rt S0 + Arb SA + Ark V) and state_dot_a = SA for the wave's
// value columns, into `out` (p.out set). Ends with a barrier.
template <typename T, bool kOut>
__device__ __forceinline__ void piece_forward_state(PieceSmem& sm, Slab& S,
                                                    const PieceRows& rows,
                                                    const TrainParams& p, int32_t t0, int ntok,
                                                    PieceOut& out) {
  using St = typename IoTraits<T>::storage;
  const int tid = lane_tid();
  const int w = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, n = lane & 15;
  __builtin_amdgcn_s_setprio(1);
  i16x4 s_op[kPD / 16];
#pragma unroll
  for (int kb = 0; kb < kPD / 16; ++kb) s_op[kb] = to_operand(S.x[kb]);
  const i16x4 v_op = lds_operand_tr<kPS>(sm.vt, 0, 16 * w, g, n);
  f32x4 rhs = zero4();
#pragma unroll
  for (int c = 0; c < kPD / 32; ++c) {
    rhs = mfma32(lds_operand32<kPS>(sm.at, n, 32 * c, g), cat(s_op[2 * c], s_op[2 * c + 1]), rhs);
  }
  rhs = mfma32(lo32(lds_operand<kTriStride>(sm.tri[kTLak], n, 4 * g)), lo32(v_op), rhs);
  const f32x4 sa =
      mfma32(lo32(lds_operand<kTriStride>(sm.tri[kTT], n, 4 * g)), lo32(to_operand(rhs)), zero4());
  const i16x4 sa_op = to_operand(sa);
  if (kOut && p.out != nullptr) {
    // Y^T = S0^T Rt^T + [SA^T | V^T] [Arb^T ; Ark^T]: lane (g, n) holds
    // y[t = n][16w + 4g + j].
    f32x4 yt = zero4();
#pragma unroll
    for (int c = 0; c < kPD / 32; ++c) {
      yt = mfma32(cat(s_op[2 * c], s_op[2 * c + 1]), lds_operand32<kPS>(sm.rt, n, 32 * c, g), yt);
    }
    yt = mfma32(cat(sa_op, v_op), cat(lds_operand<kTriStride>(sm.tri[kTArb], n, 4 * g),
                                      lds_operand<kTriStride>(sm.tri[kTArk], n, 4 * g)),
                yt);
    out.y = u32x2{pack2<T>(p.scale * yt[0], p.scale * yt[1]),
                  pack2<T>(p.scale * yt[2], p.scale * yt[3])};
    out.sa = sa;
    out.t0 = t0;
    out.ntok = ntok;
    out.lo = rows.lo;
    out.hi = rows.hi;
    out.on = rows.on;
  }
  const i16x8 sav = cat(sa_op, v_op);
#pragma unroll
  for (int kb = 0; kb < kPD / 16; ++kb) {
    const i16x8 a = cat(lds_operand_tr<kPS>(sm.bh, 0, 16 * kb, g, n),
                        lds_operand_tr<kPS>(sm.kh, 0, 16 * kb, g, n));
    f32x4 sn = mfma32(a, sav, S.x[kb]);
#pragma unroll
    for (int j = 0; j < 4; ++j) S.x[kb][j] = sn[j] * sm.gc[16 * kb + 4 * g + j];
  }
  __builtin_amdgcn_s_setprio(0);
  __syncthreads();
}

// The backward of the prepared (sub-)piece [lo, hi) of the piece at token t0
// (ntok tokens):
// intra products, the column phase (dV stored; dS <- dS0), the gradient
// matrices and the tokens phase (key gradients stored). S is the pass's start
// state. Ends with a barrier.
template <typename T>
__device__ __forceinline__ void piece_backward(PieceSmem& sm, const PieceRows& rows,
                                               const TrainParams& p, int head, int32_t t0,
                                               int ntok, const Slab& S, Slab& dS) {
  using St = typename IoTraits<T>::storage;
  const int tid = lane_tid();
  const int w = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, n = lane & 15;
  piece_intra(sm);

  const uint32_t row_bytes = static_cast<uint32_t>(p.num_heads) * kPD * 2;
  const int64_t base = (static_cast<int64_t>(t0) * p.num_heads + head) * kPD;
  const uint32_t range = static_cast<uint32_t>(ntok) * row_bytes;
  // Stores of token n, 4 consecutive features from f: masked tokens go to
  // kDropOffset (dropped), so every lane issues the same stores.
  auto store4 = [&](void* dst, int f, float x0, float x1, float x2, float x3) {
    const auto rs = buffer_rsrc(static_cast<St*>(dst) + base, range);
    const u32x2 q = {pack2<T>(x0, x1), pack2<T>(x2, x3)};
    __builtin_amdgcn_raw_buffer_store_b64(
        q, rs, rows.on ? static_cast<uint32_t>(n) * row_bytes + 2 * f : kDropOffset, 0, 0);
  };

  // ---- columns: value columns 16w .. 16w+15 ----
  // Every vector memory load of this wave has landed: the start state read
  // here, and the next piece's rows staged before it (read after the barrier
  // that ends this phase).
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int kb = 0; kb < kPD / 16; ++kb) {
    lds_store_transposed(sm.s0 + 16 * w * kPS + 16 * kb, kPS, g, n, S.x[kb]);
    lds_store_transposed(sm.ds + 16 * w * kPS + 16 * kb, kPS, g, n, dS.x[kb]);
  }
  i16x4 s_op[kPD / 16];
#pragma unroll
  for (int kb = 0; kb < kPD / 16; ++kb) s_op[kb] = to_operand(S.x[kb]);
  const i16x4 v_op = lds_operand_tr<kPS>(sm.vt, 0, 16 * w, g, n);
  const i16x4 dy_op = lds_operand_tr<kPS>(sm.dy, 0, 16 * w, g, n);
  auto tri16 = [&](int m) { return lds_operand<kTriStride>(sm.tri[m], n, 4 * g); };
  auto trit = [&](int m) { return lds_operand_tr<kTriStride>(sm.tri[m], 0, 0, g, n); };

  // rhs = At S0 + Lak V, then SA^T = rhs^T T^T into the SA tile ([t][v]).
  f32x4 rhs = zero4();
#pragma unroll
  for (int c = 0; c < kPD / 32; ++c) {
    rhs = mfma32(lds_operand32<kPS>(sm.at, n, 32 * c, g), cat(s_op[2 * c], s_op[2 * c + 1]), rhs);
  }
  rhs = mfma32(lo32(tri16(kTLak)), lo32(v_op), rhs);
  const f32x4 sat = mfma32(lo32(to_operand(rhs)), lo32(tri16(kTT)), zero4());
  lds_store_transposed(sm.sa + 16 * w, kPS, g, n, sat);

  // dU = g o dS (in place); dSA = Bh dU + Arb^T dYs; dZ = T^T dSA.
#pragma unroll
  for (int kb = 0; kb < kPD / 16; ++kb) {
#pragma unroll
    for (int j = 0; j < 4; ++j) dS.x[kb][j] *= sm.gc[16 * kb + 4 * g + j];
  }
  i16x4 du_op[kPD / 16];
#pragma unroll
  for (int kb = 0; kb < kPD / 16; ++kb) du_op[kb] = to_operand(dS.x[kb]);
  f32x4 dsa = zero4();
#pragma unroll
  for (int c = 0; c < kPD / 32; ++c) {
    dsa = mfma32(lds_operand32<kPS>(sm.bh, n, 32 * c, g), cat(du_op[2 * c], du_op[2 * c + 1]), dsa);
  }
  dsa = mfma32(lo32(trit(kTArb)), lo32(dy_op), dsa);
  const i16x4 dsa_op = to_operand(dsa);
  const f32x4 dz = mfma32(lo32(trit(kTT)), lo32(dsa_op), zero4());
  const f32x4 dzt = mfma32(lo32(dsa_op), lo32(trit(kTT)), zero4());
  lds_store_transposed(sm.dz + 16 * w, kPS, g, n, dzt);
  const i16x4 dz_op = to_operand(dz);
  const i16x8 ydz = cat(dy_op, dz_op);

  // dV^T = dU^T Kh^T + [dYs^T | dZ^T] [Ark ; Lak]: lane (g, n) holds
  // dV[t = n][16w + 4g + j].
  f32x4 dvt = zero4();
#pragma unroll
  for (int c = 0; c < kPD / 32; ++c) {
    dvt = mfma32(cat(du_op[2 * c], du_op[2 * c + 1]), lds_operand32<kPS>(sm.kh, n, 32 * c, g), dvt);
  }
  dvt = mfma32(ydz, cat(trit(kTArk), trit(kTLak)), dvt);
  store4(p.dv, 16 * w + 4 * g, dvt[0], dvt[1], dvt[2], dvt[3]);

  // dS0 = dU + [Rt^T | At^T] [dYs ; dZ], per key block, in place.
#pragma unroll
  for (int kb = 0; kb < kPD / 16; ++kb) {
    const i16x8 a = cat(lds_operand_tr<kPS>(sm.rt, 0, 16 * kb, g, n),
                        lds_operand_tr<kPS>(sm.at, 0, 16 * kb, g, n));
    dS.x[kb] = mfma32(a, ydz, dS.x[kb]);
  }
  __builtin_amdgcn_s_setprio(0);
  __syncthreads();

  // ---- gradient matrices (waves 0-3) ----
  if (w < 4) {
    __builtin_amdgcn_s_setprio(1);
    const uint16_t* X = w < 2 ? sm.dy : sm.dz;          // t side
    const uint16_t* Y = (w & 1) == 0 ? sm.sa : sm.vt;   // i side
    f32x4 acc = zero4();
#pragma unroll
    for (int c = 0; c < kPD; c += 32) {
      acc = mfma32(lds_operand32<kPS>(Y, n, c, g), lds_operand32<kPS>(X, n, c, g), acc);
    }
    const bool strict = w >= 2;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = 4 * g + j;
      acc[j] = (strict ? i < n : i <= n) ? acc[j] : 0.0f;
    }
    lds_store_transposed(sm.grad[w], kTriStride, g, n, acc);
    __builtin_amdgcn_s_setprio(0);
  }

  // ---- tokens: keys 16w .. 16w+15; lane (g, n) = keys 16w + 4g + j, token n ----
  // Products over the values (need no gradient matrix).
  auto tr_vk = [&](const uint16_t* tile, int c) {
    return cat(lds_operand_tr<kPS>(tile, c, 16 * w, g, n),
               lds_operand_tr<kPS>(tile, c + 16, 16 * w, g, n));
  };
  f32x4 drt = zero4(), dat = zero4(), dbt = zero4(), dkt = zero4(), dgk = zero4();
#pragma unroll
  for (int c = 0; c < kPD; c += 32) {
    const i16x8 s0a = tr_vk(sm.s0, c);
    const i16x8 dsa_ = tr_vk(sm.ds, c);
    drt = mfma32(s0a, lds_operand32<kPS>(sm.dy, n, c, g), drt);
    dat = mfma32(s0a, lds_operand32<kPS>(sm.dz, n, c, g), dat);
    dbt = mfma32(dsa_, lds_operand32<kPS>(sm.sa, n, c, g), dbt);
    dkt = mfma32(dsa_, lds_operand32<kPS>(sm.vt, n, c, g), dkt);
    dgk = mfma32(s0a, dsa_, dgk);
  }
  // dg[key] = (S0 dS^T)[key][key]: the diagonal lanes publish it.
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (4 * g + j == n) sm.dg[16 * w + n] = dgk[j];
  }
  __syncthreads();  // gradient matrices (and dg) in LDS

  __builtin_amdgcn_s_setprio(1);
  const i16x4 bht = lds_operand_tr<kPS>(sm.bh, 0, 16 * w, g, n);
  const i16x4 kht = lds_operand_tr<kPS>(sm.kh, 0, 16 * w, g, n);
  const i16x4 att = lds_operand_tr<kPS>(sm.at, 0, 16 * w, g, n);
  const i16x4 rtt = lds_operand_tr<kPS>(sm.rt, 0, 16 * w, g, n);
  auto gT = [&](int m) { return lds_operand<kTriStride>(sm.grad[m], n, 4 * g); };  // B = M^T
  auto gN = [&](int m) { return lds_operand_tr<kTriStride>(sm.grad[m], 0, 0, g, n); };  // B = M
  drt = mfma32(cat(bht, kht), cat(gT(kGArb), gT(kGArk)), drt);
  dat = mfma32(cat(bht, kht), cat(gT(kGLab), gT(kGLak)), dat);
  const f32x4 dbh = mfma32(cat(att, rtt), cat(gN(kGLab), gN(kGArb)), zero4());
  const f32x4 dkh = mfma32(cat(att, rtt), cat(gN(kGLak), gN(kGArk)), zero4());
  __builtin_amdgcn_s_setprio(0);

  const int f0 = 16 * w + 4 * g;
  const float4 gk4 = *reinterpret_cast<const float4*>(&sm.gc[f0]);
  const float4 dg4 = *reinterpret_cast<const float4*>(&sm.dg[f0]);
  const float gk[4] = {gk4.x, gk4.y, gk4.z, gk4.w};
  const float dgv[4] = {dg4.x, dg4.y, dg4.z, dg4.w};
  // The decay terms multiply the scaled gradients by the bf16 tile values the
  // products used (not by the exact scaled inputs): the terms are large and
  // cancel, and they cancel to rounding only against the same operands.
  auto tile4 = [&](const uint16_t* tile, float (&x)[4]) {
    const uint2 q = *reinterpret_cast<const uint2*>(tile + n * kPS + f0);
    x[0] = bf16_float(static_cast<uint16_t>(q.x & 0xffffu));
    x[1] = bf16_float(static_cast<uint16_t>(q.x >> 16));
    x[2] = bf16_float(static_cast<uint16_t>(q.y & 0xffffu));
    x[3] = bf16_float(static_cast<uint16_t>(q.y >> 16));
  };
  float rt4[4], at4[4], bh4[4], kh4[4];
  tile4(sm.rt, rt4);
  tile4(sm.at, at4);
  tile4(sm.bh, bh4);
  tile4(sm.kh, kh4);
  float o_r[4], o_k[4], o_a[4], o_b[4], o_w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float dbc = dbh[j] + gk[j] * dbt[j];
    const float dkc = dkh[j] + gk[j] * dkt[j];
    const float e2 = dat[j] * at4[j];
    const float e1 = drt[j] * rt4[j] - dbc * bh4[j] - dkc * kh4[j];
    const float e3 = gk[j] * (dbt[j] * bh4[j] + dkt[j] * kh4[j]);
    const float dlg = suffix16_sum(e1 + e2) - e2 + rowsum16(e3) + gk[j] * dgv[j];
    o_r[j] = drt[j] * rows.fg[j];
    o_a[j] = dat[j] * rows.fgp[j];
    o_b[j] = rows.fgn[j] * dbc;
    o_k[j] = rows.fgn[j] * dkc;
    o_w[j] = dlg * rows.dwf[j];
  }
  store4(p.dr, f0, o_r[0], o_r[1], o_r[2], o_r[3]);
  store4(p.dk, f0, o_k[0], o_k[1], o_k[2], o_k[3]);
  store4(p.da, f0, o_a[0], o_a[1], o_a[2], o_a[3]);
  store4(p.db, f0, o_b[0], o_b[1], o_b[2], o_b[3]);
  store4(p.ddecay, f0, o_w[0], o_w[1], o_w[2], o_w[3]);
  __syncthreads();  // the next pass rewrites every tile
}

template <typename T, DecayMode M>
__global__ __launch_bounds__(kPThreads, 1) void piece_bwd_kernel(TrainParams p) {
  __shared__ PieceSmem sm;
  __shared__ __align__(16) RowStage stage;
  using St = typename IoTraits<T>::storage;
  const int tid = threadIdx.x;
  const int w = tid >> 6, lane = tid & 63;
  const int g = lane >> 4;
  const int unit = blockIdx.x;
  const int seq = unit / p.num_heads;
  const int head = unit % p.num_heads;
  const int64_t hd = static_cast<int64_t>(p.num_heads) * kPD;
  const int64_t unit_state =
      (static_cast<int64_t>(seq) * p.num_heads + head) * static_cast<int64_t>(kPD) * kPD;
  const float nan = __int_as_float(0x7fc00000);

  float bias[4] = {0.f, 0.f, 0.f, 0.f};
  if constexpr (M == DecayMode::kLogits) {
    if (p.bias != nullptr) {
      const St* bp = static_cast<const St*>(p.bias) + head * kPD + 16 * w + 4 * g;
      const uint2 q = *reinterpret_cast<const uint2*>(bp);
      unpack4<T>(q, bias);
    }
  }

  Slab dS;
  if (p.dstate_final != nullptr) {
    load_slab16(dS, p.dstate_final + unit_state);
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  } else {
#pragma unroll
    for (int kb = 0; kb < kPD / 16; ++kb) dS.x[kb] = zero4();
  }

  // Fail closed, as the per-token backward: from a chunk longer than one
  // piece without interior states on (walking backwards), the unit's
  // gradients are NaN.
  auto nan_fill = [&](const Chunk& ch) {
    const int64_t nt = static_cast<int64_t>(ch.end - ch.start);
    void* const outs[6] = {p.dr, p.dk, p.db, p.ddecay, p.da, p.dv};
    for (int64_t item = tid; item < nt * 6 * kPD; item += kPThreads) {
      const int32_t t = ch.start + static_cast<int32_t>(item / (6 * kPD));
      const int gi = static_cast<int>((item / kPD) % 6);
      const int e = static_cast<int>(item % kPD);
      static_cast<St*>(outs[gi])[t * hd + head * kPD + e] = from_f32<T>(nan);
    }
  };

  int c_begin, c_end;
  chunk_range(p, seq, c_begin, c_end);
  bool failed = false;
  PieceRows rows;
  // have: the rows of the piece at t0 are staged in LDS (loaded while the
  // piece after it computed).
  bool have = false;
  for (int c = c_end - 1; c >= c_begin; --c) {
    const Chunk whole = chunk_at<kPD>(p, seq, head, c);
    const int len = whole.end - whole.start;
    const int pieces = len > kPiece ? (len + kPiece - 1) / kPiece : 1;
    if (pieces > 1 && p.interior == nullptr) failed = true;
    if (failed) {
      nan_fill(whole);
      continue;
    }
    for (int pj = pieces - 1; pj >= 0; --pj) {
      const int32_t t0 = whole.start + kPiece * pj;
      const int ntok = min(kPiece, whole.end - t0);
      if (ntok <= 0) continue;
      // The piece's start state: the chunk's (fp32) or an interior one (bf16).
      auto load_start = [&](Slab& S) {
        if (pj == 0) {
          load_slab16(S, p.ckpt + whole.ckpt_off);
        } else {
          load_slab_bf16(S, interior_block(p, head, t0));
        }
      };
      // The next piece (walking backwards): this chunk's previous piece, else
      // the last piece of the chunk before when that chunk will not fail.
      // Found here, before the start state's loads are issued: reading the
      // chunk metadata waits for every load in flight.
      int32_t t0n = 0;
      int ntokn = 0;
      if (pj > 0) {
        t0n = t0 - kPiece;
        ntokn = kPiece;
      } else if (c > c_begin) {
        const Chunk wn = chunk_at<kPD>(p, seq, head, c - 1);
        const int lenn = wn.end - wn.start;
        const int piecesn = lenn > kPiece ? (lenn + kPiece - 1) / kPiece : 1;
        if (!(piecesn > 1 && p.interior == nullptr)) {
          t0n = wn.start + kPiece * (piecesn - 1);
          ntokn = min(kPiece, wn.end - t0n);
        }
      }
      // The piece's rows: staged while the piece after it computed (its
      // column phase waited for them, and barriers followed), or now. Once
      // every wave has read them, the next piece's rows are staged, then the
      // start state is loaded.
      if (!have) {
        piece_rows_to_lds<T>(stage, p, head, t0, ntok);
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        __syncthreads();
      }
      PieceLoad L;
      piece_load_staged(L, stage);
      __syncthreads();
      have = ntokn > 0;
      if (have) piece_rows_to_lds<T>(stage, p, head, t0n, ntokn);
      Slab S;
      load_start(S);
      piece_stage<T, M, true>(sm, rows, L, p, bias, 0, ntok);
      bool ok = true;
#pragma unroll
      for (int i = 0; i < kPWaves; ++i) ok = ok && sm.span_ok[i] != 0;
      ok = __builtin_amdgcn_readfirstlane(ok ? 1 : 0) != 0;


      // One pass sequence with a single copy of each phase. A piece within
      // the span limit is one backward pass over [0, ntok), on the rows just
      // staged. Strong decay: 4-token sub-pieces s = nsub - 1 .. 0, each
      // preceded by forward passes over sub-pieces 0 .. s - 1 from the piece
      // start state, every pass on rows loaded again from global memory.
      const int nsub = (ntok + 3) / 4;
      int sub = ok ? 0 : nsub - 1;
      int q = 0;
      bool prepared = ok;
      for (;;) {
        const bool fwd = !ok && q < sub;
        const int lo = ok ? 0 : 4 * (fwd ? q : sub);
        const int hi = ok ? ntok : min(lo + 4, ntok);
        if (!prepared) {
          if (!ok && q == 0 && sub != nsub - 1) load_start(S);
          piece_prepare<T, M>(sm, rows, p, bias, head, t0, ntok, lo, hi);
        }
        prepared = false;
        if (fwd) {
          piece_intra(sm);
          PieceOut unused;
          piece_forward_state<T, false>(sm, S, rows, p, t0, ntok, unused);
          ++q;
          continue;
        }
        piece_backward<T>(sm, rows, p, head, t0, ntok, S, dS);
        if (sub == 0) break;
        --sub;
        q = 0;
      }
    }
  }

  if (p.dstate0 != nullptr) {
    if (failed) {
#pragma unroll
      for (int kb = 0; kb < kPD / 16; ++kb) dS.x[kb] = f32x4{nan, nan, nan, nan};
    }
    store_slab16(p.dstate0 + unit_state, dS);
  }
}

// The head-size-128 training forward, with the outputs and checkpoint layout
// of the per-token kernels (train_recurrent.hip). Per chunk of the unit: the state at the chunk start (ckpt), at every further 16-token piece
// start (interior, slot (piece start) / 16), y and state_dot_a per token, and
// the final state. kFill: the interior replay (one chunk per unit, only the
// interior states; chunks of at most 16 tokens are skipped and a chunk's last
// piece is not computed).
template <typename T, DecayMode M, bool kFill>
__global__ __launch_bounds__(kPThreads, 1) void piece_fwd_kernel(TrainParams p) {
  __shared__ PieceSmem sm;
  using St = typename IoTraits<T>::storage;
  const int tid = threadIdx.x;
  const int w = tid >> 6, lane = tid & 63;
  const int g = lane >> 4;
  const int unit = blockIdx.x;
  const int seq = unit / p.num_heads;
  const int head = unit % p.num_heads;
  const int64_t unit_state =
      (static_cast<int64_t>(seq) * p.num_heads + head) * static_cast<int64_t>(kPD) * kPD;

  float bias[4] = {0.f, 0.f, 0.f, 0.f};
  if constexpr (M == DecayMode::kLogits) {
    if (p.bias != nullptr) {
      const St* bp = static_cast<const St*>(p.bias) + head * kPD + 16 * w + 4 * g;
      const uint2 q = *reinterpret_cast<const uint2*>(bp);
      unpack4<T>(q, bias);
    }
  }
  Slab S;
  if (p.state != nullptr) {
    load_slab16(S, p.state + unit_state);
  } else {
#pragma unroll
    for (int kb = 0; kb < kPD / 16; ++kb) S.x[kb] = zero4();
  }
  // The initial state lands before the piece loop (kWaitVmcnt0).
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);

  int c_begin, c_end;
  chunk_range(p, seq, c_begin, c_end);
  PieceRows rows;
  // The rows of the next piece to compute are loaded while the current one
  // is computed (have: L holds the piece at t0). A pass's outputs are stored
  // at the start of the next piece, after its wait for those rows: on gfx9
  // that wait (vmcnt) also waits for every store issued before it, and these
  // then have had a whole piece to complete.
  PieceLoad L;
  bool have = false;
  PieceOut held;
  bool pending = false;
  for (int c = c_begin; c < c_end; ++c) {
    const Chunk ch = chunk_at<kPD>(p, seq, head, c);
    const int len = ch.end - ch.start;
    if (kFill && len <= kPiece) continue;
    const int pieces = len > kPiece ? (len + kPiece - 1) / kPiece : 1;
    for (int pj = 0; pj < pieces; ++pj) {
      const int32_t t0 = ch.start + kPiece * pj;
      const int ntok = min(kPiece, ch.end - t0);
      const bool stop = ntok <= 0 || (kFill && t0 + kPiece >= ch.end);
      if (!stop && !have) piece_load<T, false>(L, p, head, t0, ntok);
      __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
      if (pending) store_piece_out<T>(held, p, head);
      pending = false;
      if (pj == 0 && !kFill && p.ckpt != nullptr) store_slab16(p.ckpt + ch.ckpt_off, S);
      if (pj > 0 && p.interior != nullptr) store_slab_bf16(interior_block(p, head, t0), S);
      if (stop) break;
      piece_stage<T, M, false>(sm, rows, L, p, bias, 0, ntok);
      bool ok = true;
#pragma unroll
      for (int i = 0; i < kPWaves; ++i) ok = ok && sm.span_ok[i] != 0;
      ok = __builtin_amdgcn_readfirstlane(ok ? 1 : 0) != 0;

      // The next piece that computes: the chunk's next piece, else the next
      // chunk's first (only once its range is checked). Its rows go to L,
      // which the stage above consumed.
      int32_t t0n = 0;
      int ntokn = 0;
      if (pj + 1 < pieces) {
        t0n = t0 + kPiece;
        ntokn = (kFill && t0n + kPiece >= ch.end) ? 0 : min(kPiece, ch.end - t0n);
      } else if (c + 1 < c_end) {
        const Chunk chn = chunk_at<kPD>(p, seq, head, c + 1);
        if (!(kFill && chn.end - chn.start <= kPiece)) {
          t0n = chn.start;
          ntokn = min(kPiece, chn.end - chn.start);
        }
      }
      have = ntokn > 0;
      if (have) piece_load<T, false>(L, p, head, t0n, ntokn);

      if (ok) {
        // One pass over [0, ntok); its outputs are stored with the next piece.
        piece_intra(sm);
        piece_forward_state<T, !kFill>(sm, S, rows, p, t0, ntok, held);
        pending = !kFill && p.out != nullptr;
      } else {
        // Strong decay: 4-token sub-pieces in order, each continuing from the
        // state the one before it left, on rows loaded again (L holds the
        // next piece); outputs stored right away.
        for (int sub = 0; 4 * sub < ntok; ++sub) {
          const int lo = 4 * sub, hi = min(lo + 4, ntok);
          PieceLoad Ls;
          piece_load<T, false>(Ls, p, head, t0, ntok);
          piece_stage<T, M, false>(sm, rows, Ls, p, bias, lo, hi);
          piece_intra(sm);
          PieceOut o;
          piece_forward_state<T, !kFill>(sm, S, rows, p, t0, ntok, o);
          if (!kFill && p.out != nullptr) store_piece_out<T>(o, p, head);
        }
      }
    }
  }
  if (pending) store_piece_out<T>(held, p, head);

  if (p.state != nullptr && !kFill) store_slab16(p.state + unit_state, S);
}

template <typename T, DecayMode M>
int launch_piece(const TrainParams& p, int units, bool backward, hipStream_t stream) {
  if (backward) {
    hipLaunchKernelGGL((piece_bwd_kernel<T, M>), dim3(units), dim3(kPThreads), 0, stream, p);
    return check_launch("piece_bwd_kernel");
  }
  if (p.fill_only) {
    hipLaunchKernelGGL((piece_fwd_kernel<T, M, true>), dim3(units), dim3(kPThreads), 0, stream,
                       p);
  } else {
    hipLaunchKernelGGL((piece_fwd_kernel<T, M, false>), dim3(units), dim3(kPThreads), 0, stream,
                       p);
  }
  return check_launch("piece_fwd_kernel");
}

}  // namespace

int launch_piece_train(const TrainParams& p, int io_dtype, int decay_mode, int units,
                       bool backward, hipStream_t stream) {
  const bool logits = decay_mode == FRWKV_DECAY_LOGITS;
  if (!logits && decay_mode != FRWKV_DECAY_RAW_W) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT, "unknown decay mode %d", decay_mode);
  }
  if (!logits && p.bias != nullptr) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "decay_bias is only defined for the logits decay mode");
  }
  switch (io_dtype) {
    case FRWKV_DTYPE_BF16:
      return logits ? launch_piece<Bf16, DecayMode::kLogits>(p, units, backward, stream)
                    : launch_piece<Bf16, DecayMode::kRawW>(p, units, backward, stream);
    case FRWKV_DTYPE_F16:
      return logits ? launch_piece<F16, DecayMode::kLogits>(p, units, backward, stream)
                    : launch_piece<F16, DecayMode::kRawW>(p, units, backward, stream);
    default:
      return set_error(FRWKV_ERR_UNSUPPORTED,
                       "training kernels take float16 or bfloat16 tokens (io dtype %d)",
                       io_dtype);
  }
}

}  // namespace frwkv
