// Chunked WKV7 backward on bf16 MFMA (training: StateTune and pretraining).
//
// Replaces the reference's StateTune backward
// (csrc/sm90/tmix/wkv7/statetune_recurrent_fp32io16_backward.cu:49-676),
// which rebuilds S_{t-1} = (S_t - k v^T - b sa^T) / w token by token; that
// division loses all precision over a 64-token chunk. This kernel never
// divides by the decay: the forward stores the state at every caller chunk
// start (the StateTune boundary output) and, for caller chunks longer than
// 64 tokens, at every further 64-token piece start (interior checkpoints);
// the backward recomputes each piece's forward quantities from those states.
//
// One 512-thread workgroup per (sequence, head) walks its pieces in reverse,
// carrying the state adjoint dS (dL/dS at the current piece end) in
// registers. With the chunk notation of the forward kernel (At, Rt, Bh, Kh,
// g = 2^GC, Lab, Lak, Arb, Ark, T = (I - Lab)^{-1}, SA) and dYs = scale dY,
// per piece:
//   dSA = Arb^T dYs + Bh (g o dS)            dZ  = T^T dSA
//   dV  = Ark^T dYs + Lak^T dZ + Kh (g o dS)
//   dS0 = g o dS + Rt^T dYs + At^T dZ        (the adjoint of the piece before)
//   dArb = lower(dYs SA^T)   dArk = lower(dYs V^T)
//   dLab = strict(dZ SA^T)   dLak = strict(dZ V^T)
//   dRt = dYs S0^T + dArb Bh + dArk Kh       dAt = dZ S0^T + dLab Bh + dLak Kh
//   dBh = dLab^T At + dArb^T Rt              dKh = dLak^T At + dArk^T Rt
//   dBt = SA dS^T                            dKt = V dS^T     (Bt = Bh diag g)
//   dg  = rowsum(S0 o dS)
// and the raw gradients follow elementwise: dr = dRt 2^G, da = dAt 2^Gp,
// db = 2^-G (dBh + g dBt), dk = 2^-G (dKh + g dKt). With e1_t = dRt Rt -
// (dBh + g dBt) Bh - (dKh + g dKt) Kh, e2_t = dAt At, e3_t = g (dBt Bh +
// dKt Kh) per feature, the gradient of the log2 retention is
//   dlg_j = sum_{t>=j} (e1_t + e2_t) - e2_j + sum_t e3_t + dg g,
// so dw = dlg / w (the ln 2 of d(log2 w)/dw cancels) and, for logits,
// dx = dlg (-e^{-1/2} sigmoid(x) (1 - sigmoid(x))).
//
// Work decomposition (8 waves, two per SIMD; wave w, lane (g, n) with
// g = lane / 16, n = lane % 16):
//   prepare   token layout: wave w owns tokens 16p .. 16p+15 (p = w % 4) and
//             features 32h .. 32h+31 (h = w / 4); lane (g, n) holds token
//             16p + n, features 32h + 8g .. +7. Decodes the rows, scans the
//             decay over tokens (DPP inside a 16-lane row plus block sums)
//             and writes the operand tiles At, Rt, Bh, Kh, dYs, V.
//   intra     Lab, Lak, Arb, Ark ([t][i] blocks) and the diagonal inverses T;
//             waves 0-3 the diagonal blocks, waves 4-7 the off-diagonal ones.
//   columns   wave w < 4 runs the forward chain SA for value columns
//             16w .. 16w+15; wave w + 4 the adjoint chain dSA, dZ, dV, dS0
//             for the same columns (dS lives in its accumulators).
//   matrices  dArb, dArk, dLab, dLak ([t][i] blocks), five blocks per wave.
//   tokens    the token layout again: the gradient products come out with
//             lane (g, n) holding token 16p + n and features 32h + 8g .. +7,
//             the lanes that hold the raw rows, so the elementwise chain rule
//             needs no reload and every gradient store is 16 bytes per lane
//             (64 contiguous bytes per 4 lanes).
// Every transposed operand is read through gfx950's LDS transpose read from
// the one stored copy. Every HBM input of a piece is loaded while the piece
// after it computes.
//
// Pieces: a caller chunk [s, e) is walked as 64-token pieces s + 64 j. The
// state at piece j > 0 comes from the interior checkpoint at frame
// (s + 64 j) / 64; interior starts of different chunks are more than 64
// tokens apart, so frames are unique and the interior buffer has
// ceil(total_tokens / 64) entries per head. A piece whose decay span exceeds
// the single-reference limit (80 log2 units) runs as sub-pieces of 16
// tokens, or 4 where a 16-token block still exceeds it: sub-piece r starts
// from the state recomputed by forward steps over sub-pieces 0 .. r-1 from the
// piece start, so the backward stays exact for any decay (at a cost quadratic
// in the number of sub-pieces, which only such pieces pay).

#include "capi_internal.h"
#include "chunk_common.h"

namespace frwkv {
namespace {

constexpr int kBwdThreads = 512;

struct BwdSmem {
  uint16_t at[kOpTile];   // At  [t][k]
  uint16_t rt[kOpTile];   // Rt  [t][k]
  uint16_t bh[kOpTile];   // Bh  [t][k]
  uint16_t kh[kOpTile];   // Kh  [t][k]
  uint16_t dy[kOpTile];   // dYs [t][v]
  uint16_t vv[kOpTile];   // V   [t][v]
  uint16_t sa[kOpTile];   // SA  [t][v]
  uint16_t dz[kOpTile];   // dZ  [t][v]
  uint16_t s0[kOpTile];   // S0  [v][k]
  uint16_t ds[kOpTile];   // dS  [v][k] (adjoint at the piece end)
  uint16_t dv[kOpTile];   // dV  [t][v] in the io dtype (staged for row stores)
  union {
    struct {
      uint16_t tri[4][kTriBlocks * kTriBlock];  // Lab, Lak, Arb, Ark: [t][i]
      uint16_t tinv[4][kTriBlock];              // T_pp [t][i]
    } f;
    uint16_t grad[4][kTriBlocks * kTriBlock];   // dArb, dArk, dLab, dLak: [t][i]
  } u;
  float blk[4][kHead];    // per-block products of the retention
  float gc[kHead];        // 2^GC
  float dgam[4][kHead];   // partial rowsum(S0 o dS) per column slab
  float car1[4][kHead];   // per-block totals of e1 + e2
  float car3[4][kHead];   // per-block totals of e3
  // The state adjoint dS of the adjoint waves between their column phases:
  // [slab][kb][lane] x 4 floats (the lane's C-layout values), 16 bytes per
  // lane and consecutive lanes consecutive, so the accesses are
  // conflict-free. Keeping it here frees 16 registers per lane in the other
  // phases.
  f32x4 dstash[4][4][64];
};
static_assert(sizeof(BwdSmem) <= 160 * 1024, "one workgroup per CU");

enum FwdTri { kLab = 0, kLak = 1, kArb = 2, kArk = 3 };
enum GradTri { kGArb = 0, kGArk = 1, kGLab = 2, kGLak = 3 };

struct ChunkBwdParams {
  int32_t num_heads;
  int32_t total_tokens;
  int32_t num_segments;
  const int32_t* seg_offsets;
  const int32_t* seg_starts;
  const int32_t* seg_ends;
  const float* checkpoint;      // [num_segments, H, 64, 64]: state at each segment start
  const float* interior;        // [ceil(N/64), H, 64, 64] piece-start states, or null
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
  // Dense layout: > 0 means every sequence has dense_t tokens (one segment)
  // and checkpoint is [B, H, dense_t / 16, D, D], the state every 16 tokens.
  int32_t dense_t;
};

__device__ __forceinline__ const __attribute__((address_space(4))) ChunkBwdParams& args() {
  return kernel_args<ChunkBwdParams>();
}

// Raw token rows of one piece in the token layout (16 bytes per tensor).
struct TokRows {
  uint4 r, w, k, a, b, dy, v;
};

// A piece and where its start state lives.
struct Piece {
  int c0, ntok;      // first token, token count (0: none)
  int64_t ckpt;      // float index of its 64 x 64 start state
  bool from_interior;
};

__device__ __forceinline__ const uint16_t* tri_blk(const uint16_t* m, int p, int q) {
  return m + tri_index(p, q) * kTriBlock;
}

// Inclusive prefix / suffix sums over the 16 lanes of a DPP row.
template <int N>
__device__ __forceinline__ float row_shr_add(float x) {
  return x + __int_as_float(
                 __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x110 + N, 0xf, 0xf, true));
}
template <int N>
__device__ __forceinline__ float row_shl_add(float x) {
  return x + __int_as_float(
                 __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x100 + N, 0xf, 0xf, true));
}
__device__ __forceinline__ float prefix16(float x) {
  return row_shr_add<8>(row_shr_add<4>(row_shr_add<2>(row_shr_add<1>(x))));
}
__device__ __forceinline__ float suffix16(float x) {
  return row_shl_add<8>(row_shl_add<4>(row_shl_add<2>(row_shl_add<1>(x))));
}
// Products over the 16 lanes of a DPP row (n = lane % 16): lanes n < N keep
// x (the shifted-in value reads 0, and the select restores x).
template <int N>
__device__ __forceinline__ float row_shr_mul(float x, int n) {
  const float y = x * __int_as_float(
                          __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x110 + N, 0xf, 0xf, true));
  return n >= N ? y : x;
}
__device__ __forceinline__ float prefix16_mul(float x, int n) {
  return row_shr_mul<8>(row_shr_mul<4>(row_shr_mul<2>(row_shr_mul<1>(x, n), n), n), n);
}
// The exclusive product from the inclusive one: lane n takes lane n - 1's,
// lane 0 the empty product 1.
__device__ __forceinline__ float exclusive16(float incl, int n) {
  const float y = __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(incl), 0x111, 0xf, 0xf, true));
  return n >= 1 ? y : 1.0f;
}

// Stores a C-layout block (lane (g, n) holds X[4g + j][n]) into a row-major
// [row][col] bf16 tile at dst: four 2-byte stores per lane, the 16 lanes of a
// group writing 32 consecutive bytes of one row.
__device__ __forceinline__ void lds_store_rows(uint16_t* dst, int stride, int g, int n,
                                               f32x4 c) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    dst[(4 * g + j) * stride + n] = static_cast<uint16_t>(pack_bf16x2(c[j], 0.0f) & 0xffffu);
  }
}

// Transpose read (see lds_operand_tr) whose column groups are 8 apart:
// lane (g, i) receives X[t0 + 4g + e][c0 + 8 (i / 4) + i % 4], so the rows
// m = 4g' + j of a product with this A operand are features
// c0 + 8 g' + j: with c0 = 32h + 4u, lane (g, n) of the product holds
// features 32h + 8g + 4u + j, the token layout's features.
template <int Stride>
__device__ __forceinline__ i16x4 lds_tr_q8(const uint16_t* tile, int t0, int c0, int g, int n) {
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  const uint16_t* src = tile + (t0 + 4 * g + (n >> 2)) * Stride + c0 + 8 * (n & 3);
  const v4i16 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4i16*)(src));
  return i16x4{x[0], x[1], x[2], x[3]};
}

// 32-wide K steps: two 16-blocks concatenated (see mfma32).
template <int Stride>
__device__ __forceinline__ i16x8 tr32(const uint16_t* tile, int t0, int c0, int g, int n) {
  return cat(lds_operand_tr<Stride>(tile, t0, c0, g, n),
             lds_operand_tr<Stride>(tile, t0 + 16, c0, g, n));
}
template <int Stride>
__device__ __forceinline__ i16x8 tr32_q8(const uint16_t* tile, int t0, int c0, int g, int n) {
  return cat(lds_tr_q8<Stride>(tile, t0, c0, g, n), lds_tr_q8<Stride>(tile, t0 + 16, c0, g, n));
}

__device__ __forceinline__ i16x8 lo32(i16x4 x) { return cat(x, i16x4{0, 0, 0, 0}); }

template <typename T>
__device__ __forceinline__ void unpack8v(uint4 q, float (&x)[8]) {
  unpack8<T>(q, x);
}

// 8 floats -> 8 values of the io dtype, one 16-byte word.
template <typename T>
__device__ __forceinline__ u32x4 pack8(const float (&x)[8]) {
  return u32x4{pack2<T>(x[0], x[1]), pack2<T>(x[2], x[3]), pack2<T>(x[4], x[5]),
               pack2<T>(x[6], x[7])};
}

// Decay-span verdicts of a prepared range, uniform over the workgroup.
struct Spans {
  bool whole;
  bool block[4];
  __device__ __forceinline__ bool block_ok(int q) const {
    return q == 0 ? block[0] : q == 1 ? block[1] : q == 2 ? block[2] : block[3];
  }
};

// Sub-piece r of a strong-decay piece: 16-token blocks whose span is within
// the limit stay whole, the others split in four 4-token sub-pieces.
__device__ __forceinline__ int sub_count(const Spans& s) {
  int c = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) c += s.block[q] ? 1 : 4;
  return c;
}
__device__ __forceinline__ void sub_range(const Spans& s, int r, int& lo, int& hi) {
  int idx = 0;
  lo = hi = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int cnt = s.block[q] ? 1 : 4;
    if (r >= idx && r < idx + cnt) {
      const int len = s.block[q] ? 16 : 4;
      lo = 16 * q + (r - idx) * len;
      hi = lo + len;
    }
    idx += cnt;
  }
}

// Prepare: decodes the lane's token row over [lo, hi) (tokens outside are
// zero rows), writes the operand tiles, the per-block decay sums and 2^GC,
// and returns the spans. Ends with a barrier.
template <typename T, DecayMode M>
__device__ Spans prepare_piece(BwdSmem& sm, const TokRows& rows, const uint4& bias_raw,
                               int lo, int hi, float scale) {
  const int tid = lane_tid();
  const int wave = uniform(tid >> 6);
  const int lane = tid & 63;
  const int g = lane >> 4, n = lane & 15;
  const int p = wave & 3, h = wave >> 2;
  const int t = 16 * p + n;
  const int f0 = 32 * h + 8 * g;
  const bool on = t >= lo && t < hi;

  __syncthreads();  // earlier readers of the tiles are done

  // Retentions (1 outside [lo, hi)) and the cumulative decay as products:
  // 2^G(t) = prod_{j<=t} w_j by a product scan over the block's 16 tokens
  // (one DPP row) and the products of the earlier blocks. Every product that
  // reaches an operand has a span within the limit (>= 2^-80, a normal fp32
  // number); a pass whose span exceeds it is redone as sub-pieces.
  float wr[8], G[8];
  {
    float x[8], bias[8];
    unpack8<T>(rows.w, x);
    unpack8<T>(bias_raw, bias);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float xin = x[e];
      if constexpr (M == DecayMode::kLogits) xin += bias[e];
      const float r = clamped_retention<M>(xin);
      wr[e] = on ? r : 1.0f;
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) G[e] = prefix16_mul(wr[e], n);
  if (n == 15) {
    *reinterpret_cast<float4*>(&sm.blk[p][f0]) = make_float4(G[0], G[1], G[2], G[3]);
    *reinterpret_cast<float4*>(&sm.blk[p][f0 + 4]) = make_float4(G[4], G[5], G[6], G[7]);
  }
  __syncthreads();

  float total[8], carry[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) total[e] = carry[e] = 1.0f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float4 x0 = *reinterpret_cast<const float4*>(&sm.blk[q][f0]);
    const float4 x1 = *reinterpret_cast<const float4*>(&sm.blk[q][f0 + 4]);
    const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (q < p) carry[e] *= xs[e];
      total[e] *= xs[e];
    }
  }
  // Spans over all 64 features: lane l looks at feature l.
  Spans spans;
  {
    float bprod = 1.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float x = sm.blk[q][lane];
      bprod *= x;
      spans.block[q] = __builtin_amdgcn_ballot_w64(!(x >= kSpanFloor)) == 0;
    }
    spans.whole = __builtin_amdgcn_ballot_w64(!(bprod >= kSpanFloor)) == 0;
  }

  // Scaled operand rows: At = a 2^Gp, Rt = r 2^G, Bh = b 2^-G, Kh = k 2^-G.
  float up[8], upp[8], dn[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float g = G[e] * carry[e];
    const float gp = exclusive16(G[e], n) * carry[e];
    up[e] = on ? g : 0.0f;
    upp[e] = on ? gp : 0.0f;
    dn[e] = on ? __builtin_amdgcn_rcpf(g) : 0.0f;
  }
  auto row = [&](uint16_t* tile, uint4 raw, const float (&f)[8], float s) {
    float x[8];
    unpack8<T>(raw, x);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] *= f[e] * s;
    store8_bf16(tile + t * kOpStride + f0, x);
  };
  row(sm.at, rows.a, upp, 1.0f);
  row(sm.rt, rows.r, up, 1.0f);
  row(sm.bh, rows.b, dn, 1.0f);
  row(sm.kh, rows.k, dn, 1.0f);
  float ones[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) ones[e] = on ? 1.0f : 0.0f;
  row(sm.dy, rows.dy, ones, scale);
  row(sm.vv, rows.v, ones, 1.0f);
  if (p == 0 && n == 0) {
    *reinterpret_cast<float4*>(&sm.gc[f0]) = make_float4(total[0], total[1], total[2], total[3]);
    *reinterpret_cast<float4*>(&sm.gc[f0 + 4]) = make_float4(total[4], total[5], total[6], total[7]);
  }
  __syncthreads();
  return spans;
}

// Intra-piece matrices Lab, Lak, Arb, Ark ([t][i]) and the diagonal inverses
// T_pp = (I - Lab_pp)^{-1}. Waves 0-3: the diagonal block pair (w, w) and its
// inverse; waves 4-7: three of the twelve off-diagonal half-pairs each. A
// block M[t][i] = sum_k X[t][k] Y[i][k] is computed transposed (A = Y rows,
// B = X rows) so that each lane writes 4 consecutive i of one row t. issue(i)
// runs between product groups (prefetch of the piece before). Ends with a
// barrier.
template <typename Issue>
__device__ __forceinline__ void intra_piece(BwdSmem& sm, Issue&& issue) {
  const int tid = lane_tid();
  const int wave = uniform(tid >> 6);
  const int lane = tid & 63;
  const int g = lane >> 4, n = lane & 15;

  auto store = [&](int m, int p, int q, f32x4 acc, bool strict) {
    if (p == q) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = 4 * g + j;
        acc[j] = (strict ? (i < n) : (i <= n)) ? acc[j] : 0.0f;
      }
    }
    lds_store_transposed(sm.u.f.tri[m] + tri_index(p, q) * kTriBlock, kTriStride, g, n, acc);
  };
  auto group = [&](int p, int q, bool with_b, bool with_k, f32x4* lab_c) {
    f32x4 lab = zero4(), lak = zero4(), arb = zero4(), ark = zero4(), labc = zero4();
#pragma unroll
    for (int c = 0; c < 64; c += 32) {
      const i16x8 xa = lds_operand32<kOpStride>(sm.at, 16 * p + n, c, g);
      const i16x8 xr = lds_operand32<kOpStride>(sm.rt, 16 * p + n, c, g);
      if (with_b) {
        const i16x8 yb = lds_operand32<kOpStride>(sm.bh, 16 * q + n, c, g);
        lab = mfma32(yb, xa, lab);
        arb = mfma32(yb, xr, arb);
        if (lab_c != nullptr) labc = mfma32(xa, yb, labc);
      }
      if (with_k) {
        const i16x8 yk = lds_operand32<kOpStride>(sm.kh, 16 * q + n, c, g);
        lak = mfma32(yk, xa, lak);
        ark = mfma32(yk, xr, ark);
      }
    }
    if (with_b) {
      store(kLab, p, q, lab, true);
      store(kArb, p, q, arb, false);
    }
    if (with_k) {
      store(kLak, p, q, lak, true);
      store(kArk, p, q, ark, false);
    }
    if (lab_c != nullptr) {
      // lab: lane (g, n) holds L[n][4g + j]; labc: L[4g + j][n] (strict lower).
      f32x4 lr = lab, lc = labc;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        lr[j] = (4 * g + j < n) ? lr[j] : 0.0f;
        lc[j] = (n < 4 * g + j) ? lc[j] : 0.0f;
      }
      lab_c[0] = lr;
      lab_c[1] = lc;
    }
  };

  __builtin_amdgcn_s_setprio(1);
  if (wave < 4) {
    f32x4 l[2];
    issue(0);
    group(wave, wave, true, true, l);
    issue(1);
    // (I - L)^{-1} = (I + L)(I + L^2)(I + L^4)(I + L^8) for strictly lower
    // 16 x 16 L. With X_R "lane (g, n) holds X[n][4g + j]" and X_C the C
    // layout, Z = X Y is Z_C = mfma(X_R, Y_C) and Z_R = mfma(Y_C, X_R).
    const i16x4 lr = to_operand(l[0]), lc = to_operand(l[1]);
    const i16x4 p2c = to_operand(mfma16(lr, lc, zero4()));
    const i16x4 p2r = to_operand(mfma16(lc, lr, zero4()));
    const i16x4 p4c = to_operand(mfma16(p2r, p2c, zero4()));
    const i16x4 p4r = to_operand(mfma16(p2c, p2r, zero4()));
    const i16x4 p8c = to_operand(mfma16(p4r, p4c, zero4()));
    f32x4 tt = l[0];
#pragma unroll
    for (int j = 0; j < 4; ++j) tt[j] += (4 * g + j == n) ? 1.0f : 0.0f;
    tt = mfma16(p2c, to_operand(tt), tt);
    tt = mfma16(p4c, to_operand(tt), tt);
    tt = mfma16(p8c, to_operand(tt), tt);
    lds_store_transposed(sm.u.f.tinv[wave], kTriStride, g, n, tt);  // T [t][i]
    issue(2);
  } else {
    // Off-diagonal half-pairs: pair index item / 2 over (1,0) (2,0) (2,1)
    // (3,0) (3,1) (3,2), half item % 2 ({Lab, Arb} share Bh_q, {Lak, Ark}
    // share Kh_q).
#pragma unroll
    for (int r = 0; r < 3; ++r) {
      const int item = (wave - 4) + 4 * r;
      const int pair = item >> 1;
      const int p = pair < 1 ? 1 : (pair < 3 ? 2 : 3);
      const int q = pair - (p * (p - 1)) / 2;
      issue(r);
      group(p, q, (item & 1) == 0, (item & 1) == 1, nullptr);
    }
  }
  __builtin_amdgcn_s_setprio(0);
  __syncthreads();
}

// Forward chain of value columns 16 cs .. 16 cs + 15 (S0 in C layout):
// SA = T (At S0 + Lak V) in C layout (lane (g, n): SA[16 pb + 4g + j][16 cs + n]).
__device__ __forceinline__ void sa_chain(const BwdSmem& sm, const f32x4 (&S0)[4], int cs,
                                         int g, int n, f32x4 (&sa)[4], i16x4 (&sab)[4],
                                         i16x4 (&vs)[4]) {
  g = (lane_tid() & 63) >> 4;
  n = lane_tid() & 15;
#pragma unroll
  for (int q = 0; q < 4; ++q) vs[q] = lds_operand_tr<kOpStride>(sm.vv, 16 * q, 16 * cs, g, n);
  const i16x8 s01 = cat(to_operand(S0[0]), to_operand(S0[1]));
  const i16x8 s23 = cat(to_operand(S0[2]), to_operand(S0[3]));
  const i16x8 v01 = cat(vs[0], vs[1]), v23 = cat(vs[2], vs[3]);
  auto L = [&](int m, int p, int q) {
    return lds_operand<kTriStride>(tri_blk(sm.u.f.tri[m], p, q), n, 4 * g);
  };
  f32x4 rhs[4];
#pragma unroll
  for (int pb = 0; pb < 4; ++pb)
    rhs[pb] = mfma32(lds_operand32<kOpStride>(sm.at, 16 * pb + n, 0, g), s01, zero4());
#pragma unroll
  for (int pb = 0; pb < 4; ++pb)
    rhs[pb] = mfma32(lds_operand32<kOpStride>(sm.at, 16 * pb + n, 32, g), s23, rhs[pb]);
  rhs[0] = mfma32(lo32(L(kLak, 0, 0)), lo32(vs[0]), rhs[0]);
  rhs[1] = mfma32(cat(L(kLak, 1, 0), L(kLak, 1, 1)), v01, rhs[1]);
  rhs[2] = mfma32(cat(L(kLak, 2, 0), L(kLak, 2, 1)), v01, rhs[2]);
  rhs[3] = mfma32(cat(L(kLak, 3, 0), L(kLak, 3, 1)), v01, rhs[3]);
  rhs[2] = mfma32(lo32(L(kLak, 2, 2)), lo32(vs[2]), rhs[2]);
  rhs[3] = mfma32(cat(L(kLak, 3, 2), L(kLak, 3, 3)), v23, rhs[3]);
  auto Tm = [&](int pb) { return lds_operand<kTriStride>(sm.u.f.tinv[pb], n, 4 * g); };
  sa[0] = mfma32(lo32(Tm(0)), lo32(to_operand(rhs[0])), zero4());
  sab[0] = to_operand(sa[0]);
  rhs[1] = mfma32(lo32(L(kLab, 1, 0)), lo32(sab[0]), rhs[1]);
  sa[1] = mfma32(lo32(Tm(1)), lo32(to_operand(rhs[1])), zero4());
  sab[1] = to_operand(sa[1]);
  const i16x8 sa01 = cat(sab[0], sab[1]);
  rhs[2] = mfma32(cat(L(kLab, 2, 0), L(kLab, 2, 1)), sa01, rhs[2]);
  rhs[3] = mfma32(cat(L(kLab, 3, 0), L(kLab, 3, 1)), sa01, rhs[3]);
  sa[2] = mfma32(lo32(Tm(2)), lo32(to_operand(rhs[2])), zero4());
  sab[2] = to_operand(sa[2]);
  rhs[3] = mfma32(lo32(L(kLab, 3, 2)), lo32(sab[2]), rhs[3]);
  sa[3] = mfma32(lo32(Tm(3)), lo32(to_operand(rhs[3])), zero4());
  sab[3] = to_operand(sa[3]);
}

// State after the prepared range: S' = diag(2^GC) (S0 + Bh^T SA + Kh^T V).
__device__ __forceinline__ void state_step(const BwdSmem& sm, f32x4 (&S)[4], int g, int n,
                                           const i16x4 (&sab)[4], const i16x4 (&vs)[4]) {
  g = (lane_tid() & 63) >> 4;
  n = lane_tid() & 15;
  const i16x8 sa01 = cat(sab[0], sab[1]), sa23 = cat(sab[2], sab[3]);
  const i16x8 v01 = cat(vs[0], vs[1]), v23 = cat(vs[2], vs[3]);
  f32x4 sn[4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) sn[kb] = mfma32(tr32<kOpStride>(sm.bh, 0, 16 * kb, g, n), sa01, S[kb]);
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) sn[kb] = mfma32(tr32<kOpStride>(sm.bh, 32, 16 * kb, g, n), sa23, sn[kb]);
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) sn[kb] = mfma32(tr32<kOpStride>(sm.kh, 0, 16 * kb, g, n), v01, sn[kb]);
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) sn[kb] = mfma32(tr32<kOpStride>(sm.kh, 32, 16 * kb, g, n), v23, sn[kb]);
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    const float4 gc4 = *reinterpret_cast<const float4*>(&sm.gc[16 * kb + 4 * g]);
    S[kb][0] = sn[kb][0] * gc4.x;
    S[kb][1] = sn[kb][1] * gc4.y;
    S[kb][2] = sn[kb][2] * gc4.z;
    S[kb][3] = sn[kb][3] * gc4.w;
  }
}

// Adjoint chain of value columns 16 cs .. 16 cs + 15, first part: dSA, dZ
// (written to the dz tile and returned as operands), the partial dg of these
// columns, and dS0 without its dZ term (ds0). S0 is the piece-start state
// slab (fp32, C layout). adjoint_finish completes dS0 after the columns
// phase's mid barrier; the forward waves form dV meanwhile (dv_partial,
// dv_finish).
template <typename T>
__device__ __forceinline__ void adjoint_chain(BwdSmem& sm, const f32x4 (&S0)[4], int cs, int g,
                                              int n, int lane, f32x4 (&ds0)[4], i16x8& dz01,
                                              i16x8& dz23) {
  lane = lane_tid() & 63;
  g = lane >> 4;
  n = lane & 15;
  f32x4 dS[4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) dS[kb] = sm.dstash[cs][kb][lane];
  i16x4 dys[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) dys[q] = lds_operand_tr<kOpStride>(sm.dy, 16 * q, 16 * cs, g, n);
  auto L = [&](int m, int p, int q) {  // block (p, q) as stored: [t][i]
    return lds_operand<kTriStride>(tri_blk(sm.u.f.tri[m], p, q), n, 4 * g);
  };
  auto Lt = [&](int m, int p, int q) {  // block (p, q) transposed: [i][t]
    return lds_operand_tr<kTriStride>(tri_blk(sm.u.f.tri[m], p, q), 0, 0, g, n);
  };

  // g o dS (operand over keys) and the partial rowsums of S0 o dS; the dS
  // tile [v][k] for the tokens phase.
  i16x4 gds[4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    const float4 gc4 = *reinterpret_cast<const float4*>(&sm.gc[16 * kb + 4 * g]);
    const float gcv[4] = {gc4.x, gc4.y, gc4.z, gc4.w};
    f32x4 x;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[j] = gcv[j] * dS[kb][j];
      const float s = suffix16(S0[kb][j] * dS[kb][j]);
      if (n == 0) sm.dgam[cs][16 * kb + 4 * g + j] = s;
    }
    gds[kb] = to_operand(x);
    lds_store_transposed(sm.ds + (16 * cs) * kOpStride + 16 * kb, kOpStride, g, n, dS[kb]);
  }
  const i16x8 gds01 = cat(gds[0], gds[1]), gds23 = cat(gds[2], gds[3]);
  const i16x8 dy01 = cat(dys[0], dys[1]), dy23 = cat(dys[2], dys[3]);

  // dSA_p = Bh_p (g o dS) + sum_{q>=p} Arb^T(q, p) dYs_q.
  f32x4 dsa[4];
#pragma unroll
  for (int pb = 0; pb < 4; ++pb)
    dsa[pb] = mfma32(lds_operand32<kOpStride>(sm.bh, 16 * pb + n, 0, g), gds01, zero4());
#pragma unroll
  for (int pb = 0; pb < 4; ++pb)
    dsa[pb] = mfma32(lds_operand32<kOpStride>(sm.bh, 16 * pb + n, 32, g), gds23, dsa[pb]);
  dsa[0] = mfma32(cat(Lt(kArb, 0, 0), Lt(kArb, 1, 0)), dy01, dsa[0]);
  dsa[0] = mfma32(cat(Lt(kArb, 2, 0), Lt(kArb, 3, 0)), dy23, dsa[0]);
  dsa[1] = mfma32(lo32(Lt(kArb, 1, 1)), lo32(dys[1]), dsa[1]);
  dsa[1] = mfma32(cat(Lt(kArb, 2, 1), Lt(kArb, 3, 1)), dy23, dsa[1]);
  dsa[2] = mfma32(cat(Lt(kArb, 2, 2), Lt(kArb, 3, 2)), dy23, dsa[2]);
  dsa[3] = mfma32(lo32(Lt(kArb, 3, 3)), lo32(dys[3]), dsa[3]);

  // The part of dS0 that does not need dZ first, so its products fill the
  // latencies of the dZ chain: dS0 <- g o dS + Rt^T dYs.
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    const float4 gc4 = *reinterpret_cast<const float4*>(&sm.gc[16 * kb + 4 * g]);
    f32x4 acc = {gc4.x * dS[kb][0], gc4.y * dS[kb][1], gc4.z * dS[kb][2], gc4.w * dS[kb][3]};
    acc = mfma32(tr32<kOpStride>(sm.rt, 0, 16 * kb, g, n), dy01, acc);
    ds0[kb] = mfma32(tr32<kOpStride>(sm.rt, 32, 16 * kb, g, n), dy23, acc);
  }

  // dZ = T^T dSA: dZ_p = T_pp^T (dSA_p + sum_{q>p} Lab^T(q, p) dZ_q).
  auto Tt = [&](int pb) {
    return lds_operand_tr<kTriStride>(sm.u.f.tinv[pb], 0, 0, g, n);
  };
  f32x4 dz[4];
  i16x4 dzb[4];
  dz[3] = mfma32(lo32(Tt(3)), lo32(to_operand(dsa[3])), zero4());
  dzb[3] = to_operand(dz[3]);
  dsa[2] = mfma32(lo32(Lt(kLab, 3, 2)), lo32(dzb[3]), dsa[2]);
  dz[2] = mfma32(lo32(Tt(2)), lo32(to_operand(dsa[2])), zero4());
  dzb[2] = to_operand(dz[2]);
  dz23 = cat(dzb[2], dzb[3]);
  dsa[1] = mfma32(cat(Lt(kLab, 2, 1), Lt(kLab, 3, 1)), dz23, dsa[1]);
  dsa[0] = mfma32(cat(Lt(kLab, 2, 0), Lt(kLab, 3, 0)), dz23, dsa[0]);
  dz[1] = mfma32(lo32(Tt(1)), lo32(to_operand(dsa[1])), zero4());
  dzb[1] = to_operand(dz[1]);
  dsa[0] = mfma32(lo32(Lt(kLab, 1, 0)), lo32(dzb[1]), dsa[0]);
  dz[0] = mfma32(lo32(Tt(0)), lo32(to_operand(dsa[0])), zero4());
  dzb[0] = to_operand(dz[0]);
  dz01 = cat(dzb[0], dzb[1]);
#pragma unroll
  for (int pb = 0; pb < 4; ++pb)
    lds_store_rows(sm.dz + (16 * pb) * kOpStride + 16 * cs, kOpStride, g, n, dz[pb]);
}

// Second part, after the mid barrier: dS0 = g o dS + Rt^T dYs + At^T dZ into
// the stash (dS for the range before).
__device__ __forceinline__ void adjoint_finish(BwdSmem& sm, int cs, f32x4 (&ds0)[4],
                                               const i16x8& dz01, const i16x8& dz23) {
  const int lane = lane_tid() & 63;
  const int g = lane >> 4, n = lane & 15;
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    f32x4 acc = mfma32(tr32<kOpStride>(sm.at, 0, 16 * kb, g, n), dz01, ds0[kb]);
    acc = mfma32(tr32<kOpStride>(sm.at, 32, 16 * kb, g, n), dz23, acc);
    sm.dstash[cs][kb][lane] = acc;
  }
}

// dV^T of value columns 16 cs .. 16 cs + 15 on the forward waves (lane (g, n)
// ends with dV[16 pb + n][16 cs + 4g .. +3]). dv_partial, before the mid
// barrier: the terms without dZ, (g o dS)^T Kh^T + sum_{q>=pb} dYs_q^T
// Ark(q, pb), with dS read from the adjoint waves' stash (same slab and lane,
// read before they overwrite it). dv_finish, after it: the dZ terms
// sum_{q>=pb} dZ_q^T Lak(q, pb) from the dz tile, then the dv tile.
__device__ __forceinline__ void dv_partial(const BwdSmem& sm, int cs, f32x4 (&dvt)[4]) {
  const int lane = lane_tid() & 63;
  const int g = lane >> 4, n = lane & 15;
  i16x4 gds[4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    const f32x4 dS = sm.dstash[cs][kb][lane];
    const float4 gc4 = *reinterpret_cast<const float4*>(&sm.gc[16 * kb + 4 * g]);
    f32x4 x;
    x[0] = gc4.x * dS[0];
    x[1] = gc4.y * dS[1];
    x[2] = gc4.z * dS[2];
    x[3] = gc4.w * dS[3];
    gds[kb] = to_operand(x);
  }
  const i16x8 gds01 = cat(gds[0], gds[1]), gds23 = cat(gds[2], gds[3]);
  i16x4 dys[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) dys[q] = lds_operand_tr<kOpStride>(sm.dy, 16 * q, 16 * cs, g, n);
  const i16x8 dy01 = cat(dys[0], dys[1]), dy23 = cat(dys[2], dys[3]);
  auto Lb = [&](int m, int q, int pb) {  // B[k = t][n = i] = M[t][i] of block (q, pb)
    return lds_operand_tr<kTriStride>(tri_blk(sm.u.f.tri[m], q, pb), 0, 0, g, n);
  };
#pragma unroll
  for (int pb = 0; pb < 4; ++pb)
    dvt[pb] = mfma32(gds01, lds_operand32<kOpStride>(sm.kh, 16 * pb + n, 0, g), zero4());
#pragma unroll
  for (int pb = 0; pb < 4; ++pb)
    dvt[pb] = mfma32(gds23, lds_operand32<kOpStride>(sm.kh, 16 * pb + n, 32, g), dvt[pb]);
  dvt[0] = mfma32(dy01, cat(Lb(kArk, 0, 0), Lb(kArk, 1, 0)), dvt[0]);
  dvt[0] = mfma32(dy23, cat(Lb(kArk, 2, 0), Lb(kArk, 3, 0)), dvt[0]);
  dvt[1] = mfma32(lo32(dys[1]), lo32(Lb(kArk, 1, 1)), dvt[1]);
  dvt[1] = mfma32(dy23, cat(Lb(kArk, 2, 1), Lb(kArk, 3, 1)), dvt[1]);
  dvt[2] = mfma32(dy23, cat(Lb(kArk, 2, 2), Lb(kArk, 3, 2)), dvt[2]);
  dvt[3] = mfma32(lo32(dys[3]), lo32(Lb(kArk, 3, 3)), dvt[3]);
}

template <typename T>
__device__ __forceinline__ void dv_finish(BwdSmem& sm, int cs, f32x4 (&dvt)[4]) {
  const int lane = lane_tid() & 63;
  const int g = lane >> 4, n = lane & 15;
  i16x4 dzb[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) dzb[q] = lds_operand_tr<kOpStride>(sm.dz, 16 * q, 16 * cs, g, n);
  const i16x8 dz01 = cat(dzb[0], dzb[1]), dz23 = cat(dzb[2], dzb[3]);
  auto Lb = [&](int m, int q, int pb) {
    return lds_operand_tr<kTriStride>(tri_blk(sm.u.f.tri[m], q, pb), 0, 0, g, n);
  };
  dvt[0] = mfma32(dz01, cat(Lb(kLak, 0, 0), Lb(kLak, 1, 0)), dvt[0]);
  dvt[0] = mfma32(dz23, cat(Lb(kLak, 2, 0), Lb(kLak, 3, 0)), dvt[0]);
  dvt[1] = mfma32(lo32(dzb[1]), lo32(Lb(kLak, 1, 1)), dvt[1]);
  dvt[1] = mfma32(dz23, cat(Lb(kLak, 2, 1), Lb(kLak, 3, 1)), dvt[1]);
  dvt[2] = mfma32(dz23, cat(Lb(kLak, 2, 2), Lb(kLak, 3, 2)), dvt[2]);
  dvt[3] = mfma32(lo32(dzb[3]), lo32(Lb(kLak, 3, 3)), dvt[3]);
#pragma unroll
  for (int pb = 0; pb < 4; ++pb) {
    uint2 q;
    q.x = pack2<T>(dvt[pb][0], dvt[pb][1]);
    q.y = pack2<T>(dvt[pb][2], dvt[pb][3]);
    *reinterpret_cast<uint2*>(sm.dv + (16 * pb + n) * kOpStride + 16 * cs + 4 * g) = q;
  }
}

// The four gradient matrices, 40 (matrix, block) items: M[t][i] = sum_v
// X[t][v] Y[i][v] (X = dYs or dZ, Y = SA or V, all four [t][v] tiles),
// computed as M^T in C layout and stored [t][i]. Wave w takes matrix w / 2
// and the block rows {3, 0} (w even) or {2, 1} (w odd): five blocks, whose
// operands are two row blocks of X and the four (three) row blocks of Y, each
// read from LDS once (6 or 5 operand reads for 5 products, instead of 10).
// Ends with a barrier.
__device__ __forceinline__ void gradient_matrices(BwdSmem& sm) {
  const int tid = lane_tid();
  const int wave = uniform(tid >> 6);
  const int lane = tid & 63;
  const int g = lane >> 4, n = lane & 15;
  const int m = wave >> 1;  // kGArb, kGArk, kGLab, kGLak
  const bool odd = (wave & 1) != 0;
  const bool from_dz = m >= 2;
  const uint16_t* xt = from_dz ? sm.dz : sm.dy;
  const uint16_t* yt = (m & 1) != 0 ? sm.vv : sm.sa;
  const int pa = odd ? 2 : 3, pz = odd ? 1 : 0;
  __builtin_amdgcn_s_setprio(1);
  i16x8 xa[2], xz[2], y[4][2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    xa[h] = lds_operand32<kOpStride>(xt, 16 * pa + n, 32 * h, g);
    xz[h] = lds_operand32<kOpStride>(xt, 16 * pz + n, 32 * h, g);
#pragma unroll
    for (int q = 0; q < 4; ++q) y[q][h] = lds_operand32<kOpStride>(yt, 16 * q + n, 32 * h, g);
  }
  auto block = [&](const i16x8 (&x)[2], int pb, int q) {
    f32x4 mt = mfma32(y[q][0], x[0], zero4());  // lane (g, n): M[16 pb + n][16 q + 4g + j]
    mt = mfma32(y[q][1], x[1], mt);
    if (pb == q) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int ii = 4 * g + j;
        mt[j] = (from_dz ? (ii < n) : (ii <= n)) ? mt[j] : 0.0f;
      }
    }
    lds_store_transposed(sm.u.grad[m] + tri_index(pb, q) * kTriBlock, kTriStride, g, n, mt);
  };
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    if (q <= pa) block(xa, pa, q);
  }
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    if (q <= pz) block(xz, pz, q);
  }
  __builtin_amdgcn_s_setprio(0);
  __syncthreads();
}

// One backward step over the prepared range [lo, hi) of a piece, after
// prepare and intra: columns, matrices and the token gradients (stored for
// tokens in the range only). S0 is the state at the range start (C layout);
// The adjoint waves' dS (in the LDS stash) is the adjoint at the range end on
// entry and at its start on return.
template <typename T, DecayMode M>
__device__ void run_backward_step(BwdSmem& sm, const ChunkBwdParams& p, const TokRows& cur,
                                  const uint4& bias, const f32x4 (&S0)[4], int lo, int hi,
                                  const Piece& pc, int heads, int head, uint32_t row_bytes,
                                  uint32_t tok_off) {
  const int tid = lane_tid();
  const int wave = uniform(tid >> 6);
  const int lane = tid & 63;
  const int g = lane >> 4, n = lane & 15;
  const int pt = wave & 3, hf = wave >> 2;
  const int cs = wave & 3;
  const int t = 16 * pt + n;
  const int f0 = 32 * hf + 8 * g;
  const bool on = t >= lo && t < hi;

  // ---------------------------------------------------------- columns --
  // Two parts around a mid barrier. Forward waves: the SA chain and the
  // dZ-free part of dV, then dV's dZ terms. Adjoint waves: dSA, the dZ chain
  // (dz tile) and dS0 without its dZ term, then that term. The adjoint
  // waves' dZ chain is the phase's critical path: they run at a higher wave
  // priority than the forward waves sharing their SIMDs.
  if (wave < 4) {
    __builtin_amdgcn_s_setprio(1);
  } else {
    __builtin_amdgcn_s_setprio(2);
  }
  f32x4 dvt[4], ds0[4];
  i16x8 dz01, dz23;
  if (wave < 4) {
    f32x4 sa[4];
    i16x4 sab[4], vs[4];
    sa_chain(sm, S0, cs, g, n, sa, sab, vs);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      lds_store_rows(sm.sa + (16 * q) * kOpStride + 16 * cs, kOpStride, g, n, sa[q]);
      lds_store_transposed(sm.s0 + (16 * cs) * kOpStride + 16 * q, kOpStride, g, n, S0[q]);
    }
    dv_partial(sm, cs, dvt);
  } else {
    adjoint_chain<T>(sm, S0, cs, g, n, lane, ds0, dz01, dz23);
  }
  __syncthreads();
  if (wave < 4) {
    dv_finish<T>(sm, cs, dvt);
  } else {
    adjoint_finish(sm, cs, ds0, dz01, dz23);
  }
  __builtin_amdgcn_s_setprio(0);
  __syncthreads();

  // --------------------------------------------------------- matrices --
  gradient_matrices(sm);

  // ----------------------------------------------------------- tokens --
  // Two passes that share no operand: pass A forms dRt, dAt (products with
  // S0, Bh^T, Kh^T), pass B dBc = dBh + g dBt and dKc = dKh + g dKt (products
  // with dS, At^T, Rt^T), each for both of the lane's feature quarters u
  // (features f0 + 4u .. +3). Only one pass's accumulators are live at a time.
  auto Gf = [&](int m, int pp, int q) {  // B[k = i][n = t]: block (pp, q) as stored
    return lds_operand<kTriStride>(tri_blk(sm.u.grad[m], pp, q), n, 4 * g);
  };
  auto Gt = [&](int m, int pp, int q) {  // B[k = t][n = i]: block (pp, q) transposed
    return lds_operand_tr<kTriStride>(tri_blk(sm.u.grad[m], pp, q), 0, 0, g, n);
  };
  // Feature e of a packed row of 8 io values.
  auto raw = [](const uint4& q, int e) {
    const uint32_t word = e < 2 ? q.x : e < 4 ? q.y : e < 6 ? q.z : q.w;
    return to_f32<T>(static_cast<uint16_t>((e & 1) ? (word >> 16) : (word & 0xffffu)));
  };
  // Four bf16 of the lane's own tile row (token t, features fb .. fb + 3):
  // the decay gradient's terms take At, Rt, Bh, Kh as prepared.
  auto tile4 = [&](const uint16_t* tile, int fb) {
    return *reinterpret_cast<const uint2*>(tile + t * kOpStride + fb);
  };
  auto half = [](const uint2& q, int j) {
    const uint32_t w = j < 2 ? q.x : q.y;
    return bf16_float(static_cast<uint16_t>((j & 1) ? (w >> 16) : (w & 0xffffu)));
  };
  // Packed gradient words (two features each) and, per feature, the decay
  // gradient's in-block suffix sum of e1 + e2 minus e2.
  uint32_t wr[4], wa[4], wb[4], wk[4];
  float sfx[8];
  // Decay factors of the lane's 8 features, recomputed exactly as in
  // prepare: the row's product scan times the earlier blocks' products.
  float up[8], upp[8];
  {
    float carry[8] = {1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 1.0f};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (q < pt) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const float4 c = *reinterpret_cast<const float4*>(&sm.blk[q][f0 + 4 * u]);
          carry[4 * u + 0] *= c.x;
          carry[4 * u + 1] *= c.y;
          carry[4 * u + 2] *= c.z;
          carry[4 * u + 3] *= c.w;
        }
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float xin = raw(cur.w, e);
      if constexpr (M == DecayMode::kLogits) xin += raw(bias, e);
      const float wv = on ? clamped_retention<M>(xin) : 1.0f;
      // Both scans run in every lane: the lane before the first one of a
      // sub-piece range holds the empty product that the exclusive scan reads.
      const float Gi = prefix16_mul(wv, n);
      const float Ge = exclusive16(Gi, n);
      up[e] = on ? Gi * carry[e] : 0.0f;
      upp[e] = on ? Ge * carry[e] : 0.0f;
    }
  }
  // Both feature quarters u (features f0 + 4u .. +3) in each pass: the
  // operands that do not depend on u (dYs, dZ, SA, V rows and the gradient
  // blocks) are read once for both.
  float e12[8];
  // (No raised wave priority here, unlike the other MFMA phases: with all
  // eight waves in this phase at once it made the kernel 1.5% slower.)
  // ---- pass A: dRt = dYs S0^T + dArb Bh + dArk Kh, dAt = dZ S0^T + dLab Bh + dLak Kh.
  {
    f32x4 acc_r[2] = {zero4(), zero4()}, acc_a[2] = {zero4(), zero4()};
#pragma unroll
    for (int c = 0; c < 64; c += 32) {
      const i16x8 dyo = lds_operand32<kOpStride>(sm.dy, t, c, g);
      const i16x8 dzo = lds_operand32<kOpStride>(sm.dz, t, c, g);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const i16x8 s0a = tr32_q8<kOpStride>(sm.s0, c, 32 * hf + 4 * u, g, n);
        acc_r[u] = mfma32(s0a, dyo, acc_r[u]);
        acc_a[u] = mfma32(s0a, dzo, acc_a[u]);
      }
    }
    // Source blocks q <= pt: A = Bh^T / Kh^T (rows: features), B = the
    // gradient blocks (pt, q) as stored.
    auto src = [&](int q, bool pair) {
      auto gb = [&](int m) {
        return pair ? cat(Gf(m, pt, q), Gf(m, pt, q + 1)) : lo32(Gf(m, pt, q));
      };
      const i16x8 g_arb = gb(kGArb), g_ark = gb(kGArk), g_lab = gb(kGLab), g_lak = gb(kGLak);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int c0 = 32 * hf + 4 * u;
        const i16x8 bq = pair ? cat(lds_tr_q8<kOpStride>(sm.bh, 16 * q, c0, g, n),
                                    lds_tr_q8<kOpStride>(sm.bh, 16 * q + 16, c0, g, n))
                              : lo32(lds_tr_q8<kOpStride>(sm.bh, 16 * q, c0, g, n));
        const i16x8 kq = pair ? cat(lds_tr_q8<kOpStride>(sm.kh, 16 * q, c0, g, n),
                                    lds_tr_q8<kOpStride>(sm.kh, 16 * q + 16, c0, g, n))
                              : lo32(lds_tr_q8<kOpStride>(sm.kh, 16 * q, c0, g, n));
        acc_r[u] = mfma32(bq, g_arb, acc_r[u]);
        acc_r[u] = mfma32(kq, g_ark, acc_r[u]);
        acc_a[u] = mfma32(bq, g_lab, acc_a[u]);
        acc_a[u] = mfma32(kq, g_lak, acc_a[u]);
      }
    };
    if (pt == 0) {
      src(0, false);
    } else if (pt == 1) {
      src(0, true);
    } else if (pt == 2) {
      src(0, true);
      src(2, false);
    } else {
      src(0, true);
      src(2, true);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int fb = f0 + 4 * u;
      const uint2 rt4 = tile4(sm.rt, fb), at4 = tile4(sm.at, fb);
      float gr4[4], ga4[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int e = 4 * u + jj;
        gr4[jj] = acc_r[u][jj] * up[e];
        ga4[jj] = acc_a[u][jj] * upp[e];
        const float e2 = acc_a[u][jj] * half(at4, jj);
        e12[e] = acc_r[u][jj] * half(rt4, jj) + e2;
        sfx[e] = -e2;
      }
      wr[2 * u] = pack2<T>(gr4[0], gr4[1]);
      wr[2 * u + 1] = pack2<T>(gr4[2], gr4[3]);
      wa[2 * u] = pack2<T>(ga4[0], ga4[1]);
      wa[2 * u + 1] = pack2<T>(ga4[2], ga4[3]);
    }
  }
  // Token rows of the piece: the buffer range ends at its last token; inside
  // the piece only tokens of [lo, hi) are written.
  using S16 = typename IoTraits<T>::storage;
  auto rsrc = [&](void* x) {
    return buffer_rsrc(static_cast<S16*>(x) + (static_cast<int64_t>(pc.c0) * heads + head) * kHead,
                       static_cast<uint32_t>(pc.ntok) * row_bytes);
  };
  // Lanes of tokens outside [lo, hi) store to kDropOffset (dropped): no
  // branch, so every pass issues the same stores and the compiler's in-order
  // wait counts for the next piece's row loads stay exact.
  const uint32_t st_off = on ? tok_off : kDropOffset;
  __builtin_amdgcn_raw_buffer_store_b128(u32x4{wr[0], wr[1], wr[2], wr[3]}, rsrc(args().dr),
                                         st_off, 0, 0);
  __builtin_amdgcn_raw_buffer_store_b128(u32x4{wa[0], wa[1], wa[2], wa[3]}, rsrc(args().da),
                                         st_off, 0, 0);
  {
    const uint2 d0 = *reinterpret_cast<const uint2*>(sm.dv + t * kOpStride + f0);
    const uint2 d1 = *reinterpret_cast<const uint2*>(sm.dv + t * kOpStride + f0 + 4);
    __builtin_amdgcn_raw_buffer_store_b128(u32x4{d0.x, d0.y, d1.x, d1.y}, rsrc(args().dv), st_off,
                                           0, 0);
  }

  // ---- pass B: dBc = dLab^T At + dArb^T Rt + g (SA dS^T), dKc likewise
  // with dLak, dArk and V.
  {
    f32x4 acc_b[2] = {zero4(), zero4()}, acc_k[2] = {zero4(), zero4()};
    f32x4 acc_bt[2] = {zero4(), zero4()}, acc_kt[2] = {zero4(), zero4()};
#pragma unroll
    for (int c = 0; c < 64; c += 32) {
      const i16x8 sao = lds_operand32<kOpStride>(sm.sa, t, c, g);
      const i16x8 vvo = lds_operand32<kOpStride>(sm.vv, t, c, g);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const i16x8 dsa = tr32_q8<kOpStride>(sm.ds, c, 32 * hf + 4 * u, g, n);
        acc_bt[u] = mfma32(dsa, sao, acc_bt[u]);
        acc_kt[u] = mfma32(dsa, vvo, acc_kt[u]);
      }
    }
    // Target blocks qt >= pt: A = At^T / Rt^T, B = the gradient blocks
    // (qt, pt) transposed.
    auto dst = [&](int qt, bool pair) {
      auto gb = [&](int m) {
        return pair ? cat(Gt(m, qt, pt), Gt(m, qt + 1, pt)) : lo32(Gt(m, qt, pt));
      };
      const i16x8 g_lab = gb(kGLab), g_arb = gb(kGArb), g_lak = gb(kGLak), g_ark = gb(kGArk);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int c0 = 32 * hf + 4 * u;
        const i16x8 aq = pair ? cat(lds_tr_q8<kOpStride>(sm.at, 16 * qt, c0, g, n),
                                    lds_tr_q8<kOpStride>(sm.at, 16 * qt + 16, c0, g, n))
                              : lo32(lds_tr_q8<kOpStride>(sm.at, 16 * qt, c0, g, n));
        const i16x8 rq = pair ? cat(lds_tr_q8<kOpStride>(sm.rt, 16 * qt, c0, g, n),
                                    lds_tr_q8<kOpStride>(sm.rt, 16 * qt + 16, c0, g, n))
                              : lo32(lds_tr_q8<kOpStride>(sm.rt, 16 * qt, c0, g, n));
        acc_b[u] = mfma32(aq, g_lab, acc_b[u]);
        acc_b[u] = mfma32(rq, g_arb, acc_b[u]);
        acc_k[u] = mfma32(aq, g_lak, acc_k[u]);
        acc_k[u] = mfma32(rq, g_ark, acc_k[u]);
      }
    };
    if (pt == 0) {
      dst(0, true);
      dst(2, true);
    } else if (pt == 1) {
      dst(1, false);
      dst(2, true);
    } else if (pt == 2) {
      dst(2, true);
    } else {
      dst(3, false);
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int fb = f0 + 4 * u;
      const float4 gc4 = *reinterpret_cast<const float4*>(&sm.gc[fb]);
      const float gcv[4] = {gc4.x, gc4.y, gc4.z, gc4.w};
      const uint2 bh4 = tile4(sm.bh, fb), kh4 = tile4(sm.kh, fb);
      float gb4[4], gk4[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int e = 4 * u + jj;
        const float dn = on ? __builtin_amdgcn_rcpf(up[e]) : 0.0f;
        const float dBc = acc_b[u][jj] + gcv[jj] * acc_bt[u][jj];
        const float dKc = acc_k[u][jj] + gcv[jj] * acc_kt[u][jj];
        gb4[jj] = dn * dBc;
        gk4[jj] = dn * dKc;
        const float bh_v = half(bh4, jj), kh_v = half(kh4, jj);
        const float suf = suffix16(e12[e] - dBc * bh_v - dKc * kh_v);
        const float tot3 = suffix16(gcv[jj] * (acc_bt[u][jj] * bh_v + acc_kt[u][jj] * kh_v));
        sfx[e] += suf;
        if (n == 0) {
          sm.car1[pt][fb + jj] = suf;
          sm.car3[pt][fb + jj] = tot3;
        }
      }
      wb[2 * u] = pack2<T>(gb4[0], gb4[1]);
      wb[2 * u + 1] = pack2<T>(gb4[2], gb4[3]);
      wk[2 * u] = pack2<T>(gk4[0], gk4[1]);
      wk[2 * u + 1] = pack2<T>(gk4[2], gk4[3]);
    }
  }

  __builtin_amdgcn_raw_buffer_store_b128(u32x4{wb[0], wb[1], wb[2], wb[3]}, rsrc(args().db),
                                         st_off, 0, 0);
  __builtin_amdgcn_raw_buffer_store_b128(u32x4{wk[0], wk[1], wk[2], wk[3]}, rsrc(args().dk),
                                         st_off, 0, 0);
  __syncthreads();  // block carries of the decay gradient

  float dw[8];
#pragma unroll
  for (int h4 = 0; h4 < 2; ++h4) {
    const int fb = f0 + 4 * h4;
    float4 later = make_float4(0.f, 0.f, 0.f, 0.f), all3 = later, dgam = later;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 c1 = *reinterpret_cast<const float4*>(&sm.car1[q][fb]);
      const float4 c3 = *reinterpret_cast<const float4*>(&sm.car3[q][fb]);
      const float4 dg = *reinterpret_cast<const float4*>(&sm.dgam[q][fb]);
      if (q > pt) {
        later.x += c1.x; later.y += c1.y; later.z += c1.z; later.w += c1.w;
      }
      all3.x += c3.x; all3.y += c3.y; all3.z += c3.z; all3.w += c3.w;
      dgam.x += dg.x; dgam.y += dg.y; dgam.z += dg.z; dgam.w += dg.w;
    }
    const float4 gc4 = *reinterpret_cast<const float4*>(&sm.gc[fb]);
    const float lat[4] = {later.x, later.y, later.z, later.w};
    const float a3[4] = {all3.x, all3.y, all3.z, all3.w};
    const float dgv[4] = {dgam.x, dgam.y, dgam.z, dgam.w};
    const float gcv[4] = {gc4.x, gc4.y, gc4.z, gc4.w};
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int e = 4 * h4 + jj;
      const float dlg = sfx[e] + lat[jj] + a3[jj] + dgv[jj] * gcv[jj];
      float xin = raw(cur.w, e);
      if constexpr (M == DecayMode::kLogits) {
        xin += raw(bias, e);
        const float sig = __builtin_amdgcn_rcpf(1.0f + fast_exp2(-kLog2E * xin));
        dw[e] = dlg * (-kExpNegHalf) * sig * (1.0f - sig);
      } else {
        // log2 w is clamped to [-20, 0]: zero derivative for w outside [2^-20, 1].
        dw[e] = (xin < 0x1p-20f || xin > 1.0f) ? 0.0f : dlg * __builtin_amdgcn_rcpf(xin);
      }
    }
  }
  __builtin_amdgcn_raw_buffer_store_b128(pack8<T>(dw), rsrc(args().ddecay), st_off, 0, 0);
}

// kDense: the pretraining layout (dense_t > 0), a separate instantiation so
// that the StateTune path's piece walk carries no dense-layout branches (18
// fewer SGPRs spilled to VGPR lanes; 2% faster at config 4, same bits).
template <typename T, DecayMode M, bool kDense>
__global__ __launch_bounds__(kBwdThreads, 1) void chunk_bwd_kernel(ChunkBwdParams p) {
  __shared__ BwdSmem sm;

  const int tid = lane_tid();
  const int wave = uniform(tid >> 6);
  const int lane = tid & 63;
  const int g = lane >> 4, n = lane & 15;
  const int pt = wave & 3, hf = wave >> 2;  // token layout: block, feature half
  const int cs = wave & 3;                  // column slab (columns phase)
  const bool adjoint = wave >= 4;
  const int heads = p.num_heads;
  const int seq = blockIdx.x / heads;
  const int head = blockIdx.x % heads;
  const int f0 = 32 * hf + 8 * g;
  constexpr bool dense = kDense;
  const int seg_lo = dense ? 0 : uniform(max(p.seg_offsets[seq], 0));
  const int seg_hi = dense ? 1 : uniform(min(p.seg_offsets[seq + 1], p.num_segments));

  // Decay bias of the lane's 8 features, packed (zero: no bias).
  uint4 bias = make_uint4(0u, 0u, 0u, 0u);
  if constexpr (M == DecayMode::kLogits) {
    if (p.bias != nullptr) bias = load_row8<T>(p.bias, static_cast<int64_t>(head) * kHead + f0);
  }

  const uint32_t row_bytes = static_cast<uint32_t>(heads) * kHead * 2;
  // Lane's byte offset in a piece's rows (token 16 pt + n, features f0 ..).
  const uint32_t tok_off = static_cast<uint32_t>(16 * pt + n) * row_bytes + 2 * f0;
  // State slab (columns 16 cs ..): element (row, col) of a 64 x 64 fp32
  // state at byte 4 (64 row + col); lane (g, n) holds rows 16 kb + 4g + j.
  const uint32_t s_off = static_cast<uint32_t>((4 * g) * kHead + 16 * cs + n) * 4;
  const int64_t unit_state = (static_cast<int64_t>(seq) * heads + head) * kHead * kHead;

  // dS: dL/dS at the end of the current piece, kept by the adjoint waves in
  // the LDS stash (each lane reads back only what it wrote).
  if (adjoint) {
    const auto rs = buffer_rsrc(p.dstate_final != nullptr ? p.dstate_final + unit_state : nullptr,
                                p.dstate_final != nullptr ? kHead * kHead * 4 : 0);
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      f32x4 x;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        x[j] = __uint_as_float(
            __builtin_amdgcn_raw_buffer_load_b32(rs, s_off, (16 * kb + j) * kHead * 4, 0));
      sm.dstash[cs][kb][lane] = x;
    }
  }
  bool failed = false;

  // Segment bounds, 64 segments at a time in VGPR lanes, read back with
  // readlane (a per-segment memory read would need a vmcnt wait, which on
  // gfx9's in-order counter also waits for every gradient store in flight).
  int cache_base = seg_hi;
  int starts_v = 0, ends_v = 0;
  auto seg_bounds = [&](int seg, int& tb, int& te) {
    if (dense) {
      tb = seq * p.dense_t;
      te = tb + p.dense_t;
      return;
    }
    if (seg < cache_base) {
      cache_base = uniform(max(seg - 63, seg_lo));
      const int idx = cache_base + lane;
      starts_v = idx <= seg ? args().seg_starts[idx] : 0;
      ends_v = idx <= seg ? args().seg_ends[idx] : 0;
      __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt(0)
    }
    tb = uniform(max(__builtin_amdgcn_readlane(starts_v, seg - cache_base), 0));
    te = uniform(min(__builtin_amdgcn_readlane(ends_v, seg - cache_base), p.total_tokens));
  };
  auto piece_of = [&](int seg, int tb, int te, int j) {
    Piece pc;
    pc.c0 = tb + kChunk * j;
    pc.ntok = uniform(max(min(te - pc.c0, kChunk), 0));
    pc.from_interior = j > 0 && !dense;
    if (dense) {
      pc.ckpt = ((static_cast<int64_t>(seq) * heads + head) * (p.dense_t / 16) + 4 * j) *
                kHead * kHead;
    } else if (j == 0) {
      pc.ckpt = (static_cast<int64_t>(seg) * heads + head) * kHead * kHead;
    } else {
      pc.ckpt = (static_cast<int64_t>(pc.c0 / kChunk) * heads + head) * kHead * kHead;
    }
    return pc;
  };
  auto npieces = [](int tb, int te) { return te > tb ? (te - tb + kChunk - 1) / kChunk : 0; };
  // The state slab of a piece start (fp32, C layout); zeros when absent.
  auto load_state = [&](const Piece& pc, f32x4 (&S)[4]) {
    const float* src = nullptr;
    if (pc.ntok > 0) {
      const float* interior = args().interior;
      src = pc.from_interior ? (interior != nullptr ? interior + pc.ckpt : nullptr)
                             : args().checkpoint + pc.ckpt;
    }
    const auto ck = buffer_rsrc(src, src != nullptr ? kHead * kHead * 4 : 0);
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        S[kb][j] = __uint_as_float(
            __builtin_amdgcn_raw_buffer_load_b32(ck, s_off, (16 * kb + j) * kHead * 4, 0));
  };
  // Token rows of a piece; rows past its tokens read as zero (buffer range).
  using S16 = typename IoTraits<T>::storage;
  auto ld16 = [&](const void* x, const Piece& pc) {
    const bool ok = x != nullptr && pc.ntok > 0;
    const auto rs = buffer_rsrc(
        ok ? static_cast<const S16*>(x) + (static_cast<int64_t>(pc.c0) * heads + head) * kHead
           : nullptr,
        ok ? static_cast<uint32_t>(pc.ntok) * row_bytes : 0u);
    const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(rs, tok_off, 0, 0);
    return make_uint4(q.x, q.y, q.z, q.w);
  };
  // Row loads in three groups (issued between product groups).
  auto load_group = [&](const Piece& pc, TokRows& rows, int grp) {
    if (grp == 0) {
      rows.w = ld16(args().decay, pc);
      rows.r = ld16(args().r, pc);
      rows.a = ld16(args().a, pc);
    } else if (grp == 1) {
      rows.b = ld16(args().b, pc);
      rows.k = ld16(args().k, pc);
    } else {
      rows.dy = ld16(args().dy, pc);
      rows.v = ld16(args().v, pc);
    }
  };

  // Pieces in reverse over the segments in reverse. advance() moves
  // (sg, b, e, jj) to the piece before: jj - 1, else the last piece of the
  // nearest earlier non-empty segment; false when there is none.
  auto advance = [&](int& sg, int& b, int& e, int& jj) {
    if (jj > 0) {
      --jj;
      return true;
    }
    while (--sg >= seg_lo) {
      seg_bounds(sg, b, e);
      const int np = npieces(b, e);
      if (np > 0) {
        jj = np - 1;
        return true;
      }
    }
    return false;
  };
  // A whole piece issues the six gradient stores between its loads of the
  // next piece's rows and that piece's prepare; paths that load rows without
  // them issue as many dropped stores, so that on every path into the prepare
  // the compiler counts them and waits for the row loads alone (the memory
  // counter retires in order; at a join the compiler keeps the path with the
  // fewest instructions after the loads).
  auto pad_after_rows = [&]() {
    const auto nrs = buffer_rsrc(static_cast<float*>(nullptr), 0u);
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      __builtin_amdgcn_raw_buffer_store_b32(0u, nrs, kDropOffset, 4 * i, 0);
    }
  };
  int seg = seg_hi, tb = 0, te = 0, j = 0;
  bool have = advance(seg, tb, te, j);
  TokRows nxt;
  if (have) {
    const Piece first = piece_of(seg, tb, te, j);
#pragma unroll
    for (int grp = 0; grp < 3; ++grp) load_group(first, nxt, grp);
  }
  pad_after_rows();

  while (have) {
    const Piece pc = piece_of(seg, tb, te, j);
    if (pc.from_interior && p.interior == nullptr) failed = true;
    int pseg = seg, ptb = tb, pte = te, pj = j;
    const bool have_prev = advance(pseg, ptb, pte, pj);
    const Piece prev = have_prev ? piece_of(pseg, ptb, pte, pj) : Piece{0, 0, 0, false};

    // The piece-start state: loaded now, first read in the column phase.
    f32x4 S[4];
    load_state(pc, S);
    const TokRows cur = nxt;
    const Spans spans = prepare_piece<T, M>(sm, cur, bias, 0, pc.ntok, p.scale);
    if (spans.whole) {
      intra_piece(sm, [&](int i) { load_group(prev, nxt, i); });
      run_backward_step<T, M>(sm, p, cur, bias, S, 0, pc.ntok, pc, heads, head, row_bytes,
                              tok_off);
    } else {
      // Strong decay: sub-pieces in reverse, each from the state recomputed
      // by forward steps from the piece start.
      const int nsub = sub_count(spans);
      for (int r = nsub - 1; r >= 0; --r) {
        load_state(pc, S);
        for (int i = 0; i < r; ++i) {
          int lo, hi;
          sub_range(spans, i, lo, hi);
          prepare_piece<T, M>(sm, cur, bias, lo, min(hi, pc.ntok), p.scale);
          intra_piece(sm, [](int) {});
          // Both roles step the slab: the adjoint waves need the state (dg).
          f32x4 sa[4];
          i16x4 sab[4], vs[4];
          sa_chain(sm, S, cs, g, n, sa, sab, vs);
          state_step(sm, S, g, n, sab, vs);
        }
        int lo, hi;
        sub_range(spans, r, lo, hi);
        prepare_piece<T, M>(sm, cur, bias, lo, min(hi, pc.ntok), p.scale);
        intra_piece(sm, [](int) {});
        run_backward_step<T, M>(sm, p, cur, bias, S, lo, min(hi, pc.ntok), pc, heads, head,
                                row_bytes, tok_off);
      }
#pragma unroll
      for (int grp = 0; grp < 3; ++grp) load_group(prev, nxt, grp);
      pad_after_rows();
    }
    seg = pseg;
    tb = ptb;
    te = pte;
    j = pj;
    have = have_prev;
  }

  // Gradient of the initial state (the adjoint waves' stash).
  if (p.dstate0 != nullptr && adjoint) {
    const auto rs0 = buffer_rsrc(p.dstate0 + unit_state, kHead * kHead * 4);
    const float kNaN = __int_as_float(0x7fc00000);
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const f32x4 x = sm.dstash[cs][kb][lane];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(failed ? kNaN : x[jj]), rs0,
                                              s_off, (16 * kb + jj) * kHead * 4, 0);
    }
  }
}

template <typename T, DecayMode M>
int launch_bwd(const ChunkBwdParams& p, int units, hipStream_t stream) {
  if (p.num_heads > kMaxChunkHeads) {
    return set_error(FRWKV_ERR_UNSUPPORTED, "chunked kernels take at most %d heads, got %d",
                     kMaxChunkHeads, p.num_heads);
  }
  if (p.dense_t > 0) {
    hipLaunchKernelGGL((chunk_bwd_kernel<T, M, true>), dim3(units), dim3(kBwdThreads), 0,
                       stream, p);
  } else {
    hipLaunchKernelGGL((chunk_bwd_kernel<T, M, false>), dim3(units), dim3(kBwdThreads), 0,
                       stream, p);
  }
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

int dispatch_bwd(const ChunkBwdParams& p, int io_dtype, int decay_mode, int units,
                 hipStream_t s) {
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

}  // namespace
}  // namespace frwkv

namespace {
constexpr size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }
}  // namespace

extern "C" size_t frwkv_statetune_backward_workspace_bytes(int32_t head_size, int32_t num_heads,
                                                           int32_t total_tokens,
                                                           int interior_given) {
  size_t bytes = align256(frwkv_train_slice_bytes(head_size, num_heads, total_tokens));
  if (!interior_given) bytes += frwkv_statetune_interior_bytes(head_size, num_heads, total_tokens);
  return bytes;
}

extern "C" int frwkv_statetune_backward(
    int io_dtype, int decay_mode, int32_t num_sequences, int32_t num_heads, int32_t head_size,
    int32_t total_tokens, int32_t num_chunks, const int32_t* sequence_chunk_offsets,
    const int32_t* chunk_token_starts, const int32_t* chunk_token_ends, const float* boundary,
    const float* interior, const void* r, const void* decay, const void* decay_bias,
    const void* k, const void* v, const void* a, const void* b, const void* grad_output,
    const float* grad_final_state, void* grad_r, void* grad_decay, void* grad_k, void* grad_v,
    void* grad_a, void* grad_b, float* grad_initial_state, void* workspace,
    size_t workspace_bytes, float scale, void* stream) {
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
  if (head_size != 64 && head_size != 128 && head_size != 256) {
    return set_error(FRWKV_ERR_UNSUPPORTED, "head size must be 64, 128, or 256, got %d",
                     head_size);
  }
  // Workspace: the gradient slices (head size 256), then, when interior is
  // null, the interior states this call recomputes from the boundaries. A
  // call without interior states always needs the workspace: whether some
  // chunk is longer than one piece is only known on the device.
  const size_t slice_bytes = frwkv_train_slice_bytes(head_size, num_heads, total_tokens);
  const size_t need = frwkv_statetune_backward_workspace_bytes(head_size, num_heads,
                                                               total_tokens, interior != nullptr);
  const bool fill = interior == nullptr;
  if ((slice_bytes > 0 || fill) && (workspace == nullptr || workspace_bytes < need)) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_statetune_backward: workspace of %zu bytes given, %zu needed",
                     workspace != nullptr ? workspace_bytes : static_cast<size_t>(0), need);
  }
  float* slices = slice_bytes > 0 ? static_cast<float*>(workspace) : nullptr;
  if (fill) {
    float* filled = reinterpret_cast<float*>(static_cast<char*>(workspace) + align256(slice_bytes));
    const int rc = frwkv_statetune_interior(io_dtype, decay_mode, num_heads, head_size,
                                            total_tokens, num_chunks, chunk_token_starts,
                                            chunk_token_ends, boundary, r, decay, decay_bias, k,
                                            v, a, b, filled, stream);
    if (rc != FRWKV_OK) return rc;
    interior = filled;
  }
  if (head_size == 128 || head_size == 256) {
    return frwkv_train_recurrent_backward(
        io_dtype, decay_mode, num_sequences, num_heads, head_size, total_tokens,
        sequence_chunk_offsets, chunk_token_starts, chunk_token_ends, num_chunks, /*dense_t=*/0,
        boundary, r, decay, decay_bias, k, v, a, b, grad_output, grad_final_state, grad_r,
        grad_decay, grad_k, grad_v, grad_a, grad_b, grad_initial_state, interior, slices, scale,
        stream);
  }
  ChunkBwdParams p{};
  p.num_heads = num_heads;
  p.total_tokens = total_tokens;
  p.num_segments = num_chunks;
  p.seg_offsets = sequence_chunk_offsets;
  p.seg_starts = chunk_token_starts;
  p.seg_ends = chunk_token_ends;
  p.checkpoint = boundary;
  p.interior = interior;
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
  return dispatch_bwd(p, io_dtype, decay_mode, num_sequences * num_heads,
                      static_cast<hipStream_t>(stream));
}

extern "C" size_t frwkv_pretrain_backward_workspace_bytes(int32_t batch, int32_t tokens,
                                                          int32_t num_heads, int32_t head_size) {
  if (batch <= 0 || tokens <= 0 || static_cast<int64_t>(batch) * tokens > INT32_MAX) return 0;
  return frwkv_train_slice_bytes(head_size, num_heads, batch * tokens);
}

extern "C" int frwkv_pretrain_backward(int io_dtype, int decay_mode, int32_t batch,
                                       int32_t tokens, int32_t num_heads, int32_t head_size,
                                       const void* r, const void* decay, const void* k,
                                       const void* v, const void* a, const void* b,
                                       const void* grad_output, const float* boundary,
                                       void* grad_r, void* grad_decay, void* grad_k,
                                       void* grad_v, void* grad_a, void* grad_b,
                                       void* workspace, size_t workspace_bytes, void* stream) {
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
    const size_t need = frwkv_train_slice_bytes(head_size, num_heads, batch * tokens);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
      return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                       "frwkv_pretrain_backward: workspace of %zu bytes given, %zu needed",
                       workspace != nullptr ? workspace_bytes : static_cast<size_t>(0), need);
    }
    return frwkv_train_recurrent_backward(
        io_dtype, decay_mode, batch, num_heads, head_size, batch * tokens, nullptr, nullptr,
        nullptr, 0, tokens, boundary, r, decay, /*decay_bias=*/nullptr, k, v, a, b, grad_output,
        /*grad_final_state=*/nullptr, grad_r, grad_decay, grad_k, grad_v, grad_a, grad_b,
        /*grad_initial_state=*/nullptr, /*interior=*/nullptr,
        need > 0 ? static_cast<float*>(workspace) : nullptr, 1.0f, stream);
  }
  if (head_size != 64) {
    return set_error(FRWKV_ERR_UNSUPPORTED, "head size must be 64, 128, or 256, got %d",
                     head_size);
  }
  ChunkBwdParams p{};
  p.num_heads = num_heads;
  p.total_tokens = batch * tokens;
  p.dense_t = tokens;
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
  return dispatch_bwd(p, io_dtype, decay_mode, batch * num_heads,
                      static_cast<hipStream_t>(stream));
}
