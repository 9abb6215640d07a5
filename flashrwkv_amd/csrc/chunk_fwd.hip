// Chunked WKV7 forward on bf16 MFMA (prefill and training forward).
//
// Replaces the reference's infer_chunk_bf16_k1/k2 kernels
// (csrc/sm120/tmix/wkv7/infer_chunk_bf16_forward_varlen.cu:42-334) and the
// StateTune forward kernel (csrc/sm90/tmix/wkv7/statetune_recurrent_fp32io16_forward.cu:32-224)
// with one algorithm: the exact chunked form of the recurrence, whose results
// equal the per-token recurrence up to rounding (the reference K1/K2 pair
// does not: its per-chunk transforms are cumulative from the sequence start).
//
// Recurrence (state S is [K,V], per token t):
//   sa_t = S_{t-1}^T a_t;  S_t = diag(w_t) S_{t-1} + b_t sa_t^T + k_t v_t^T;
//   y_t = scale S_t^T r_t.
// Chunk form, tokens t = 0..63 of a chunk, G_t = sum_{j<=t} log2 w_j
// (inclusive), Gp_t = G_t - log2 w_t, GC = G_63, S0 = state at chunk start:
//   At = a 2^Gp, Rt = r 2^G, Bh = b 2^-G, Kh = k 2^-G;
//   Lab = strict_lower(At Bh^T), Lak = strict_lower(At Kh^T),
//   Arb = lower(Rt Bh^T),        Ark = lower(Rt Kh^T);
//   SA = (I - Lab)^{-1} (At S0 + Lak V)       (rows are sa_t)
//   Y  = scale (Rt S0 + Arb SA + Ark V)
//   S' = diag(2^GC) (S0 + Bh^T SA + Kh^T V).
// (The last product is accumulated in fp32 and scaled once: every term
// carries the common factor 2^GC, so this keeps the relative precision of
// scaling Bh, Kh by 2^GC first.)
// Every exponent above is <= 0 except the 2^-G of Bh/Kh, bounded by the
// chunk's decay span -GC. The kernel keeps that span <= 80 (log2 units): a
// chunk whose span is larger is processed as 16-token sub-chunks, and a
// 16-token block whose span is still larger as 4-token sub-chunks. The
// per-token log2 retention is clamped to [-20, 0] (w in [2^-20, 1]), so
// 4-token spans never exceed 80; below 2^-20 the clamp changes S_t by less
// than 1e-6 |S_{t-1}|, far under bf16 resolution.
//
// Work decomposition (one 256-thread workgroup per (sequence, head), two
// workgroups per CU: 80 KB of LDS and at most 256 registers per lane):
//   * prepare: the chunk's 64 tokens x 64 features are decoded once (two
//     tokens x 8 features per thread), the cumulative decay is a wave
//     shuffle scan plus a cross-wave carry, and the scaled operands go to LDS
//     as bf16 [token][feature] tiles (products contracting over tokens read
//     them through gfx950's LDS transpose read);
//   * intra-chunk products: the 40 lower-triangular 16x16 blocks of Lab,
//     Lak, Arb, Ark (stored packed) are spread over the four waves; wave p
//     also inverts the diagonal block I - Lab_pp (forward substitution);
//   * state-dependent part: wave w owns value columns 16w..16w+15. Its slice
//     of the fp32 state lives in MFMA accumulators for the whole sequence;
//     the block forward substitution SA_p = T_pp (rhs_p + sum_q Lab_pq SA_q),
//     the output tiles and the state update chain through registers, so this
//     part has no barrier.
// The token rows of chunk c+1 are loaded while chunk c computes.
#include "capi_internal.h"
#include "wkv7_device.h"
#include "wkv7_mfma.h"
#include "chunk_common.h"

namespace frwkv {
namespace {

struct ChunkSmem {
  uint16_t at[kOpTile];   // [t][k]
  uint16_t rt[kOpTile];   // [t][k]
  uint16_t bh[kOpTile];   // [t][k]
  uint16_t kh[kOpTile];   // [t][k]
  uint16_t vt[kOpTile];   // V [t][v]
  uint16_t tri[4][kTriBlocks * kTriBlock];  // Lab, Lak, Arb, Ark: [t][i]
  // Decay scan carry (prepare only). Not shared with the tiles: the scan
  // writes it before the barrier after which the tiles may be overwritten.
  float wave_tot[4][kHead];
  uint16_t tinv[4][kTriBlock];  // (I - Lab_pp)^{-1}, [t][i]
  float gc[kHead];              // 2^GC per key feature
  float gsub[3][kHead];         // 2^G at tokens 15, 31, 47 (16-token boundaries)
};
static_assert(sizeof(ChunkSmem) <= 80 * 1024, "two workgroups per CU need <= 80 KB of LDS");

// Split-precision variant (the recurrent operator's long sequences): the
// products whose bf16 rounding dominates the error against the per-token
// fp32 recurrence are taken on split operands x = hi + lo (split_bf16x2),
// which leaves about 2^-17 relative error per operand instead of 2^-9:
//   Ark = Rt Kh^T   from Rt, Kh split (three products: hi hi, lo hi, hi lo),
//                   stored split, so Ark V is two products;
//   Lak = At Kh^T   with Kh split (two products);
//   Rt S0           with Rt and S0 split (three products);
//   Kh^T V          in the state update, Kh split (two products).
// The remaining bf16 roundings (At, Bh, Lab, Arb, T, SA) enter through the
// b sa^T term only. These tiles hold the low halves; the high halves stay in
// ChunkSmem. The extra 23 KB of LDS leave one workgroup per CU.
struct PreciseTiles {
  uint16_t rt_lo[kOpTile];                  // [t][k]
  uint16_t kh_lo[kOpTile];                  // [t][k]
  uint16_t ark_lo[kTriBlocks * kTriBlock];  // [t][i]
};
struct NoPreciseTiles {};
template <bool kPrecise>
struct ExtraTilesOf {
  using type = NoPreciseTiles;
};
template <>
struct ExtraTilesOf<true> {
  using type = PreciseTiles;
};
template <bool kPrecise>
using ExtraTiles = typename ExtraTilesOf<kPrecise>::type;

__device__ __forceinline__ const uint16_t* tri_block(const ChunkSmem& sm, int m, int p, int q) {
  return sm.tri[m] + tri_index(p, q) * kTriBlock;
}

struct ChunkFwdParams {
  int32_t num_heads;
  // Packed varlen batches of at most 64 sequences (cu_seqlens mode) run
  // their sequences longest first: workgroup b takes the sequence of length
  // rank b / H. 0 keeps the natural order.
  int32_t longest_first_sequences;
  int32_t total_tokens;
  int32_t state_slots;
  const int32_t* cu_seqlens;    // sequence token ranges when seg_offsets == null
  const int32_t* seg_offsets;   // [B+1] segment lists (StateTune chunks) or null
  const int32_t* seg_starts;
  const int32_t* seg_ends;
  int32_t num_segments;         // length of seg_starts / seg_ends / boundary
  const int32_t* slots;         // [B] state slot per sequence, or null (identity)
  const int32_t* status;        // metadata status word, or null
  void* state;
  const void* r;
  const void* decay;
  const void* bias;
  const void* k;
  const void* v;
  const void* a;
  const void* b;
  void* out;
  float* boundary;              // state at each segment start, or null
  float* state_dot_a;           // per-token a^T S_{t-1}, or null
  float scale;
  int64_t out_elems;
  // Dense layout: > 0 means every sequence has dense_t tokens (sequence s
  // covers tokens s * dense_t ..), with no cu_seqlens or segment arrays.
  int32_t dense_t;
  // 1: boundary is [B, H, dense_t / 16, D, D], the state every 16 tokens.
  int32_t boundary16;
  // 1: the initial states are read and never written back (replay from
  // stored boundaries).
  int32_t read_only_state;
  // [ceil(total_tokens / 64), H, D, D] or null: the state at every 64-token
  // piece start inside a segment (not at the segment start), at slot
  // (piece start) / 64. Interior starts of different segments lie more than
  // 64 tokens apart, so the slots are distinct.
  float* interior;
  // 1 (replay layout, one segment per unit): only the interior states are
  // wanted; segments of at most 64 tokens have none and are skipped, and a
  // segment's last piece is not computed.
  int32_t fill_only;
};

// Token rows of one chunk held by a thread: r, w, k, a, b for 2 tokens x 8
// features (prepare layout), and two 16-byte pieces of the chunk's V tile
// (piece tid + 256 s: token (tid + 256 s) / 8, features 8 ((tid + 256 s) % 8)
// .. +7). V goes through LDS to reach the MFMA operand layout.
struct ChunkRows {
  uint4 r[2], w[2], k[2], a[2], b[2];
  uint4 v[2];
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

// Decay-span verdicts of a prepared range, uniform over the workgroup: is
// the span of the whole range, resp. of each 16-token block, within the
// limit of the single-reference factorisation?
struct Spans {
  bool whole;
  bool block[4];

  // block[q] for a runtime q without indexing a private array.
  __device__ __forceinline__ bool block_ok(int q) const {
    return q == 0 ? block[0] : q == 1 ? block[1] : q == 2 ? block[2] : block[3];
  }
};

// Decodes the thread's rows restricted to tokens [lo, hi) of the chunk,
// scans the decay and writes the scaled operand tiles At, Rt, Bh, Kh
// ([t][k]) and the V tile. Ends with a barrier. kFull: the range is the
// whole 64-token chunk, so no token needs masking.
//
// Per feature, the thread's tokens t0 and t0 + 1 need 2^Gp(t0), 2^G(t0)
// (= 2^Gp(t0 + 1)), 2^G(t0 + 1), 2^-G(t0), 2^-G(t0 + 1): two exponentials
// and products with the retentions w = 2^lg (G(t) = Gp(t) + lg(t)).
template <typename T, DecayMode M, bool kFull, bool kPrecise>
__device__ Spans prepare(ChunkSmem& sm, ExtraTiles<kPrecise>& ext, const ChunkRows& rows,
                         const float (&bias)[8], int lo, int hi) {
  const int tid = threadIdx.x;
  const int wave = uniform(tid >> 6);
  const int lane = tid & 63;
  const int tp = lane & 7;   // token pair
  const int kg = lane >> 3;  // feature group
  const int t0 = 16 * wave + 2 * tp;
  const bool on0 = kFull || (t0 >= lo && t0 < hi);
  const bool on1 = kFull || (t0 + 1 >= lo && t0 + 1 < hi);

  // Retentions; tokens outside [lo, hi) get w = 1 (no decay, and their operand
  // rows are zero below).
  float w0[8], w1[8];
  {
    float x0[8], x1[8];
    unpack8<T>(rows.w[0], x0);
    unpack8<T>(rows.w[1], x1);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if constexpr (M == DecayMode::kLogits) {
        x0[e] += bias[e];
        x1[e] += bias[e];
      }
      const float r0 = clamped_retention<M>(x0[e]);
      const float r1 = clamped_retention<M>(x1[e]);
      w0[e] = on0 ? r0 : 1.0f;
      w1[e] = on1 ? r1 : 1.0f;
    }
  }

  // The cumulative decay as products, 2^G(t) = prod_{j<=t} w_j: an inclusive
  // product scan over the wave's 8 token pairs (the 8 lanes of a feature
  // group), then the carry of earlier waves through LDS. Every product that
  // reaches an operand has a span within the limit, so it stays a normal
  // fp32 number (>= 2^-80); a pass whose span exceeds the limit is
  // discarded and redone as sub-chunks.
  float incl[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float x = w0[e] * w1[e];
    x = scan8_mul<1>(x, tp);
    x = scan8_mul<2>(x, tp);
    incl[e] = scan8_mul<4>(x, tp);
  }
  if (tp == 7) {
#pragma unroll
    for (int e = 0; e < 8; ++e) sm.wave_tot[wave][8 * kg + e] = incl[e];
  }
  // The carries are in LDS, and every reader of the previous pass's tiles
  // (its state pass) is done: the tiles below may be overwritten.
  __syncthreads();

  // Block products x_q (q = 0..3, one per wave's 16 tokens); the carry into
  // this wave is the product of the blocks before it (a wave-uniform count).
  float up_p[8], g1[8], total[8];
  float xq[4][8];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float4 xa = *reinterpret_cast<const float4*>(&sm.wave_tot[q][8 * kg]);
    const float4 xb = *reinterpret_cast<const float4*>(&sm.wave_tot[q][8 * kg + 4]);
    xq[q][0] = xa.x; xq[q][1] = xa.y; xq[q][2] = xa.z; xq[q][3] = xa.w;
    xq[q][4] = xb.x; xq[q][5] = xb.y; xq[q][6] = xb.z; xq[q][7] = xb.w;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float lo2 = xq[0][e] * xq[1][e];
    const float hi2 = xq[2][e] * xq[3][e];
    total[e] = lo2 * hi2;
    float base = 1.0f;
    if (wave == 1) base = xq[0][e];
    if (wave == 2) base = lo2;
    if (wave == 3) base = lo2 * xq[2][e];
    g1[e] = base * incl[e];                   // 2^G(t0 + 1)
    up_p[e] = base * scan8_exclusive(incl[e], tp);  // 2^Gp(t0)
  }
  // A span exceeds the limit when its decay product is below 2^-kSpanLimit;
  // min reductions over the thread's 8 features, then a ballot. Every wave
  // covers all 64 features, so the ballots agree.
  auto within = [](const float (&x)[8]) {
    float m = x[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) m = fminf(m, x[e]);
    return __builtin_amdgcn_ballot_w64(!(m >= kSpanFloor)) == 0;
  };
  Spans spans;
  spans.whole = within(total);
#pragma unroll
  for (int q = 0; q < 4; ++q) spans.block[q] = within(xq[q]);

  // Scale factors of the thread's two token rows, zero outside [lo, hi).
  float fa0[8], fa1[8], fr0[8], fr1[8], fd0[8], fd1[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float up0 = up_p[e] * w0[e];                // 2^G(t0) = 2^Gp(t0 + 1)
    const float dn1 = __builtin_amdgcn_rcpf(g1[e]);   // 2^-G(t0 + 1)
    const float dn0 = dn1 * w1[e];                    // 2^-G(t0)
    fa0[e] = on0 ? up_p[e] : 0.0f;
    fa1[e] = on1 ? up0 : 0.0f;
    fr0[e] = on0 ? up0 : 0.0f;
    fr1[e] = on1 ? g1[e] : 0.0f;
    fd0[e] = on0 ? dn0 : 0.0f;
    fd1[e] = on1 ? dn1 : 0.0f;
  }
  auto tile_rows = [&](uint16_t* tile, uint4 q0, uint4 q1, const float (&f0)[8],
                       const float (&f1)[8]) {
    float x0[8], x1[8];
    unpack8<T>(q0, x0);
    unpack8<T>(q1, x1);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x0[e] *= f0[e];
      x1[e] *= f1[e];
    }
    store8_bf16(tile + t0 * kOpStride + 8 * kg, x0);
    store8_bf16(tile + (t0 + 1) * kOpStride + 8 * kg, x1);
  };
  // Rt and Kh as split pairs in the precise variant.
  auto split_rows = [&](uint16_t* tile, uint16_t* tile_lo, uint4 q0, uint4 q1,
                        const float (&f0)[8], const float (&f1)[8]) {
    float x0[8], x1[8];
    unpack8<T>(q0, x0);
    unpack8<T>(q1, x1);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x0[e] *= f0[e];
      x1[e] *= f1[e];
    }
    const int o0 = t0 * kOpStride + 8 * kg, o1 = o0 + kOpStride;
    store8_bf16_split(tile + o0, tile_lo + o0, x0);
    store8_bf16_split(tile + o1, tile_lo + o1, x1);
  };
  tile_rows(sm.at, rows.a[0], rows.a[1], fa0, fa1);
  if constexpr (kPrecise) {
    split_rows(sm.rt, ext.rt_lo, rows.r[0], rows.r[1], fr0, fr1);
  } else {
    tile_rows(sm.rt, rows.r[0], rows.r[1], fr0, fr1);
  }
  tile_rows(sm.bh, rows.b[0], rows.b[1], fd0, fd1);
  if constexpr (kPrecise) {
    split_rows(sm.kh, ext.kh_lo, rows.k[0], rows.k[1], fd0, fd1);
  } else {
    tile_rows(sm.kh, rows.k[0], rows.k[1], fd0, fd1);
  }
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int piece = tid + 256 * s;
    store_piece_bf16<T>(sm.vt + (piece >> 3) * kOpStride + 8 * (piece & 7), rows.v[s]);
  }
  if (wave == 0 && tp == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) sm.gc[8 * kg + e] = total[e];
  }
  if (wave < 3 && tp == 7) {
    // Token t0 + 1 = 16 wave + 15 ends a 16-token block.
#pragma unroll
    for (int e = 0; e < 8; ++e) sm.gsub[wave][8 * kg + e] = g1[e];
  }
  __syncthreads();
  return spans;
}

// Intra-chunk products: the 40 lower-triangular 16x16 blocks of Lab, Lak,
// Arb, Ark, plus the inverse of each diagonal block I - Lab_pp. Ends with a
// barrier.
//
// A stored block is M[t][i] = sum_k X[t][k] Y[i][k] (X = At or Rt for the
// target block p, Y = Bh or Kh for the source block q); it is computed
// transposed (A operand = Y rows, B operand = X rows) so each lane writes 4
// consecutive i of one row t. Blocks sharing operands are computed together:
// wave w does all four matrices of its diagonal pair (w, w), then three of
// the twelve off-diagonal half-pairs ({Lab, Arb} share Bh_q, {Lak, Ark}
// share Kh_q; both share At_p and Rt_p).
//
// issue(i), i = 0..5, is called between the product groups: the caller
// issues one sixth of the next chunk's row loads there, so the loads enter
// the memory system while the products run instead of stalling the wave on
// a burst of 12 outstanding 16-byte loads.
template <bool kPrecise, typename Issue>
__device__ __forceinline__ void intra_chunk(ChunkSmem& sm, ExtraTiles<kPrecise>& ext,
                                            Issue&& issue) {
  // MFMA phases run at raised wave priority: the other workgroup on the CU
  // is then usually in its VALU-heavy prepare, and the arbiter keeps the
  // matrix pipe fed from this one.
  __builtin_amdgcn_s_setprio(1);
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int g = lane >> 4;
  const int n = lane & 15;

  auto store = [&](int m, int p, int q, f32x4 acc, bool strict, bool diag) {
    if (diag) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = 4 * g + j;
        const bool keep = strict ? (i < n) : (i <= n);
        acc[j] = keep ? acc[j] : 0.0f;
      }
    }
    lds_store_transposed(sm.tri[m] + tri_index(p, q) * kTriBlock, kTriStride, g, n, acc);
  };

  auto group = [&](int p, int q, bool with_b, bool with_k, bool diag) {
    f32x4 lab = zero4(), lak = zero4(), arb = zero4(), ark = zero4();
    f32x4 lak_c = zero4(), ark_c = zero4();  // precise: the low-half products
#pragma unroll
    for (int c = 0; c < 64; c += 32) {
      const i16x8 xa = lds_operand32<kOpStride>(sm.at, 16 * p + n, c, g);
      const i16x8 xr = lds_operand32<kOpStride>(sm.rt, 16 * p + n, c, g);
      if (with_b) {
        const i16x8 yb = lds_operand32<kOpStride>(sm.bh, 16 * q + n, c, g);
        lab = mfma32(yb, xa, lab);
        arb = mfma32(yb, xr, arb);
      }
      if (with_k) {
        const i16x8 yk = lds_operand32<kOpStride>(sm.kh, 16 * q + n, c, g);
        lak = mfma32(yk, xa, lak);
        ark = mfma32(yk, xr, ark);
        if constexpr (kPrecise) {
          const i16x8 yk_lo = lds_operand32<kOpStride>(ext.kh_lo, 16 * q + n, c, g);
          const i16x8 xr_lo = lds_operand32<kOpStride>(ext.rt_lo, 16 * p + n, c, g);
          lak_c = mfma32(yk_lo, xa, lak_c);
          ark_c = mfma32(yk_lo, xr, ark_c);
          ark_c = mfma32(yk, xr_lo, ark_c);
        }
      }
    }
    if (with_b) {
      store(kLab, p, q, lab, true, diag);
      store(kArb, p, q, arb, false, diag);
    }
    if (with_k) {
      if constexpr (kPrecise) {
        lak += lak_c;
        ark += ark_c;
      }
      store(kLak, p, q, lak, true, diag);
      if constexpr (kPrecise) {
        if (diag) {
#pragma unroll
          for (int j = 0; j < 4; ++j) ark[j] = (4 * g + j <= n) ? ark[j] : 0.0f;
        }
        lds_store_transposed_split(sm.tri[kArk] + tri_index(p, q) * kTriBlock,
                                   ext.ark_lo + tri_index(p, q) * kTriBlock, kTriStride, g, n,
                                   ark);
      } else {
        store(kArk, p, q, ark, false, diag);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // Diagonal pair first; its Lab block feeds the inverse.
  issue(0);
  group(wave, wave, true, true, true);
  issue(1);
  // T_pp = (I - L)^{-1} for the strictly lower 16 x 16 block L = Lab_pp:
  // L^16 = 0, so (I - L)^{-1} = (I + L)(I + L^2)(I + L^4)(I + L^8). All
  // factors are polynomials in L and commute. With X_R the register layout
  // "lane (g, n) holds X[n][4g + j]" (A operand of X, C layout of X^T) and
  // X_C the C layout of X (B operand of X), a product Z = X Y is
  // Z_C = mfma(X_R, Y_C) and Z_R = mfma(Y_C, X_R).
  {
    f32x4 l_r = zero4(), l_c = zero4();
#pragma unroll
    for (int c = 0; c < 64; c += 32) {
      const i16x8 xa = lds_operand32<kOpStride>(sm.at, 16 * wave + n, c, g);
      const i16x8 yb = lds_operand32<kOpStride>(sm.bh, 16 * wave + n, c, g);
      l_r = mfma32(yb, xa, l_r);  // lane (g, n): L[n][4g + j]
      l_c = mfma32(xa, yb, l_c);  // lane (g, n): L[4g + j][n]
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      l_r[j] = (4 * g + j < n) ? l_r[j] : 0.0f;
      l_c[j] = (n < 4 * g + j) ? l_c[j] : 0.0f;
    }
    const i16x4 lr = to_operand(l_r), lc = to_operand(l_c);
    const i16x4 p2c = to_operand(mfma16(lr, lc, zero4()));
    const i16x4 p2r = to_operand(mfma16(lc, lr, zero4()));
    const i16x4 p4c = to_operand(mfma16(p2r, p2c, zero4()));
    const i16x4 p4r = to_operand(mfma16(p2c, p2r, zero4()));
    const i16x4 p8c = to_operand(mfma16(p4r, p4c, zero4()));
    f32x4 t = l_r;  // T1 = I + L
#pragma unroll
    for (int j = 0; j < 4; ++j) t[j] += (4 * g + j == n) ? 1.0f : 0.0f;
    t = mfma16(p2c, to_operand(t), t);  // T2 = T1 + P2 T1
    t = mfma16(p4c, to_operand(t), t);  // T3 = T2 + P4 T2
    t = mfma16(p8c, to_operand(t), t);  // T  = T3 + P8 T3
    lds_store_transposed(sm.tinv[wave], kTriStride, g, n, t);
  }
  issue(2);

  // Off-diagonal half-pairs: pair index item / 2 over (1,0) (2,0) (2,1)
  // (3,0) (3,1) (3,2), half item % 2 ({Lab, Arb} or {Lak, Ark}).
#pragma unroll
  for (int r = 0; r < 3; ++r) {
    const int item = wave + 4 * r;
    const int pair = item >> 1;
    const int p = pair < 1 ? 1 : (pair < 3 ? 2 : 3);
    const int q = pair - (p * (p - 1)) / 2;
    group(p, q, (item & 1) == 0, (item & 1) == 1, false);
    issue(3 + r);
  }
  __builtin_amdgcn_s_setprio(0);
  __syncthreads();
}

// State-dependent part of one prepared (sub-)chunk for wave w's value
// columns. Tokens outside [lo, hi) are zero rows of every operand; their
// output stores go to kDropOffset and are dropped (no branch around them, so
// every pass issues the same stores).
// out_rs / sda_rs cover the chunk's rows of the output and of state_dot_a
// (row t at byte t * row_bytes, resp. 2 * t * row_bytes); sda_rs is unused
// when with_sda is false.
// sub_rs / nsub: the first nsub (at most 3) 16-token boundary states of the
// chunk (after tokens 15, 31, 47) go to sub_rs, one [D][D] fp32 block each;
// nsub is 0 except for whole-chunk passes of the every-16-tokens layout.
template <typename T, bool kPrecise>
__device__ void state_pass(const ChunkSmem& sm, const ExtraTiles<kPrecise>& ext, f32x4 (&S)[4],
                           const uint16_t* vtile, __amdgpu_buffer_rsrc_t out_rs,
                           __amdgpu_buffer_rsrc_t sda_rs, bool with_sda, uint32_t row_bytes,
                           float scale, int lo, int hi, __amdgpu_buffer_rsrc_t sub_rs,
                           int nsub) {
  __builtin_amdgcn_s_setprio(1);  // MFMA phase (see intra_chunk)
  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int lane = tid & 63;
  const int g = lane >> 4;
  const int n = lane & 15;
  // The wave's V columns in operand layout: vs[q] holds V[16q + 4g + e][16w + n].
  i16x4 vs[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) vs[q] = lds_operand_tr<kOpStride>(vtile, 16 * q, 16 * w, g, n);

  // Operands: S0 (C layout; B operand of products over keys, A operand of
  // the transposed output product), V slice, then SA as it is solved. A
  // 32-wide K step concatenates two 16-blocks (see mfma32).
  i16x8 s01, s23;
  i16x8 s01_lo, s23_lo;  // precise: S0 = hi + lo for the output product
  if constexpr (kPrecise) {
    i16x4 h[4], l[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) to_operand_split(S[kb], h[kb], l[kb]);
    s01 = cat(h[0], h[1]);
    s23 = cat(h[2], h[3]);
    s01_lo = cat(l[0], l[1]);
    s23_lo = cat(l[2], l[3]);
  } else {
    const i16x4 s0 = to_operand(S[0]), s1 = to_operand(S[1]);
    const i16x4 s2 = to_operand(S[2]), s3 = to_operand(S[3]);
    s01 = cat(s0, s1);
    s23 = cat(s2, s3);
  }
  const i16x8 v01 = cat(vs[0], vs[1]), v23 = cat(vs[2], vs[3]);
  auto tri16 = [&](int m, int p, int q) {
    return lds_operand<kTriStride>(tri_block(sm, m, p, q), n, 4 * g);
  };
  auto tri32 = [&](int m, int p, int q) {  // blocks (p, q) and (p, q + 1)
    return cat(tri16(m, p, q), tri16(m, p, q + 1));
  };
  // A single 16-wide K block as a 32-wide step with a zero upper half: every
  // accumulator chain then uses one MFMA shape (same issue cost as the
  // 16-wide form).
  const i16x4 z4 = {0, 0, 0, 0};
  auto lo32 = [&](i16x4 x) { return cat(x, z4); };

  // rhs_p = At_p S0 + sum_{q<=p} Lak_pq V_q: four independent chains.
  f32x4 rhs[4];
#pragma unroll
  for (int pb = 0; pb < 4; ++pb) {
    rhs[pb] = mfma32(lds_operand32<kOpStride>(sm.at, 16 * pb + n, 0, g), s01, zero4());
  }
#pragma unroll
  for (int pb = 0; pb < 4; ++pb) {
    rhs[pb] = mfma32(lds_operand32<kOpStride>(sm.at, 16 * pb + n, 32, g), s23, rhs[pb]);
  }
  rhs[0] = mfma32(lo32(tri16(kLak, 0, 0)), lo32(vs[0]), rhs[0]);
  rhs[1] = mfma32(tri32(kLak, 1, 0), v01, rhs[1]);
  rhs[2] = mfma32(tri32(kLak, 2, 0), v01, rhs[2]);
  rhs[3] = mfma32(tri32(kLak, 3, 0), v01, rhs[3]);
  rhs[2] = mfma32(lo32(tri16(kLak, 2, 2)), lo32(vs[2]), rhs[2]);
  rhs[3] = mfma32(tri32(kLak, 3, 2), v23, rhs[3]);

  // Block forward substitution SA_p = T_pp (rhs_p + sum_{q<p} Lab_pq SA_q).
  auto tinv = [&](int pb) { return lds_operand<kTriStride>(sm.tinv[pb], n, 4 * g); };
  f32x4 sa[4];
  i16x4 sab[4];
  sa[0] = mfma32(lo32(tinv(0)), lo32(to_operand(rhs[0])), zero4());
  sab[0] = to_operand(sa[0]);
  rhs[1] = mfma32(lo32(tri16(kLab, 1, 0)), lo32(sab[0]), rhs[1]);
  sa[1] = mfma32(lo32(tinv(1)), lo32(to_operand(rhs[1])), zero4());
  sab[1] = to_operand(sa[1]);
  const i16x8 sa01 = cat(sab[0], sab[1]);
  rhs[2] = mfma32(tri32(kLab, 2, 0), sa01, rhs[2]);
  rhs[3] = mfma32(tri32(kLab, 3, 0), sa01, rhs[3]);
  sa[2] = mfma32(lo32(tinv(2)), lo32(to_operand(rhs[2])), zero4());
  sab[2] = to_operand(sa[2]);
  rhs[3] = mfma32(lo32(tri16(kLab, 3, 2)), lo32(sab[2]), rhs[3]);
  sa[3] = mfma32(lo32(tinv(3)), lo32(to_operand(rhs[3])), zero4());
  sab[3] = to_operand(sa[3]);
  const i16x8 sa23 = cat(sab[2], sab[3]);

  if (with_sda) {
    const uint32_t off = static_cast<uint32_t>(4 * g) * 2 * row_bytes + 4 * (16 * w + n);
#pragma unroll
    for (int pb = 0; pb < 4; ++pb) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = 16 * pb + 4 * g + j;
        __builtin_amdgcn_raw_buffer_store_b32(
            __float_as_uint(sa[pb][j]), sda_rs, (t >= lo && t < hi) ? off : kDropOffset,
            static_cast<int>((16 * pb + j) * 2 * row_bytes), 0);
      }
    }
  }

  // Y^T blocks (rows v of w, cols t of block p) and S' = diag(2^GC) (S0 +
  // Bh^T SA + Kh^T V): eight independent chains. Bh^T and Kh^T (A operands
  // over tokens) come from the [t][k] tiles through the transpose read.
  auto tr32 = [&](const uint16_t* tile, int kb, int c) {
    return cat(lds_operand_tr<kOpStride>(tile, c, 16 * kb, g, n),
               lds_operand_tr<kOpStride>(tile, c + 16, 16 * kb, g, n));
  };
  f32x4 y[4], sn[4];
  if (nsub > 0) {
    // The state update in 16-token steps: after block q the accumulator
    // holds S0 + sum_{t < 16(q+1)} (Bh_t^T SA_t + Kh_t^T V_t), which scaled
    // by 2^G(16q + 15) is the state after that block.
    const uint32_t b_off = static_cast<uint32_t>((4 * g) * kHead + 16 * w + n) * 4;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) sn[kb] = S[kb];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        sn[kb] = mfma32(lo32(lds_operand_tr<kOpStride>(sm.bh, 16 * q, 16 * kb, g, n)),
                        lo32(sab[q]), sn[kb]);
        sn[kb] = mfma32(lo32(lds_operand_tr<kOpStride>(sm.kh, 16 * q, 16 * kb, g, n)),
                        lo32(vs[q]), sn[kb]);
        if constexpr (kPrecise) {
          sn[kb] = mfma32(lo32(lds_operand_tr<kOpStride>(ext.kh_lo, 16 * q, 16 * kb, g, n)),
                          lo32(vs[q]), sn[kb]);
        }
      }
      if (q < 3 && q < nsub) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float x = sn[kb][j] * sm.gsub[q][16 * kb + 4 * g + j];
            __builtin_amdgcn_raw_buffer_store_b32(
                __float_as_uint(x), sub_rs, b_off,
                static_cast<int>((q * kHead * kHead + (16 * kb + j) * kHead) * 4), 0);
          }
        }
      }
    }
  } else {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) sn[kb] = mfma32(tr32(sm.bh, kb, 0), sa01, S[kb]);
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) sn[kb] = mfma32(tr32(sm.bh, kb, 32), sa23, sn[kb]);
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) sn[kb] = mfma32(tr32(sm.kh, kb, 0), v01, sn[kb]);
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) sn[kb] = mfma32(tr32(sm.kh, kb, 32), v23, sn[kb]);
    if constexpr (kPrecise) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) sn[kb] = mfma32(tr32(ext.kh_lo, kb, 0), v01, sn[kb]);
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) sn[kb] = mfma32(tr32(ext.kh_lo, kb, 32), v23, sn[kb]);
    }
  }
#pragma unroll
  for (int pb = 0; pb < 4; ++pb) {
    y[pb] = mfma32(s01, lds_operand32<kOpStride>(sm.rt, 16 * pb + n, 0, g), zero4());
  }
#pragma unroll
  for (int pb = 0; pb < 4; ++pb) {
    y[pb] = mfma32(s23, lds_operand32<kOpStride>(sm.rt, 16 * pb + n, 32, g), y[pb]);
  }
  if constexpr (kPrecise) {
    // Rt S0 = Rt_hi S0_hi + Rt_hi S0_lo + Rt_lo S0_hi.
#pragma unroll
    for (int pb = 0; pb < 4; ++pb) {
      const i16x8 r01 = lds_operand32<kOpStride>(sm.rt, 16 * pb + n, 0, g);
      const i16x8 r23 = lds_operand32<kOpStride>(sm.rt, 16 * pb + n, 32, g);
      y[pb] = mfma32(s01_lo, r01, y[pb]);
      y[pb] = mfma32(s23_lo, r23, y[pb]);
      y[pb] = mfma32(s01, lds_operand32<kOpStride>(ext.rt_lo, 16 * pb + n, 0, g), y[pb]);
      y[pb] = mfma32(s23, lds_operand32<kOpStride>(ext.rt_lo, 16 * pb + n, 32, g), y[pb]);
    }
    // Ark V with the low half of Ark.
    auto ark16 = [&](int p, int q) {
      return lds_operand<kTriStride>(ext.ark_lo + tri_index(p, q) * kTriBlock, n, 4 * g);
    };
    auto ark32 = [&](int p, int q) { return cat(ark16(p, q), ark16(p, q + 1)); };
    y[0] = mfma32(lo32(vs[0]), lo32(ark16(0, 0)), y[0]);
    y[1] = mfma32(v01, ark32(1, 0), y[1]);
    y[2] = mfma32(v01, ark32(2, 0), y[2]);
    y[3] = mfma32(v01, ark32(3, 0), y[3]);
    y[2] = mfma32(lo32(vs[2]), lo32(ark16(2, 2)), y[2]);
    y[3] = mfma32(v23, ark32(3, 2), y[3]);
  }
  y[0] = mfma32(lo32(sab[0]), lo32(tri16(kArb, 0, 0)), y[0]);
  y[1] = mfma32(sa01, tri32(kArb, 1, 0), y[1]);
  y[2] = mfma32(sa01, tri32(kArb, 2, 0), y[2]);
  y[3] = mfma32(sa01, tri32(kArb, 3, 0), y[3]);
  y[0] = mfma32(lo32(vs[0]), lo32(tri16(kArk, 0, 0)), y[0]);
  y[1] = mfma32(v01, tri32(kArk, 1, 0), y[1]);
  y[2] = mfma32(v01, tri32(kArk, 2, 0), y[2]);
  y[3] = mfma32(v01, tri32(kArk, 3, 0), y[3]);
  y[2] = mfma32(lo32(sab[2]), lo32(tri16(kArb, 2, 2)), y[2]);
  y[3] = mfma32(sa23, tri32(kArb, 3, 2), y[3]);
  y[2] = mfma32(lo32(vs[2]), lo32(tri16(kArk, 2, 2)), y[2]);
  y[3] = mfma32(v23, tri32(kArk, 3, 2), y[3]);
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
    for (int j = 0; j < 4; ++j) S[kb][j] = sn[kb][j] * sm.gc[16 * kb + 4 * g + j];
  }
  __builtin_amdgcn_s_setprio(0);

  // Lane (g, n) stores Y[16p + n][16w + 4g .. 16w + 4g + 3] (8 bytes).
  const uint32_t y_off = static_cast<uint32_t>(n) * row_bytes + 2 * (16 * w + 4 * g);
#pragma unroll
  for (int pb = 0; pb < 4; ++pb) {
    const int t = 16 * pb + n;
    u32x2 q;
    q.x = pack2<T>(scale * y[pb][0], scale * y[pb][1]);
    q.y = pack2<T>(scale * y[pb][2], scale * y[pb][3]);
    __builtin_amdgcn_raw_buffer_store_b64(q, out_rs, (t >= lo && t < hi) ? y_off : kDropOffset,
                                          static_cast<int>(16 * pb * row_bytes), 0);
  }
}

// The sequence of the given rank in order of decreasing length (ties in
// index order), for batches of at most 64 sequences: lane s holds sequence
// s's length, counts the sequences ahead of it, and the lane whose count is
// the rank names the sequence. Wave-uniform; every wave computes it alike.
__device__ __forceinline__ int sequence_by_length_rank(const ChunkFwdParams& p, int rank,
                                                       int lane) {
  const int count = p.longest_first_sequences;
  const int len = lane < count ? p.cu_seqlens[lane + 1] - p.cu_seqlens[lane] : -1;
  int ahead = 0;
  for (int j = 0; j < count; ++j) {
    const int lj = __builtin_amdgcn_readlane(len, j);
    ahead += (lj > len || (lj == len && j < lane)) ? 1 : 0;
  }
  const uint64_t hit = __builtin_amdgcn_ballot_w64(lane < count && ahead == rank);
  return hit != 0 ? static_cast<int>(__builtin_ctzll(hit)) : rank;
}

// kLean: the instantiation for calls with none of the optional layouts --
// no segment lists, boundary or interior states, every-16-token checkpoints,
// state_dot_a, read-only or absent state (the prefill op and the recurrent
// operator's chunk route). Those paths then compile away, and with them the
// scalar registers their descriptors and offsets would hold across the chunk
// loop (spilled to VGPR lanes and reloaded every chunk otherwise).
template <typename T, DecayMode M, typename PoolT, bool kPrecise, bool kLean>
__global__ __launch_bounds__(kChunkThreads, kPrecise ? 1 : 2) void chunk_fwd_kernel(
    ChunkFwdParams p) {
  __shared__ ChunkSmem sm;
  __shared__ ExtraTiles<kPrecise> ext;
  using S16 = typename IoTraits<T>::storage;

  if (p.status != nullptr && p.status[0] != 0) {
    fill_nan<T>(static_cast<S16*>(p.out), p.out_elems);
    return;
  }
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int g = lane >> 4;
  const int n = lane & 15;
  const int tp = lane & 7;   // token pair
  const int kg = lane >> 3;  // feature group
  const int heads = p.num_heads;
  int seq = blockIdx.x / heads;
  if (p.longest_first_sequences > 0) seq = sequence_by_length_rank(p, seq, lane);
  const int head = blockIdx.x % heads;
  // Metadata values are workgroup-uniform; readfirstlane keeps them (and
  // every buffer descriptor derived from them) in scalar registers.
  const int slot = uniform(p.slots != nullptr ? p.slots[seq] : seq);
  if (slot < 0 || slot >= p.state_slots) return;

  // Segments: the lists of seg_offsets, or (seg_offsets null, seg_starts
  // given) exactly one segment per sequence, segment s for sequence s.
  const bool segmented = !kLean && p.seg_starts != nullptr;
  const bool fill_only = !kLean && p.fill_only;
  const bool boundary16 = !kLean && p.boundary16;
  float* const boundary = kLean ? nullptr : p.boundary;
  float* const interior = kLean ? nullptr : p.interior;
  float* const state_dot_a = kLean ? nullptr : p.state_dot_a;
  const bool has_state = kLean || p.state != nullptr;
  int seg_lo = 0, seg_hi = 1;
  if (!kLean && p.seg_offsets != nullptr) {
    seg_lo = uniform(max(p.seg_offsets[seq], 0));
    seg_hi = uniform(min(p.seg_offsets[seq + 1], p.num_segments));
  } else if (segmented) {
    seg_lo = seq;
    seg_hi = min(seq + 1, p.num_segments);
  }

  // Interior-state fill (replay layout, one segment per unit): a segment of
  // at most one chunk has no interior state, so its unit ends before it
  // loads the start state or any token row.
  if (fill_only) {
    if (seg_lo >= seg_hi) return;
    const int tb = uniform(max(p.seg_starts[seg_lo], 0));
    const int te = uniform(min(p.seg_ends[seg_lo], p.total_tokens));
    if (te - tb <= kChunk) return;
  }

  float bias[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) bias[e] = 0.0f;
  if constexpr (M == DecayMode::kLogits) {
    if (p.bias != nullptr) {
      unpack8<T>(load_row8<T>(p.bias, static_cast<int64_t>(head) * kHead + 8 * kg), bias);
    }
  }

  // Wave w's state slice: S[16kb + 4g + j][16w + n] in S[kb][j]. Element
  // (row, col) of a 64 x 64 state is at byte (row * 64 + col) * size.
  using PS = typename IoTraits<PoolT>::storage;
  constexpr int kPoolBytes = static_cast<int>(sizeof(PS));
  const int64_t sbase = (static_cast<int64_t>(slot) * heads + head) * kHead * kHead;
  const auto state_rs =
      has_state
          ? buffer_rsrc(static_cast<PS*>(p.state) + sbase, kHead * kHead * kPoolBytes)
          : buffer_rsrc(static_cast<PS*>(nullptr), 0u);
  const uint32_t s_off = static_cast<uint32_t>((4 * g) * kHead + 16 * wave + n) * kPoolBytes;
  // A null state means S0 = 0 and no final state (the pretraining layout).
  f32x4 S[4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int so = (16 * kb + j) * kHead * kPoolBytes;
      if (!has_state) {
        S[kb][j] = 0.0f;
      } else if constexpr (kPoolBytes == 4) {
        S[kb][j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(state_rs, s_off, so, 0));
      } else {
        S[kb][j] = to_f32<PoolT>(__builtin_amdgcn_raw_buffer_load_b16(state_rs, s_off, so, 0));
      }
    }
  }

  // Segment bounds, 64 segments at a time in VGPR lanes (lane i: segment
  // cache_base + i), read back with readlane: a per-segment memory read would
  // need a vmcnt wait, which on gfx9's in-order counter also waits for every
  // output store still in flight.
  int cache_base = seg_hi;
  int starts_v = 0, ends_v = 0;
  auto seg_range = [&](int seg, int& t_begin, int& t_end) {
    if (segmented) {
      if (seg < cache_base || seg >= cache_base + 64) {
        cache_base = seg;
        const int idx = seg + lane;
        starts_v = idx < seg_hi ? p.seg_starts[idx] : 0;
        ends_v = idx < seg_hi ? p.seg_ends[idx] : 0;
        __builtin_amdgcn_s_waitcnt(0xF70);  // vmcnt(0): nothing pending at the join
      }
      t_begin = __builtin_amdgcn_readlane(starts_v, seg - cache_base);
      t_end = __builtin_amdgcn_readlane(ends_v, seg - cache_base);
    } else if (p.dense_t > 0) {
      t_begin = seq * p.dense_t;
      t_end = t_begin + p.dense_t;
    } else {
      t_begin = p.cu_seqlens[seq];
      t_end = p.cu_seqlens[seq + 1];
    }
    t_begin = uniform(max(t_begin, 0));
    t_end = uniform(min(t_end, p.total_tokens));
  };
  // Chunk following (seg, c0): c0 + 64 in the same segment, else the start
  // of the next non-empty segment. Returns false at the end of the sequence.
  auto next_chunk = [&](int& seg, int& c0, int& c_end) {
    c0 += kChunk;
    while (c0 >= c_end) {
      if (++seg >= seg_hi) return false;
      seg_range(seg, c0, c_end);
    }
    return true;
  };
  using S16c = typename IoTraits<T>::storage;
  const uint32_t row_bytes = static_cast<uint32_t>(heads) * kHead * 2;
  // Per-lane byte offset inside a chunk's rows in the prepare layout (token
  // 16w + 2tp [+1], features 8kg..8kg+7).
  const uint32_t prep_off = static_cast<uint32_t>(16 * wave + 2 * tp) * row_bytes + 16 * kg;
  // Row loads of one chunk in six pieces (piece i: tensor w, a, r, b, k, v
  // in prepare's order of use), two 16-byte loads per lane each.
  auto load_piece = [&](ChunkRows& rows, int c0, int ntok, int piece) {
    const int64_t base = (static_cast<int64_t>(c0) * heads + head) * kHead;
    const uint32_t bytes = static_cast<uint32_t>(ntok) * row_bytes;
    const void* src = piece == 0 ? p.decay : piece == 1 ? p.a : piece == 2 ? p.r
                    : piece == 3 ? p.b : piece == 4 ? p.k : p.v;
    const auto rs = buffer_rsrc(static_cast<const S16c*>(src) + base, bytes);
    uint4* dst = piece == 0 ? rows.w : piece == 1 ? rows.a : piece == 2 ? rows.r
               : piece == 3 ? rows.b : piece == 4 ? rows.k : rows.v;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      uint32_t off;
      int so;
      if (piece == 5) {
        const int v_piece = tid + 256 * s;
        off = static_cast<uint32_t>(v_piece >> 3) * row_bytes + 16 * (v_piece & 7);
        so = 0;
      } else {
        off = prep_off;
        so = s * static_cast<int>(row_bytes);
      }
      const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rs, off, so, 0);
      dst[s] = make_uint4(x.x, x.y, x.z, x.w);
    }
  };
  auto load_rows = [&](ChunkRows& rows, int c0, int ntok) {
#pragma unroll
    for (int piece = 0; piece < 6; ++piece) load_piece(rows, c0, ntok, piece);
  };
  // The main path issues the state pass's output stores between a chunk's
  // row loads and the prepare that reads them. Paths that load rows without
  // a state pass after them issue as many dropped stores, so that on every
  // path into the prepare the compiler counts them and waits for the loads
  // alone (the memory counter retires in order; at a join the compiler keeps
  // the path with the fewest instructions after the loads).
  auto pad_after_rows = [&]() {
    const auto nrs = buffer_rsrc(static_cast<float*>(nullptr), 0u);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      __builtin_amdgcn_raw_buffer_store_b32(0u, nrs, kDropOffset, 4 * i, 0);
    }
  };

  ChunkRows rows;
  {
    int seg = seg_lo, c0 = 0, c_end = 0;
    if (seg < seg_hi) seg_range(seg, c0, c_end);
    if (seg < seg_hi && c0 < c_end) load_rows(rows, c0, min(kChunk, c_end - c0));
    pad_after_rows();
  }
  for (int seg = seg_lo; seg < seg_hi; ++seg) {
    int t_begin, t_end;
    seg_range(seg, t_begin, t_end);
    // The state at the segment start, written after the first chunk's
    // prepare: stores issued here, between the row loads of that chunk
    // (made during the previous chunk) and their first use, would be waited
    // for with them (the memory counter retires in order). Segments that
    // reach no prepare (empty, or skipped by fill_only) store it here.
    auto store_boundary = [&]() {
      const auto brs = buffer_rsrc(
          boundary + (static_cast<int64_t>(seg) * heads + head) * kHead * kHead,
          kHead * kHead * 4);
      const uint32_t b_off = static_cast<uint32_t>((4 * g) * kHead + 16 * wave + n) * 4;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(S[kb][j]), brs, b_off,
                                                (16 * kb + j) * kHead * 4, 0);
        }
      }
    };
    const bool want_boundary = boundary != nullptr && !boundary16;
    const bool defer_boundary = t_end > t_begin && !fill_only;
    if (want_boundary && !defer_boundary) store_boundary();
    if (fill_only && t_end - t_begin <= kChunk) continue;
    for (int c0 = t_begin; c0 < t_end; c0 += kChunk) {
      const int ntok = min(kChunk, t_end - c0);
      if (interior != nullptr && c0 > t_begin) {
        const auto irs = buffer_rsrc(
            interior + (static_cast<int64_t>(c0 / kChunk) * heads + head) * kHead * kHead,
            kHead * kHead * 4);
        const uint32_t i_off = static_cast<uint32_t>((4 * g) * kHead + 16 * wave + n) * 4;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(S[kb][j]), irs, i_off,
                                                  (16 * kb + j) * kHead * 4, 0);
          }
        }
      }
      if (fill_only && c0 + kChunk >= t_end) break;
      int nseg = seg, nc0 = c0, nend = t_end;
      const bool has_next = next_chunk(nseg, nc0, nend);
      // Every-16-tokens boundary layout [B, H, dense_t / 16, D, D]: the state
      // at token c0 + i (i a multiple of 16) of this sequence.
      const int64_t b16_base = (static_cast<int64_t>(seq) * heads + head) * (p.dense_t / 16) +
                               (c0 - t_begin) / 16;
      auto b16_rs = [&](int i, int count) {
        if (!boundary16 || count <= 0) return buffer_rsrc(static_cast<float*>(nullptr), 0u);
        return buffer_rsrc(boundary + (b16_base + i / 16) * kHead * kHead,
                           static_cast<uint32_t>(count) * kHead * kHead * 4);
      };
      auto store_b16 = [&](int i) {
        const auto brs = b16_rs(i, 1);
        const uint32_t b_off = static_cast<uint32_t>((4 * g) * kHead + 16 * wave + n) * 4;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(S[kb][j]), brs, b_off,
                                                  (16 * kb + j) * kHead * 4, 0);
          }
        }
      };
      if (boundary16) store_b16(0);
      // One pass over [lo, hi) per iteration. The first pass prepares the
      // whole chunk; if its decay span is above the limit (strong decay), the
      // chunk is redone as 16-token sub-chunks, or 4-token ones where a
      // 16-token block is still too strong, and `rows` keeps this chunk's
      // rows until the last pass. Otherwise the next chunk's rows are loaded
      // right after the first prepare, while the products run.
      Spans spans{};
      bool whole = true, first = true;
      int lo = 0, hi = ntok;
      for (;;) {
        const Spans cur = (lo == 0 && hi == kChunk)
                              ? prepare<T, M, true, kPrecise>(sm, ext, rows, bias, lo, hi)
                              : prepare<T, M, false, kPrecise>(sm, ext, rows, bias, lo, hi);
        if (first) {
          if (want_boundary && defer_boundary && c0 == t_begin) store_boundary();
          first = false;
          spans = cur;
          whole = cur.whole;
          if (!whole) {
            hi = min(spans.block[0] ? 16 : 4, ntok);
            continue;
          }
        }
        // A whole chunk's pass requests the next chunk's rows in pieces
        // during the products. The request is unconditional: with no next
        // chunk the range is empty and the loads return zeros (a skipped
        // load would make the compiler's in-order wait counts too strict).
        if (whole) {
          intra_chunk<kPrecise>(sm, ext, [&](int piece) {
            load_piece(rows, has_next ? nc0 : c0, has_next ? min(kChunk, nend - nc0) : 0,
                       piece);
          });
        } else {
          intra_chunk<kPrecise>(sm, ext, [](int) {});
        }
        {
          const int64_t base = (static_cast<int64_t>(c0) * heads + head) * kHead;
          const auto out_rs = buffer_rsrc(
              p.out != nullptr ? static_cast<S16c*>(p.out) + base : nullptr,
              p.out != nullptr ? static_cast<uint32_t>(ntok) * row_bytes : 0u);
          const auto sda_rs = buffer_rsrc(
              state_dot_a != nullptr ? state_dot_a + base : nullptr,
              state_dot_a != nullptr ? 2u * static_cast<uint32_t>(ntok) * row_bytes : 0u);
          const int nsub = (boundary16 && whole) ? (ntok - 1) / 16 : 0;
          state_pass<T, kPrecise>(sm, ext, S, sm.vt, out_rs, sda_rs, state_dot_a != nullptr,
                                  row_bytes, p.scale, lo, hi, b16_rs(16, nsub), nsub);
        }
        if (whole) break;
        if (boundary16 && hi % 16 == 0 && hi < ntok) store_b16(hi);
        lo = hi;
        if (lo >= ntok) break;
        const int q = lo >> 4;
        hi = min(lo + (spans.block_ok(q) ? 16 : 4), min(16 * q + 16, ntok));
      }
      if (!whole) {
        load_rows(rows, has_next ? nc0 : c0, has_next ? min(kChunk, nend - nc0) : 0);
        pad_after_rows();
      }
    }
  }

  if (!has_state || (!kLean && p.read_only_state)) return;
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int so = (16 * kb + j) * kHead * kPoolBytes;
      if constexpr (kPoolBytes == 4) {
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(S[kb][j]), state_rs, s_off, so, 0);
      } else {
        __builtin_amdgcn_raw_buffer_store_b16(from_f32<PoolT>(S[kb][j]), state_rs, s_off, so, 0);
      }
    }
  }
}

template <typename T, DecayMode M, typename PoolT, bool kPrecise = false>
int launch_chunk(const ChunkFwdParams& p, int units, hipStream_t stream) {
  if (p.num_heads > kMaxChunkHeads) {
    return set_error(FRWKV_ERR_UNSUPPORTED, "chunked kernels take at most %d heads, got %d",
                     kMaxChunkHeads, p.num_heads);
  }
  const bool lean = p.seg_starts == nullptr && p.seg_offsets == nullptr &&
                    p.boundary == nullptr && p.state_dot_a == nullptr &&
                    p.interior == nullptr && !p.fill_only && !p.boundary16 &&
                    !p.read_only_state && p.state != nullptr;
  if (lean) {
    hipLaunchKernelGGL((chunk_fwd_kernel<T, M, PoolT, kPrecise, true>), dim3(units),
                       dim3(kChunkThreads), 0, stream, p);
  } else {
    hipLaunchKernelGGL((chunk_fwd_kernel<T, M, PoolT, kPrecise, false>), dim3(units),
                       dim3(kChunkThreads), 0, stream, p);
  }
  return check_launch("chunk_fwd_kernel");
}

template <typename T, typename PoolT>
int dispatch_chunk_decay(const ChunkFwdParams& p, int decay_mode, int units,
                         hipStream_t stream) {
  if (decay_mode == FRWKV_DECAY_LOGITS) {
    return launch_chunk<T, DecayMode::kLogits, PoolT>(p, units, stream);
  }
  if (decay_mode == FRWKV_DECAY_RAW_W) {
    if (p.bias != nullptr) {
      return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                       "decay_bias is only defined for the logits decay mode");
    }
    return launch_chunk<T, DecayMode::kRawW, PoolT>(p, units, stream);
  }
  return set_error(FRWKV_ERR_INVALID_ARGUMENT, "unknown decay mode %d", decay_mode);
}

template <typename PoolT>
int dispatch_chunk_io(const ChunkFwdParams& p, int io_dtype, int decay_mode, int units,
                      hipStream_t stream) {
  switch (io_dtype) {
    case FRWKV_DTYPE_BF16:
      return dispatch_chunk_decay<Bf16, PoolT>(p, decay_mode, units, stream);
    case FRWKV_DTYPE_F16:
      return dispatch_chunk_decay<F16, PoolT>(p, decay_mode, units, stream);
    default:
      return set_error(FRWKV_ERR_UNSUPPORTED,
                       "chunked kernels take float16 or bfloat16 tokens (io dtype %d)",
                       io_dtype);
  }
}

int check_token_pointers(const void* r, const void* decay, const void* k, const void* v,
                         const void* a, const void* b, const void* out) {
  if (!r || !decay || !k || !v || !a || !b || !out) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT, "null token pointer argument");
  }
  return FRWKV_OK;
}

}  // namespace
}  // namespace frwkv

extern "C" int frwkv_chunk_forward(
    int io_dtype, int decay_mode, int pool_dtype, int32_t num_sequences,
    int32_t num_heads, int32_t head_size, int32_t total_tokens, int32_t state_pool_size,
    const int32_t* cu_seqlens, const int32_t* state_indices,
    const int32_t* metadata_status, void* state_pool, const void* r, const void* decay,
    const void* decay_bias, const void* k, const void* v, const void* a, const void* b,
    void* output, float scale, void* stream) {
  using namespace frwkv;
  if (!cu_seqlens || !state_indices || !metadata_status || !state_pool) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT, "frwkv_chunk_forward: null pointer argument");
  }
  int rc = check_token_pointers(r, decay, k, v, a, b, output);
  if (rc != FRWKV_OK) return rc;
  if (head_size != 64) {
    return set_error(FRWKV_ERR_UNSUPPORTED, "chunked kernels support head size 64, got %d",
                     head_size);
  }
  if (num_sequences <= 0 || num_sequences > 65535 || num_heads <= 0 || total_tokens <= 0 ||
      state_pool_size <= 0) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_chunk_forward: sizes must be positive (B=%d, H=%d, N=%d, slots=%d)",
                     num_sequences, num_heads, total_tokens, state_pool_size);
  }
  if (!__builtin_isfinite(scale)) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT, "scale must be finite");
  }
  ChunkFwdParams p{};
  p.num_heads = num_heads;
  p.longest_first_sequences = num_sequences <= 64 ? num_sequences : 0;
  p.total_tokens = total_tokens;
  p.state_slots = state_pool_size;
  p.cu_seqlens = cu_seqlens;
  p.slots = state_indices;
  p.status = metadata_status;
  p.state = state_pool;
  p.r = r;
  p.decay = decay;
  p.bias = decay_bias;
  p.k = k;
  p.v = v;
  p.a = a;
  p.b = b;
  p.out = output;
  p.scale = scale;
  p.out_elems = static_cast<int64_t>(total_tokens) * num_heads * head_size;
  const int units = num_sequences * num_heads;
  auto s = static_cast<hipStream_t>(stream);
  if (pool_dtype == FRWKV_DTYPE_F32) return dispatch_chunk_io<float>(p, io_dtype, decay_mode, units, s);
  if (pool_dtype == FRWKV_DTYPE_BF16) return dispatch_chunk_io<Bf16>(p, io_dtype, decay_mode, units, s);
  return set_error(FRWKV_ERR_UNSUPPORTED, "state pool must be float32 or bfloat16 (dtype %d)",
                   pool_dtype);
}

extern "C" int frwkv_statetune_forward(
    int io_dtype, int decay_mode, int32_t num_sequences, int32_t num_heads,
    int32_t head_size, int32_t total_tokens, int32_t num_chunks,
    const int32_t* sequence_chunk_offsets, const int32_t* chunk_token_starts,
    const int32_t* chunk_token_ends, float* state, const void* r, const void* decay,
    const void* decay_bias, const void* k, const void* v, const void* a, const void* b,
    void* output, float* boundary, float* state_dot_a, float* interior, float scale,
    void* stream) {
  using namespace frwkv;
  if (!sequence_chunk_offsets || !chunk_token_starts || !chunk_token_ends || !state ||
      !boundary || !state_dot_a) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_statetune_forward: null pointer argument");
  }
  int rc = check_token_pointers(r, decay, k, v, a, b, output);
  if (rc != FRWKV_OK) return rc;
  if (num_sequences <= 0 || num_heads <= 0 || total_tokens <= 0 || num_chunks <= 0) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_statetune_forward: sizes must be positive");
  }
  if (!__builtin_isfinite(scale)) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT, "scale must be finite");
  }
  if (head_size == 128 || head_size == 256) {
    return frwkv_train_recurrent_forward(io_dtype, decay_mode, num_sequences, num_heads,
                                         head_size, total_tokens, sequence_chunk_offsets,
                                         chunk_token_starts, chunk_token_ends, num_chunks,
                                         /*dense_t=*/0,
                                         state, r, decay, decay_bias, k, v, a, b, output,
                                         boundary, state_dot_a, interior, /*fill_only=*/0,
                                         scale, stream);
  }
  if (head_size != 64) {
    return set_error(FRWKV_ERR_UNSUPPORTED, "head size must be 64, 128, or 256, got %d",
                     head_size);
  }
  ChunkFwdParams p{};
  p.num_heads = num_heads;
  p.total_tokens = total_tokens;
  p.state_slots = num_sequences;
  p.seg_offsets = sequence_chunk_offsets;
  p.seg_starts = chunk_token_starts;
  p.seg_ends = chunk_token_ends;
  p.num_segments = num_chunks;
  p.state = state;
  p.r = r;
  p.decay = decay;
  p.bias = decay_bias;
  p.k = k;
  p.v = v;
  p.a = a;
  p.b = b;
  p.out = output;
  p.boundary = boundary;
  p.state_dot_a = state_dot_a;
  p.interior = interior;
  p.scale = scale;
  p.out_elems = static_cast<int64_t>(total_tokens) * num_heads * head_size;
  return dispatch_chunk_io<float>(p, io_dtype, decay_mode, num_sequences * num_heads,
                                  static_cast<hipStream_t>(stream));
}

extern "C" size_t frwkv_statetune_interior_bytes(int32_t head_size, int32_t num_heads,
                                                 int32_t total_tokens) {
  if (num_heads <= 0 || total_tokens <= 0) return 0;
  const int64_t piece = head_size == 64 ? 64 : 16;
  const int64_t slots = (total_tokens + piece - 1) / piece;
  // Head size 128 keeps the states in bf16 (the piece kernels' own order).
  const int64_t bytes = head_size == 128 ? 2 : 4;
  return static_cast<size_t>(slots * num_heads * head_size * head_size * bytes);
}

extern "C" int frwkv_statetune_interior(int io_dtype, int decay_mode, int32_t num_heads,
                                        int32_t head_size, int32_t total_tokens,
                                        int32_t num_chunks, const int32_t* chunk_token_starts,
                                        const int32_t* chunk_token_ends, const float* boundary,
                                        const void* r, const void* decay, const void* decay_bias,
                                        const void* k, const void* v, const void* a,
                                        const void* b, float* interior, void* stream) {
  using namespace frwkv;
  if (!chunk_token_starts || !chunk_token_ends || !boundary || !interior || !r || !decay ||
      !k || !v || !a || !b) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT, "frwkv_statetune_interior: null pointer argument");
  }
  if (num_chunks <= 0 || num_heads <= 0 || total_tokens <= 0) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_statetune_interior: sizes must be positive");
  }
  if (head_size == 128 || head_size == 256) {
    return frwkv_train_recurrent_forward(io_dtype, decay_mode, num_chunks, num_heads, head_size,
                                         total_tokens, nullptr, chunk_token_starts,
                                         chunk_token_ends, num_chunks, /*dense_t=*/0,
                                         const_cast<float*>(boundary), r, decay, decay_bias, k,
                                         v, a, b, nullptr, nullptr, nullptr, interior,
                                         /*fill_only=*/1, 1.0f, stream);
  }
  if (head_size != 64) {
    return set_error(FRWKV_ERR_UNSUPPORTED, "head size must be 64, 128, or 256, got %d",
                     head_size);
  }
  ChunkFwdParams p{};
  p.num_heads = num_heads;
  p.total_tokens = total_tokens;
  p.state_slots = num_chunks;
  p.seg_starts = chunk_token_starts;
  p.seg_ends = chunk_token_ends;
  p.num_segments = num_chunks;
  p.state = const_cast<float*>(boundary);
  p.read_only_state = 1;
  p.r = r;
  p.decay = decay;
  p.bias = decay_bias;
  p.k = k;
  p.v = v;
  p.a = a;
  p.b = b;
  p.interior = interior;
  p.fill_only = 1;
  p.scale = 1.0f;
  return dispatch_chunk_io<float>(p, io_dtype, decay_mode, num_chunks * num_heads,
                                  static_cast<hipStream_t>(stream));
}

extern "C" int frwkv_pretrain_forward(int io_dtype, int decay_mode, int32_t batch,
                                      int32_t tokens, int32_t num_heads, int32_t head_size,
                                      const void* r, const void* decay, const void* k,
                                      const void* v, const void* a, const void* b,
                                      void* output, float* boundary, float* state_dot_a,
                                      void* stream) {
  using namespace frwkv;
  if (!boundary || !state_dot_a) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT, "frwkv_pretrain_forward: null pointer argument");
  }
  int rc = check_token_pointers(r, decay, k, v, a, b, output);
  if (rc != FRWKV_OK) return rc;
  if (batch <= 0 || tokens <= 0 || num_heads <= 0 || tokens % 16 != 0) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_pretrain_forward: B, H > 0 and T a positive multiple of 16 "
                     "(B=%d, T=%d, H=%d)", batch, tokens, num_heads);
  }
  if (static_cast<int64_t>(batch) * tokens > INT32_MAX) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT, "frwkv_pretrain_forward: B * T too large");
  }
  if (head_size == 128 || head_size == 256) {
    return frwkv_train_recurrent_forward(io_dtype, decay_mode, batch, num_heads, head_size,
                                         batch * tokens, nullptr, nullptr, nullptr, 0, tokens,
                                         /*state=*/nullptr, r, decay, /*decay_bias=*/nullptr, k,
                                         v, a, b, output, boundary, state_dot_a,
                                         /*interior=*/nullptr, /*fill_only=*/0, 1.0f, stream);
  }
  if (head_size != 64) {
    return set_error(FRWKV_ERR_UNSUPPORTED, "head size must be 64, 128, or 256, got %d",
                     head_size);
  }
  ChunkFwdParams p{};
  p.num_heads = num_heads;
  p.total_tokens = batch * tokens;
  p.state_slots = batch;
  p.dense_t = tokens;
  p.boundary16 = 1;
  p.r = r;
  p.decay = decay;
  p.k = k;
  p.v = v;
  p.a = a;
  p.b = b;
  p.out = output;
  p.boundary = boundary;
  p.state_dot_a = state_dot_a;
  p.scale = 1.0f;
  p.out_elems = static_cast<int64_t>(batch) * tokens * num_heads * head_size;
  return dispatch_chunk_io<float>(p, io_dtype, decay_mode, batch * num_heads,
                                  static_cast<hipStream_t>(stream));
}

extern "C" int frwkv_chunk_replay(int io_dtype, int decay_mode, int32_t num_chunks,
                                  int32_t num_heads, int32_t head_size, int32_t total_tokens,
                                  const int32_t* chunk_token_starts,
                                  const int32_t* chunk_token_ends, const float* boundary,
                                  const void* r, const void* decay, const void* decay_bias,
                                  const void* k, const void* v, const void* a, const void* b,
                                  void* output, float* state_dot_a, float scale,
                                  void* stream) {
  using namespace frwkv;
  if (!chunk_token_starts || !chunk_token_ends || !boundary || !state_dot_a) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT, "frwkv_chunk_replay: null pointer argument");
  }
  int rc = check_token_pointers(r, decay, k, v, a, b, output);
  if (rc != FRWKV_OK) return rc;
  if (num_chunks <= 0 || num_heads <= 0 || total_tokens <= 0) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT, "frwkv_chunk_replay: sizes must be positive");
  }
  if (!__builtin_isfinite(scale)) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT, "scale must be finite");
  }
  if (head_size != 64) {
    // Other head sizes: the fp32 per-token kernel, one unit per chunk.
    return frwkv_replay_recurrent(io_dtype, decay_mode, num_chunks, num_heads, head_size,
                                  total_tokens, chunk_token_starts, chunk_token_ends,
                                  boundary, r, decay, decay_bias, k, v, a, b, output,
                                  state_dot_a, scale, stream);
  }
  ChunkFwdParams p{};
  p.num_heads = num_heads;
  p.total_tokens = total_tokens;
  p.state_slots = num_chunks;
  p.seg_starts = chunk_token_starts;
  p.seg_ends = chunk_token_ends;
  p.num_segments = num_chunks;
  p.state = const_cast<float*>(boundary);
  p.read_only_state = 1;
  p.r = r;
  p.decay = decay;
  p.bias = decay_bias;
  p.k = k;
  p.v = v;
  p.a = a;
  p.b = b;
  p.out = output;
  p.state_dot_a = state_dot_a;
  p.scale = scale;
  p.out_elems = static_cast<int64_t>(total_tokens) * num_heads * head_size;
  return dispatch_chunk_io<float>(p, io_dtype, decay_mode, num_chunks * num_heads,
                                  static_cast<hipStream_t>(stream));
}

// The recurrent operator's route for long sequences (called by
// frwkv_recurrent_forward): bf16 tokens, head size 64, fp32 pool, the
// split-precision variant of the chunk kernel. Arguments as there; the
// caller has checked pointers and sizes.
int frwkv_recurrent_chunked_forward(int decay_mode, int32_t num_sequences, int32_t num_heads,
                                    int32_t total_tokens, int32_t state_pool_size,
                                    const int32_t* cu_seqlens, const int32_t* state_indices,
                                    const int32_t* metadata_status, float* state_pool,
                                    const void* r, const void* decay, const void* decay_bias,
                                    const void* k, const void* v, const void* a, const void* b,
                                    void* output, float scale, void* stream) {
  using namespace frwkv;
  ChunkFwdParams p{};
  p.num_heads = num_heads;
  p.longest_first_sequences = num_sequences <= 64 ? num_sequences : 0;
  p.total_tokens = total_tokens;
  p.state_slots = state_pool_size;
  p.cu_seqlens = cu_seqlens;
  p.slots = state_indices;
  p.status = metadata_status;
  p.state = state_pool;
  p.r = r;
  p.decay = decay;
  p.bias = decay_bias;
  p.k = k;
  p.v = v;
  p.a = a;
  p.b = b;
  p.out = output;
  p.scale = scale;
  p.out_elems = static_cast<int64_t>(total_tokens) * num_heads * kHead;
  const int units = num_sequences * num_heads;
  auto s = static_cast<hipStream_t>(stream);
  if (decay_mode == FRWKV_DECAY_LOGITS) {
    return launch_chunk<Bf16, DecayMode::kLogits, float, true>(p, units, s);
  }
  if (decay_mode == FRWKV_DECAY_RAW_W) {
    if (decay_bias != nullptr) {
      return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                       "decay_bias is only defined for the logits decay mode");
    }
    return launch_chunk<Bf16, DecayMode::kRawW, float, true>(p, units, s);
  }
  return set_error(FRWKV_ERR_INVALID_ARGUMENT, "unknown decay mode %d", decay_mode);
}
