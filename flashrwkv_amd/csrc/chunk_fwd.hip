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
//   At = a 2^Gp, Rt = r 2^G, Bh = b 2^-G, Kh = k 2^-G, Bt = b 2^(GC-G),
//   Kt = k 2^(GC-G);
//   Lab = strict_lower(At Bh^T), Lak = strict_lower(At Kh^T),
//   Arb = lower(Rt Bh^T),        Ark = lower(Rt Kh^T);
//   SA = (I - Lab)^{-1} (At S0 + Lak V)       (rows are sa_t)
//   Y  = scale (Rt S0 + Arb SA + Ark V)
//   S' = diag(2^GC) S0 + Bt^T SA + Kt^T V.
// Every exponent above is <= 0 except the 2^-G of Bh/Kh, bounded by the
// chunk's decay span -GC. The kernel keeps that span <= 80 (log2 units): a
// chunk whose span is larger is processed as 16-token sub-chunks, and a
// 16-token block whose span is still larger as 4-token sub-chunks. The
// per-token log2 retention is clamped to [-20, 0] (w in [2^-20, 1]), so
// 4-token spans never exceed 80; below 2^-20 the clamp changes S_t by less
// than 1e-6 |S_{t-1}|, far under bf16 resolution.
//
// Work decomposition (one 256-thread workgroup per (sequence, head)):
//   * prepare: the chunk's 64 tokens x 64 features are decoded once (two
//     tokens x 8 features per thread), the cumulative decay is a wave
//     shuffle scan plus a cross-wave carry, and the scaled operands go to LDS
//     as bf16 ([token][feature] tiles and, for products contracting over
//     tokens, [feature][token] tiles);
//   * intra-chunk products: the 40 lower-triangular 16x16 tiles of Lab,
//     Lak, Arb, Ark are spread over the four waves; wave p also inverts the
//     diagonal block I - Lab_pp in fp32 (forward substitution);
//   * state-dependent part: wave w owns value columns 16w..16w+15. Its slice
//     of the fp32 state lives in MFMA accumulators for the whole sequence;
//     the block forward substitution SA_p = T_pp (rhs_p + sum_q Lab_pq SA_q),
//     the output tiles and the state update chain through registers, so this
//     part has no barrier.
#include "capi_internal.h"
#include "wkv7_device.h"
#include "wkv7_mfma.h"

namespace frwkv {
namespace {

constexpr int kChunk = 64;
constexpr int kHead = 64;
constexpr int kChunkThreads = 256;
constexpr float kSpanLimit = 80.0f;   // log2 units
constexpr float kLog2Min = -20.0f;    // per-token clamp of log2 retention

struct ChunkSmem {
  uint16_t at[kTileElems];   // [t][k]
  uint16_t rt[kTileElems];   // [t][k]
  uint16_t bh[kTileElems];   // [t][k]
  uint16_t kh[kTileElems];   // [t][k]
  uint16_t btT[kTileElems];  // [k][t]
  uint16_t ktT[kTileElems];  // [k][t]
  uint16_t vT[kTileElems];   // [v][t]
  uint16_t lab[kTileElems];  // [t][i]
  uint16_t lak[kTileElems];
  uint16_t arb[kTileElems];
  uint16_t ark[kTileElems];
  uint16_t tinv[4][16 * 24];  // (I - Lab_pp)^{-1}, [t][i], row stride 24
  float lpp[4][16 * 16];      // fp32 Lab_pp, [t][i]
  float gc[kHead];            // 2^GC per key feature
  float wave_tot[4][kHead];   // per-wave sums of log2 retention
};

struct ChunkFwdParams {
  int32_t num_heads;
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
};

// Raw token rows held by one thread: 2 tokens x 8 features of each input.
struct RawRows {
  uint4 r[2], w[2], k[2], v[2], a[2], b[2];
};

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

template <typename PoolT>
__device__ __forceinline__ float pool_load(const void* base, int64_t i) {
  return to_f32<PoolT>(static_cast<const typename IoTraits<PoolT>::storage*>(base)[i]);
}

template <typename PoolT>
__device__ __forceinline__ void pool_store(void* base, int64_t i, float x) {
  static_cast<typename IoTraits<PoolT>::storage*>(base)[i] = from_f32<PoolT>(x);
}

// log2 of the retention, clamped to [kLog2Min, 0].
template <DecayMode M>
__device__ __forceinline__ float log2_retention(float x) {
  const float lg = decay_log<M>(x) * kLog2E;
  return fminf(fmaxf(lg, kLog2Min), 0.0f);
}

struct Spans {
  float all;       // -GC over the prepared range
  float block[4];  // per 16-token block
};

// Decodes the thread's raw rows restricted to tokens [lo, hi) of the chunk,
// scans the decay and writes every scaled operand tile. Ends with a barrier.
template <typename T, DecayMode M>
__device__ Spans prepare(ChunkSmem& sm, const RawRows& raw, const float (&bias)[8],
                         int lo, int hi) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int tp = lane >> 3;
  const int kg = lane & 7;
  const int t0 = 16 * wave + 2 * tp;

  __syncthreads();  // earlier readers of the tiles are done

  float lg[2][8], rr[2][8], kk[2][8], vv[2][8], aa[2][8], bb[2][8];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const bool active = (t0 + s >= lo) && (t0 + s < hi);
    float wraw[8];
    unpack8<T>(raw.w[s], wraw);
    unpack8<T>(raw.r[s], rr[s]);
    unpack8<T>(raw.k[s], kk[s]);
    unpack8<T>(raw.v[s], vv[s]);
    unpack8<T>(raw.a[s], aa[s]);
    unpack8<T>(raw.b[s], bb[s]);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      lg[s][e] = active ? log2_retention<M>(wraw[e] + bias[e]) : 0.0f;
      if (!active) {
        rr[s][e] = 0.0f;
        kk[s][e] = 0.0f;
        vv[s][e] = 0.0f;
        aa[s][e] = 0.0f;
        bb[s][e] = 0.0f;
      }
    }
  }

  // Inclusive scan over the wave's 8 token pairs (lanes 8 apart share kg).
  float incl[8], pair[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    pair[e] = lg[0][e] + lg[1][e];
    incl[e] = pair[e];
  }
#pragma unroll
  for (int off = 8; off < 64; off <<= 1) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float y = __shfl_up(incl[e], off, 64);
      if (lane >= off) incl[e] += y;
    }
  }
  if (tp == 7) {
#pragma unroll
    for (int e = 0; e < 8; ++e) sm.wave_tot[wave][8 * kg + e] = incl[e];
  }
  __syncthreads();

  float base[8], total[8];
  Spans spans;
#pragma unroll
  for (int q = 0; q < 4; ++q) spans.block[q] = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    base[e] = 0.0f;
    total[e] = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float x = sm.wave_tot[q][8 * kg + e];
      if (q < wave) base[e] += x;
      total[e] += x;
      spans.block[q] = fmaxf(spans.block[q], -x);
    }
  }
  float span_all = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) span_all = fmaxf(span_all, -total[e]);
  // Max over the 8 feature groups (lane bits 0..2): every lane of every wave
  // ends with the same values, so branches on them are uniform.
#pragma unroll
  for (int off = 1; off < 8; off <<= 1) {
    span_all = fmaxf(span_all, __shfl_xor(span_all, off, 64));
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      spans.block[q] = fmaxf(spans.block[q], __shfl_xor(spans.block[q], off, 64));
    }
  }
  spans.all = span_all;

  float gtok[2][8], gprev[2][8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float excl = base[e] + incl[e] - pair[e];
    gprev[0][e] = excl;
    gtok[0][e] = excl + lg[0][e];
    gprev[1][e] = gtok[0][e];
    gtok[1][e] = gtok[0][e] + lg[1][e];
  }

  float btv[2][8], ktv[2][8];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int t = t0 + s;
    float atv[8], rtv[8], bhv[8], khv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float up = exp2f(gprev[s][e]);
      const float ug = exp2f(gtok[s][e]);
      const float dn = exp2f(-gtok[s][e]);
      const float tail = exp2f(total[e] - gtok[s][e]);
      atv[e] = aa[s][e] * up;
      rtv[e] = rr[s][e] * ug;
      bhv[e] = bb[s][e] * dn;
      khv[e] = kk[s][e] * dn;
      btv[s][e] = bb[s][e] * tail;
      ktv[s][e] = kk[s][e] * tail;
    }
    uint4 q;
    q = make_uint4(pack_bf16x2(atv[0], atv[1]), pack_bf16x2(atv[2], atv[3]),
                   pack_bf16x2(atv[4], atv[5]), pack_bf16x2(atv[6], atv[7]));
    *reinterpret_cast<uint4*>(sm.at + t * kTileStride + 8 * kg) = q;
    q = make_uint4(pack_bf16x2(rtv[0], rtv[1]), pack_bf16x2(rtv[2], rtv[3]),
                   pack_bf16x2(rtv[4], rtv[5]), pack_bf16x2(rtv[6], rtv[7]));
    *reinterpret_cast<uint4*>(sm.rt + t * kTileStride + 8 * kg) = q;
    q = make_uint4(pack_bf16x2(bhv[0], bhv[1]), pack_bf16x2(bhv[2], bhv[3]),
                   pack_bf16x2(bhv[4], bhv[5]), pack_bf16x2(bhv[6], bhv[7]));
    *reinterpret_cast<uint4*>(sm.bh + t * kTileStride + 8 * kg) = q;
    q = make_uint4(pack_bf16x2(khv[0], khv[1]), pack_bf16x2(khv[2], khv[3]),
                   pack_bf16x2(khv[4], khv[5]), pack_bf16x2(khv[6], khv[7]));
    *reinterpret_cast<uint4*>(sm.kh + t * kTileStride + 8 * kg) = q;
  }
  // Token-contiguous tiles: the thread's two tokens form one 32-bit pair.
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int row = (8 * kg + e) * kTileStride + t0;
    *reinterpret_cast<uint32_t*>(sm.btT + row) = pack_bf16x2(btv[0][e], btv[1][e]);
    *reinterpret_cast<uint32_t*>(sm.ktT + row) = pack_bf16x2(ktv[0][e], ktv[1][e]);
    *reinterpret_cast<uint32_t*>(sm.vT + row) = pack_bf16x2(vv[0][e], vv[1][e]);
  }
  if (wave == 0 && tp == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) sm.gc[8 * kg + e] = exp2f(total[e]);
  }
  __syncthreads();
  return spans;
}

// Intra-chunk products: 40 lower-triangular 16x16 tiles of Lab, Lak, Arb,
// Ark, plus the fp32 inverse of each diagonal block I - Lab_pp. Ends with a
// barrier.
__device__ void intra_chunk(ChunkSmem& sm) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int g = lane >> 4;
  const int n = lane & 15;

  // Tile (matrix m, target block p, source block q <= p). The stored tile
  // is M[t][i] = sum_k X[t][k] Y[i][k]; it is computed transposed (A = Y
  // rows, B = X rows) so each lane writes 4 consecutive i of one row t.
  auto tile = [&](int m, int p, int q) {
    const uint16_t* x = (m < 2) ? sm.at : sm.rt;
    const uint16_t* y = (m & 1) ? sm.kh : sm.bh;
    uint16_t* dst = (m == 0) ? sm.lab : (m == 1) ? sm.lak : (m == 2) ? sm.arb : sm.ark;
    f32x4 acc = zero4();
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      acc = mfma16(lds_operand(y, 16 * q + n, 16 * kb + 4 * g),
                   lds_operand(x, 16 * p + n, 16 * kb + 4 * g), acc);
    }
    const bool strict = m < 2;
    const int t = 16 * p + n;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = 16 * q + 4 * g + j;
      const bool keep = strict ? (i < t) : (i <= t);
      acc[j] = keep ? acc[j] : 0.0f;
    }
    lds_store_transposed(dst + (16 * p) * kTileStride + 16 * q, kTileStride, g, n, acc);
    if (m == 0 && p == q) {
#pragma unroll
      for (int j = 0; j < 4; ++j) sm.lpp[p][n * 16 + 4 * g + j] = acc[j];
    }
  };

  // Wave w first computes the diagonal Lab(w, w) and inverts it.
  tile(0, wave, wave);
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (lane < 16) {
    // Column j of (I - L)^{-1}: x = e_j + L x, rows in order.
    const float* l = sm.lpp[wave];
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float acc = (i == lane) ? 1.0f : 0.0f;
#pragma unroll
      for (int m = 0; m < i; ++m) acc = fmaf(l[i * 16 + m], x[m], acc);
      x[i] = acc;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) sm.tinv[wave][i * 24 + lane] = to_bf16_bits(x[i]);
  }

  // The other 36 tiles, 9 per wave.
  int item = 0;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
#pragma unroll
      for (int q = 0; q <= p; ++q) {
        if (m == 0 && p == q) continue;
        if ((item & 3) == wave) tile(m, p, q);
        ++item;
      }
    }
  }
  __syncthreads();
}

// State-dependent part of one prepared (sub-)chunk for wave w's value
// columns. Tokens outside [lo, hi) are zero rows of every operand; their
// outputs are not stored.
template <typename T>
__device__ void state_pass(const ChunkSmem& sm, f32x4 (&S)[4], const ChunkFwdParams& p,
                           int head, int64_t chunk_base, int lo, int hi) {
  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int lane = tid & 63;
  const int g = lane >> 4;
  const int n = lane & 15;

  i16x4 sb[4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) sb[kb] = to_operand(S[kb]);

  // rhs_p = At_p S0 + sum_q Lak_pq V_q      (rows t of block p, cols v of w)
  f32x4 sa[4];
  i16x4 sab[4];
#pragma unroll
  for (int pb = 0; pb < 4; ++pb) {
    f32x4 acc = zero4();
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      acc = mfma16(lds_operand(sm.at, 16 * pb + n, 16 * kb + 4 * g), sb[kb], acc);
    }
#pragma unroll
    for (int q = 0; q <= pb; ++q) {
      acc = mfma16(lds_operand(sm.lak, 16 * pb + n, 16 * q + 4 * g),
                   lds_operand(sm.vT, 16 * w + n, 16 * q + 4 * g), acc);
    }
    // Block forward substitution: SA_p = T_pp (rhs_p + sum_{q<p} Lab_pq SA_q).
#pragma unroll
    for (int q = 0; q < pb; ++q) {
      acc = mfma16(lds_operand(sm.lab, 16 * pb + n, 16 * q + 4 * g), sab[q], acc);
    }
    sa[pb] = mfma16(lds_operand<24>(sm.tinv[pb], n, 4 * g), to_operand(acc), zero4());
    sab[pb] = to_operand(sa[pb]);
  }

  const int heads = p.num_heads;
  if (p.state_dot_a != nullptr) {
#pragma unroll
    for (int pb = 0; pb < 4; ++pb) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = 16 * pb + 4 * g + j;
        if (t >= lo && t < hi) {
          p.state_dot_a[((chunk_base + t) * heads + head) * kHead + 16 * w + n] = sa[pb][j];
        }
      }
    }
  }

  // Y^T tiles: rows v of w, cols t of block p.
  using S16 = typename IoTraits<T>::storage;
  S16* out = static_cast<S16*>(p.out);
#pragma unroll
  for (int pb = 0; pb < 4; ++pb) {
    f32x4 acc = zero4();
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      acc = mfma16(sb[kb], lds_operand(sm.rt, 16 * pb + n, 16 * kb + 4 * g), acc);
    }
#pragma unroll
    for (int q = 0; q <= pb; ++q) {
      acc = mfma16(sab[q], lds_operand(sm.arb, 16 * pb + n, 16 * q + 4 * g), acc);
      acc = mfma16(lds_operand(sm.vT, 16 * w + n, 16 * q + 4 * g),
                   lds_operand(sm.ark, 16 * pb + n, 16 * q + 4 * g), acc);
    }
    const int t = 16 * pb + n;
    if (t >= lo && t < hi) {
      store4<T>(out + ((chunk_base + t) * heads + head) * kHead + 16 * w + 4 * g,
                p.scale * acc[0], p.scale * acc[1], p.scale * acc[2], p.scale * acc[3]);
    }
  }

  // S' = diag(2^GC) S0 + Bt^T SA + Kt^T V.
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    f32x4 acc;
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = S[kb][j] * sm.gc[16 * kb + 4 * g + j];
#pragma unroll
    for (int pb = 0; pb < 4; ++pb) {
      acc = mfma16(lds_operand(sm.btT, 16 * kb + n, 16 * pb + 4 * g), sab[pb], acc);
      acc = mfma16(lds_operand(sm.ktT, 16 * kb + n, 16 * pb + 4 * g),
                   lds_operand(sm.vT, 16 * w + n, 16 * pb + 4 * g), acc);
    }
    S[kb] = acc;
  }
}

template <typename T, DecayMode M, typename PoolT>
__global__ __launch_bounds__(kChunkThreads, 1) void chunk_fwd_kernel(ChunkFwdParams p) {
  __shared__ ChunkSmem sm;
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
  const int tp = lane >> 3;
  const int kg = lane & 7;
  const int heads = p.num_heads;
  const int seq = blockIdx.x / heads;
  const int head = blockIdx.x % heads;
  const int slot = p.slots != nullptr ? p.slots[seq] : seq;
  if (slot < 0 || slot >= p.state_slots) return;

  int seg_lo = 0, seg_hi = 1;
  if (p.seg_offsets != nullptr) {
    seg_lo = max(p.seg_offsets[seq], 0);
    seg_hi = min(p.seg_offsets[seq + 1], p.num_segments);
  }

  float bias[8];
  if constexpr (M == DecayMode::kLogits) {
    if (p.bias != nullptr) {
      unpack8<T>(load_row8<T>(p.bias, static_cast<int64_t>(head) * kHead + 8 * kg), bias);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) bias[e] = 0.0f;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) bias[e] = 0.0f;
  }

  // Wave w's state slice: S[16kb + 4g + j][16w + n] in acc[kb][j].
  const int64_t sbase = (static_cast<int64_t>(slot) * heads + head) * kHead * kHead;
  f32x4 S[4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      S[kb][j] = pool_load<PoolT>(p.state, sbase + (16 * kb + 4 * g + j) * kHead + 16 * wave + n);
    }
  }

  for (int seg = seg_lo; seg < seg_hi; ++seg) {
    int t_begin, t_end;
    if (p.seg_offsets != nullptr) {
      t_begin = p.seg_starts[seg];
      t_end = p.seg_ends[seg];
    } else {
      t_begin = p.cu_seqlens[seq];
      t_end = p.cu_seqlens[seq + 1];
    }
    t_begin = max(t_begin, 0);
    t_end = min(t_end, p.total_tokens);
    if (p.boundary != nullptr) {
      const int64_t bbase = (static_cast<int64_t>(seg) * heads + head) * kHead * kHead;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          p.boundary[bbase + (16 * kb + 4 * g + j) * kHead + 16 * wave + n] = S[kb][j];
        }
      }
    }
    for (int c0 = t_begin; c0 < t_end; c0 += kChunk) {
      const int ntok = min(kChunk, t_end - c0);
      RawRows raw;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int t = 16 * wave + 2 * tp + s;
        if (t < ntok) {
          const int64_t off = ((static_cast<int64_t>(c0) + t) * heads + head) * kHead + 8 * kg;
          raw.r[s] = load_row8<T>(p.r, off);
          raw.w[s] = load_row8<T>(p.decay, off);
          raw.k[s] = load_row8<T>(p.k, off);
          raw.v[s] = load_row8<T>(p.v, off);
          raw.a[s] = load_row8<T>(p.a, off);
          raw.b[s] = load_row8<T>(p.b, off);
        } else {
          raw.r[s] = raw.w[s] = raw.k[s] = raw.v[s] = raw.a[s] = raw.b[s] =
              make_uint4(0, 0, 0, 0);
        }
      }
      const Spans spans = prepare<T, M>(sm, raw, bias, 0, ntok);
      if (spans.all <= kSpanLimit) {
        intra_chunk(sm);
        state_pass<T>(sm, S, p, head, c0, 0, ntok);
      } else {
        // Strong decay: 16-token sub-chunks, or 4-token ones where needed.
        for (int q = 0; q < 4 && 16 * q < ntok; ++q) {
          const int hi16 = min(16 * q + 16, ntok);
          const int step = spans.block[q] <= kSpanLimit ? 16 : 4;
          for (int lo = 16 * q; lo < hi16; lo += step) {
            const int hi = min(lo + step, hi16);
            prepare<T, M>(sm, raw, bias, lo, hi);
            intra_chunk(sm);
            state_pass<T>(sm, S, p, head, c0, lo, hi);
          }
        }
      }
    }
  }

#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      pool_store<PoolT>(p.state, sbase + (16 * kb + 4 * g + j) * kHead + 16 * wave + n,
                        S[kb][j]);
    }
  }
}

template <typename T, DecayMode M, typename PoolT>
int launch_chunk(const ChunkFwdParams& p, int units, hipStream_t stream) {
  hipLaunchKernelGGL((chunk_fwd_kernel<T, M, PoolT>), dim3(units), dim3(kChunkThreads), 0,
                     stream, p);
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
    void* output, float* boundary, float* state_dot_a, float scale, void* stream) {
  using namespace frwkv;
  if (!sequence_chunk_offsets || !chunk_token_starts || !chunk_token_ends || !state ||
      !boundary || !state_dot_a) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_statetune_forward: null pointer argument");
  }
  int rc = check_token_pointers(r, decay, k, v, a, b, output);
  if (rc != FRWKV_OK) return rc;
  if (head_size != 64) {
    return set_error(FRWKV_ERR_UNSUPPORTED, "chunked kernels support head size 64, got %d",
                     head_size);
  }
  if (num_sequences <= 0 || num_heads <= 0 || total_tokens <= 0 || num_chunks <= 0) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_statetune_forward: sizes must be positive");
  }
  if (!__builtin_isfinite(scale)) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT, "scale must be finite");
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
  p.scale = scale;
  p.out_elems = static_cast<int64_t>(total_tokens) * num_heads * head_size;
  return dispatch_chunk_io<float>(p, io_dtype, decay_mode, num_sequences * num_heads,
                                  static_cast<hipStream_t>(stream));
}
