// Per-token WKV7 training kernels for head size 256.
//
// The chunked MFMA kernels (chunk_fwd.hip, chunk_bwd.hip) are built around
// D = 64 tiles and the piece kernels (piece_train.hip) around D = 128. These
// kernels serve the StateTune and pretraining entry points at D = 256, which
// the reference accepts too
// (flashrwkv2/tmix/wkv7/statetune.py:57-58, pretrain.py:16-17; kernels
// csrc/sm90/tmix/wkv7/statetune_recurrent_fp32io16_{forward,backward}.cu and
// pretrain_recurrent_bf16_forward.cu). They run the recurrence token by token
// in fp32:
//   sa_t = S_{t-1}^T a_t,  S_t = diag(w_t) S_{t-1} + b_t sa_t^T + k_t v_t^T,
//   y_t = scale S_t^T r_t                                     (S is [K,V]).
//
// Layout. A wave owns CW value columns of one (sequence, head) state: lane
// (rg, cg) = (lane / (CW/4), lane % (CW/4)) holds key rows rg*R .. rg*R+R-1
// (R = D*CW/256) of columns 4cg..4cg+3 as float4 registers, so a sum over
// keys is a wave reduction and no recurrence step needs another wave. A
// workgroup of NW waves covers NW*CW columns; a (sequence, head) unit spans
// D/(NW*CW) workgroups ("groups"). Token rows are staged in LDS 16 tokens at
// a time, the decay transform computed once per element there.
//
// Forward: each group walks the chunks of its sequence and writes, for its
// columns, the state at every chunk start (the StateTune boundary output, or
// the pretraining state every 16 tokens), y, a^T S_{t-1} and the final state.
// The next 16-token piece is loaded while the current one computes.
//
// Backward: the adjoint A = dL/dS_t is column-local as well:
//   A += scale r_t dy_t^T,   dsa = A^T b_t,   dv_t = A^T k_t,
//   A <- diag(w_t) A + a_t dsa^T,
// while the per-key gradients are sums over value columns
//   dr = scale S_t dy,  dk = A v,  db = A sa,  dw = rowsum(A o S_{t-1}),
//   da = S_{t-1} dsa,
// which each wave forms over its columns and the workgroup adds up in LDS in
// a fixed wave order. With more than one group per unit, each group writes its
// sums to its own fp32 slice and a second kernel adds the slices in group
// order, so the gradients are deterministic. Chunks are walked in reverse and
// must be at most 16 tokens; S_{t-1} is recomputed from the chunk's stored
// start state (never by dividing by the decay) or from a register copy of the
// state 8 tokens into the chunk.
//
// The recomputed states are bitwise equal to the forward's: both kernels use
// the same lane layout per head size, the same fma forms and the same
// reduction order.
#include "capi_internal.h"
#include "train_common.h"
#include "wkv7_device.h"

#include <algorithm>

namespace frwkv {
namespace {

// Columns per wave and waves per workgroup for each head size. The two fp32
// state slabs (state and adjoint) of a lane take 2 * D * CW / 64 registers.
template <int D> struct TrainShape;
template <> struct TrainShape<256> { static constexpr int kCW = 8, kNW = 8; };

// The retention of the training kernels: raw retention clamped to
// [2^-20, 1], as the MFMA training kernels (head sizes 64 and 128) take it,
// so every head size trains on the same function.
template <DecayMode M>
__device__ __forceinline__ float train_retention(float x) {
  if constexpr (M == DecayMode::kLogits) {
    return decay_retention<M>(x);
  } else {
    return __builtin_amdgcn_fmed3f(x, 0x1p-20f, 1.0f);
  }
}

template <int D>
struct Layout {
  static constexpr int kCW = TrainShape<D>::kCW;
  static constexpr int kNW = TrainShape<D>::kNW;
  static constexpr int kThreads = 64 * kNW;
  static constexpr int kCg = kCW / 4;           // lanes across a wave's columns
  static constexpr int kNg = 64 / kCg;          // key row groups per wave
  static constexpr int kRpl = D / kNg;          // key rows per lane
  static constexpr int kCols = kCW * kNW;       // columns per workgroup
  static constexpr int kGroups = D / kCols;     // workgroups per (sequence, head)
  static_assert(kRpl % 4 == 0 && kGroups * kCols == D, "layout");
};


template <int kCtrl>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), kCtrl, 0xF, 0xF, true));
}

// Sum over the key row groups of a wave: lanes sharing lane % kCg. Inside a
// 16-lane DPP row, rotations by kCg, 2 kCg, ... (row_ror) gather one residue
// class; the four rows are then added across lanes xor 16 and xor 32, either
// with the VALU lane swaps (kSwap: the backward, whose single wave per SIMD
// waits on every LDS round trip) or with LDS-crossbar shuffles (the forward,
// whose VALU is the busier unit). Addition is commutative, so both forms give
// the same bits and the backward's recomputed states match the forward's.
template <int kCg, bool kSwap>
__device__ __forceinline__ float sum_keys(float x) {
  if constexpr (kCg <= 2) x += dpp<0x122>(x);  // row_ror:2
  x += dpp<0x124>(x);                          // row_ror:4
  x += dpp<0x128>(x);                          // row_ror:8
  if constexpr (kSwap) {
    return add_xor32(add_xor16(x));
  } else {
    x += __shfl_xor(x, 16, 64);
    return x + __shfl_xor(x, 32, 64);
  }
}

template <int kCg, bool kSwap>
__device__ __forceinline__ float4 sum_keys4(float4 x) {
  return make_float4(sum_keys<kCg, kSwap>(x.x), sum_keys<kCg, kSwap>(x.y),
                     sum_keys<kCg, kSwap>(x.z), sum_keys<kCg, kSwap>(x.w));
}

// Sum over the kCg column lanes of a row group (quad_perm xor 1, xor 2).
template <int kCg>
__device__ __forceinline__ float sum_cols(float x) {
  x += dpp<0xB1>(x);
  if constexpr (kCg == 4) x += dpp<0x4E>(x);
  return x;
}

__device__ __forceinline__ float dot4(float4 a, float4 b) {
  return fmaf(a.x, b.x, fmaf(a.y, b.y, fmaf(a.z, b.z, a.w * b.w)));
}

template <typename T>
__device__ __forceinline__ void decode4(uint2 q, float (&out)[4]) {
  out[0] = to_f32<T>(static_cast<uint16_t>(q.x & 0xffffu));
  out[1] = to_f32<T>(static_cast<uint16_t>(q.x >> 16));
  out[2] = to_f32<T>(static_cast<uint16_t>(q.y & 0xffffu));
  out[3] = to_f32<T>(static_cast<uint16_t>(q.y >> 16));
}

template <typename T>
__device__ __forceinline__ float4 decode4f(uint2 q) {
  float f[4];
  decode4<T>(q, f);
  return make_float4(f[0], f[1], f[2], f[3]);
}

__device__ __forceinline__ uint2 load8(const void* base, int64_t elem) {
  return *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + elem);
}

__device__ __forceinline__ uint2 lds8(const uint16_t* p) {
  return *reinterpret_cast<const uint2*>(p);
}

// A lane's slab of a [D,D] fp32 state at `base` (rows row0.., columns col..col+3).
template <int D, int kRpl>
__device__ __forceinline__ void load_slab(float4 (&s)[kRpl], const float* base, int row0,
                                          int col) {
  const float* p = base + row0 * D + col;
#pragma unroll
  for (int j = 0; j < kRpl; ++j) s[j] = *reinterpret_cast<const float4*>(p + j * D);
}

template <int D, int kRpl>
__device__ __forceinline__ void store_slab(float* base, const float4 (&s)[kRpl], int row0,
                                           int col) {
  float* p = base + row0 * D + col;
#pragma unroll
  for (int j = 0; j < kRpl; ++j) *reinterpret_cast<float4*>(p + j * D) = s[j];
}

// One forward step on a lane's state slab: s <- diag(w) s + b sa^T + k v^T
// with sa = s^T a (returned, the lane's 4 columns), token rows read from LDS.
// The fma forms are those of the inference kernels.
template <int D, typename T, bool kSwap>
__device__ __forceinline__ float4 step_state(float4 (&s)[Layout<D>::kRpl], const uint16_t* a_row,
                                             const uint16_t* b_row, const uint16_t* k_row,
                                             const float* w_row, float4 vv, int row0) {
  constexpr int kRpl = Layout<D>::kRpl;
  float4 sa = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int q = 0; q < kRpl / 4; ++q) {
    float aa[4];
    decode4<T>(lds8(a_row + row0 + 4 * q), aa);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4 x = s[4 * q + j];
      sa.x = fmaf(aa[j], x.x, sa.x);
      sa.y = fmaf(aa[j], x.y, sa.y);
      sa.z = fmaf(aa[j], x.z, sa.z);
      sa.w = fmaf(aa[j], x.w, sa.w);
    }
  }
  sa = sum_keys4<Layout<D>::kCg, kSwap>(sa);
#pragma unroll
  for (int q = 0; q < kRpl / 4; ++q) {
    float bb[4], kk[4];
    decode4<T>(lds8(b_row + row0 + 4 * q), bb);
    decode4<T>(lds8(k_row + row0 + 4 * q), kk);
    const float4 ww = *reinterpret_cast<const float4*>(w_row + row0 + 4 * q);
    const float wj[4] = {ww.x, ww.y, ww.z, ww.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float4& x = s[4 * q + j];
      x.x = fmaf(wj[j], x.x, fmaf(bb[j], sa.x, kk[j] * vv.x));
      x.y = fmaf(wj[j], x.y, fmaf(bb[j], sa.y, kk[j] * vv.y));
      x.z = fmaf(wj[j], x.z, fmaf(bb[j], sa.z, kk[j] * vv.z));
      x.w = fmaf(wj[j], x.w, fmaf(bb[j], sa.w, kk[j] * vv.w));
    }
  }
  return sa;
}

// Staging of a 16-token piece into LDS. Row tensors (indexed by key) are
// staged for all D keys, column tensors for the workgroup's columns only. A
// thread moves 4 consecutive elements (8 bytes) per quad.
template <int D>
struct Staging {
  using L = Layout<D>;
  static constexpr int kRowQuads = kPiece * D / 4;
  static constexpr int kColQuads = kPiece * L::kCols / 4;
  static constexpr int kRowPer = kRowQuads / L::kThreads;                     // >= 1
  static constexpr int kColPer = (kColQuads + L::kThreads - 1) / L::kThreads;  // 1
  static_assert(kRowQuads % L::kThreads == 0 && kColPer == 1, "staging split");
  __device__ static int row_tok(int tid, int u) { return (tid + u * L::kThreads) / (D / 4); }
  __device__ static int row_elem(int tid, int u) {
    return 4 * ((tid + u * L::kThreads) % (D / 4));
  }
  __device__ static int col_tok(int tid) { return tid / (L::kCols / 4); }
  __device__ static int col_elem(int tid) { return 4 * (tid % (L::kCols / 4)); }
  __device__ static bool col_active(int tid) { return tid < kColQuads; }
};

// ------------------------------------------------------------- forward ----

template <int D>
struct FwdStage {
  static constexpr int kCols = Layout<D>::kCols;
  uint16_t r[kPiece][D], k[kPiece][D], a[kPiece][D], b[kPiece][D];
  uint16_t v[kPiece][kCols];
  float w[kPiece][D];  // retention
};

template <int D, typename T, DecayMode M>
__global__ __launch_bounds__(Layout<D>::kThreads) void train_fwd_kernel(TrainParams p) {
  using L = Layout<D>;
  using Sg = Staging<D>;
  constexpr int kRpl = L::kRpl;
  __shared__ FwdStage<D> st[2];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int cg = lane % L::kCg, rg = lane / L::kCg;
  const int row0 = rg * kRpl;
  const int unit = blockIdx.x / L::kGroups;
  const int group = blockIdx.x % L::kGroups;
  const int col0 = group * L::kCols;
  const int wcol = L::kCW * wave + 4 * cg;  // lane's first column within the group
  const int col = col0 + wcol;
  const int seq = unit / p.num_heads;
  const int head = unit % p.num_heads;
  const int64_t hd = static_cast<int64_t>(p.num_heads) * D;
  const int64_t head_off = static_cast<int64_t>(head) * D;

  float bias4[Sg::kRowPer][4];
#pragma unroll
  for (int u = 0; u < Sg::kRowPer; ++u) {
#pragma unroll
    for (int j = 0; j < 4; ++j) bias4[u][j] = 0.0f;
    if (p.bias != nullptr) decode4<T>(load8(p.bias, head_off + Sg::row_elem(tid, u)), bias4[u]);
  }

  struct Regs {
    uint2 r[Sg::kRowPer], k[Sg::kRowPer], a[Sg::kRowPer], b[Sg::kRowPer], x[Sg::kRowPer];
    uint2 v;
  };
  auto load_piece = [&](Regs& g, int32_t t0, int n) {
#pragma unroll
    for (int u = 0; u < Sg::kRowPer; ++u) {
      const int i = Sg::row_tok(tid, u);
      if (i < n) {
        const int64_t e = (t0 + i) * hd + head_off + Sg::row_elem(tid, u);
        g.r[u] = load8(p.r, e);
        g.k[u] = load8(p.k, e);
        g.a[u] = load8(p.a, e);
        g.b[u] = load8(p.b, e);
        g.x[u] = load8(p.decay, e);
      }
    }
    const int i = Sg::col_tok(tid);
    if (Sg::col_active(tid) && i < n) {
      g.v = load8(p.v, (t0 + i) * hd + head_off + col0 + Sg::col_elem(tid));
    }
  };
  auto store_piece = [&](FwdStage<D>& s, const Regs& g, int n) {
#pragma unroll
    for (int u = 0; u < Sg::kRowPer; ++u) {
      const int i = Sg::row_tok(tid, u), e = Sg::row_elem(tid, u);
      if (i < n) {
        *reinterpret_cast<uint2*>(&s.r[i][e]) = g.r[u];
        *reinterpret_cast<uint2*>(&s.k[i][e]) = g.k[u];
        *reinterpret_cast<uint2*>(&s.a[i][e]) = g.a[u];
        *reinterpret_cast<uint2*>(&s.b[i][e]) = g.b[u];
        float x[4];
        decode4<T>(g.x[u], x);
        *reinterpret_cast<float4*>(&s.w[i][e]) = make_float4(
            train_retention<M>(x[0] + bias4[u][0]), train_retention<M>(x[1] + bias4[u][1]),
            train_retention<M>(x[2] + bias4[u][2]), train_retention<M>(x[3] + bias4[u][3]));
      }
    }
    const int i = Sg::col_tok(tid);
    if (Sg::col_active(tid) && i < n) {
      *reinterpret_cast<uint2*>(&s.v[i][Sg::col_elem(tid)]) = g.v;
    }
  };

  const int64_t unit_state =
      (static_cast<int64_t>(seq) * p.num_heads + head) * static_cast<int64_t>(D) * D;
  float4 s[kRpl];
  if (p.state != nullptr) {
    load_slab<D, kRpl>(s, p.state + unit_state, row0, col);
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  } else {
#pragma unroll
    for (int j = 0; j < kRpl; ++j) s[j] = make_float4(0.f, 0.f, 0.f, 0.f);
  }

  int c_begin, c_end;
  chunk_range(p, seq, c_begin, c_end);
  // Piece cursor (chunk c, first token t0). Every chunk has at least one
  // piece; an empty chunk's single piece only writes its start state.
  int c = c_begin;
  Chunk ch{};
  if (c < c_end) ch = chunk_at<D>(p, seq, head, c);
  int32_t t0 = ch.start;
  Regs g{};
  int buf = 0;
  if (c < c_end) {
    const int n0 = min(kPiece, ch.end - t0);
    load_piece(g, t0, n0);
    store_piece(st[0], g, n0);
  }
  __syncthreads();

  if (p.fill_only && (c >= c_end || ch.end - ch.start <= kPiece)) return;
  while (c < c_end) {
    const int n = min(kPiece, ch.end - t0);
    const bool first = t0 == ch.start;
    if (!first && p.interior != nullptr) {
      store_slab<D, kRpl>(p.interior + (static_cast<int64_t>(t0 / kPiece) * p.num_heads + head) *
                                           static_cast<int64_t>(D) * D,
                          s, row0, col);
    }
    if (p.fill_only && t0 + kPiece >= ch.end) break;
    int c_n = c;
    Chunk ch_n = ch;
    int32_t t0_n = t0 + kPiece;
    if (t0_n >= ch.end) {
      c_n = c + 1;
      if (c_n < c_end) {
        ch_n = chunk_at<D>(p, seq, head, c_n);
        t0_n = ch_n.start;
      }
    }
    const bool has_next = c_n < c_end;
    const int n_n = has_next ? min(kPiece, ch_n.end - t0_n) : 0;
    if (n_n > 0) load_piece(g, t0_n, n_n);

    if (first && p.ckpt != nullptr) store_slab<D, kRpl>(p.ckpt + ch.ckpt_off, s, row0, col);
    const FwdStage<D>& cur = st[buf];
    for (int i = 0; i < n; ++i) {
      const float4 vv = decode4f<T>(lds8(&cur.v[i][wcol]));
      const float4 sa =
          step_state<D, T, false>(s, cur.a[i], cur.b[i], cur.k[i], cur.w[i], vv, row0);
      float4 y = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int q = 0; q < kRpl / 4; ++q) {
        float rr[4];
        decode4<T>(lds8(&cur.r[i][row0 + 4 * q]), rr);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float4 x = s[4 * q + j];
          y.x = fmaf(rr[j], x.x, y.x);
          y.y = fmaf(rr[j], x.y, y.y);
          y.z = fmaf(rr[j], x.z, y.z);
          y.w = fmaf(rr[j], x.w, y.w);
        }
      }
      y = sum_keys4<L::kCg, false>(y);
      if (rg == 0 && p.out != nullptr) {
        const int64_t e = (t0 + i) * hd + head_off + col;
        *reinterpret_cast<float4*>(p.state_dot_a + e) = sa;
        store4<T>(static_cast<typename IoTraits<T>::storage*>(p.out) + e, p.scale * y.x,
                  p.scale * y.y, p.scale * y.z, p.scale * y.w);
      }
    }
    if (n_n > 0) store_piece(st[buf ^ 1], g, n_n);
    __syncthreads();
    c = c_n;
    ch = ch_n;
    t0 = t0_n;
    buf ^= 1;
  }

  if (p.state != nullptr && !p.fill_only) {
    store_slab<D, kRpl>(p.state + unit_state, s, row0, col);
  }
}

// ------------------------------------------------------------ backward ----

template <int D>
struct BwdSmem {
  static constexpr int kCols = Layout<D>::kCols;
  static constexpr int kNW = Layout<D>::kNW;
  uint16_t r[kPiece][D], k[kPiece][D], a[kPiece][D], b[kPiece][D];
  uint16_t v[kPiece][kCols], dy[kPiece][kCols];
  float w[kPiece][D];    // retention
  float dwf[kPiece][D];  // d retention / d decay input (1 for the raw retention)
  // Per-wave partial sums over the wave's columns: [buffer][wave][gradient][key]
  // with gradients dr, dk, db, dw, da.
  float red[2][kNW][5][D];
};

template <int D, typename T, DecayMode M>
__global__ __launch_bounds__(Layout<D>::kThreads) void train_bwd_kernel(TrainParams p) {
  using L = Layout<D>;
  using Sg = Staging<D>;
  using St = typename IoTraits<T>::storage;
  constexpr int kRpl = L::kRpl;
  constexpr int kThreads = L::kThreads;
  constexpr int kGroups = L::kGroups;
  static_assert(sizeof(BwdSmem<D>) <= 160 * 1024, "backward LDS budget");
  __shared__ BwdSmem<D> sm;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int cg = lane % L::kCg, rg = lane / L::kCg;
  const int row0 = rg * kRpl;
  const int unit = blockIdx.x / kGroups;
  const int group = blockIdx.x % kGroups;
  const int col0 = group * L::kCols;
  const int wcol = L::kCW * wave + 4 * cg;
  const int col = col0 + wcol;
  const int seq = unit / p.num_heads;
  const int head = unit % p.num_heads;
  const int64_t hd = static_cast<int64_t>(p.num_heads) * D;
  const int64_t head_off = static_cast<int64_t>(head) * D;
  const int64_t slice = static_cast<int64_t>(p.total_tokens) * hd;  // elements per gradient
  const int64_t unit_state =
      (static_cast<int64_t>(seq) * p.num_heads + head) * static_cast<int64_t>(D) * D;
  const float nan = __int_as_float(0x7fc00000);

  float bias4[Sg::kRowPer][4];
#pragma unroll
  for (int u = 0; u < Sg::kRowPer; ++u) {
#pragma unroll
    for (int j = 0; j < 4; ++j) bias4[u][j] = 0.0f;
    if (p.bias != nullptr) decode4<T>(load8(p.bias, head_off + Sg::row_elem(tid, u)), bias4[u]);
  }

  // Adjoint of the state at the current position.
  float4 A[kRpl];
  if (p.dstate_final != nullptr) {
    load_slab<D, kRpl>(A, p.dstate_final + unit_state, row0, col);
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  } else {
#pragma unroll
    for (int j = 0; j < kRpl; ++j) A[j] = make_float4(0.f, 0.f, 0.f, 0.f);
  }

  // Where this workgroup's per-key gradient gi of element `off` goes.
  auto key_store = [&](int gi, int64_t off, float4 x) {
    if constexpr (kGroups == 1) {
      void* const outs[5] = {p.dr, p.dk, p.db, p.ddecay, p.da};
      store4<T>(static_cast<St*>(outs[gi]) + off, x.x, x.y, x.z, x.w);
    } else {
      *reinterpret_cast<float4*>(p.accum + (group * 5 + gi) * slice + off) = x;
    }
  };

  // Fail closed: from a chunk longer than one piece without interior states
  // on (walking backwards), the unit's gradients are NaN.
  auto nan_fill = [&](const Chunk& ch) {
    const int64_t n = static_cast<int64_t>(ch.end - ch.start);
    const float4 nan4 = make_float4(nan, nan, nan, nan);
    for (int64_t item = tid; item < n * (5 * (D / 4)); item += kThreads) {
      const int32_t t = ch.start + static_cast<int32_t>(item / (5 * (D / 4)));
      const int gi = static_cast<int>(item % (5 * (D / 4))) / (D / 4);
      const int e = 4 * static_cast<int>(item % (D / 4));
      key_store(gi, t * hd + head_off + e, nan4);
    }
    for (int64_t item = tid; item < n * (L::kCols / 4); item += kThreads) {
      const int32_t t = ch.start + static_cast<int32_t>(item / (L::kCols / 4));
      const int e = col0 + 4 * static_cast<int>(item % (L::kCols / 4));
      store4<T>(static_cast<St*>(p.dv) + t * hd + head_off + e, nan, nan, nan, nan);
    }
  };

  int c_begin, c_end;
  chunk_range(p, seq, c_begin, c_end);
  bool failed = false;
  int buf = 0;

  for (int c = c_end - 1; c >= c_begin; --c) {
    const Chunk whole = chunk_at<D>(p, seq, head, c);
    const int len = whole.end - whole.start;
    // Pieces of kPiece tokens from the chunk start; piece j > 0 starts from
    // the interior state at slot (its first token) / kPiece.
    const int pieces = len > kPiece ? (len + kPiece - 1) / kPiece : 1;
    if (pieces > 1 && p.interior == nullptr) failed = true;
    if (failed) {
      nan_fill(whole);
      continue;
    }
   for (int pj = pieces - 1; pj >= 0; --pj) {
    Chunk ch;
    ch.start = whole.start + kPiece * pj;
    ch.end = min(ch.start + kPiece, whole.end);
    const float* ck =
        pj == 0 ? p.ckpt + whole.ckpt_off
                : p.interior + (static_cast<int64_t>(ch.start / kPiece) * p.num_heads + head) *
                                   static_cast<int64_t>(D) * D;
    const int n = ch.end - ch.start;
    if (n == 0) continue;

    // Stage the chunk (the previous chunk's last reads ended at a barrier).
#pragma unroll
    for (int u = 0; u < Sg::kRowPer; ++u) {
      const int i = Sg::row_tok(tid, u), e = Sg::row_elem(tid, u);
      if (i < n) {
        const int64_t g = (ch.start + i) * hd + head_off + e;
        *reinterpret_cast<uint2*>(&sm.r[i][e]) = load8(p.r, g);
        *reinterpret_cast<uint2*>(&sm.k[i][e]) = load8(p.k, g);
        *reinterpret_cast<uint2*>(&sm.a[i][e]) = load8(p.a, g);
        *reinterpret_cast<uint2*>(&sm.b[i][e]) = load8(p.b, g);
        float x[4];
        decode4<T>(load8(p.decay, g), x);
        float w4[4], f4[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float xb = x[j] + bias4[u][j];
          w4[j] = train_retention<M>(xb);
          if constexpr (M == DecayMode::kLogits) {
            // dw/dx = w * (-e^{-1/2}) sigmoid(x) (1 - sigmoid(x))
            const float sig = 1.0f / (1.0f + exp2f(-kLog2E * xb));
            f4[j] = w4[j] * (-kExpNegHalf) * sig * (1.0f - sig);
          } else {
            // Raw retention is clamped to [2^-20, 1], with zero derivative
            // outside (as torch.clamp).
            f4[j] = (xb >= 0x1p-20f && xb <= 1.0f) ? 1.0f : 0.0f;
          }
        }
        *reinterpret_cast<float4*>(&sm.w[i][e]) = make_float4(w4[0], w4[1], w4[2], w4[3]);
        *reinterpret_cast<float4*>(&sm.dwf[i][e]) = make_float4(f4[0], f4[1], f4[2], f4[3]);
      }
    }
    {
      const int i = Sg::col_tok(tid), e = Sg::col_elem(tid);
      if (Sg::col_active(tid) && i < n) {
        const int64_t g = (ch.start + i) * hd + head_off + col0 + e;
        *reinterpret_cast<uint2*>(&sm.v[i][e]) = load8(p.v, g);
        *reinterpret_cast<uint2*>(&sm.dy[i][e]) =
            p.dy != nullptr ? load8(p.dy, g) : make_uint2(0u, 0u);
      }
    }
    __syncthreads();

    auto step = [&](float4 (&s)[kRpl], int i) {
      const float4 vv = decode4f<T>(lds8(&sm.v[i][wcol]));
      step_state<D, T, true>(s, sm.a[i], sm.b[i], sm.k[i], sm.w[i], vv, row0);
    };
    // S^8, the state 8 tokens into the chunk (when the chunk is longer).
    float4 cm[kRpl];
    if (n > 8) {
      load_slab<D, kRpl>(cm, ck, row0, col);
      for (int i = 0; i < 8; ++i) step(cm, i);
    }

    for (int jt = n - 1; jt >= 0; --jt) {
      // S^jt = the state before token jt of the chunk.
      float4 s[kRpl];
      int i0 = 0;
      if (jt >= 8) {
#pragma unroll
        for (int j = 0; j < kRpl; ++j) s[j] = cm[j];
        i0 = 8;
      } else {
        load_slab<D, kRpl>(s, ck, row0, col);
      }
      for (int i = i0; i < jt; ++i) step(s, i);

      // Token jt.
      const float4 vv = decode4f<T>(lds8(&sm.v[jt][wcol]));
      float4 dys = decode4f<T>(lds8(&sm.dy[jt][wcol]));
      dys = make_float4(p.scale * dys.x, p.scale * dys.y, p.scale * dys.z, p.scale * dys.w);
      float4 sa = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int q = 0; q < kRpl / 4; ++q) {
        float aa[4];
        decode4<T>(lds8(&sm.a[jt][row0 + 4 * q]), aa);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float4 x = s[4 * q + j];
          sa.x = fmaf(aa[j], x.x, sa.x);
          sa.y = fmaf(aa[j], x.y, sa.y);
          sa.z = fmaf(aa[j], x.z, sa.z);
          sa.w = fmaf(aa[j], x.w, sa.w);
        }
      }
      sa = sum_keys4<L::kCg, true>(sa);

      float(&red)[5][D] = sm.red[buf][wave];
      float4 dsa = make_float4(0.f, 0.f, 0.f, 0.f), dv = dsa;
#pragma unroll
      for (int q = 0; q < kRpl / 4; ++q) {
        float rr[4], bb[4], kk[4];
        decode4<T>(lds8(&sm.r[jt][row0 + 4 * q]), rr);
        decode4<T>(lds8(&sm.b[jt][row0 + 4 * q]), bb);
        decode4<T>(lds8(&sm.k[jt][row0 + 4 * q]), kk);
        const float4 ww = *reinterpret_cast<const float4*>(&sm.w[jt][row0 + 4 * q]);
        const float wj[4] = {ww.x, ww.y, ww.z, ww.w};
        float pr[4], pk[4], pb[4], pw[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float4& Aj = A[4 * q + j];
          const float4 x = s[4 * q + j];
          Aj.x = fmaf(rr[j], dys.x, Aj.x);
          Aj.y = fmaf(rr[j], dys.y, Aj.y);
          Aj.z = fmaf(rr[j], dys.z, Aj.z);
          Aj.w = fmaf(rr[j], dys.w, Aj.w);
          float4 st;
          st.x = fmaf(wj[j], x.x, fmaf(bb[j], sa.x, kk[j] * vv.x));
          st.y = fmaf(wj[j], x.y, fmaf(bb[j], sa.y, kk[j] * vv.y));
          st.z = fmaf(wj[j], x.z, fmaf(bb[j], sa.z, kk[j] * vv.z));
          st.w = fmaf(wj[j], x.w, fmaf(bb[j], sa.w, kk[j] * vv.w));
          pr[j] = sum_cols<L::kCg>(dot4(st, dys));
          pk[j] = sum_cols<L::kCg>(dot4(Aj, vv));
          pb[j] = sum_cols<L::kCg>(dot4(Aj, sa));
          pw[j] = sum_cols<L::kCg>(dot4(Aj, x));
          dsa.x = fmaf(bb[j], Aj.x, dsa.x);
          dsa.y = fmaf(bb[j], Aj.y, dsa.y);
          dsa.z = fmaf(bb[j], Aj.z, dsa.z);
          dsa.w = fmaf(bb[j], Aj.w, dsa.w);
          dv.x = fmaf(kk[j], Aj.x, dv.x);
          dv.y = fmaf(kk[j], Aj.y, dv.y);
          dv.z = fmaf(kk[j], Aj.z, dv.z);
          dv.w = fmaf(kk[j], Aj.w, dv.w);
        }
        if (cg == 0) {
          const int r4 = row0 + 4 * q;
          *reinterpret_cast<float4*>(&red[0][r4]) = make_float4(pr[0], pr[1], pr[2], pr[3]);
          *reinterpret_cast<float4*>(&red[1][r4]) = make_float4(pk[0], pk[1], pk[2], pk[3]);
          *reinterpret_cast<float4*>(&red[2][r4]) = make_float4(pb[0], pb[1], pb[2], pb[3]);
          *reinterpret_cast<float4*>(&red[3][r4]) = make_float4(pw[0], pw[1], pw[2], pw[3]);
        }
      }
      dsa = sum_keys4<L::kCg, true>(dsa);
      dv = sum_keys4<L::kCg, true>(dv);
      const int32_t t = ch.start + jt;
      if (rg == 0) {
        store4<T>(static_cast<St*>(p.dv) + t * hd + head_off + col, dv.x, dv.y, dv.z, dv.w);
      }
#pragma unroll
      for (int q = 0; q < kRpl / 4; ++q) {
        float aa[4];
        decode4<T>(lds8(&sm.a[jt][row0 + 4 * q]), aa);
        const float4 ww = *reinterpret_cast<const float4*>(&sm.w[jt][row0 + 4 * q]);
        const float wj[4] = {ww.x, ww.y, ww.z, ww.w};
        float pa[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float4& Aj = A[4 * q + j];
          pa[j] = sum_cols<L::kCg>(dot4(s[4 * q + j], dsa));
          Aj.x = fmaf(wj[j], Aj.x, aa[j] * dsa.x);
          Aj.y = fmaf(wj[j], Aj.y, aa[j] * dsa.y);
          Aj.z = fmaf(wj[j], Aj.z, aa[j] * dsa.z);
          Aj.w = fmaf(wj[j], Aj.w, aa[j] * dsa.w);
        }
        if (cg == 0) {
          *reinterpret_cast<float4*>(&red[4][row0 + 4 * q]) =
              make_float4(pa[0], pa[1], pa[2], pa[3]);
        }
      }
      __syncthreads();

      // Sum the waves' partials in wave order and store the per-key gradients.
      for (int item = tid; item < 5 * (D / 4); item += kThreads) {
        const int gi = item / (D / 4);
        const int e = 4 * (item % (D / 4));
        float4 acc = *reinterpret_cast<const float4*>(&sm.red[buf][0][gi][e]);
#pragma unroll
        for (int w2 = 1; w2 < L::kNW; ++w2) {
          const float4 x = *reinterpret_cast<const float4*>(&sm.red[buf][w2][gi][e]);
          acc.x += x.x;
          acc.y += x.y;
          acc.z += x.z;
          acc.w += x.w;
        }
        if (gi == 3) {
          const float4 f = *reinterpret_cast<const float4*>(&sm.dwf[jt][e]);
          acc = make_float4(acc.x * f.x, acc.y * f.y, acc.z * f.z, acc.w * f.w);
        }
        key_store(gi, t * hd + head_off + e, acc);
      }
      buf ^= 1;
    }
    __syncthreads();  // staging of the next piece overwrites the rows
   }
  }

  if (p.dstate0 != nullptr) {
    if (failed) {
#pragma unroll
      for (int j = 0; j < kRpl; ++j) A[j] = make_float4(nan, nan, nan, nan);
    }
    store_slab<D, kRpl>(p.dstate0 + unit_state, A, row0, col);
  }
}

// Per-group fp32 slices [groups, 5, n] -> dr, dk, db, ddecay, da in the io
// dtype, adding the slices in group order.
template <typename T, int kGroups>
__global__ void train_slices_store_kernel(const float* accum, int64_t n, void* dr, void* dk,
                                          void* db, void* ddecay, void* da) {
  using St = typename IoTraits<T>::storage;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t n4 = n / 4;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < 5 * n4;
       i += stride) {
    const int gi = static_cast<int>(i / n4);
    const int64_t e = 4 * (i % n4);
    float4 x = *reinterpret_cast<const float4*>(accum + gi * n + e);
#pragma unroll
    for (int g = 1; g < kGroups; ++g) {
      const float4 y = *reinterpret_cast<const float4*>(accum + (g * 5 + gi) * n + e);
      x.x += y.x;
      x.y += y.y;
      x.z += y.z;
      x.w += y.w;
    }
    void* const outs[5] = {dr, dk, db, ddecay, da};
    store4<T>(static_cast<St*>(outs[gi]) + e, x.x, x.y, x.z, x.w);
  }
}

template <int D, typename T, DecayMode M>
int launch_train_forward(const TrainParams& p, int units, hipStream_t stream) {
  using L = Layout<D>;
  hipLaunchKernelGGL((train_fwd_kernel<D, T, M>), dim3(units * L::kGroups), dim3(L::kThreads),
                     0, stream, p);
  return check_launch("train_fwd_kernel");
}

template <int D, typename T, DecayMode M>
int launch_train_backward(const TrainParams& p, int units, hipStream_t stream) {
  using L = Layout<D>;
  hipLaunchKernelGGL((train_bwd_kernel<D, T, M>), dim3(units * L::kGroups), dim3(L::kThreads),
                     0, stream, p);
  int rc = check_launch("train_bwd_kernel");
  if constexpr (L::kGroups > 1) {
    if (rc != FRWKV_OK) return rc;
    const int64_t n = static_cast<int64_t>(p.total_tokens) * p.num_heads * D;
    const int blocks = static_cast<int>(std::min<int64_t>((5 * n / 4 + 255) / 256, 8192));
    hipLaunchKernelGGL((train_slices_store_kernel<T, L::kGroups>), dim3(blocks), dim3(256), 0,
                       stream, p.accum, n, p.dr, p.dk, p.db, p.ddecay, p.da);
    rc = check_launch("train_slices_store_kernel");
  }
  return rc;
}

int slice_groups(int head_size) {
  switch (head_size) {
    case 256:
      return Layout<256>::kGroups;
    default:
      return 1;
  }
}

template <typename T, DecayMode M>
int dispatch_train(const TrainParams& p, int head_size, int units, bool backward,
                   hipStream_t s) {
  switch (head_size) {
    case 256:
      return backward ? launch_train_backward<256, T, M>(p, units, s)
                      : launch_train_forward<256, T, M>(p, units, s);
    default:
      return set_error(FRWKV_ERR_UNSUPPORTED,
                       "the per-token training kernels take head size 256, got %d",
                       head_size);
  }
}

template <typename T>
int dispatch_train_decay(const TrainParams& p, int decay_mode, int head_size, int units,
                         bool backward, hipStream_t s) {
  if (decay_mode == FRWKV_DECAY_LOGITS) {
    return dispatch_train<T, DecayMode::kLogits>(p, head_size, units, backward, s);
  }
  if (decay_mode == FRWKV_DECAY_RAW_W) {
    if (p.bias != nullptr) {
      return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                       "decay_bias is only defined for the logits decay mode");
    }
    return dispatch_train<T, DecayMode::kRawW>(p, head_size, units, backward, s);
  }
  return set_error(FRWKV_ERR_INVALID_ARGUMENT, "unknown decay mode %d", decay_mode);
}

int dispatch_train_io(const TrainParams& p, int io_dtype, int decay_mode, int head_size,
                      int units, bool backward, hipStream_t s) {
  switch (io_dtype) {
    case FRWKV_DTYPE_BF16:
      return dispatch_train_decay<Bf16>(p, decay_mode, head_size, units, backward, s);
    case FRWKV_DTYPE_F16:
      return dispatch_train_decay<F16>(p, decay_mode, head_size, units, backward, s);
    default:
      return set_error(FRWKV_ERR_UNSUPPORTED,
                       "training kernels take float16 or bfloat16 tokens (io dtype %d)",
                       io_dtype);
  }
}

}  // namespace
}  // namespace frwkv

int frwkv_train_recurrent_forward(int io_dtype, int decay_mode, int32_t num_sequences,
                                  int32_t num_heads, int32_t head_size, int32_t total_tokens,
                                  const int32_t* seg_offsets, const int32_t* seg_starts,
                                  const int32_t* seg_ends, int32_t num_chunks, int32_t dense_t,
                                  float* state,
                                  const void* r, const void* decay, const void* decay_bias,
                                  const void* k, const void* v, const void* a, const void* b,
                                  void* output, float* boundary, float* state_dot_a,
                                  float* interior, int fill_only, float scale, void* stream) {
  using namespace frwkv;
  TrainParams p{};
  p.interior = interior;
  p.fill_only = fill_only;
  p.num_heads = num_heads;
  p.total_tokens = total_tokens;
  p.num_sequences = num_sequences;
  p.seg_offsets = seg_offsets;
  p.seg_starts = seg_starts;
  p.seg_ends = seg_ends;
  p.num_chunks = num_chunks;
  p.dense_t = dense_t;
  p.state = state;
  p.ckpt = boundary;
  p.state_dot_a = state_dot_a;
  p.r = r;
  p.decay = decay;
  p.bias = decay_bias;
  p.k = k;
  p.v = v;
  p.a = a;
  p.b = b;
  p.out = output;
  p.scale = scale;
  if (head_size == 128) {
    return launch_piece_train(p, io_dtype, decay_mode, num_sequences * num_heads,
                              /*backward=*/false, static_cast<hipStream_t>(stream));
  }
  return dispatch_train_io(p, io_dtype, decay_mode, head_size, num_sequences * num_heads,
                           /*backward=*/false, static_cast<hipStream_t>(stream));
}

int frwkv_train_recurrent_backward(int io_dtype, int decay_mode, int32_t num_sequences,
                                   int32_t num_heads, int32_t head_size, int32_t total_tokens,
                                   const int32_t* seg_offsets, const int32_t* seg_starts,
                                   const int32_t* seg_ends, int32_t num_chunks,
                                   int32_t dense_t, const float* boundary, const void* r, const void* decay,
                                   const void* decay_bias, const void* k, const void* v,
                                   const void* a, const void* b, const void* grad_output,
                                   const float* grad_final_state, void* grad_r,
                                   void* grad_decay, void* grad_k, void* grad_v, void* grad_a,
                                   void* grad_b, float* grad_initial_state,
                                   const float* interior, float* slices, float scale,
                                   void* stream) {
  using namespace frwkv;
  TrainParams p{};
  p.interior = const_cast<float*>(interior);
  p.num_heads = num_heads;
  p.total_tokens = total_tokens;
  p.num_sequences = num_sequences;
  p.seg_offsets = seg_offsets;
  p.seg_starts = seg_starts;
  p.seg_ends = seg_ends;
  p.num_chunks = num_chunks;
  p.dense_t = dense_t;
  p.ckpt = const_cast<float*>(boundary);
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
  const auto s = static_cast<hipStream_t>(stream);
  if (slice_groups(head_size) > 1) {
    if (slices == nullptr) {
      return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                       "training backward at head size %d needs the gradient-slice workspace",
                       head_size);
    }
    p.accum = slices;
  }
  if (head_size == 128) {
    return launch_piece_train(p, io_dtype, decay_mode, num_sequences * num_heads,
                              /*backward=*/true, s);
  }
  const int rc = dispatch_train_io(p, io_dtype, decay_mode, head_size,
                                   num_sequences * num_heads, /*backward=*/true, s);
  return rc;
}

size_t frwkv_train_slice_bytes(int32_t head_size, int32_t num_heads, int32_t total_tokens) {
  const int groups = frwkv::slice_groups(head_size);
  if (groups <= 1 || num_heads <= 0 || total_tokens <= 0) return 0;
  return static_cast<size_t>(groups) * 5 * static_cast<size_t>(total_tokens) * num_heads *
         head_size * sizeof(float);
}
