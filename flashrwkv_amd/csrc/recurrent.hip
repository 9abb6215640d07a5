// fp32-state WKV7 recurrent forward (decode and short state-carry sequences).
//
// Replaces the reference's wkv_fp32_v2_kernel / wkv_fp32_v2_small_warp_kernel
// and their dispatch (csrc/sm120/tmix/wkv7/infer_recurrent_fp32io16_forward_varlen.cu:90-275,
// 369-508). Same contract: packed [N,H,D] tokens, [slots,H,D,D] fp32 pool laid
// out [K,V] and updated in place at state_indices, fail-closed NaN output when
// the metadata status word is non-zero.
//
// The same kernel runs the fp16-state family (reference
// csrc/sm120/tmix/wkv7/infer_recurrent_fp16_forward_varlen.cu, contract
// tests/tmix/wkv7/test.py:214-264): the pool holds fp16, the retention enters
// as delta = fp16(w - 1 + dither(phase)) with phase = elapsed[slot] + h*D +
// key + token offset, and every token's state S + S*delta + b sa^T + k v^T
// is rounded to fp16 before the output reads it. Arithmetic between those
// rounding points is fp32, as in the reference's oracle.
//
// MI355X design. The value columns of a state are independent given the token
// vectors (sa[v], y[v] and S[:,v] only touch column v), so the work unit is a
// wave owning a slab of CW columns of one (sequence, head) state:
//   * lane l holds a group cg of NC = 4 columns (NC = 2 in the 8-column
//     slabs that launches over few states use) for RPL consecutive key rows
//     of row group rg (NG = 64/(CW/NC) row groups), i.e. RPL float4 (float2)
//     registers; the wave's loads and stores of a state slab are 16-byte
//     (8-byte) per lane;
//   * token vectors of the lane's RPL rows are contiguous and read directly
//     from global memory (lanes sharing rows share the cache line);
//   * S^T a and S^T r reduce first in-lane over RPL rows, then across the
//     row groups. Multi-token shapes (CW = 16) put rg in the low lane bits
//     (rg = l % NG), so that sum is a butterfly of DPP lane permutations
//     inside a 16-lane row with no LDS-crossbar exchange on the token-to-token
//     dependency chain (1.7x faster on long sequences); the decode shape
//     (CW = 64) keeps rg in the high bits (rg = l / 16) for whole-row loads;
//   * waves never synchronise with each other, so the kernel has no barrier.
// Decode (T=1) is HBM-bound: per (sequence, head) it moves the 16 KiB state in
// and out plus 7 token rows; everything is issued up front. State traffic is
// nontemporal and decode launches one wave per workgroup: on MI355X that pair
// measured fastest (6.07 TB/s at B=256, H=40, above a plain 168 MB copy).
#include "capi_internal.h"
#include "wkv7_device.h"
#include "wkv7_mfma.h"

namespace frwkv {
namespace {


// State pool element type.
enum class StateKind : int { kFp32 = 0, kFp16 = 1 };

template <StateKind SK>
struct StateTraits {
  using storage = float;
};
template <>
struct StateTraits<StateKind::kFp16> {
  using storage = uint16_t;
};

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Four consecutive state columns, streamed (each state slab moves once).
template <StateKind SK>
__device__ __forceinline__ float4 load_state4(const typename StateTraits<SK>::storage* p) {
  if constexpr (SK == StateKind::kFp32) {
    return load_f4_stream(p);
  } else {
    const u32x2_t q = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
    return make_float4(f16_to_f32(static_cast<uint16_t>(q.x & 0xffffu)),
                       f16_to_f32(static_cast<uint16_t>(q.x >> 16)),
                       f16_to_f32(static_cast<uint16_t>(q.y & 0xffffu)),
                       f16_to_f32(static_cast<uint16_t>(q.y >> 16)));
  }
}

// NC consecutive state columns (NC = 4 or 2) of a lane: float4 or float2.
// The kernel names the components (x, y[, z, w]) rather than indexing a
// vector: indexed forms changed the schedule of the four-column kernels
// (decode included) for no gain.
template <int NC>
struct ColVec {
  using type = float4;
};
template <>
struct ColVec<2> {
  using type = float2;
};

template <typename V>
__device__ __forceinline__ V zero_cols() {
  if constexpr (sizeof(V) == 16) return make_float4(0.f, 0.f, 0.f, 0.f);
  else return make_float2(0.f, 0.f);
}

template <StateKind SK>
__device__ __forceinline__ float2 load_state2(const typename StateTraits<SK>::storage* p) {
  if constexpr (SK == StateKind::kFp32) {
    const u32x2_t q = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
    return make_float2(__uint_as_float(q.x), __uint_as_float(q.y));
  } else {
    const uint32_t q = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
    return make_float2(f16_to_f32(static_cast<uint16_t>(q & 0xffffu)),
                       f16_to_f32(static_cast<uint16_t>(q >> 16)));
  }
}

template <StateKind SK>
__device__ __forceinline__ void store_state2(typename StateTraits<SK>::storage* p, float2 v) {
  if constexpr (SK == StateKind::kFp32) {
    const u32x2_t q = {__float_as_uint(v.x), __float_as_uint(v.y)};
    __builtin_nontemporal_store(q, reinterpret_cast<u32x2_t*>(p));
  } else {
    // v holds fp16 values already; the conversion is exact.
    __builtin_nontemporal_store(pack2<F16>(v.x, v.y), reinterpret_cast<uint32_t*>(p));
  }
}

// Two consecutive output values (16-bit io: 4 bytes; fp32: 8 bytes).
template <typename T>
__device__ __forceinline__ void store2(typename IoTraits<T>::storage* p, float x0, float x1) {
  if constexpr (__is_same(T, float)) {
    *reinterpret_cast<float2*>(p) = make_float2(x0, x1);
  } else {
    *reinterpret_cast<uint32_t*>(p) = pack2<T>(x0, x1);
  }
}

template <typename T>
__device__ __forceinline__ void store2_buf(__amdgpu_buffer_rsrc_t rs, uint32_t voffset,
                                           int soffset, float x0, float x1) {
  if constexpr (__is_same(T, float)) {
    const u32x2_t q = {__float_as_uint(x0), __float_as_uint(x1)};
    __builtin_amdgcn_raw_buffer_store_b64(q, rs, voffset, soffset, 0);
  } else {
    __builtin_amdgcn_raw_buffer_store_b32(pack2<T>(x0, x1), rs, voffset, soffset, 0);
  }
}

template <StateKind SK>
__device__ __forceinline__ void store_state4(typename StateTraits<SK>::storage* p, float4 v) {
  if constexpr (SK == StateKind::kFp32) {
    store_f4_stream(p, v);
  } else {
    // v holds fp16 values already; the conversion is exact.
    u32x2_t q;
    q.x = pack2<F16>(v.x, v.y);
    q.y = pack2<F16>(v.z, v.w);
    __builtin_nontemporal_store(q, reinterpret_cast<u32x2_t*>(p));
  }
}

__device__ __forceinline__ float round_f16(float x) {
  return static_cast<float>(static_cast<_Float16>(x));
}

// Phase dither of the fp16-state delta: the signed 32-bit value of
// phase * 2654435769 (mod 2^32), times 2^-41, so |dither| <= 2^-10.
constexpr uint32_t kDitherMultiplier = 2654435769u;
constexpr float kDitherUnit = 4.547473508864641e-13f;  // 2^-41

__device__ __forceinline__ float phase_dither(uint32_t phase) {
  return kDitherUnit * static_cast<float>(static_cast<int32_t>(kDitherMultiplier * phase));
}

// Sum over the NG row groups of recurrent_fp32_kernel's lane layout, where
// the row group is the low log2(NG) bits of the lane id: a butterfly of DPP
// permutations inside a 16-lane row (xor 1 and xor 2 by quad_perm, xor 7 by
// row_half_mirror, xor 15 by row_mirror; the masks span the 4 low bits). Each
// step adds a lane pair symmetrically, so every lane of a group ends with the
// same bits, and no step leaves the row (no LDS-crossbar exchange).
template <int kCtrl>
__device__ __forceinline__ float dpp_read(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), kCtrl, 0xF, 0xF, true));
}

template <int NG>
__device__ __forceinline__ float reduce_row_groups(float x) {
  static_assert(NG == 4 || NG == 16, "row groups fill a quad or a DPP row");
  x += dpp_read<0xB1>(x);  // quad_perm [1,0,3,2]
  x += dpp_read<0x4E>(x);  // quad_perm [2,3,0,1]
  if constexpr (NG == 16) {
    x += dpp_read<0x141>(x);  // row_half_mirror
    x += dpp_read<0x140>(x);  // row_mirror
  }
  return x;
}

// The decode shape (one wave per state, CW = 64) keeps its row groups in the
// high lane bits instead: lanes 16 rg .. 16 rg + 15 then read whole 256-byte
// state rows per load instruction (measured 57 us against 68 us per config-1
// step with the low-bit layout), and its single token has no dependency chain
// to shorten.
template <int CW>
struct RowLayout {
  static constexpr bool kLow = CW != 64;  // row group in the low lane bits
};

template <int NG, bool kLow>
__device__ __forceinline__ float sum_row_groups(float x) {
  if constexpr (kLow) {
    return reduce_row_groups<NG>(x);
  } else {
    static_assert(NG == 4, "high-bit row groups are the lanes' two top bits");
    return add_xor32(add_xor16(x));
  }
}

// Sum over 4 row groups held in the high lane bits (xor 16, xor 32): the
// fused TMix kernel's layout.
__device__ __forceinline__ float reduce_row_groups_high(float x) {
  return add_xor32(add_xor16(x));
}

// Unit ranges: sequence s covers tokens cu_seqlens[s] .. cu_seqlens[s+1]-1,
// or cu_seqlens[s] .. seg_ends[s]-1 when seg_ends is given (independent
// chunks, the replay stage). state_dot_a (optional) receives a_t^T S_{t-1};
// read_only_state keeps the pool unwritten (the replay stage starts from
// stored boundaries); status may be null (no metadata word to check).
// elapsed is the fp16-state family's per-slot phase origin.
struct RecurrentKernelParams {
  int32_t num_heads, num_units;
  int64_t output_elements;
  int32_t total_tokens, state_pool_size;
  const int32_t* cu_seqlens;
  const int32_t* seg_ends;
  const int32_t* slots;
  const int32_t* status;
  const int32_t* elapsed;
  void* state;
  float* state_dot_a;
  int32_t read_only_state;
  float scale;
};

template <int D, int CW, int WG, typename T, DecayMode M, StateKind SK, bool kBuf = false>
__global__ __launch_bounds__(WG) void recurrent_fp32_kernel(
    RecurrentKernelParams p,
    const typename IoTraits<T>::storage* __restrict__ r_ptr,
    const typename IoTraits<T>::storage* __restrict__ decay_ptr,
    const typename IoTraits<T>::storage* __restrict__ bias_ptr,
    const typename IoTraits<T>::storage* __restrict__ k_ptr,
    const typename IoTraits<T>::storage* __restrict__ v_ptr,
    const typename IoTraits<T>::storage* __restrict__ a_ptr,
    const typename IoTraits<T>::storage* __restrict__ b_ptr,
    typename IoTraits<T>::storage* __restrict__ out_ptr) {
  const int32_t num_heads = p.num_heads;
  const int32_t total_tokens = p.total_tokens;
  const float scale = p.scale;
  constexpr int kWavesPerUnit = D / CW;
  constexpr int kNc = CW == 8 ? 2 : 4;  // state columns per lane (one vector)
  constexpr int kCg = CW / kNc;       // lanes per row group
  constexpr int kNg = 64 / kCg;       // row groups per wave
  constexpr int kRpl = D / kNg;       // key rows per lane
  static_assert(kRpl % 4 == 0, "lane rows load in 4-element pieces");
  using VC = typename ColVec<kNc>::type;

  if (p.status != nullptr && p.status[0] != 0) {
    fill_nan<T>(out_ptr, p.output_elements);
    return;
  }
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * (WG / 64) + (threadIdx.x >> 6);
  const int unit = wave / kWavesPerUnit;
  if (unit >= p.num_units) return;
  const int slab = wave % kWavesPerUnit;
  const int seq = unit / num_heads;
  const int head = unit % num_heads;
  constexpr bool kLowRows = RowLayout<CW>::kLow;
  const int rg = kLowRows ? lane % kNg : lane / kCg;
  const int cg = kLowRows ? lane / kNg : lane % kCg;
  const int row0 = rg * kRpl;
  const int col = slab * CW + kNc * cg;

  // One wave handles one sequence, so its bounds and slot are wave-uniform;
  // readfirstlane makes the token loop's branches scalar.
  const int32_t t_begin = __builtin_amdgcn_readfirstlane(p.cu_seqlens[seq]);
  const int32_t t_end = __builtin_amdgcn_readfirstlane(
      p.seg_ends != nullptr ? p.seg_ends[seq] : p.cu_seqlens[seq + 1]);
  const int32_t slot = __builtin_amdgcn_readfirstlane(p.slots != nullptr ? p.slots[seq] : seq);
  // Validated metadata never fails these; they keep a bad direct launch from
  // touching memory outside the tensors.
  if (t_begin < 0 || t_end > total_tokens || t_begin >= t_end || slot < 0 ||
      slot >= p.state_pool_size) {
    return;
  }

  using SS = typename StateTraits<SK>::storage;
  SS* sbase = static_cast<SS*>(p.state) +
              ((static_cast<int64_t>(slot) * num_heads + head) * D) * D;
  VC s[kRpl];
#pragma unroll
  for (int j = 0; j < kRpl; ++j) {
    if constexpr (kNc == 4) {
      s[j] = load_state4<SK>(sbase + static_cast<int64_t>(row0 + j) * D + col);
    } else {
      s[j] = load_state2<SK>(sbase + static_cast<int64_t>(row0 + j) * D + col);
    }
  }
  // fp16 state: phase of key row0 at the first token.
  uint32_t phase0 = 0;
  if constexpr (SK == StateKind::kFp16) {
    phase0 = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(p.elapsed[slot])) +
             static_cast<uint32_t>(head * D + row0) - static_cast<uint32_t>(t_begin);
  }

  float bias[kRpl];
  if (bias_ptr != nullptr) {
    load_vec<T, kRpl>(bias_ptr + head * D + row0, bias);
  } else {
#pragma unroll
    for (int j = 0; j < kRpl; ++j) bias[j] = 0.0f;
  }

  // Token rows are independent of the state, so their loads run ahead of the
  // recurrence: a register ring holds the raw rows of the next kPrefetch
  // tokens, and each step issues the loads of the token kPrefetch positions
  // later before it computes. Long sequences are otherwise bound by one HBM
  // round trip per token. Decode (one token, one wave per state) loads each
  // token in place instead: it needs many waves per SIMD to cover HBM latency,
  // so its register count must stay low.
  struct TokenRows {
    RawRow<T, kRpl> a, w, b, k, r;
    RawRow<T, kNc> v;
  };
  // kBuf (prefetching shapes, tensors under 2 GiB): buffer loads whose
  // per-lane offset is fixed and whose token offset is one scalar, so a
  // token's six row loads need no address arithmetic in the vector unit.
  constexpr uint32_t kEsize = IoTraits<T>::kBytes;
  const uint32_t tensor_bytes =
      kBuf ? static_cast<uint32_t>(total_tokens) * static_cast<uint32_t>(num_heads * D) * kEsize
           : 0u;
  // The ranges differ by a few bytes past each tensor's end (no access goes
  // there): with identical upper descriptor words the compiler shares them
  // between the descriptors and copies them back into place before every
  // load, ten scalar moves per token.
  const auto rs_a = buffer_rsrc(a_ptr, tensor_bytes);
  const auto rs_w = buffer_rsrc(decay_ptr, tensor_bytes + 4);
  const auto rs_b = buffer_rsrc(b_ptr, tensor_bytes + 8);
  const auto rs_k = buffer_rsrc(k_ptr, tensor_bytes + 12);
  const auto rs_r = buffer_rsrc(r_ptr, tensor_bytes + 16);
  const auto rs_v = buffer_rsrc(v_ptr, tensor_bytes + 20);
  const auto rs_out = buffer_rsrc(out_ptr, tensor_bytes);
  const uint32_t vo_rows = static_cast<uint32_t>(head * D + row0) * kEsize;
  const uint32_t vo_cols = static_cast<uint32_t>(head * D + col) * kEsize;
  const uint32_t token_bytes = static_cast<uint32_t>(num_heads * D) * kEsize;
  auto load_token = [&](TokenRows& dst, int32_t t) {
    if constexpr (kBuf) {
      const int so = static_cast<int>(static_cast<uint32_t>(t) * token_bytes);
      load_raw_buf<T, kRpl>(rs_a, vo_rows, so, dst.a);
      load_raw_buf<T, kRpl>(rs_w, vo_rows, so, dst.w);
      load_raw_buf<T, kRpl>(rs_b, vo_rows, so, dst.b);
      load_raw_buf<T, kRpl>(rs_k, vo_rows, so, dst.k);
      load_raw_buf<T, kRpl>(rs_r, vo_rows, so, dst.r);
      load_raw_buf<T, kNc>(rs_v, vo_cols, so, dst.v);
    } else {
      const int64_t base = (static_cast<int64_t>(t) * num_heads + head) * D;
      load_raw<T, kRpl>(a_ptr + base + row0, dst.a);
      load_raw<T, kRpl>(decay_ptr + base + row0, dst.w);
      load_raw<T, kRpl>(b_ptr + base + row0, dst.b);
      load_raw<T, kRpl>(k_ptr + base + row0, dst.k);
      load_raw<T, kRpl>(r_ptr + base + row0, dst.r);
      load_raw<T, kNc>(v_ptr + base + col, dst.v);
    }
  };
  // About 96 registers of ring; the one-wave decode shape loads in place.
  constexpr int kTokenWords = 5 * RawRow<T, kRpl>::kWords + RawRow<T, kNc>::kWords;
  constexpr int kRing = 96 / kTokenWords < 1 ? 1 : (96 / kTokenWords > 8 ? 8 : 96 / kTokenWords);
  constexpr int kPrefetch = (CW == 64) ? 1 : kRing;
  TokenRows ring[kPrefetch];
  if constexpr (kPrefetch > 1) {
#pragma unroll
    for (int j = 0; j < kPrefetch; ++j) {
      if (t_begin + j < t_end) load_token(ring[j], t_begin + j);
    }
  }

  for (int32_t t0 = t_begin; t0 < t_end; t0 += kPrefetch) {
#pragma unroll
    for (int jp = 0; jp < kPrefetch; ++jp) {
      const int32_t t = t0 + jp;
      if (t >= t_end) break;
      if constexpr (kPrefetch == 1) load_token(ring[0], t);
      float rr[kRpl], ww[kRpl], kk[kRpl], aa[kRpl], bb[kRpl], vv[kNc];
      decode_raw<T, kRpl>(ring[jp].a, aa);
      decode_raw<T, kRpl>(ring[jp].w, ww);
      decode_raw<T, kRpl>(ring[jp].b, bb);
      decode_raw<T, kRpl>(ring[jp].k, kk);
      decode_raw<T, kRpl>(ring[jp].r, rr);
      decode_raw<T, kNc>(ring[jp].v, vv);
      if constexpr (kPrefetch > 1) {
        // Unconditional (the last token again past the end): a skipped load
        // would make the ring registers a join of two paths, copied per token.
        load_token(ring[jp], min(t + kPrefetch, t_end - 1));
      }

      VC sa = zero_cols<VC>();
#pragma unroll
      for (int j = 0; j < kRpl; ++j) {
        sa.x = fmaf(aa[j], s[j].x, sa.x);
        sa.y = fmaf(aa[j], s[j].y, sa.y);
        if constexpr (kNc == 4) {
          sa.z = fmaf(aa[j], s[j].z, sa.z);
          sa.w = fmaf(aa[j], s[j].w, sa.w);
        }
      }
      sa.x = sum_row_groups<kNg, kLowRows>(sa.x);
      sa.y = sum_row_groups<kNg, kLowRows>(sa.y);
      if constexpr (kNc == 4) {
        sa.z = sum_row_groups<kNg, kLowRows>(sa.z);
        sa.w = sum_row_groups<kNg, kLowRows>(sa.w);
      }
      if (p.state_dot_a != nullptr && rg == 0) {
        *reinterpret_cast<VC*>(
            p.state_dot_a + (static_cast<int64_t>(t) * num_heads + head) * D + col) = sa;
      }

      VC y = zero_cols<VC>();
#pragma unroll
      for (int j = 0; j < kRpl; ++j) {
        // (The raw-retention prefetch path skips the zero bias; the decode
        // shape keeps the add: without it the compiler reorders the
        // one-token body and the HBM-bound launch runs 1.6% slower.)
        const float w = decay_retention<M>(
            (kPrefetch > 1 && M != DecayMode::kLogits) ? ww[j] : ww[j] + bias[j]);
        if constexpr (SK == StateKind::kFp32) {
          s[j].x = fmaf(w, s[j].x, fmaf(bb[j], sa.x, kk[j] * vv[0]));
          s[j].y = fmaf(w, s[j].y, fmaf(bb[j], sa.y, kk[j] * vv[1]));
          if constexpr (kNc == 4) {
            s[j].z = fmaf(w, s[j].z, fmaf(bb[j], sa.z, kk[j] * vv[2]));
            s[j].w = fmaf(w, s[j].w, fmaf(bb[j], sa.w, kk[j] * vv[3]));
          }
        } else {
          const uint32_t phase = phase0 + static_cast<uint32_t>(j + t);
          const float delta = round_f16(w - 1.0f + phase_dither(phase));
          s[j].x = round_f16(fmaf(kk[j], vv[0], fmaf(bb[j], sa.x, fmaf(s[j].x, delta, s[j].x))));
          s[j].y = round_f16(fmaf(kk[j], vv[1], fmaf(bb[j], sa.y, fmaf(s[j].y, delta, s[j].y))));
          if constexpr (kNc == 4) {
            s[j].z =
                round_f16(fmaf(kk[j], vv[2], fmaf(bb[j], sa.z, fmaf(s[j].z, delta, s[j].z))));
            s[j].w =
                round_f16(fmaf(kk[j], vv[3], fmaf(bb[j], sa.w, fmaf(s[j].w, delta, s[j].w))));
          }
        }
        y.x = fmaf(rr[j], s[j].x, y.x);
        y.y = fmaf(rr[j], s[j].y, y.y);
        if constexpr (kNc == 4) {
          y.z = fmaf(rr[j], s[j].z, y.z);
          y.w = fmaf(rr[j], s[j].w, y.w);
        }
      }
      y.x = sum_row_groups<kNg, kLowRows>(y.x);
      y.y = sum_row_groups<kNg, kLowRows>(y.y);
      if constexpr (kNc == 4) {
        y.z = sum_row_groups<kNg, kLowRows>(y.z);
        y.w = sum_row_groups<kNg, kLowRows>(y.w);
      }
      if (rg == 0) {
        if constexpr (kBuf) {
          const int so = static_cast<int>(static_cast<uint32_t>(t) * token_bytes);
          if constexpr (kNc == 4) {
            store4_buf<T>(rs_out, vo_cols, so, scale * y.x, scale * y.y, scale * y.z,
                          scale * y.w);
          } else {
            store2_buf<T>(rs_out, vo_cols, so, scale * y.x, scale * y.y);
          }
        } else {
          const int64_t base = (static_cast<int64_t>(t) * num_heads + head) * D;
          if constexpr (kNc == 4) {
            store4<T>(out_ptr + base + col, scale * y.x, scale * y.y, scale * y.z,
                      scale * y.w);
          } else {
            store2<T>(out_ptr + base + col, scale * y.x, scale * y.y);
          }
        }
      }
    }
  }

  if (p.read_only_state) return;
#pragma unroll
  for (int j = 0; j < kRpl; ++j) {
    if constexpr (kNc == 4) {
      store_state4<SK>(sbase + static_cast<int64_t>(row0 + j) * D + col, s[j]);
    } else {
      store_state2<SK>(sbase + static_cast<int64_t>(row0 + j) * D + col, s[j]);
    }
  }
}

struct RecurrentArgs {
  int32_t num_sequences, num_heads, head_size, total_tokens, max_seqlen,
      state_pool_size;
  const int32_t* cu;
  const int32_t* slots;
  const int32_t* status;
  void* state;
  const void *r, *decay, *bias, *k, *v, *a, *b;
  void* out;
  float scale;
  hipStream_t stream;
  const int32_t* seg_ends = nullptr;
  float* state_dot_a = nullptr;
  int32_t read_only_state = 0;
  const int32_t* elapsed = nullptr;
};

template <int D, int CW, int WG, typename T, DecayMode M, StateKind SK, bool kBuf = false>
int launch_recurrent(const RecurrentArgs& p) {
  using S = typename IoTraits<T>::storage;
  const int units = p.num_sequences * p.num_heads;
  const int64_t waves = static_cast<int64_t>(units) * (D / CW);
  const int blocks = static_cast<int>((waves + WG / 64 - 1) / (WG / 64));
  const int64_t out_elems = static_cast<int64_t>(p.total_tokens) * p.num_heads * D;
  RecurrentKernelParams kp{};
  kp.num_heads = p.num_heads;
  kp.num_units = units;
  kp.output_elements = out_elems;
  kp.total_tokens = p.total_tokens;
  kp.state_pool_size = p.state_pool_size;
  kp.cu_seqlens = p.cu;
  kp.seg_ends = p.seg_ends;
  kp.slots = p.slots;
  kp.status = p.status;
  kp.elapsed = p.elapsed;
  kp.state = p.state;
  kp.state_dot_a = p.state_dot_a;
  kp.read_only_state = p.read_only_state;
  kp.scale = p.scale;
  hipLaunchKernelGGL((recurrent_fp32_kernel<D, CW, WG, T, M, SK, kBuf>), dim3(blocks),
                     dim3(WG), 0, p.stream, kp, static_cast<const S*>(p.r),
                     static_cast<const S*>(p.decay), static_cast<const S*>(p.bias),
                     static_cast<const S*>(p.k), static_cast<const S*>(p.v),
                     static_cast<const S*>(p.a), static_cast<const S*>(p.b),
                     static_cast<S*>(p.out));
  return check_launch("recurrent_fp32_kernel");
}

// fp16-state decode shape (head size 64, one wave per state, a few tokens
// per sequence). Lane (rg, cg) = (lane / 8, lane % 8) holds key rows
// 8 rg .. 8 rg + 7 of value columns 8 cg .. 8 cg + 7: every state access is
// 16 bytes per lane (8 fp16), and the 8 lanes of a row group cover one whole
// 128-byte state row per load instruction. Token rows are 16-byte loads too
// (the lane's 8 key features, or its 8 value columns). Sums over key rows
// add the lane's 8 rows, then the 8 row groups held in lane bits 3..5
// (row_ror 8 inside a DPP row, then the 16- and 32-lane swaps); each step
// adds a lane pair symmetrically, so every lane of a column ends with the
// same bits. Same arithmetic and rounding points as recurrent_fp32_kernel's
// fp16-state path.
//
// Registers: the state and the token rows stay packed, two fp16 per register
// (32 + 24 registers), and every product reads its fp16 operands through the
// mixed-precision fma's half selects. The kernel then fits 5 waves per SIMD
// (92 registers) instead of 4 (118 with one value per register): 10,240
// states of config 1 run in two rounds of 5,120 resident waves, not in 2.5
// rounds of 4,096 (32.3 -> 30.3 us per step).
__device__ __forceinline__ float sum_row_groups8(float x) {
  x += dpp_read<0x128>(x);  // row_ror 8: lane ^ 8 inside the 16-lane row
  return add_xor32(add_xor16(x));
}

__device__ __forceinline__ uint4 load_x8(const uint16_t* p) {
  return *reinterpret_cast<const uint4*>(p);
}

// Word i of a packed row of 8 fp16 (i uniform after unrolling).
__device__ __forceinline__ uint32_t word_of(const uint4& q, int i) {
  return i == 0 ? q.x : i == 1 ? q.y : i == 2 ? q.z : q.w;
}

// Half e & 1 of a word of two fp16, as fp32 (exact).
__device__ __forceinline__ float half_of(uint32_t w, int e) {
  return static_cast<float>(
      __builtin_bit_cast(_Float16, static_cast<uint16_t>((e & 1) ? (w >> 16) : (w & 0xffffu))));
}

// Element e of a packed row of 8 fp16, as fp32.
__device__ __forceinline__ float elem_of(const uint4& q, int e) {
  return half_of(word_of(q, e >> 1), e);
}

// Two fp16 results in one register: lo = fp16(k * v_lo + t0) and
// hi = fp16(k * v_hi + t1), each rounded once from the fused multiply-add
// (v_fma_mixlo_f16 / v_fma_mixhi_f16; MIXHI keeps the low half). k is half
// kh of kw, v_lo and v_hi are the two halves of vw, t0 and t1 are fp32. The
// compiler does not form the MIXHI write into a shared register by itself.
template <int kh>
__device__ __forceinline__ uint32_t fma_pair_f16(uint32_t kw, uint32_t vw, float t0, float t1) {
  uint32_t w;
  if constexpr (kh == 0) {
    asm("v_fma_mixlo_f16 %0, %1, %2, %3 op_sel_hi:[1,1,0]\n\t"
        "v_fma_mixhi_f16 %0, %1, %2, %4 op_sel:[0,1,0] op_sel_hi:[1,1,0]"
        : "=&v"(w)
        : "v"(kw), "v"(vw), "v"(t0), "v"(t1));
  } else {
    asm("v_fma_mixlo_f16 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,1,0]\n\t"
        "v_fma_mixhi_f16 %0, %1, %2, %4 op_sel:[1,1,0] op_sel_hi:[1,1,0]"
        : "=&v"(w)
        : "v"(kw), "v"(vw), "v"(t0), "v"(t1));
  }
  return w;
}

__global__ __launch_bounds__(64, 5) void recurrent_fp16_decode_kernel(
    RecurrentKernelParams p, const uint16_t* __restrict__ r_ptr,
    const uint16_t* __restrict__ decay_ptr, const uint16_t* __restrict__ bias_ptr,
    const uint16_t* __restrict__ k_ptr, const uint16_t* __restrict__ v_ptr,
    const uint16_t* __restrict__ a_ptr, const uint16_t* __restrict__ b_ptr,
    uint16_t* __restrict__ out_ptr) {
  constexpr int D = 64;
  if (p.status != nullptr && p.status[0] != 0) {
    fill_nan<F16>(out_ptr, p.output_elements);
    return;
  }
  const int unit = blockIdx.x;
  if (unit >= p.num_units) return;
  const int lane = threadIdx.x & 63;
  const int num_heads = p.num_heads;
  const int seq = unit / num_heads;
  const int head = unit % num_heads;
  const int rg = lane >> 3, cg = lane & 7;
  const int row0 = 8 * rg, col = 8 * cg;
  const int32_t t_begin = __builtin_amdgcn_readfirstlane(p.cu_seqlens[seq]);
  const int32_t t_end = __builtin_amdgcn_readfirstlane(p.cu_seqlens[seq + 1]);
  const int32_t slot = __builtin_amdgcn_readfirstlane(p.slots[seq]);
  if (t_begin < 0 || t_end > p.total_tokens || t_begin >= t_end || slot < 0 ||
      slot >= p.state_pool_size) {
    return;
  }
  uint16_t* sbase = static_cast<uint16_t*>(p.state) +
                    ((static_cast<int64_t>(slot) * num_heads + head) * D) * D;
  // sp[j][i]: state row row0 + j, columns col + 2i (low half) and col + 2i + 1.
  uint32_t sp[8][4];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const u32x4 q = __builtin_nontemporal_load(
        reinterpret_cast<const u32x4*>(sbase + (row0 + j) * D + col));
    sp[j][0] = q.x;
    sp[j][1] = q.y;
    sp[j][2] = q.z;
    sp[j][3] = q.w;
  }
  auto state = [&](int j, int c) { return half_of(sp[j][c >> 1], c); };
  float bias[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (bias_ptr != nullptr) {
    const uint4 qb = load_x8(bias_ptr + head * D + row0);
#pragma unroll
    for (int e = 0; e < 8; ++e) bias[e] = elem_of(qb, e);
  }
  const uint32_t phase0 = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(p.elapsed[slot])) +
                          static_cast<uint32_t>(head * D + row0) - static_cast<uint32_t>(t_begin);

  for (int32_t t = t_begin; t < t_end; ++t) {
    const int64_t base = (static_cast<int64_t>(t) * num_heads + head) * D;
    const uint4 qa = load_x8(a_ptr + base + row0), qx = load_x8(decay_ptr + base + row0);
    const uint4 qb = load_x8(b_ptr + base + row0), qk = load_x8(k_ptr + base + row0);
    const uint4 qr = load_x8(r_ptr + base + row0), qv = load_x8(v_ptr + base + col);
    float sa[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc = fmaf(elem_of(qa, j), state(j, c), acc);
      sa[c] = sum_row_groups8(acc);
    }
    float y[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float w = decay_retention<DecayMode::kLogits>(elem_of(qx, j) + bias[j]);
      const float delta =
          round_f16(w - 1.0f + phase_dither(phase0 + static_cast<uint32_t>(j + t)));
      const float bj = elem_of(qb, j), rj = elem_of(qr, j);
#pragma unroll
      for (int c = 0; c < 8; c += 2) {
        const float s0 = state(j, c), s1 = state(j, c + 1);
        const float t0 = fmaf(bj, sa[c], fmaf(s0, delta, s0));
        const float t1 = fmaf(bj, sa[c + 1], fmaf(s1, delta, s1));
        sp[j][c >> 1] = (j & 1) == 0
                            ? fma_pair_f16<0>(word_of(qk, j >> 1), word_of(qv, c >> 1), t0, t1)
                            : fma_pair_f16<1>(word_of(qk, j >> 1), word_of(qv, c >> 1), t0, t1);
        y[c] = fmaf(rj, state(j, c), y[c]);
        y[c + 1] = fmaf(rj, state(j, c + 1), y[c + 1]);
      }
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) y[c] = sum_row_groups8(y[c]);
    if (rg == 0) {
      u32x4 q;
      q.x = pack2<F16>(p.scale * y[0], p.scale * y[1]);
      q.y = pack2<F16>(p.scale * y[2], p.scale * y[3]);
      q.z = pack2<F16>(p.scale * y[4], p.scale * y[5]);
      q.w = pack2<F16>(p.scale * y[6], p.scale * y[7]);
      *reinterpret_cast<u32x4*>(out_ptr + base + col) = q;
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const u32x4 q = {sp[j][0], sp[j][1], sp[j][2], sp[j][3]};
    __builtin_nontemporal_store(q, reinterpret_cast<u32x4*>(sbase + (row0 + j) * D + col));
  }
}

int launch_fp16_decode(const RecurrentArgs& p) {
  const int units = p.num_sequences * p.num_heads;
  RecurrentKernelParams kp{};
  kp.num_heads = p.num_heads;
  kp.num_units = units;
  kp.output_elements = static_cast<int64_t>(p.total_tokens) * p.num_heads * 64;
  kp.total_tokens = p.total_tokens;
  kp.state_pool_size = p.state_pool_size;
  kp.cu_seqlens = p.cu;
  kp.slots = p.slots;
  kp.status = p.status;
  kp.elapsed = p.elapsed;
  kp.state = p.state;
  kp.scale = p.scale;
  using S = uint16_t;
  hipLaunchKernelGGL(recurrent_fp16_decode_kernel, dim3(units), dim3(64), 0, p.stream, kp,
                     static_cast<const S*>(p.r), static_cast<const S*>(p.decay),
                     static_cast<const S*>(p.bias), static_cast<const S*>(p.k),
                     static_cast<const S*>(p.v), static_cast<const S*>(p.a),
                     static_cast<const S*>(p.b), static_cast<S*>(p.out));
  return check_launch("recurrent_fp16_decode_kernel");
}

// SIMDs of an MI355X (256 CUs x 4), the gfx950 part this library is built for.
constexpr int64_t kSimdCount = 1024;

// Smallest max_seqlen that the recurrent operator routes to the chunk kernel.
constexpr int32_t kChunkedMinSeqlen = 64;

// Token tensors small enough for 32-bit buffer offsets (below 2 GiB).
template <int D, typename T>
bool buffer_addressable(const RecurrentArgs& p) {
  return static_cast<int64_t>(p.total_tokens) * p.num_heads * D * IoTraits<T>::kBytes <
         (int64_t{1} << 31);
}

template <typename T, DecayMode M, StateKind SK = StateKind::kFp32>
int dispatch_head_size(const RecurrentArgs& p) {
  switch (p.head_size) {
    case 64:
      // Decode keeps one wave per state (fewest redundant decay evaluations);
      // longer sequences split the state over 4 waves for more parallelism.
      if (p.max_seqlen > 0 && p.max_seqlen <= 2) {
        if constexpr (SK == StateKind::kFp16) return launch_fp16_decode(p);
        return launch_recurrent<64, 64, 64, T, M, SK>(p);
      }
      // Few states: 8-column slabs (8 waves per state), so that the launch
      // fills more SIMDs and each wave's token step is half as long. Beyond
      // one wave per SIMD the 16-column slabs' fewer redundant decay and
      // token-row evaluations win (same-box, B x H = 32 .. 128: 23-24%
      // faster; 256: 2.5% slower).
      if (static_cast<int64_t>(p.num_sequences) * p.num_heads * 8 <= kSimdCount) {
        if (buffer_addressable<64, T>(p)) return launch_recurrent<64, 8, 256, T, M, SK, true>(p);
        return launch_recurrent<64, 8, 256, T, M, SK>(p);
      }
      if (buffer_addressable<64, T>(p)) return launch_recurrent<64, 16, 256, T, M, SK, true>(p);
      return launch_recurrent<64, 16, 256, T, M, SK>(p);
    case 128:
      if (buffer_addressable<128, T>(p)) return launch_recurrent<128, 16, 256, T, M, SK, true>(p);
      return launch_recurrent<128, 16, 256, T, M, SK>(p);
    case 256:
      if (buffer_addressable<256, T>(p)) return launch_recurrent<256, 16, 256, T, M, SK, true>(p);
      return launch_recurrent<256, 16, 256, T, M, SK>(p);
    default:
      return set_error(FRWKV_ERR_UNSUPPORTED,
                       "recurrent head size must be 64, 128, or 256, got %d",
                       p.head_size);
  }
}

template <typename T>
int dispatch_decay(const RecurrentArgs& p, int decay_mode) {
  if (decay_mode == FRWKV_DECAY_LOGITS) return dispatch_head_size<T, DecayMode::kLogits>(p);
  if (decay_mode == FRWKV_DECAY_RAW_W) {
    if (p.bias != nullptr) {
      return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                       "decay_bias is only defined for the logits decay mode");
    }
    return dispatch_head_size<T, DecayMode::kRawW>(p);
  }
  return set_error(FRWKV_ERR_INVALID_ARGUMENT, "unknown decay mode %d", decay_mode);
}

// Fused TMix chain for decode and short sequences (head size 64, fp32 pool,
// one wave per (sequence, head) state; lane (rg, cg) = (lane / 16, lane % 16)
// holds key rows 16rg..16rg+15 of value columns 4cg..4cg+3). Per token it runs, without writing the intermediates:
//   producer (reference kk_a_gate): u = k k_k, kk = u / max(|u|, 1e-12),
//     gate = sigmoid(a0 + a12), k' = k (gate k_a + 1 - k_a);
//   WKV7 step with k', a = -kk, b = kk gate (S += b (a^T S), the RWKV-7
//     update as the benchmark configs state it), y = scale S^T r;
//   consumer (reference lnx_rkvres_xg): out = ((y - mean) rstd ln_w + ln_b
//     + rkv v) g with rstd = 1 / sqrt(var + 64e-5), rkv = sum r k' r_k.
// Norms over key features reduce across the four row groups (xor 16, 32),
// norms over value columns across the 16 column-group lanes (xor 1..8).
struct FusedTmixParams {
  const void* a12;
  const void* g;
  const void* k_k;
  const void* a0;
  const void* k_a;
  const void* r_k;
  const void* ln_weight;
  const void* ln_bias;
};

__device__ __forceinline__ float sigmoid_fast(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-kLog2E * x));
}

// Sum over the 16 lanes of a DPP row (the DPP butterfly of reduce_row_groups).
__device__ __forceinline__ float reduce_col_groups(float x) {
  return reduce_row_groups<16>(x);
}

template <typename T, DecayMode M>
__global__ __launch_bounds__(64, 2) void recurrent_tmix_fused_kernel(
    RecurrentKernelParams p, FusedTmixParams f,
    const typename IoTraits<T>::storage* __restrict__ r_ptr,
    const typename IoTraits<T>::storage* __restrict__ decay_ptr,
    const typename IoTraits<T>::storage* __restrict__ bias_ptr,
    const typename IoTraits<T>::storage* __restrict__ k_ptr,
    const typename IoTraits<T>::storage* __restrict__ v_ptr,
    typename IoTraits<T>::storage* __restrict__ out_ptr) {
  using S = typename IoTraits<T>::storage;
  constexpr int D = 64;
  constexpr int kRpl = 16;
  const int32_t num_heads = p.num_heads;
  if (p.status != nullptr && p.status[0] != 0) {
    fill_nan<T>(out_ptr, p.output_elements);
    return;
  }
  const int lane = threadIdx.x & 63;
  const int unit = blockIdx.x;
  if (unit >= p.num_units) return;
  const int seq = unit / num_heads;
  const int head = unit % num_heads;
  const int cg = lane % 16;
  const int rg = lane / 16;
  const int row0 = rg * kRpl;
  const int col = 4 * cg;
  const int32_t t_begin = __builtin_amdgcn_readfirstlane(p.cu_seqlens[seq]);
  const int32_t t_end = __builtin_amdgcn_readfirstlane(p.cu_seqlens[seq + 1]);
  const int32_t slot = __builtin_amdgcn_readfirstlane(p.slots[seq]);
  if (t_begin < 0 || t_end > p.total_tokens || t_begin >= t_end || slot < 0 ||
      slot >= p.state_pool_size) {
    return;
  }
  float* sbase = static_cast<float*>(p.state) +
                 ((static_cast<int64_t>(slot) * num_heads + head) * D) * D;
  float4 s[kRpl];
#pragma unroll
  for (int j = 0; j < kRpl; ++j) {
    s[j] = load_state4<StateKind::kFp32>(sbase + static_cast<int64_t>(row0 + j) * D + col);
  }
  // Per-head vectors: the lane's 16 key rows of k_k, a0, k_a, r_k (kept raw,
  // decoded per token) and its 4 value columns of the norm weight and bias.
  const int64_t hrow = static_cast<int64_t>(head) * D;
  RawRow<T, kRpl> kkp_raw, a0_raw, ka_raw, rk_raw;
  load_raw<T, kRpl>(static_cast<const S*>(f.k_k) + hrow + row0, kkp_raw);
  load_raw<T, kRpl>(static_cast<const S*>(f.a0) + hrow + row0, a0_raw);
  load_raw<T, kRpl>(static_cast<const S*>(f.k_a) + hrow + row0, ka_raw);
  load_raw<T, kRpl>(static_cast<const S*>(f.r_k) + hrow + row0, rk_raw);
  float lnw[4], lnb[4];
  load_vec<T, 4>(static_cast<const S*>(f.ln_weight) + hrow + col, lnw);
  load_vec<T, 4>(static_cast<const S*>(f.ln_bias) + hrow + col, lnb);
  float bias[kRpl];
  if (bias_ptr != nullptr) {
    load_vec<T, kRpl>(bias_ptr + hrow + row0, bias);
  } else {
#pragma unroll
    for (int j = 0; j < kRpl; ++j) bias[j] = 0.0f;
  }

  // Element j of a raw row (rows stay packed; decoding on use keeps the
  // register count, and so the number of waves per SIMD, close to the plain
  // decode kernel's).
  auto at = [](const auto& raw, int j) {
    const uint32_t w = raw.w[j >> 1];
    return to_f32<T>(static_cast<uint16_t>((j & 1) ? (w >> 16) : (w & 0xffffu)));
  };
  for (int32_t t = t_begin; t < t_end; ++t) {
    const int64_t base = (static_cast<int64_t>(t) * num_heads + head) * D;
    RawRow<T, kRpl> a12_raw, w_raw, k_raw, r_raw;
    load_raw<T, kRpl>(static_cast<const S*>(f.a12) + base + row0, a12_raw);
    load_raw<T, kRpl>(decay_ptr + base + row0, w_raw);
    load_raw<T, kRpl>(k_ptr + base + row0, k_raw);
    load_raw<T, kRpl>(r_ptr + base + row0, r_raw);
    float vv[4], gg[4];
    load_vec<T, 4>(v_ptr + base + col, vv);
    load_vec<T, 4>(static_cast<const S*>(f.g) + base + col, gg);

    // Producer: the norm of u = k k_k over the head's 64 key features.
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < kRpl; ++j) {
      const float u = at(k_raw, j) * at(kkp_raw, j);
      ss = fmaf(u, u, ss);
    }
    const float inv =
        __builtin_amdgcn_rcpf(fmaxf(__builtin_sqrtf(reduce_row_groups_high(ss)), 1.0e-12f));
    // WKV7 step. sa = S^T a with a = -kk; then, row by row, the rest of the
    // producer (gate, b = kk gate, k' = k (gate k_a + 1 - k_a)), the update,
    // y = S^T r and the residual dot rkv = sum r k' r_k. Each producer value
    // is computed once, where it is used.
    float4 sa = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < kRpl; ++j) {
      const float a_j = -(at(k_raw, j) * at(kkp_raw, j) * inv);
      sa.x = fmaf(a_j, s[j].x, sa.x);
      sa.y = fmaf(a_j, s[j].y, sa.y);
      sa.z = fmaf(a_j, s[j].z, sa.z);
      sa.w = fmaf(a_j, s[j].w, sa.w);
    }
    sa.x = reduce_row_groups_high(sa.x);
    sa.y = reduce_row_groups_high(sa.y);
    sa.z = reduce_row_groups_high(sa.z);
    sa.w = reduce_row_groups_high(sa.w);
    float4 y = make_float4(0.f, 0.f, 0.f, 0.f);
    float rkv = 0.0f;
#pragma unroll
    for (int j = 0; j < kRpl; ++j) {
      const float kraw = at(k_raw, j);
      const float kkn = kraw * at(kkp_raw, j) * inv;
      const float gate = sigmoid_fast(at(a0_raw, j) + at(a12_raw, j));
      const float ka = at(ka_raw, j);
      const float b_j = kkn * gate;
      const float k_j = kraw * fmaf(gate, ka, 1.0f - ka);
      const float w = decay_retention<M>(at(w_raw, j) + bias[j]);
      const float rj = at(r_raw, j);
      rkv = fmaf(rj * k_j, at(rk_raw, j), rkv);
      s[j].x = fmaf(w, s[j].x, fmaf(b_j, sa.x, k_j * vv[0]));
      s[j].y = fmaf(w, s[j].y, fmaf(b_j, sa.y, k_j * vv[1]));
      s[j].z = fmaf(w, s[j].z, fmaf(b_j, sa.z, k_j * vv[2]));
      s[j].w = fmaf(w, s[j].w, fmaf(b_j, sa.w, k_j * vv[3]));
      y.x = fmaf(rj, s[j].x, y.x);
      y.y = fmaf(rj, s[j].y, y.y);
      y.z = fmaf(rj, s[j].z, y.z);
      y.w = fmaf(rj, s[j].w, y.w);
    }
    rkv = reduce_row_groups_high(rkv);
    const float x[4] = {p.scale * reduce_row_groups_high(y.x), p.scale * reduce_row_groups_high(y.y),
                        p.scale * reduce_row_groups_high(y.z), p.scale * reduce_row_groups_high(y.w)};

    // Consumer: per-head norm of the output, residual and gate.
    const float mean = reduce_col_groups(x[0] + x[1] + x[2] + x[3]) * (1.0f / D);
    float dev[4], sq = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      dev[c] = x[c] - mean;
      sq = fmaf(dev[c], dev[c], sq);
    }
    const float rstd = __builtin_amdgcn_rsqf(reduce_col_groups(sq) * (1.0f / D) + 64.0e-5f);
    float o[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      o[c] = fmaf(dev[c] * rstd, lnw[c], fmaf(rkv, vv[c], lnb[c])) * gg[c];
    }
    if (rg == 0) store4<T>(out_ptr + base + col, o[0], o[1], o[2], o[3]);
  }

#pragma unroll
  for (int j = 0; j < kRpl; ++j) {
    store_state4<StateKind::kFp32>(sbase + static_cast<int64_t>(row0 + j) * D + col, s[j]);
  }
}

template <typename T, DecayMode M>
int launch_tmix_fused(const RecurrentArgs& a, const FusedTmixParams& f) {
  using S = typename IoTraits<T>::storage;
  RecurrentKernelParams kp{};
  kp.num_heads = a.num_heads;
  kp.num_units = a.num_sequences * a.num_heads;
  kp.output_elements = static_cast<int64_t>(a.total_tokens) * a.num_heads * 64;
  kp.total_tokens = a.total_tokens;
  kp.state_pool_size = a.state_pool_size;
  kp.cu_seqlens = a.cu;
  kp.slots = a.slots;
  kp.status = a.status;
  kp.state = a.state;
  kp.scale = a.scale;
  hipLaunchKernelGGL((recurrent_tmix_fused_kernel<T, M>), dim3(kp.num_units), dim3(64), 0,
                     a.stream, kp, f, static_cast<const S*>(a.r),
                     static_cast<const S*>(a.decay), static_cast<const S*>(a.bias),
                     static_cast<const S*>(a.k), static_cast<const S*>(a.v),
                     static_cast<S*>(a.out));
  return check_launch("recurrent_tmix_fused_kernel");
}

template <typename T>
int dispatch_tmix_fused(const RecurrentArgs& a, const FusedTmixParams& f, int decay_mode) {
  if (decay_mode == FRWKV_DECAY_LOGITS) return launch_tmix_fused<T, DecayMode::kLogits>(a, f);
  if (decay_mode == FRWKV_DECAY_RAW_W) {
    if (a.bias != nullptr) {
      return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                       "decay_bias is only defined for the logits decay mode");
    }
    return launch_tmix_fused<T, DecayMode::kRawW>(a, f);
  }
  return set_error(FRWKV_ERR_INVALID_ARGUMENT, "unknown decay mode %d", decay_mode);
}

}  // namespace
}  // namespace frwkv

extern "C" int frwkv_recurrent_forward(
    int io_dtype, int decay_mode, int32_t num_sequences, int32_t num_heads,
    int32_t head_size, int32_t total_tokens, int32_t max_seqlen,
    int32_t state_pool_size, const int32_t* cu_seqlens,
    const int32_t* state_indices, const int32_t* metadata_status,
    float* state_pool, const void* r, const void* decay, const void* decay_bias,
    const void* k, const void* v, const void* a, const void* b, void* output,
    float scale, void* stream) {
  using namespace frwkv;
  if (!cu_seqlens || !state_indices || !metadata_status || !state_pool || !r ||
      !decay || !k || !v || !a || !b || !output) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_recurrent_forward: null pointer argument");
  }
  if (num_sequences <= 0 || num_sequences > 65535 || num_heads <= 0 ||
      total_tokens <= 0 || state_pool_size <= 0) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_recurrent_forward: sizes must be positive "
                     "(B=%d, H=%d, N=%d, slots=%d)",
                     num_sequences, num_heads, total_tokens, state_pool_size);
  }
  if (!__builtin_isfinite(scale)) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT, "scale must be finite");
  }
  // Long bf16 sequences at head size 64 take the split-precision chunk
  // kernel: its products keep about 2^-17 relative error per operand, so the
  // outputs stay within the per-token kernel's tolerances, at several times
  // its speed once sequences span a few chunks.
  if (io_dtype == FRWKV_DTYPE_BF16 && head_size == 64 && max_seqlen >= kChunkedMinSeqlen) {
    return frwkv_recurrent_chunked_forward(decay_mode, num_sequences, num_heads, total_tokens,
                                           state_pool_size, cu_seqlens, state_indices,
                                           metadata_status, state_pool, r, decay, decay_bias,
                                           k, v, a, b, output, scale, stream);
  }
  RecurrentArgs p{num_sequences, num_heads, head_size, total_tokens, max_seqlen,
                  state_pool_size, cu_seqlens, state_indices, metadata_status,
                  state_pool, r, decay, decay_bias, k, v, a, b, output, scale,
                  static_cast<hipStream_t>(stream)};
  switch (io_dtype) {
    case FRWKV_DTYPE_BF16:
      return dispatch_decay<Bf16>(p, decay_mode);
    case FRWKV_DTYPE_F16:
      return dispatch_decay<F16>(p, decay_mode);
    case FRWKV_DTYPE_F32:
      return dispatch_decay<float>(p, decay_mode);
    default:
      return set_error(FRWKV_ERR_INVALID_ARGUMENT, "unknown io dtype %d", io_dtype);
  }
}

// Replay stage for head sizes other than 64 (called by frwkv_chunk_replay):
// unit c runs tokens chunk_token_starts[c] .. chunk_token_ends[c]-1 from
// boundary[c], which stays unwritten, and writes output and a^T S_{t-1}.
int frwkv_replay_recurrent(int io_dtype, int decay_mode, int32_t num_chunks, int32_t num_heads,
                           int32_t head_size, int32_t total_tokens,
                           const int32_t* chunk_token_starts, const int32_t* chunk_token_ends,
                           const float* boundary, const void* r, const void* decay,
                           const void* decay_bias, const void* k, const void* v,
                           const void* a, const void* b, void* output, float* state_dot_a,
                           float scale, void* stream) {
  using namespace frwkv;
  RecurrentArgs p{num_chunks, num_heads, head_size, total_tokens, /*max_seqlen=*/-1,
                  num_chunks, chunk_token_starts, /*slots=*/nullptr, /*status=*/nullptr,
                  const_cast<float*>(boundary), r, decay, decay_bias, k, v, a, b, output,
                  scale, static_cast<hipStream_t>(stream)};
  p.seg_ends = chunk_token_ends;
  p.state_dot_a = state_dot_a;
  p.read_only_state = 1;
  switch (io_dtype) {
    case FRWKV_DTYPE_BF16:
      return dispatch_decay<Bf16>(p, decay_mode);
    case FRWKV_DTYPE_F16:
      return dispatch_decay<F16>(p, decay_mode);
    default:
      return set_error(FRWKV_ERR_UNSUPPORTED,
                       "replay takes float16 or bfloat16 tokens (io dtype %d)", io_dtype);
  }
}

// fp16-state family: fp16 tokens, decay logits, fp16 pool, per-slot elapsed
// phase origins (read, not advanced: frwkv_advance_i32_varlen does that).
extern "C" int frwkv_recurrent_fp16_forward(
    int32_t num_sequences, int32_t num_heads, int32_t head_size, int32_t total_tokens,
    int32_t max_seqlen, int32_t state_pool_size, const int32_t* cu_seqlens,
    const int32_t* state_indices, const int32_t* metadata_status,
    const int32_t* elapsed_state_pool, void* state_pool, const void* r,
    const void* decay_logits, const void* decay_bias, const void* k, const void* v,
    const void* a, const void* b, void* output, float scale, void* stream) {
  using namespace frwkv;
  if (!cu_seqlens || !state_indices || !metadata_status || !elapsed_state_pool ||
      !state_pool || !r || !decay_logits || !k || !v || !a || !b || !output) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_recurrent_fp16_forward: null pointer argument");
  }
  if (num_sequences <= 0 || num_sequences > 65535 || num_heads <= 0 ||
      total_tokens <= 0 || state_pool_size <= 0) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_recurrent_fp16_forward: sizes must be positive "
                     "(B=%d, H=%d, N=%d, slots=%d)",
                     num_sequences, num_heads, total_tokens, state_pool_size);
  }
  if (!__builtin_isfinite(scale)) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT, "scale must be finite");
  }
  RecurrentArgs p{num_sequences, num_heads, head_size, total_tokens, max_seqlen,
                  state_pool_size, cu_seqlens, state_indices, metadata_status,
                  state_pool, r, decay_logits, decay_bias, k, v, a, b, output, scale,
                  static_cast<hipStream_t>(stream)};
  p.elapsed = elapsed_state_pool;
  return dispatch_head_size<F16, DecayMode::kLogits, StateKind::kFp16>(p);
}

// Fused TMix chain (producer + WKV7 step + consumer) on the fp32 pool, head
// size 64; see recurrent_tmix_fused_kernel.
extern "C" int frwkv_recurrent_tmix_fused_forward(
    int io_dtype, int decay_mode, int32_t num_sequences, int32_t num_heads,
    int32_t head_size, int32_t total_tokens, int32_t state_pool_size,
    const int32_t* cu_seqlens, const int32_t* state_indices,
    const int32_t* metadata_status, float* state_pool, const void* r, const void* decay,
    const void* decay_bias, const void* k, const void* v, const void* a12, const void* g,
    const void* k_k, const void* a0, const void* k_a, const void* r_k,
    const void* ln_weight, const void* ln_bias, void* output, float scale, void* stream) {
  using namespace frwkv;
  if (!cu_seqlens || !state_indices || !metadata_status || !state_pool || !r || !decay ||
      !k || !v || !a12 || !g || !k_k || !a0 || !k_a || !r_k || !ln_weight || !ln_bias ||
      !output) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_recurrent_tmix_fused_forward: null pointer argument");
  }
  if (head_size != 64) {
    return set_error(FRWKV_ERR_UNSUPPORTED,
                     "frwkv_recurrent_tmix_fused_forward: head size 64 only, got %d",
                     head_size);
  }
  if (num_sequences <= 0 || num_sequences > 65535 || num_heads <= 0 || total_tokens <= 0 ||
      state_pool_size <= 0) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT,
                     "frwkv_recurrent_tmix_fused_forward: sizes must be positive "
                     "(B=%d, H=%d, N=%d, slots=%d)",
                     num_sequences, num_heads, total_tokens, state_pool_size);
  }
  if (!__builtin_isfinite(scale)) {
    return set_error(FRWKV_ERR_INVALID_ARGUMENT, "scale must be finite");
  }
  RecurrentArgs p{num_sequences, num_heads, head_size, total_tokens, /*max_seqlen=*/-1,
                  state_pool_size, cu_seqlens, state_indices, metadata_status,
                  state_pool, r, decay, decay_bias, k, v, /*a=*/nullptr, /*b=*/nullptr,
                  output, scale, static_cast<hipStream_t>(stream)};
  const FusedTmixParams f{a12, g, k_k, a0, k_a, r_k, ln_weight, ln_bias};
  switch (io_dtype) {
    case FRWKV_DTYPE_BF16:
      return dispatch_tmix_fused<Bf16>(p, f, decay_mode);
    case FRWKV_DTYPE_F16:
      return dispatch_tmix_fused<F16>(p, f, decay_mode);
    default:
      return set_error(FRWKV_ERR_UNSUPPORTED,
                       "the fused TMix chain takes float16 or bfloat16 tokens (io dtype %d)",
                       io_dtype);
  }
}
