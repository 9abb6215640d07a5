// MFMA and LDS-tile helpers for the chunked WKV7 kernels (gfx950, wave64).
//
// Every matrix product in the chunked kernels is a sum of 16x16x16 bf16 MFMA
// tiles (v_mfma_f32_16x16x16_bf16, fp32 accumulate). With lane l, g = l / 16
// and n = l % 16 the register layouts are:
//   A operand (4 bf16): A[m = n][k = 4g + e],  e = 0..3
//   B operand (4 bf16): B[k = 4g + e][n]
//   C / D     (4 fp32): C[m = 4g + j][n],      j = 0..3
// so an accumulator tile in C layout is, after conversion to bf16, directly
// the B operand of a product contracting over its rows, and the A operand of
// a product contracting over its columns with its transpose. Kernels chain
// products through registers this way and only stage operands that several
// waves share through LDS.
//
// LDS tiles are 64 x 64 bf16 with a padded row stride of 72 elements
// (144 bytes = 36 banks): the 16 rows an operand read touches start in 16
// distinct bank groups, so 8-byte operand reads are conflict-free within each
// 16-lane group.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace frwkv {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// Buffer resource over [base, base + bytes): loads beyond the range return
// zero and stores beyond it are dropped by the hardware. Descriptor word 3
// for gfx9-family raw buffers.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base,
                                                              uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0,
                                           static_cast<int>(bytes), 0x00020000);
}

constexpr int kTileStride = 72;                  // bf16 elements per LDS row
constexpr int kTileElems = 64 * kTileStride;     // one 64 x 64 tile

typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x4 mfma16(i16x4 a, i16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

// v_mfma_f32_16x16x32_bf16: same issue cost as the 16x16x16 form on gfx950
// for twice the work. An accumulator chain must keep one MFMA shape: with
// this toolchain, a 16x16x16 MFMA taking a 16x16x32 result as its
// accumulator a few instructions later produced wrong sums on MI355X (the
// wait states between the two were too few), so single 16-blocks are fed as
// zero-padded 32-wide steps instead. Operand register e of lane (g, n) carries
// k = 4g + e (e < 4) and k = 16 + 4g + (e - 4) (e >= 4) of the 32-wide K
// block: two 16-row blocks in C layout concatenate into one operand, and an
// LDS operand is two 8-byte reads 16 columns apart.
__device__ __forceinline__ f32x4 mfma32(i16x8 a, i16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

__device__ __forceinline__ i16x8 cat(i16x4 lo, i16x4 hi) {
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// Round-to-nearest-even fp32 -> bf16 bits.
__device__ __forceinline__ uint16_t to_bf16_bits(float x) {
  __bf16 h = static_cast<__bf16>(x);
  uint16_t bits;
  __builtin_memcpy(&bits, &h, 2);
  return bits;
}

__device__ __forceinline__ float bf16_float(uint16_t bits) {
  return __uint_as_float(static_cast<uint32_t>(bits) << 16);
}

// Two fp32 -> two round-to-nearest-even bf16 in one dword (lo in bits
// 0..15). The vector conversion selects one v_cvt_pk_bf16_f32 with both
// sources; converting the halves one by one costs a conversion per value plus
// the shift/mask/or to pack them.
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// Two fp32 split into bf16 pairs x = hi + lo: .x packs hi = bf16(x), .y packs
// lo = bf16(x - hi) (x - hi is exact in fp32), leaving a relative error of
// about 2^-17 where bf16 alone leaves 2^-9.
__device__ __forceinline__ uint2 split_bf16x2(float x0, float x1) {
  const uint32_t hi = pack_bf16x2(x0, x1);
  const float h0 = __uint_as_float(hi << 16);
  const float h1 = __uint_as_float(hi & 0xffff0000u);
  return make_uint2(hi, pack_bf16x2(x0 - h0, x1 - h1));
}

// C-layout accumulator -> bf16 operand registers (two packed conversions;
// a single 4-wide vector conversion is split into per-value conversions plus
// byte permutes when its result feeds an MFMA operand directly).
__device__ __forceinline__ i16x4 to_operand(f32x4 c) {
  const u32x2 q = {pack_bf16x2(c[0], c[1]), pack_bf16x2(c[2], c[3])};
  return __builtin_bit_cast(i16x4, q);
}

// The same as a split pair of operands, c = hi + lo (see split_bf16x2).
__device__ __forceinline__ void to_operand_split(f32x4 c, i16x4& hi, i16x4& lo) {
  const uint2 p01 = split_bf16x2(c[0], c[1]);
  const uint2 p23 = split_bf16x2(c[2], c[3]);
  const u32x2 h = {p01.x, p23.x}, l = {p01.y, p23.y};
  hi = __builtin_bit_cast(i16x4, h);
  lo = __builtin_bit_cast(i16x4, l);
}

// Operand read from an LDS tile: 4 consecutive bf16 of row `row` starting at
// column `col` (8-byte aligned). Serves as A operand (row = m, col = k0) or
// as B operand of a tile stored [n][k] (row = n, col = k0).
template <int Stride = kTileStride>
__device__ __forceinline__ i16x4 lds_operand(const uint16_t* tile, int row, int col) {
  return *reinterpret_cast<const i16x4*>(tile + row * Stride + col);
}

// 32-wide K operand from an LDS tile: columns col + 4g .. +3 and
// col + 16 + 4g .. +3 of row `row` (lane group g), matching mfma32's K order.
template <int Stride = kTileStride>
__device__ __forceinline__ i16x8 lds_operand32(const uint16_t* tile, int row, int col, int g) {
  return cat(lds_operand<Stride>(tile, row, col + 4 * g),
             lds_operand<Stride>(tile, row, col + 16 + 4 * g));
}

// B operand over tokens from a row-major [t][col] LDS tile via the gfx950
// transpose read (ds_read_b64_tr_b16): lane (g, n) receives
// X[t0 + 4g + e][c0 + n], e = 0..3, i.e. the MFMA operand layout for
// K = tokens t0 .. t0 + 15. Within a 16-lane group, lane i's element e
// comes from the 8 bytes addressed by lane 4e + i / 4, element i % 4, so
// lane j addresses row t0 + 4g + j / 4, columns c0 + 4 (j % 4) .. +3. The
// row stride (elements) must keep those addresses 8-byte aligned.
template <int Stride>
__device__ __forceinline__ i16x4 lds_operand_tr(const uint16_t* tile, int t0, int c0, int g,
                                                int n) {
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  static_assert((Stride * 2) % 8 == 0, "rows must be 8-byte aligned");
  const uint16_t* src = tile + (t0 + 4 * g + (n >> 2)) * Stride + c0 + 4 * (n & 3);
  const v4i16 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4i16*)(src));
  i16x4 r;
  r[0] = x[0];
  r[1] = x[1];
  r[2] = x[2];
  r[3] = x[3];
  return r;
}

// Stores a C-layout tile transposed: lane (g, n) writes its 4 values to
// dst[n][4g .. 4g+3] of a tile with the given row stride (one 8-byte write).
__device__ __forceinline__ void lds_store_transposed(uint16_t* dst, int stride,
                                                     int g, int n, f32x4 c) {
  uint2 q;
  q.x = pack_bf16x2(c[0], c[1]);
  q.y = pack_bf16x2(c[2], c[3]);
  *reinterpret_cast<uint2*>(dst + n * stride + 4 * g) = q;
}

// lds_store_transposed of the split pair c = hi + lo into two tiles.
__device__ __forceinline__ void lds_store_transposed_split(uint16_t* dst_hi, uint16_t* dst_lo,
                                                           int stride, int g, int n, f32x4 c) {
  const uint2 p01 = split_bf16x2(c[0], c[1]);
  const uint2 p23 = split_bf16x2(c[2], c[3]);
  *reinterpret_cast<uint2*>(dst_hi + n * stride + 4 * g) = make_uint2(p01.x, p23.x);
  *reinterpret_cast<uint2*>(dst_lo + n * stride + 4 * g) = make_uint2(p01.y, p23.y);
}

}  // namespace frwkv
