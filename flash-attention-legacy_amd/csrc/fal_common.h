// Shared device helpers for the gfx950 (CDNA4) attention kernels.
//
// Conventions used by every kernel in this library
// -------------------------------------------------
// * One wavefront is 64 lanes.  `l32 = lane & 31` and `hh = lane >> 5` split a
//   wave into two 32-lane halves.
// * Matrix products use v_mfma_f32_32x32x16_f16.  Operand layouts (verified on
//   MI355X):  A[m][k]: lane holds m = l32 and k = hh*8 + j (j = 0..7);
//             B[k][n]: lane holds n = l32 and k = hh*8 + j;
//             C[m][n]: accumulator element i holds m = (i/4)*8 + hh*4 + i%4, n = l32.
// * An accumulator tile is reused as the B operand of the next product without
//   leaving registers: elements 8t..8t+7 of a C tile are the 8 k-values of
//   k-step t, where k-slot j stands for row (j/4)*8 + hh*4 + j%4 of that
//   16-row step.  The other operand of that product is read from LDS with
//   ds_read_b64_tr_b16 so that its k-slot j names the same row.
// * ds_read_b64_tr_b16: within each 16-lane group, the 16 lanes x 4 halves
//   read form a 16x4 matrix M; lane r receives M[4j + r/4][r%4] in slot j.
//   Reading X[k0 + i/4][n0 + 4*(i%4)] from lane i of the group therefore
//   gives lane r the column X[k0 + 0..3][n0 + r].
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fal {

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef short short4v __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ f32x16 mfma32(half8 a, half8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Hardware base-2 exponential / logarithm (v_exp_f32 / v_log_f32).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// Combine a value with the one held by lane ^ 32 (the other wave half).
__device__ __forceinline__ float pair_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ half8 load_h8(const half_t* p) {
  return __builtin_bit_cast(half8, *reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ u32x4 load_u4(const half_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void store_u4(half_t* p, u32x4 v) {
  *reinterpret_cast<u32x4*>(p) = v;
}
__device__ __forceinline__ half8 zero_h8() { return half8{0, 0, 0, 0, 0, 0, 0, 0}; }
__device__ __forceinline__ f32x16 zero_f16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Transposed LDS read (see file header).  `p` already points at this lane's
// 8-byte source X[k0 + i/4][n0 + 4*(i%4)].
__device__ __forceinline__ half4 lds_read_tr(const half_t* p) {
  typedef __attribute__((address_space(3))) short4v lds_s4;
  short4v v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(p));
  return __builtin_bit_cast(half4, v);
}

// Offset (in elements) of this lane's source inside a row-major LDS tile X
// with row stride `ld`, for a transposed read of rows k0..k0+3 and columns
// n0..n0+15 where n0 = (lane & 16) picks the 16-column half of a 32-wide block.
__device__ __forceinline__ int tr_offset(int lane, int ld) {
  const int i = lane & 15;
  return (i >> 2) * ld + ((lane & 16) | ((i & 3) << 2));
}

// A/B operand (8 k-slots) for 16 rows starting at `row0` of a row-major tile:
// slot j <-> row row0 + (j/4)*8 + hh*4 + j%4, column = col0 + l32.
// `base` = tile + tr_offset(lane, ld) + col0.
__device__ __forceinline__ half8 lds_kslab_tr(const half_t* base, int row0, int hh, int ld) {
  const half4 lo = lds_read_tr(base + (row0 + hh * 4) * ld);
  const half4 hi = lds_read_tr(base + (row0 + 8 + hh * 4) * ld);
  return half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

__device__ __forceinline__ half8 cvt8(const f32x16& c, int t) {
  half8 r;
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = (half_t)c[8 * t + j];
  return r;
}

__host__ __device__ constexpr int cdiv(int a, int b) { return (a + b - 1) / b; }

}  // namespace fal
