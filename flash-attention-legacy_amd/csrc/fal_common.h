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
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

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

// ---- element-type generic forms (fp16 or bf16 operands, fp32 accumulation) ----
typedef __bf16 bf16_t;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

template <class T> struct ElemVec;
template <> struct ElemVec<half_t> { typedef half8 v8; typedef half4 v4; };
template <> struct ElemVec<bf16_t> { typedef bf16x8 v8; typedef bf16x4 v4; };
template <class T> using vec8 = typename ElemVec<T>::v8;
template <class T> using vec4 = typename ElemVec<T>::v4;

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16(half8 a, half8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// 8 consecutive elements (16 bytes) at p
template <class T>
__device__ __forceinline__ vec8<T> ld8(const T* p) {
  return __builtin_bit_cast(vec8<T>, *reinterpret_cast<const u32x4*>(p));
}
template <class T>
__device__ __forceinline__ vec8<T> zero8() {
  return __builtin_bit_cast(vec8<T>, u32x4{0, 0, 0, 0});
}
// two 4-element halves joined into the 8 k-slots of an MFMA operand
__device__ __forceinline__ half8 join8(half4 lo, half4 hi) {
  return half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}
__device__ __forceinline__ bf16x8 join8(bf16x4 lo, bf16x4 hi) {
  return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}
// transposed LDS read of 16-bit elements (see lds_read_tr), typed by the tile's element
template <class T>
__device__ __forceinline__ vec4<T> lds_tr(const T* p) {
  typedef __attribute__((address_space(3))) short4v lds_s4;
  short4v v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(p));
  return __builtin_bit_cast(vec4<T>, v);
}
// elements 8t..8t+7 of an accumulator, rounded to T
template <class T>
__device__ __forceinline__ vec8<T> cvt8t(const f32x16& c, int t) {
  vec8<T> r;
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = (T)c[8 * t + j];
  return r;
}
// sum of 8 elements into an fp32 accumulator (dot2 with ones)
__device__ __forceinline__ float sum8(half8 v, float acc) {
  const half2v one = {(half_t)1.f, (half_t)1.f};
#pragma unroll
  for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_fdot2(half2v{v[2 * j], v[2 * j + 1]}, one, acc, false);
  return acc;
}
__device__ __forceinline__ float sum8(bf16x8 v, float acc) {
  const bf16x2 one = {(bf16_t)1.f, (bf16_t)1.f};
#pragma unroll
  for (int j = 0; j < 4; ++j)
    acc = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{v[2 * j], v[2 * j + 1]}, one, acc, false);
  return acc;
}
// A/B operand (8 k-slots) of rows row0.. of a row-major tile (see lds_kslab_tr)
template <class T>
__device__ __forceinline__ vec8<T> kslab_tr(const T* base, int row0, int hh, int ld) {
  return join8(lds_tr(base + (row0 + hh * 4) * ld), lds_tr(base + (row0 + 8 + hh * 4) * ld));
}
__device__ __forceinline__ u32x4 ld_u4(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st_u4(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
// acc + sum_j a[j] * b[j] over 8 elements
__device__ __forceinline__ float dot8(half8 a, half8 b, float acc) {
#pragma unroll
  for (int j = 0; j < 4; ++j)
    acc = __builtin_amdgcn_fdot2(half2v{a[2 * j], a[2 * j + 1]}, half2v{b[2 * j], b[2 * j + 1]}, acc, false);
  return acc;
}
__device__ __forceinline__ float dot8(bf16x8 a, bf16x8 b, float acc) {
#pragma unroll
  for (int j = 0; j < 4; ++j)
    acc = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{a[2 * j], a[2 * j + 1]}, bf16x2{b[2 * j], b[2 * j + 1]}, acc,
                                          false);
  return acc;
}

// Sum of 8 fp16 values into an fp32 accumulator (v_dot2 with ones).
__device__ __forceinline__ float sum8_f16(half8 v, float acc) {
  const half2v one = {(half_t)1.f, (half_t)1.f};
#pragma unroll
  for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_fdot2(half2v{v[2 * j], v[2 * j + 1]}, one, acc, false);
  return acc;
}

// 16-byte global -> LDS copy that bypasses VGPRs (gfx950 global_load_lds_dwordx4).
// Lane i of the wave writes bytes [16 i, 16 i + 16) of `lds_wave_base`, which must be
// the same for all lanes.  Completion is tracked by vmcnt (see wait_vmcnt0).
__device__ __forceinline__ void global_to_lds16(const void* src, void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds((__attribute__((address_space(1))) void*)(src),
                                   (__attribute__((address_space(3))) void*)(lds_wave_base), 16, 0, 0);
}
// Raw buffer resource over `nbytes` bytes at `base` (loads past the end return 0).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t nbytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)nbytes, 0x00020000);
}
// 16-byte store through a raw buffer resource: a store whose offset is past the
// resource's byte count is dropped, so rows past the end of a sequence need no branch.
// The row goes in `voffset` (the range check covers it; an SGPR offset would not be).
__device__ __forceinline__ void buffer_store16(__amdgpu_buffer_rsrc_t rs, int voffset, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, rs, voffset, 0, 0);
}
// 16-byte buffer -> LDS copy (buffer_load_dwordx4 ... lds); lane i writes bytes
// [16 i, 16 i + 16) of `lds_wave_base` (uniform across the wave).
// AUX: cache-policy bits of the load.
template <int AUX = 0>
__device__ __forceinline__ void buffer_to_lds16(__amdgpu_buffer_rsrc_t rs, int voffset, void* lds_wave_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(lds_wave_base), 16,
                                           voffset, 0, 0, AUX);
}
// Segment s of a cu_seqlens array, clamped to [0, total): a malformed array (not
// monotone, or past the packed tensor) yields empty or shortened segments, never
// rows outside the tensor.
__device__ __forceinline__ void seg_bounds(const int* cu, int s, int total, int& off, int& len) {
  const int a = min(max(cu[s], 0), total);
  const int e = min(max(cu[s + 1], a), total);
  off = a;
  len = e - a;
}

__device__ __forceinline__ void wait_vmcnt0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Row-major LDS tile of D fp16 columns stored as 16-byte chunks with an XOR swizzle
// of the chunk index by the row.  The swizzle makes both access patterns used on
// these tiles free of bank conflicts:
//   * 16 consecutive rows, one chunk each (MFMA A/B fragments, ds_read_b128);
//   * 4 consecutive rows (first row a multiple of 4) x 4 aligned chunks
//     (ds_read_b64_tr_b16 of a 32-column block by a 32-lane half-wave).
// swz(r) only depends on r mod 16, so row offsets that are multiples of 16 keep it.
template <int D>
struct SwizzledTile {
  static constexpr int CPR = D / 8;   // chunks per row
  __device__ static int swz(int r) {
    if constexpr (D == 32) return (r >> 2) & 3;
    else if constexpr (D == 64) return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
    else if constexpr (D == 96) return 0;
    else return ((r & 3) << 2) | ((r >> 2) & 3);
  }
  // element offset of logical chunk c of row r
  __device__ static int offset(int r, int c) { return (r * CPR + (c ^ swz(r))) * 8; }
  // logical chunk held by physical chunk cp of row r (the swizzle is an involution)
  __device__ static int logical_chunk(int r, int cp) { return cp ^ swz(r); }
};

}  // namespace fal
