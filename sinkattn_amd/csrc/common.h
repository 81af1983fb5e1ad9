// Shared device helpers for the gfx950 kernels of libsinkattn.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef short v4i16 __attribute__((ext_vector_type(4)));

enum DType { kBF16 = 0, kF16 = 1, kF32 = 2 };

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float neg_inf() { return -__builtin_inff(); }
__device__ __forceinline__ float pos_inf() { return __builtin_inff(); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Two fp32 -> packed 16-bit floats (lo in bits 0-15), round to nearest even: one
// v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
template <int CT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi);
template <>
__device__ __forceinline__ uint32_t pack2<kBF16>(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}
template <>
__device__ __forceinline__ uint32_t pack2<kF16>(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, f16x2));
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// 32x32x16 MFMA, A/B as 8 packed 16-bit values in a u32x4.
template <int CT>
__device__ __forceinline__ f32x16 mfma32x32x16(u32x4 a, u32x4 b, f32x16 c);
template <>
__device__ __forceinline__ f32x16 mfma32x32x16<kBF16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x16 mfma32x32x16<kF16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// 16x16x32 MFMA, A/B as 8 packed 16-bit values in a u32x4.  Lane l holds row (A) or column
// (B) l % 16 and the 8 contraction elements of slice l / 16; D holds column l % 16, rows
// 4 (l / 16) .. +3.  With random 16-bit operands the matrix cores draw less power per flop in
// this shape than in 32x32x16 and the chip holds a higher clock.
template <int CT>
__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c);
template <>
__device__ __forceinline__ f32x4 mfma16x16x32<kBF16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma16x16x32<kF16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Reductions over lane pairs (l, l ^ 32), the two halves of a 32x32 MFMA column, with one
// v_permlane32_swap (a VALU op, no LDS round trip).  The swap of x with itself leaves
// (x[l], x[l + 32]) in lane l < 32 and (x[l - 32], x[l]) in lane l >= 32, so both lanes of a
// pair combine the same two values in the same order.
__device__ __forceinline__ f32x2 pair32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return f32x2{__uint_as_float(r[0]), __uint_as_float(r[1])};
}
__device__ __forceinline__ float max_xor32(float x) {
  const f32x2 p = pair32(x);
  return fmaxf(p[0], p[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
  const f32x2 p = pair32(x);
  return p[0] + p[1];
}

// The same over lane pairs (l, l ^ 16) with v_permlane16_swap: lane l of an even 16-lane row
// gets (x[l], x[l + 16]), lane l of an odd row (x[l - 16], x[l]).  Together with the pair32
// forms they reduce over the four lanes l % 16 + 16 j of a 16x16 MFMA column.
__device__ __forceinline__ f32x2 pair16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return f32x2{__uint_as_float(r[0]), __uint_as_float(r[1])};
}
__device__ __forceinline__ float max_col16(float x) {
  const f32x2 p = pair16(x);
  return max_xor32(fmaxf(p[0], p[1]));
}
__device__ __forceinline__ float sum_col16(float x) {
  const f32x2 p = pair16(x);
  return sum_xor32(p[0] + p[1]);
}

// Load 8 consecutive elements of type IT at p (16-byte aligned for 16-bit types,
// 32-byte aligned for f32) and return them as 8 packed 16-bit values of type CT.
template <int IT, int CT>
__device__ __forceinline__ u32x4 load8(const void* p);
template <>
__device__ __forceinline__ u32x4 load8<kBF16, kBF16>(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
template <>
__device__ __forceinline__ u32x4 load8<kF16, kF16>(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
template <>
__device__ __forceinline__ u32x4 load8<kF32, kBF16>(const void* p) {
  const f32x4* f = reinterpret_cast<const f32x4*>(p);
  f32x4 a = f[0], b = f[1];
  u32x4 r;
  r[0] = pack2<kBF16>(a[0], a[1]);
  r[1] = pack2<kBF16>(a[2], a[3]);
  r[2] = pack2<kBF16>(b[0], b[1]);
  r[3] = pack2<kBF16>(b[2], b[3]);
  return r;
}

// Load 2 consecutive elements as one packed pair of CT values.
template <int IT, int CT>
__device__ __forceinline__ uint32_t load2(const void* p);
template <>
__device__ __forceinline__ uint32_t load2<kBF16, kBF16>(const void* p) {
  return *reinterpret_cast<const uint32_t*>(p);
}
template <>
__device__ __forceinline__ uint32_t load2<kF16, kF16>(const void* p) {
  return *reinterpret_cast<const uint32_t*>(p);
}
template <>
__device__ __forceinline__ uint32_t load2<kF32, kBF16>(const void* p) {
  f32x2 a = *reinterpret_cast<const f32x2*>(p);
  return pack2<kBF16>(a[0], a[1]);
}

template <int IT>
struct ElemSize;
template <>
struct ElemSize<kBF16> { static constexpr int value = 2; };
template <>
struct ElemSize<kF16> { static constexpr int value = 2; };
template <>
struct ElemSize<kF32> { static constexpr int value = 4; };

// Store 4 fp32 values as 4 consecutive elements of type IT.
template <int IT>
__device__ __forceinline__ void store4(void* p, float a, float b, float c, float d);
template <>
__device__ __forceinline__ void store4<kBF16>(void* p, float a, float b, float c, float d) {
  u32x2 v;
  v[0] = pack2<kBF16>(a, b);
  v[1] = pack2<kBF16>(c, d);
  *reinterpret_cast<u32x2*>(p) = v;
}
template <>
__device__ __forceinline__ void store4<kF16>(void* p, float a, float b, float c, float d) {
  u32x2 v;
  v[0] = pack2<kF16>(a, b);
  v[1] = pack2<kF16>(c, d);
  *reinterpret_cast<u32x2*>(p) = v;
}
template <>
__device__ __forceinline__ void store4<kF32>(void* p, float a, float b, float c, float d) {
  f32x4 v;
  v[0] = a; v[1] = b; v[2] = c; v[3] = d;
  *reinterpret_cast<f32x4*>(p) = v;
}

// s_waitcnt with only a vector-memory count (gfx9 encoding: vmcnt[3:0], expcnt[6:4],
// lgkmcnt[11:8], vmcnt[15:14]); expcnt/lgkmcnt left at "no wait".
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Work-group barrier after this wave's buffer->LDS copies have landed and its own LDS
// reads have returned, so a buffer may be refilled by any wave right after it.
// (__syncthreads would do the same plus a full fence; this keeps it to the counters.)
__device__ __forceinline__ void drain_then_barrier() {
  __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (0 << 8));  // vmcnt(0) expcnt(7) lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
}

#define SA_LDS __attribute__((address_space(3)))
#define SA_CONST __attribute__((address_space(4)))

// Raw buffer resource over [base, base + bytes): loads at offsets >= bytes return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// 16 bytes per lane from rsrc+voffset into LDS at lds_wave_base + lane*16.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rs, SA_LDS void* lds_wave_base,
                                      uint32_t voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, lds_wave_base, 16, voffset, 0, 0, 0);
}

}  // namespace sa
