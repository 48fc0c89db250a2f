// Shared device helpers and the C-ABI error channel of libvdnmi.
//
// Every exported entry point returns 0 on success or a nonzero status, and leaves
// a human-readable message behind vdn_last_error(). Nothing here allocates device
// memory; callers own every buffer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define VDN_API extern "C" __attribute__((visibility("default")))

namespace vdn {

enum Status : int {
  kOk = 0,
  kInvalidArgument = 1,
  kLaunchFailed = 2,
  kUnsupported = 3,
};

// Records a formatted message for vdn_last_error() and returns `status`.
int set_error(int status, const char* fmt, ...);

// Checks the launch that was just queued on the current thread.
int check_launch(const char* what);

typedef __bf16 bf16;
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// Lane exchanges inside 16-lane DPP rows (VALU, no LDS traffic). kCtrl is the DPP control:
// quad_perm 0xB1 = lane ^ 1, 0x4E = lane ^ 2; 0x141 = half-row mirror (i <- 7 - i within 8);
// 0x140 = row mirror (i <- 15 - i); 0x100 + n = row_shl n (i <- i + n, lanes past the row's
// end read 0); 0x120 + n = row rotate right by n.
template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(v), kCtrl, 0xf, 0xf, false));
}
template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(float, dpp_u32<kCtrl>(__builtin_bit_cast(uint32_t, v)));
}

// Sum over a 16-lane DPP row. Bit-identical to the xor butterfly over lanes ^1, ^2, ^4, ^8:
// after the two quad steps every lane of quad k holds its total q_k, the half-row mirror
// adds the neighbouring quad (q0 + q1, q2 + q3) and the row mirror the other half.
__device__ __forceinline__ float sum16(float v) {
  v += dpp_f32<0xB1>(v);
  v += dpp_f32<0x4E>(v);
  v += dpp_f32<0x141>(v);
  v += dpp_f32<0x140>(v);
  return v;
}

// Sum / max over the lanes l, l ^ 16, l ^ 32, l ^ 48. Every lane gets the same bits:
// (x0 + x1) + (x2 + x3) with operand order immaterial (IEEE addition commutes).
__device__ __forceinline__ float sum_quad_rows(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const float s = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const uint32_t w = __float_as_uint(s);
  const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ float max_quad_rows(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const float s = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const uint32_t w = __float_as_uint(s);
  const auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round-to-nearest-even fp32 -> bf16 (gfx950 v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  bf16 b = static_cast<bf16>(f);
  return __builtin_bit_cast(uint16_t, b);
}

__device__ __forceinline__ float round_bf16(float f) {
  return bf16_bits_to_f32(f32_to_bf16_bits(f));
}

// Two fp32 values -> packed bf16x2 as a 32-bit word (low half = a).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  bf16x2 v;
  v[0] = static_cast<bf16>(a);
  v[1] = static_cast<bf16>(b);
  return __builtin_bit_cast(uint32_t, v);
}

// a, b = round_bf16(a), round_bf16(b) through one packed conversion (each half is rounded on
// its own, so the values are those of round_bf16). The packed word is opaque to the
// compiler: the values come back out of it with one shift or mask each, instead of being
// rounded again one conversion per value.
__device__ __forceinline__ void round_bf16_pair(float& a, float& b) {
  uint32_t p = pack_bf16x2(a, b);
  asm volatile("" : "+v"(p));
  a = __uint_as_float(p << 16);
  b = __uint_as_float(p & 0xffff0000u);
}

// fp16 storage: exact widening, round-to-nearest-even narrowing (v_cvt_f16_f32), as torch's
// float <-> half conversions.
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

__device__ __forceinline__ float round_f16(float f) {
  return static_cast<float>(static_cast<_Float16>(f));
}

// The four values of v rounded to bf16, two per conversion (as round_bf16_pair).
__device__ __forceinline__ void round_bf16_x4(f32x4& v) {
  float a = v[0], b = v[1], c = v[2], d = v[3];
  round_bf16_pair(a, b);
  round_bf16_pair(c, d);
  v = f32x4{a, b, c, d};
}

}  // namespace vdn
