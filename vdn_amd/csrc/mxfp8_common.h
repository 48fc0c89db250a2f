// MXFP8 block-32 format helpers shared by the producer kernels and the GEMM.
//
// Format (reference src/models/ops/mxfp8_quant.py:15-74, mxfp8_kernels.py:15-27):
//   * rows padded to RP = ceil(R/128)*128, K padded to KP = ceil(K/128)*128, padding is zero;
//   * per row and per 32-element K block: one E8M0 scale byte and 32 E4M3FN codes;
//   * scale bytes stored flat in the SWIZZLE_32_4_4 order, RP*KP/32 bytes.
#pragma once

#include "common.h"

namespace vdn {

// amax -> (E8M0 byte, 2^-e as fp32). Bit-level rule of the reference
// (mxfp8_kernels.py:15-22, mxfp8_quant.py:65-70): e0 = biased_exp(amax) - 135,
// bump by one when amax exceeds 1.75 * 2^(e0 + 8), clamp below at -127.
__device__ __forceinline__ uint32_t e8m0_from_amax(float amax, float* inv_out) {
  const int bits = __float_as_int(amax);
  const int e0 = ((bits >> 23) & 255) - 135;
  const float thr = __int_as_float(((e0 + 135) << 23) | 0x600000);
  int e = e0 + (amax > thr ? 1 : 0);
  e = e < -127 ? -127 : e;
  *inv_out = __int_as_float((127 - e) << 23);
  return static_cast<uint32_t>(e + 127);
}

// Byte offset of natural scale (row r, K-block c) in SWIZZLE_32_4_4 order
// (mxfp8_kernels.py:25-27). `col_tiles` = KP / 128.
__device__ __forceinline__ int64_t swizzled_scale_offset(int64_t r, int64_t c, int64_t col_tiles) {
  const int64_t tile = (r >> 7) * col_tiles + (c >> 2);
  return tile * 512 + (r & 31) * 16 + ((r & 127) >> 5) * 4 + (c & 3);
}

typedef short s16x2_t __attribute__((ext_vector_type(2)));

// 2^e as fp32 from an E8M0 byte (byte = e + 127). Byte 0 gives exponent field 0, which the
// scaled conversion below reads as 2^-127.
__device__ __forceinline__ float e8m0_scale(uint32_t byte) { return __uint_as_float(byte << 23); }

// E4M3FN codes of value / 2^e (s = e8m0_scale(byte)), four fp32 values to one word, low
// value in the low byte. On gfx950 v_cvt_scalef32_pk_fp8_f32 gives, for every bf16-valued
// input and every exponent, nonfinite inputs included, the code v_cvt_pk_fp8_f32 gives for
// value * 2^-e (RNE; measured over all 2^16 patterns, both halves of the word), without the
// multiplies.
__device__ __forceinline__ uint32_t e4m3x4_scaled(float a, float b, float c, float d, float s) {
  s16x2_t r = {0, 0};
  r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r, a, b, s, false);
  r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r, c, d, s, true);
  return __builtin_bit_cast(uint32_t, r);
}

// The two codes of value / 2^e (s = e8m0_scale(byte)) of the packed bf16 pair w (low half
// first) into byte pair kHi of `old` (the other pair kept): v_cvt_scalef32_pk_fp8_bf16, which
// gives the codes of v_cvt_scalef32_pk_fp8_f32 on the same values (measured over all 2^16
// patterns at every exponent, both byte pairs). w arrives by value: __builtin_bit_cast of a
// vector element lvalue (w4[i] of a u32x4) reads element 0 whatever i is, with this compiler.
template <bool kHi>
__device__ __forceinline__ uint32_t e4m3x2_bf16(uint32_t old, uint32_t w, float s) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(
      __builtin_bit_cast(s16x2_t, old), __builtin_bit_cast(bf16x2, w), s, kHi));
}

// Eight packed bf16 values (the low half of a word first) -> their eight codes of value / 2^e.
__device__ __forceinline__ u32x2 e4m3x8_bf16(const u32x4& w, float s) {
  u32x2 out;
  out[0] = e4m3x2_bf16<true>(e4m3x2_bf16<false>(0u, w[0], s), w[1], s);
  out[1] = e4m3x2_bf16<true>(e4m3x2_bf16<false>(0u, w[2], s), w[3], s);
  return out;
}

// Per-half maxima of the magnitude bits of eight packed bf16 values. Non-negative values
// order as their magnitude bits; a bf16 is nonfinite iff its magnitude bits reach 0x7f80.
__device__ __forceinline__ u16x2 mag8_bf16(const u32x4& w) {
  u16x2 m = {0, 0};
#pragma unroll
  for (int i = 0; i < 4; ++i) m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, w[i] & 0x7fff7fffu));
  return m;
}

// max |x| over eight packed bf16 values as fp32 (m = mag8_bf16(w)), with NaN ignored as a
// running fmaxf from 0 ignores it: the maximum is an integer one on the magnitude bits, and
// a NaN (magnitude above 0x7f80) sends the lane to the fmaxf form.
__device__ __forceinline__ float amax8_bf16(const u32x4& w, u16x2 m) {
  const uint32_t mb = m[0] > m[1] ? m[0] : m[1];
  if (mb <= 0x7f80u) return __uint_as_float(mb << 16);
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    amax = fmaxf(amax, fabsf(__uint_as_float(w[i] << 16)));
    amax = fmaxf(amax, fabsf(__uint_as_float(w[i] & 0xffff0000u)));
  }
  return amax;
}

__device__ __forceinline__ float amax8_bf16(const u32x4& w) { return amax8_bf16(w, mag8_bf16(w)); }

// Sum of squares of eight packed bf16 values added to acc, two per v_dot2_f32_bf16 (a bf16
// square is exact in fp32).
__device__ __forceinline__ float sumsq8_bf16(const u32x4& w, float acc) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t word = w[i];  // by value (see e4m3x2_bf16)
    const bf16x2 p = __builtin_bit_cast(bf16x2, word);
    acc = __builtin_amdgcn_fdot2_f32_bf16(p, p, acc, false);
  }
  return acc;
}

// torch's GELU(approximate='tanh') in fp32, rounded to bf16 by the caller:
//   0.5 x (1 + tanh(u)) = x / (1 + exp(-2u)),  u = sqrt(2/pi) (x + 0.044715 x^3).
// The second form (1 + tanh(u) = 2 sigmoid(2u)) has no cancellation in the negative tail
// and costs one hardware exp2 and one reciprocal instead of a libm tanh. The exponent
// -2u log2(e) = x (B + A x^2) is one multiply, one fma and one multiply, with
// A = 0.044715 B and B = -2 sqrt(2/pi) / ln 2. The fp32 result is within a few ulp of the
// first form, so the bf16 value agrees except where the exact value lies within those
// few ulp of a bf16 rounding boundary.
__device__ __forceinline__ float gelu_tanh(float x) {
  constexpr float kB = -2.302208198144325f;    // -2 sqrt(2/pi) / ln 2
  constexpr float kA = -0.1029432395800235f;   // 0.044715 kB
  const float z = x * __builtin_fmaf(x * x, kA, kB);
  return x * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(z));
}

// SwiGLU's gate half g * sigmoid(g), and a * silu(g), in fp32 (mxfp8_kernels.py:62-64); the
// stand-alone producer and the GEMM's producer epilogue share them, so both write the same
// bytes. The sigmoid takes the hardware exp2 and reciprocal (a few fp32 ulp from
// 1 / (1 + exp(-g)), far below the bf16 rounding of the product).
#pragma clang fp contract(off)
__device__ __forceinline__ float swiglu_gate(float g) {
  constexpr float kMinusLog2e = -1.4426950408889634f;
  const float sig = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(g * kMinusLog2e));
  return g * sig;
}
__device__ __forceinline__ float silu_mul(float a, float g) { return a * swiglu_gate(g); }
#pragma clang fp contract(on)

// The maximum of `amax` over lanes l, l ^ 1, l ^ 2, l ^ 3 (the 4 lanes of a 32-block) for an
// amax that is non-negative and never NaN (a running fmaxf from 0 ignores NaN). Such floats
// order as their bit patterns do, so the steps are unsigned maxima, which take the DPP
// operand directly.
__device__ __forceinline__ float block_amax4(float amax) {
  uint32_t b = __float_as_uint(amax);
  b = max(b, static_cast<uint32_t>(
                 __builtin_amdgcn_update_dpp(0, static_cast<int>(b), 0xB1, 0xf, 0xf, true)));
  b = max(b, static_cast<uint32_t>(
                 __builtin_amdgcn_update_dpp(0, static_cast<int>(b), 0x4E, 0xf, 0xf, true)));
  return __uint_as_float(b);
}

// The 4 scale bytes of a 16-lane group (byte i from lane 4 i of the DPP row), complete in
// the group's lane 0: lanes 0 and 8 first pair their byte with lane + 4's, then lane 0 takes
// lane 8's pair as its upper half.
__device__ __forceinline__ uint32_t scale_word16(uint32_t scale) {
  const uint32_t pair =
      scale | (static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
                   0, static_cast<int>(scale), 0x104, 0xf, 0xf, true)) << 8);  // row_shl 4
  return pair | (static_cast<uint32_t>(__builtin_amdgcn_update_dpp(
                     0, static_cast<int>(pair), 0x108, 0xf, 0xf, true)) << 16);  // row_shl 8
}

// Quantizes the 8 values a lane holds (one quarter of a 32-block), stores the 8 codes at
// `qdst` and, from the lanes with `scale_lane` set (lane 0 of each 16-lane group), the
// chunk's 4 scale bytes at `sdst`. A group is one DPP row (lanes 16k .. 16k + 15) whose lanes
// are all active: the amax and the scale bytes move between its lanes by DPP.
__device__ __forceinline__ void quantize_store8_at(const float* v, uint8_t* __restrict__ qdst,
                                                   uint8_t* __restrict__ sdst, bool scale_lane) {
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = block_amax4(amax);
  float inv;
  const uint32_t scale = e8m0_from_amax(amax, &inv);
  const float sf = e8m0_scale(scale);
  u32x2 codes;
  codes[0] = e4m3x4_scaled(v[0], v[1], v[2], v[3], sf);
  codes[1] = e4m3x4_scaled(v[4], v[5], v[6], v[7], sf);
  // 16 lanes write the chunk's 128 contiguous bytes: a streaming store of whole lines
  __builtin_nontemporal_store(codes, reinterpret_cast<u32x2*>(qdst));
  const uint32_t word = scale_word16(scale);
  if (scale_lane) *reinterpret_cast<uint32_t*>(sdst) = word;
}

// quantize_store8_at for 8 values held as packed bf16 (the low half of each word first), mag =
// mag8_bf16(w): the amax and the codes come from the packed words directly.
__device__ __forceinline__ void quantize_store8_bf16_at(const u32x4& w, u16x2 mag,
                                                        uint8_t* __restrict__ qdst,
                                                        uint8_t* __restrict__ sdst,
                                                        bool scale_lane) {
  const float amax = block_amax4(amax8_bf16(w, mag));
  float inv;
  const uint32_t scale = e8m0_from_amax(amax, &inv);
  const u32x2 codes = e4m3x8_bf16(w, e8m0_scale(scale));
  __builtin_nontemporal_store(codes, reinterpret_cast<u32x2*>(qdst));
  const uint32_t word = scale_word16(scale);
  if (scale_lane) *reinterpret_cast<uint32_t*>(sdst) = word;
}

// quantize_store8_at for lane `lane16` of the group holding row r, 128-column chunk `chunk`.
__device__ __forceinline__ void quantize_store8(const float* v, int lane16, int64_t r, int64_t chunk,
                                                int64_t kp, uint8_t* __restrict__ q,
                                                uint8_t* __restrict__ s) {
  quantize_store8_at(v, q + r * kp + chunk * 128 + lane16 * 8,
                     s + swizzled_scale_offset(r, chunk * 4, kp >> 7), lane16 == 0);
}

}  // namespace vdn
