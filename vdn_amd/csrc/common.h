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
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

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

}  // namespace vdn
