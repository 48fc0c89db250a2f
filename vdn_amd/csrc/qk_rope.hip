// QK RMSNorm + rotate-half RoPE for gfx950 (bf16 activations; fp16 and fp32 through the
// general kernel).
//
// Per (token, head) row x of D channels (reference src/models/softmax_attention/
// paper_qk_rope.py:105-140, eager semantics :82-95), with act() the rounding to the
// activation dtype (none for fp32):
//   n   = act((x * rsqrt(sum(x^2) / D + eps)) * w)             (fp32, one rounding)
//   for channel i < R: out = act(act(n_i * c_i) + act(r_i * s_i)),
//       r_i = -n_{i+R/2} (i < R/2), n_{i-R/2} (R/2 <= i < R); c, s = table values in the
//       activation dtype
//   channels i >= R pass n through.
// A row is held by D/8 lanes (8 channels each); the rotate partner is exchanged through a
// per-row LDS line, which keeps arbitrary even R <= D exact (qk_rope_kernel), or, for the
// common D = 128, through a DPP lane rotation (qk_rope_row128_kernel, qk_rope_token128_kernel).
#include "common.h"

#include <math.h>

namespace vdn {
namespace {

struct RopeArgs {
  const uint16_t* x;   // activation storage (fp32 rows are read through this pointer's bytes)
  int64_t st, sh, sd;  // token, head, channel strides (elements)
  const void* w;
  int64_t ws;
  int w_f32;
  uint16_t* out;  // contiguous [T, H, D] of the activation dtype
};

// Activation dtype of the general kernel: 0 bf16, 1 fp16, 2 fp32. Storage of a weight or a
// table that is not fp32 is the activation dtype.
template <int kT>
__device__ __forceinline__ float act_load(const void* p, int64_t i) {
  if constexpr (kT == 2) return static_cast<const float*>(p)[i];
  else if constexpr (kT == 1) return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
  else return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
}

template <int kT>
__device__ __forceinline__ float act_round(float f) {
  if constexpr (kT == 2) return f;
  else if constexpr (kT == 1) return round_f16(f);
  else return round_bf16(f);
}

// Eight consecutive values (bf16 storage or fp32) starting at element `off`, as floats;
// fp32 values are rounded to bf16 when `round` is set.
__device__ __forceinline__ void load8(const void* __restrict__ p, int f32, int64_t off, bool round,
                                      float* out) {
  if (f32) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(static_cast<const float*>(p) + off);
    const f32x4 b = *reinterpret_cast<const f32x4*>(static_cast<const float*>(p) + off + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[i] = round ? round_bf16(a[i]) : a[i];
      out[4 + i] = round ? round_bf16(b[i]) : b[i];
    }
  } else {
    const u32x4 w = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(p) + off);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = bf16_bits_to_f32(static_cast<uint16_t>(w[i] & 0xffff));
      out[2 * i + 1] = bf16_bits_to_f32(static_cast<uint16_t>(w[i] >> 16));
    }
  }
}

// Eight bf16 values of a q / k row, read once: a streaming load (the weights and the
// cos / sin rows, reused across heads, go through load8 and stay cached).
__device__ __forceinline__ void load8_row(const uint16_t* __restrict__ p, float* out) {
  const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = bf16_bits_to_f32(static_cast<uint16_t>(w[i] & 0xffff));
    out[2 * i + 1] = bf16_bits_to_f32(static_cast<uint16_t>(w[i] >> 16));
  }
}

// kVec (bf16 only): unit channel strides, 16-byte aligned rows, weights and table rows,
// rot % 8 == 0; every load is one (or two, fp32) 16-byte access per lane. kT: activation
// dtype (0 bf16, 1 fp16, 2 fp32).
template <int kD, bool kVec, int kT = 0>
__global__ void __launch_bounds__(256)
qk_rope_kernel(RopeArgs q, RopeArgs k, int64_t tokens, int heads, float eps,
               const void* __restrict__ cos_t, const void* __restrict__ sin_t, int64_t c_st,
               int64_t c_sd, int64_t s_st, int64_t s_sd, int table_f32, int rot) {
#pragma clang fp contract(off)
  static_assert(!kVec || kT == 0, "the vector form reads bf16 rows");
  constexpr int kLanes = kD / 8;
  constexpr int kRowsPerBlock = 256 / kLanes;
  __shared__ float line[kRowsPerBlock][kD + 1];
  const int sub = threadIdx.x % kLanes;
  const int slot = threadIdx.x / kLanes;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + slot;
  const int which = blockIdx.y;  // 0: q, 1: k
  const RopeArgs& a = which == 0 ? q : k;
  const bool live = row < tokens * heads;
  const int64_t t = live ? row / heads : 0;
  const int h = live ? static_cast<int>(row % heads) : 0;
  float v[8];
  const uint16_t* src = a.x + t * a.st + h * a.sh + static_cast<int64_t>(sub) * 8 * a.sd;
  if (kVec) {
    if (live) {
      load8_row(src, v);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = 0.f;
    }
  } else {
    const int64_t base = t * a.st + h * a.sh + static_cast<int64_t>(sub) * 8 * a.sd;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = live ? act_load<kT>(a.x, base + i * a.sd) : 0.f;
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss += v[i] * v[i];
#pragma unroll
  for (int off = 1; off < kLanes; off <<= 1) ss += __shfl_xor(ss, off, kLanes);
  const float inv = 1.0f / sqrtf(ss / static_cast<float>(kD) + eps);
  float n[8];
  float wv[8];
  if (kVec) {
    load8(a.w, a.w_f32, sub * 8, false, wv);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = sub * 8 + i;
      wv[i] = a.w_f32 ? static_cast<const float*>(a.w)[c * a.ws] : act_load<kT>(a.w, c * a.ws);
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int c = sub * 8 + i;
    n[i] = act_round<kT>((v[i] * inv) * wv[i]);
    line[slot][c] = n[i];
  }
  __syncthreads();
  float o[8];
  const int half = rot / 2;
  float cvv[8], svv[8];
  if (kVec && sub * 8 < rot) {
    load8(cos_t, table_f32, t * c_st + sub * 8, true, cvv);
    load8(sin_t, table_f32, t * s_st + sub * 8, true, svv);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int c = sub * 8 + i;
    if (kVec && c < rot) {
      const float other = c < half ? -line[slot][c + half] : line[slot][c - half];
      o[i] = round_bf16(round_bf16(n[i] * cvv[i]) + round_bf16(other * svv[i]));
    } else if (c < rot) {
      const float other = c < half ? -line[slot][c + half] : line[slot][c - half];
      float cv, sv;
      if (table_f32) {
        cv = act_round<kT>(static_cast<const float*>(cos_t)[t * c_st + c * c_sd]);
        sv = act_round<kT>(static_cast<const float*>(sin_t)[t * s_st + c * s_sd]);
      } else {
        cv = act_load<kT>(cos_t, t * c_st + c * c_sd);
        sv = act_load<kT>(sin_t, t * s_st + c * s_sd);
      }
      o[i] = act_round<kT>(act_round<kT>(n[i] * cv) + act_round<kT>(other * sv));
    } else {
      o[i] = n[i];
    }
  }
  if (live) {
    if constexpr (kT == 2) {
      float* dst = reinterpret_cast<float*>(a.out) + row * kD + sub * 8;
      *reinterpret_cast<f32x4*>(dst) = f32x4{o[0], o[1], o[2], o[3]};
      *reinterpret_cast<f32x4*>(dst + 4) = f32x4{o[4], o[5], o[6], o[7]};
    } else {
      uint16_t* dst = a.out + row * kD + sub * 8;
      u32x4 packed;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (kT == 1)
          packed[i] = f32_to_f16_bits(o[2 * i]) | (static_cast<uint32_t>(f32_to_f16_bits(o[2 * i + 1])) << 16);
        else
          packed[i] = pack_bf16x2(o[2 * i], o[2 * i + 1]);
      }
      *reinterpret_cast<u32x4*>(dst) = packed;
    }
  }
}

// Fast forms for 128-channel heads with unit channel strides and 16-byte rows. Arithmetic and
// rounding are those of qk_rope_kernel.
//
// qk_rope_row128_kernel: rotated over the full width (R = 128) or not rotated (R = 0); a
// 16-lane group per row, a workgroup walking kRopeGroups groups of 16 rows. The rotate-half
// partner of a lane's 8 channels is 8 lanes away in the same 16-lane row, so a DPP row
// rotation by 8 exchanges it (no LDS line, no barrier). The launcher takes it for R = 0 (the
// QK norm alone), where it streams at about 5.9 TB/s.
constexpr int kRopeGroups = 8;

// Lane l of a 16-lane row reads lane (l + 8) mod 16 (every source lane exists, so the bound
// control only lets the rotation fold into the instruction that consumes it).
__device__ __forceinline__ float row_ror8(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                               0x128, 0xf, 0xf, true));
}

__global__ void __launch_bounds__(256)
qk_rope_row128_kernel(RopeArgs q, RopeArgs k, int64_t tokens, int heads, float eps,
                      const void* __restrict__ cos_t, const void* __restrict__ sin_t,
                      int64_t c_st, int64_t s_st, int table_f32, int rot) {
#pragma clang fp contract(off)
  constexpr int kD = 128;
  const int sub = threadIdx.x & 15;
  const RopeArgs& a = blockIdx.y == 0 ? q : k;
  const int64_t rows = tokens * heads;
  float wv[8];
  load8(a.w, a.w_f32, sub * 8, false, wv);
  for (int it = 0; it < kRopeGroups; ++it) {
    const int64_t row =
        (static_cast<int64_t>(blockIdx.x) * kRopeGroups + it) * 16 + (threadIdx.x >> 4);
    if (row >= rows) break;  // uniform per 16-lane row group; nothing below synchronizes more
    const int64_t t = row / heads;
    const int h = static_cast<int>(row - t * heads);
    float v[8];
    load8_row(a.x + t * a.st + h * a.sh + sub * 8, v);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += v[i] * v[i];
    ss = sum16(ss);
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(kD) + eps);
    float n[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) n[i] = round_bf16((v[i] * inv) * wv[i]);
    float o[8];
    if (rot == kD) {
      float cvv[8], svv[8];
      load8(cos_t, table_f32, t * c_st + sub * 8, true, cvv);
      load8(sin_t, table_f32, t * s_st + sub * 8, true, svv);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float partner = row_ror8(n[i]);   // channel c + 64 (lanes 0-7) or c - 64
        const float other = sub < 8 ? -partner : partner;
        o[i] = round_bf16(round_bf16(n[i] * cvv[i]) + round_bf16(other * svv[i]));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = n[i];
    }
    u32x4 packed;
#pragma unroll
    for (int i = 0; i < 4; ++i) packed[i] = pack_bf16x2(o[2 * i], o[2 * i + 1]);
    __builtin_nontemporal_store(packed, reinterpret_cast<u32x4*>(a.out + row * kD + sub * 8));
  }
}

// qk_rope_token128_kernel: R = 128. A wave takes one token and walks its heads four at a
// time (a 16-lane group, 8 channels per lane, per head; every row load is one contiguous 1 KB
// span); the weights and the token's cos / sin row (rounded to bf16) are loaded once per
// token instead of once per row, and the partner's sign (-n_{c+64} for the first 64
// channels) is folded into the lane's sin values: (-p) s and p (-s) are the same product,
// rounding included. At [108000 tokens, 40 heads] for q and k of a fused QKV row: 1010 us for
// the row walk above, 800 us for this form; holding 2, 4 or 8 heads' loads in flight per
// group was slower (820-915 us), the registers costing more occupancy than the loads gain.
__global__ void __launch_bounds__(256)
qk_rope_token128_kernel(RopeArgs q, RopeArgs k, int64_t tokens, int heads, float eps,
                        const void* __restrict__ cos_t, const void* __restrict__ sin_t,
                        int64_t c_st, int64_t s_st, int table_f32) {
#pragma clang fp contract(off)
  constexpr int kD = 128;
  const int lane = threadIdx.x & 63, sub = lane & 15, g = lane >> 4;
  const RopeArgs& a = blockIdx.y == 0 ? q : k;
  const int64_t t =
      static_cast<int64_t>(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (t >= tokens) return;  // whole wave
  float wv[8], cvv[8], svv[8];
  load8(a.w, a.w_f32, sub * 8, false, wv);
  load8(cos_t, table_f32, t * c_st + sub * 8, true, cvv);
  load8(sin_t, table_f32, t * s_st + sub * 8, true, svv);
  if (sub < 8) {
#pragma unroll
    for (int i = 0; i < 8; ++i) svv[i] = -svv[i];
  }
  const uint16_t* const xt = a.x + t * a.st + g * a.sh + sub * 8;
  uint16_t* const ot = a.out + (t * heads + g) * kD + sub * 8;
  for (int h0 = 0; h0 < heads; h0 += 4) {
    if (h0 + g >= heads) break;  // the whole 16-lane group (its DPP steps stay in it)
    const u32x4 raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(xt + h0 * a.sh));
    float v[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(raw[i] << 16);
      v[2 * i + 1] = __uint_as_float(raw[i] & 0xffff0000u);
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += v[i] * v[i];
    ss = sum16(ss);
    const float inv = 1.0f / sqrtf(ss / static_cast<float>(kD) + eps);
    u32x4 packed;
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      float n0 = (v[i] * inv) * wv[i], n1 = (v[i + 1] * inv) * wv[i + 1];
      round_bf16_pair(n0, n1);
      float c0 = n0 * cvv[i], c1 = n1 * cvv[i + 1];
      round_bf16_pair(c0, c1);
      float s0 = row_ror8(n0) * svv[i], s1 = row_ror8(n1) * svv[i + 1];
      round_bf16_pair(s0, s1);
      packed[i / 2] = pack_bf16x2(c0 + s0, c1 + s1);
    }
    __builtin_nontemporal_store(packed, reinterpret_cast<u32x4*>(ot + h0 * kD));
  }
}

}  // namespace
}  // namespace vdn

using namespace vdn;

// Reference: paper_qk_rmsnorm_rope (src/models/softmax_attention/paper_qk_rope.py:145-211).
// q, k: [tokens, heads, D] of the activation dtype (flags bits 4-5: 0 bf16, 1 fp16, 2 fp32)
// with arbitrary element strides; weights [D] (stride w_s, fp32 per flags bit0 for q / bit1
// for k, else the activation dtype); cos/sin (nullable: norm only): [tokens, R] with strides,
// fp32 when flags bit2 else the activation dtype; qo, ko: contiguous [tokens, heads, D] of the
// activation dtype. flags bit3: q only (k, k_w and ko may be null), for a lone RMSNorm'd
// operand such as the queries of a cross-attention whose keys have another row count.
VDN_API int vdn_qk_rmsnorm_rope(const void* q, int64_t q_st, int64_t q_sh, int64_t q_sd,
                                const void* k, int64_t k_st, int64_t k_sh, int64_t k_sd,
                                const void* q_w, int64_t q_ws, const void* k_w, int64_t k_ws,
                                float eps, const void* cos_t, int64_t c_st, int64_t c_sd,
                                const void* sin_t, int64_t s_st, int64_t s_sd, int rot,
                                int flags, int64_t tokens, int heads, int head_dim, void* qo,
                                void* ko, void* stream) {
  const char* name = "vdn_qk_rmsnorm_rope";
  const bool q_only = (flags >> 3) & 1;
  if (q == nullptr || q_w == nullptr || qo == nullptr ||
      (!q_only && (k == nullptr || k_w == nullptr || ko == nullptr)))
    return set_error(kInvalidArgument, "%s: null pointer", name);
  if (heads <= 0 || tokens < 0 || (head_dim != 64 && head_dim != 128 && head_dim != 256))
    return set_error(kInvalidArgument, "%s: heads > 0 and D in {64, 128, 256} required", name);
  if ((cos_t == nullptr) != (sin_t == nullptr) || rot < 0 || rot > head_dim || rot % 2 ||
      (cos_t != nullptr && rot == 0))
    return set_error(kInvalidArgument, "%s: invalid rotary width %d", name, rot);
  const int act = (flags >> 4) & 3;
  if (act > 2) return set_error(kInvalidArgument, "%s: activation dtype must be 0, 1 or 2", name);
  if (tokens == 0) return kOk;
  const RopeArgs qa{static_cast<const uint16_t*>(q), q_st, q_sh, q_sd, q_w, q_ws, flags & 1,
                    static_cast<uint16_t*>(qo)};
  const RopeArgs ka{static_cast<const uint16_t*>(k), k_st, k_sh, k_sd, k_w, k_ws, (flags >> 1) & 1,
                    static_cast<uint16_t*>(ko)};
  const int64_t rows = tokens * heads;
  auto st = static_cast<hipStream_t>(stream);
  const int r = cos_t == nullptr ? 0 : rot;
  const int tf = (flags >> 2) & 1;
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const int64_t tab_align = tf ? 4 : 8;
  auto operand_vec = [&](const RopeArgs& o) {
    return o.sd == 1 && o.st % 8 == 0 && o.sh % 8 == 0 && al16(o.x) && o.ws == 1 && al16(o.w);
  };
  const bool vec = act == 0 && operand_vec(qa) && (q_only || operand_vec(ka)) && r % 8 == 0 &&
                   (r == 0 || (c_sd == 1 && s_sd == 1 && c_st % tab_align == 0 &&
                               s_st % tab_align == 0 && al16(cos_t) && al16(sin_t)));
#define VDN_ROPE(D)                                                                             \
  if (vec) VDN_ROPE_V(D, true, 0)                                                               \
  else if (act == 0) VDN_ROPE_V(D, false, 0)                                                    \
  else if (act == 1) VDN_ROPE_V(D, false, 1)                                                    \
  else VDN_ROPE_V(D, false, 2)
#define VDN_ROPE_V(D, V, T)                                                                     \
  hipLaunchKernelGGL((qk_rope_kernel<D, V, T>), dim3(static_cast<unsigned>((rows + 256 / (D / 8) - 1) / \
                                                                    (256 / (D / 8))),           \
                          q_only ? 1 : 2),                                                      \
                     dim3(256), 0, st, qa, ka, tokens, heads, eps, cos_t, sin_t, c_st, c_sd,    \
                     s_st, s_sd, tf, r);
  if (head_dim == 128 && vec && r == 128) {
    hipLaunchKernelGGL(qk_rope_token128_kernel,
                       dim3(static_cast<unsigned>((tokens + 3) / 4), q_only ? 1 : 2),
                       dim3(256), 0, st, qa, ka, tokens, heads, eps, cos_t, sin_t, c_st, s_st,
                       tf);
  } else if (head_dim == 128 && vec && r == 0) {
    const int64_t per_block = 16 * kRopeGroups;
    hipLaunchKernelGGL(qk_rope_row128_kernel,
                       dim3(static_cast<unsigned>((rows + per_block - 1) / per_block),
                            q_only ? 1 : 2),
                       dim3(256), 0, st, qa, ka, tokens, heads, eps, cos_t, sin_t, c_st, s_st,
                       tf, r);
  } else if (head_dim == 64) {
    VDN_ROPE(64)
  } else if (head_dim == 128) {
    VDN_ROPE(128)
  } else {
    VDN_ROPE(256)
  }
#undef VDN_ROPE
#undef VDN_ROPE_V
  return check_launch(name);
}
