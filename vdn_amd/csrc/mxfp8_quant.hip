// MXFP8 producer kernels for gfx950: block-32 E4M3FN codes + E8M0 scales in the
// SWIZZLE_32_4_4 order, written straight from bf16 activations.
//
//   vdn_mxfp8_quantize          bf16 [R,K] -> codes [RP,KP] + scales       (mxfp8_kernels.py:31-58)
//   vdn_mxfp8_act_quantize      act(bf16) rounded to bf16 -> codes+scales  (mxfp8_kernels.py:62-84;
//                               GELU-tanh and SwiGLU activations)
//   vdn_mxfp8_prenorm_quantize  RMSNorm * (1 + scale[i]) + shift[i] -> bf16 -> codes+scales
//                               (mxfp8_kernels.py:87-110, 127-139)
//
// All three are HBM-bound. Work is split into 16-lane groups that own one row and
// one 128-column chunk: each lane reads 8 contiguous bf16 (one 16-byte load), four
// lanes form one 32-element block (amax by two xor-shuffles), and lane 0 of the group
// stores the chunk's four scale bytes as one dword, because SWIZZLE_32_4_4 keeps the
// four K-blocks of a row inside a 128-column chunk contiguous.
#include "mxfp8_common.h"

#include <math.h>

namespace vdn {
namespace {

constexpr int kThreads = 256;
constexpr int kItemsPerGroup = 4;  // (row, chunk) items per 16-lane group

enum Act : int { kActNone = 0, kActGeluTanh = 1, kActSwiGLU = 2 };

__device__ __forceinline__ bool bf16_nonfinite(uint16_t h) { return (h & 0x7f80) == 0x7f80; }

// Loads 8 bf16 values of one row starting at column c0 (masked to zero outside
// [0,rows) x [0,k)). `vec` selects the 16-byte path (k % 8 == 0, aligned rows).
template <bool kVec>
__device__ __forceinline__ void load_row8(const uint16_t* __restrict__ x, int64_t r, int64_t c0,
                                          int64_t rows, int64_t k, int64_t stride,
                                          float* v, bool& bad) {
  if (kVec) {
    if (r < rows && c0 < k) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(x + r * stride + c0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint16_t lo = static_cast<uint16_t>(w[i] & 0xffff);
        const uint16_t hi = static_cast<uint16_t>(w[i] >> 16);
        bad = bad || bf16_nonfinite(lo) || bf16_nonfinite(hi);
        v[2 * i] = bf16_bits_to_f32(lo);
        v[2 * i + 1] = bf16_bits_to_f32(hi);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = 0.f;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (r < rows && c0 + i < k) {
        const uint16_t h = x[r * stride + c0 + i];
        bad |= bf16_nonfinite(h);
        v[i] = bf16_bits_to_f32(h);
      } else {
        v[i] = 0.f;
      }
    }
  }
}


template <int kAct, bool kVec>
__global__ void __launch_bounds__(kThreads)
mxfp8_quantize_kernel(const uint16_t* __restrict__ x, int64_t rows, int64_t k, int64_t stride,
                      uint8_t* __restrict__ q, uint8_t* __restrict__ s, int64_t kp, int64_t items,
                      uint32_t* __restrict__ nonfinite, uint8_t* __restrict__ finite_tiles) {
  const int lane16 = threadIdx.x & 15;
  // items < 2^31 (the host checks): 32-bit index arithmetic, one division per item
  const uint32_t ngroups = gridDim.x * (kThreads / 16);
  const uint32_t group = blockIdx.x * (kThreads / 16) + (threadIdx.x >> 4);
  const uint32_t chunks = static_cast<uint32_t>(kp >> 7);
  bool bad[kItemsPerGroup];
  float v[kItemsPerGroup][8];
  int64_t row_of[kItemsPerGroup], chunk_of[kItemsPerGroup];
  // Issue every load of the group's items before any arithmetic.
#pragma unroll
  for (int j = 0; j < kItemsPerGroup; ++j) {
    const uint32_t item = group + j * ngroups;
    const uint32_t rr = item / chunks;
    row_of[j] = rr;
    chunk_of[j] = item - rr * chunks;
    const int64_t r = item < items ? row_of[j] : rows;  // rows => zero fill
    const int64_t c0 = chunk_of[j] * 128 + lane16 * 8;
    bad[j] = false;
    if (kAct == kActSwiGLU) {
      float g[8];
      load_row8<kVec>(x, r, c0, rows, k, stride, v[j], bad[j]);
      load_row8<kVec>(x + k, r, c0, rows, k, stride, g, bad[j]);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[j][i] = round_bf16(silu_mul(v[j][i], g[i]));
    } else {
      load_row8<kVec>(x, r, c0, rows, k, stride, v[j], bad[j]);
    }
  }
  bool any_bad = false;
#pragma unroll
  for (int j = 0; j < kItemsPerGroup; ++j) {
    const uint32_t item = group + j * ngroups;
    if (item >= items) break;  // uniform across the 16-lane group
    const int64_t r = row_of[j];
    const int64_t chunk = chunk_of[j];
    if (kAct == kActGeluTanh) {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[j][i] = round_bf16(gelu_tanh(v[j][i]));
    }
    if (kAct != kActNone) {
#pragma unroll
      for (int i = 0; i < 8; ++i) bad[j] |= !(fabsf(v[j][i]) < INFINITY);
    }
    quantize_store8(v[j], lane16, r, chunk, kp, q, s);
    // Per (16-row, 256-column) tile finite flags, cleared (by every lane that saw a
    // nonfinite input or activation; all write the same 0) in a host-initialised array.
    if (finite_tiles != nullptr && bad[j])
      finite_tiles[(r >> 4) * ((kp + 255) >> 8) + (chunk >> 1)] = 0;
    any_bad |= bad[j];
  }
  if (__ballot(any_bad) != 0 && (threadIdx.x & 63) == 0) atomicOr(nonfinite, 1u);
}

// vdn_mxfp8_quantize in 32-bit offsets, for the common case: 16-byte rows and every byte
// offset of x (over the padded rows) and of the codes below 2^31. x comes in through a buffer
// resource that ends after the last row, so the padded rows read as zero without a test;
// inf / nan inputs are found from one packed 16-bit max of the exponent fields per item
// rather than a test per value. The arithmetic and the stores are those of quantize_store8.
// Two (row, chunk) items per 16-lane group, 512 threads: at [32768, 5120] bf16 (same box,
// medians of 50 launches) 91.0-91.2 us, against 91-93 with 128 or 256 threads, 93-96 with
// one or three items and 99 with eight.
constexpr int kQ32Items = 2;
constexpr int kQ32Threads = 512;

__global__ void __launch_bounds__(kQ32Threads)
mxfp8_quantize32_kernel(const uint16_t* __restrict__ x, int rows, int k, int stride,
                        uint8_t* __restrict__ q, uint8_t* __restrict__ s, int kp, uint32_t items,
                        uint32_t* __restrict__ nonfinite) {
  const int lane16 = threadIdx.x & 15;
  const uint32_t ngroups = gridDim.x * (kQ32Threads / 16);
  const uint32_t group = blockIdx.x * (kQ32Threads / 16) + (threadIdx.x >> 4);
  const uint32_t chunks = static_cast<uint32_t>(kp) >> 7;
  const uint32_t x_bytes = static_cast<uint32_t>(rows) * static_cast<uint32_t>(stride) * 2u;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(x), 0, static_cast<int>(x_bytes), 0x00020000);
  u32x4 w[kQ32Items];
  uint32_t row_of[kQ32Items], chunk_of[kQ32Items];
  // Issue every load of the group's items before any arithmetic. Columns >= k and items past
  // the end take an offset past the resource's end: those loads return zero. Item j is
  // group + j ngroups: its (row, chunk) follows from item j - 1's by adding ngroups' quotient
  // and remainder by `chunks` (one carry), one division per group instead of one per item.
  const uint32_t ng_q = ngroups / chunks, ng_r = ngroups - ng_q * chunks;
  uint32_t rr = group / chunks, cc = group - rr * chunks;
#pragma unroll
  for (int j = 0; j < kQ32Items; ++j) {
    const uint32_t item = group + j * ngroups;
    row_of[j] = rr;
    chunk_of[j] = cc;
    const uint32_t c0 = cc * 128 + lane16 * 8;
    const bool in = item < items && c0 < static_cast<uint32_t>(k);
    const uint32_t off = in ? (rr * static_cast<uint32_t>(stride) + c0) * 2u : x_bytes;
    w[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
    rr += ng_q;
    cc += ng_r;
    if (cc >= chunks) {
      cc -= chunks;
      ++rr;
    }
  }
  bool any_bad = false;
#pragma unroll
  for (int j = 0; j < kQ32Items; ++j) {
    const uint32_t item = group + j * ngroups;
    if (item >= items) break;  // uniform across the 16-lane group
    const uint32_t r = row_of[j], chunk = chunk_of[j];
    // the nonfinite test, the amax and the codes straight from the packed bf16 words
    const u16x2 m8 = mag8_bf16(w[j]);
    any_bad |= m8[0] >= 0x7f80 || m8[1] >= 0x7f80;
    const float amax = block_amax4(amax8_bf16(w[j], m8));
    float inv;
    const uint32_t scale = e8m0_from_amax(amax, &inv);
    const u32x2 codes = e4m3x8_bf16(w[j], e8m0_scale(scale));
    __builtin_nontemporal_store(
        codes, reinterpret_cast<u32x2*>(q + (r * static_cast<uint32_t>(kp) + chunk * 128 + lane16 * 8)));
    const uint32_t word = scale_word16(scale);
    if (lane16 == 0) {
      // swizzled_scale_offset(r, 4 chunk, kp / 128) in 32 bits
      const uint32_t off = ((r >> 7) * chunks + chunk) * 512 + (r & 31) * 16 + ((r & 127) >> 5) * 4;
      *reinterpret_cast<uint32_t*>(s + off) = word;
    }
  }
  if (__ballot(any_bad) != 0 && (threadIdx.x & 63) == 0) atomicOr(nonfinite, 1u);
}

// One workgroup per padded row. The row stays in registers: slice j of thread t is
// columns [8(t + 256 j), +8), so 4 consecutive lanes share a 32-block and 16 share a
// 128-column chunk, exactly as in the plain quantizer.
// Loads 8 consecutive table values (bf16 or fp32) at element offset `off` as floats.
__device__ __forceinline__ void load_table8(const void* __restrict__ t, int f32, int64_t off,
                                            float* out) {
  if (f32) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(static_cast<const float*>(t) + off);
    const f32x4 b = *reinterpret_cast<const f32x4*>(static_cast<const float*>(t) + off + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[i] = a[i];
      out[4 + i] = b[i];
    }
  } else {
    const u32x4 w = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(t) + off);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = bf16_bits_to_f32(static_cast<uint16_t>(w[i] & 0xffff));
      out[2 * i + 1] = bf16_bits_to_f32(static_cast<uint16_t>(w[i] >> 16));
    }
  }
}

__device__ __forceinline__ void unpack_bf16x8(const u32x4 w, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_bits_to_f32(static_cast<uint16_t>(w[i] & 0xffff));
    f[2 * i + 1] = bf16_bits_to_f32(static_cast<uint16_t>(w[i] >> 16));
  }
}

// Sixteen padded rows per workgroup (one per wave, kS 8-column slices per lane). When the
// rows share one AdaLN table row (the usual case: one timestep for a whole clip) the weight,
// 1 + scale and shift rows are staged once in LDS as fp32, so they are read from L2 once per
// 16 rows instead of once per row; otherwise each row reads its own table row. Arithmetic
// and rounding are those of prenorm_quantize_kernel. (A wave that walks several rows is
// slower: its next row's loads wait for the current row's arithmetic, while fresh waves
// of the next workgroups overlap them.)
constexpr int kPrenormRows = 16;
constexpr int kPrenormThreads = 64 * kPrenormRows;

// Rows of exactly kCols = 512 kS columns (every slice real), eight rows per workgroup, two
// workgroups per CU (60 KB of LDS and at most 128 VGPRs each), so one's table staging and
// load latency overlap the other's arithmetic; each wave issues its row's loads before the
// table row is staged. The row index is wave-uniform, so every address is a scalar row base
// plus a per-lane offset. The arithmetic is that of the general path in straight-line code.
// The bf16 results stay packed (the rounding conversion is the packing); a bf16 is nonfinite
// iff its magnitude bits reach 0x7f80, so one packed max per word tests two of them. (At
// [108000, 5120]: 354 us without the bf16 output and 518 us with it, against 429 and 548 us
// for sixteen rows per workgroup at one workgroup per CU, whose staging and arithmetic left
// the CU without loads in flight.)
constexpr int kFullRows = 8;
constexpr int kFullThreads = 64 * kFullRows;

template <int kS>
__global__ void __launch_bounds__(kFullThreads) __attribute__((amdgpu_waves_per_eu(4)))
prenorm_quantize_full_rows_kernel(const uint16_t* __restrict__ x, int64_t rows, int64_t stride,
                                  const void* __restrict__ weight, int weight_f32, float eps,
                                  const void* __restrict__ scale, int64_t scale_stride,
                                  const void* __restrict__ shift, int64_t shift_stride,
                                  int tables_f32, const int64_t* __restrict__ indices,
                                  uint16_t* __restrict__ y, uint8_t* __restrict__ q,
                                  uint8_t* __restrict__ s, uint8_t* __restrict__ finite,
                                  int64_t rp) {
#pragma clang fp contract(off)
  constexpr int kCols = 64 * kS * 8;
  constexpr int64_t kChunks = kCols / 128;
  __shared__ __attribute__((aligned(16))) float tab[3][kCols];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kFullRows;
  const int64_t r = r0 + wave;
  const bool in_row = r < rows;  // wave-uniform
  const int64_t idx0 = r0 < rows ? indices[r0] : 0;
  int same = 1;
  if (tid < kFullRows && r0 + tid < rows) same = indices[r0 + tid] == idx0;
  u32x4 raw[kS];
#pragma unroll
  for (int j = 0; j < kS; ++j) raw[j] = u32x4{0u, 0u, 0u, 0u};
  if (in_row) {
    const uint16_t* xrow = x + r * stride + lane * 8;
#pragma unroll
    for (int j = 0; j < kS; ++j)
      raw[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(xrow + 512 * j));
  }
  // one table row for the whole workgroup?
  const bool shared_row = __syncthreads_and(same) != 0;
  if (shared_row) {
    for (int c0 = tid * 8; c0 < kCols; c0 += kFullThreads * 8) {
      float t[8];
      load_table8(weight, weight_f32, c0, t);
      *reinterpret_cast<f32x4*>(&tab[0][c0]) = f32x4{t[0], t[1], t[2], t[3]};
      *reinterpret_cast<f32x4*>(&tab[0][c0 + 4]) = f32x4{t[4], t[5], t[6], t[7]};
      load_table8(scale, tables_f32, idx0 * scale_stride + c0, t);
#pragma unroll
      for (int i = 0; i < 8; ++i) t[i] = 1.0f + t[i];  // the (1 + scale) factor, formed once
      *reinterpret_cast<f32x4*>(&tab[1][c0]) = f32x4{t[0], t[1], t[2], t[3]};
      *reinterpret_cast<f32x4*>(&tab[1][c0 + 4]) = f32x4{t[4], t[5], t[6], t[7]};
      load_table8(shift, tables_f32, idx0 * shift_stride + c0, t);
      *reinterpret_cast<f32x4*>(&tab[2][c0]) = f32x4{t[0], t[1], t[2], t[3]};
      *reinterpret_cast<f32x4*>(&tab[2][c0 + 4]) = f32x4{t[4], t[5], t[6], t[7]};
    }
  }
  __syncthreads();
  if (r >= rp) return;  // whole wave (no barrier follows)
  // slice j of this lane: columns 8 (lane + 64 j) .. + 8, i.e. 128-column chunk 4 j + lane / 16;
  // its codes sit at row base + 8 lane + 512 j and its group's scale word at the row's
  // swizzled base + 512 (lane / 16) + 2048 j
  uint8_t* const qlane = q + r * kCols + lane * 8;
  uint8_t* const slane = s + swizzled_scale_offset(r, 0, kChunks) + (lane >> 4) * 512;
  const bool scale_lane = (lane & 15) == 0;
  if (!in_row) {  // a padding row: zero codes, the zero scale, finite
#pragma unroll
    for (int j = 0; j < kS; ++j) {
      float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      quantize_store8_at(v, qlane + 512 * j, slane + 2048 * j, scale_lane);
    }
    if (lane == 0) finite[r] = 1;
    return;
  }
  const int64_t table_row = shared_row ? idx0 : indices[r];
  // sum of squares, two products per v_dot2 on the packed words, in two chains
  float ss0 = 0.f, ss1 = 0.f;
#pragma unroll
  for (int j = 0; j < kS; ++j) {
    if (j & 1) ss1 = sumsq8_bf16(raw[j], ss1);
    else ss0 = sumsq8_bf16(raw[j], ss0);
  }
  float ss = ss0 + ss1;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  const float ms = ss / static_cast<float>(kCols) + eps;
  const float inv_rms = static_cast<float>(1.0 / sqrt(static_cast<double>(ms)));
  uint16_t* const ylane = y == nullptr ? nullptr : y + r * kCols + lane * 8;
  u16x2 mag = {0, 0};
#pragma unroll
  for (int j = 0; j < kS; ++j) {
    const int c0 = (lane + 64 * j) * 8;
    float xv[8], w[8], u[8], sh[8];
    unpack_bf16x8(raw[j], xv);
    if (shared_row) {
#pragma unroll
      for (int i = 0; i < 8; i += 4) {
        const f32x4 a = *reinterpret_cast<const f32x4*>(&tab[0][c0 + i]);
        const f32x4 b = *reinterpret_cast<const f32x4*>(&tab[1][c0 + i]);
        const f32x4 c = *reinterpret_cast<const f32x4*>(&tab[2][c0 + i]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          w[i + e] = a[e];
          u[i + e] = b[e];
          sh[i + e] = c[e];
        }
      }
    } else {
      load_table8(weight, weight_f32, c0, w);
      load_table8(scale, tables_f32, table_row * scale_stride + c0, u);
      load_table8(shift, tables_f32, table_row * shift_stride + c0, sh);
#pragma unroll
      for (int i = 0; i < 8; ++i) u[i] = 1.0f + u[i];
    }
    u32x4 packed;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float t0 = (xv[2 * i] * inv_rms) * w[2 * i];
      const float t1 = (xv[2 * i + 1] * inv_rms) * w[2 * i + 1];
      packed[i] = pack_bf16x2(t0 * u[2 * i] + sh[2 * i], t1 * u[2 * i + 1] + sh[2 * i + 1]);
    }
    const u16x2 m8 = mag8_bf16(packed);
    mag = __builtin_elementwise_max(mag, m8);
    if (y != nullptr) __builtin_nontemporal_store(packed, reinterpret_cast<u32x4*>(ylane + 512 * j));
    quantize_store8_bf16_at(packed, m8, qlane + 512 * j, slane + 2048 * j, scale_lane);
  }
  const bool any_bad = __ballot(mag[0] >= 0x7f80 || mag[1] >= 0x7f80) != 0;
  if (lane == 0) finite[r] = any_bad ? 0 : 1;
}

// Rows of other widths (K up to 512 kS columns, the last slices partial or padding).
template <int kS>
__global__ void __launch_bounds__(kPrenormThreads)
prenorm_quantize_rows_kernel(const uint16_t* __restrict__ x, int64_t rows, int64_t k,
                             int64_t stride, const void* __restrict__ weight, int weight_f32,
                             float eps, const void* __restrict__ scale, int64_t scale_stride,
                             const void* __restrict__ shift, int64_t shift_stride,
                             int tables_f32, const int64_t* __restrict__ indices,
                             uint16_t* __restrict__ y, uint8_t* __restrict__ q,
                             uint8_t* __restrict__ s, uint8_t* __restrict__ finite, int64_t kp,
                             int64_t rp) {
#pragma clang fp contract(off)
  constexpr int kCols = 64 * kS * 8;
  __shared__ __attribute__((aligned(16))) float tab[3][kCols];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kPrenormRows;
  const int64_t slices = kp >> 3;
  // one table row for the whole workgroup?
  const int64_t idx0 = r0 < rows ? indices[r0] : 0;
  int same = 1;
  if (tid < kPrenormRows && r0 + tid < rows) same = indices[r0 + tid] == idx0;
  const bool shared_row = __syncthreads_and(same) != 0;
  if (shared_row) {
    for (int64_t c = tid * 4; c < kp; c += kPrenormThreads * 4) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t cc = c + e;
        float wv = 0.f, sv = 0.f, hv = 0.f;
        if (cc < k) {
          wv = weight_f32 ? static_cast<const float*>(weight)[cc]
                          : bf16_bits_to_f32(static_cast<const uint16_t*>(weight)[cc]);
          const int64_t so = idx0 * scale_stride + cc, ho = idx0 * shift_stride + cc;
          sv = tables_f32 ? static_cast<const float*>(scale)[so]
                          : bf16_bits_to_f32(static_cast<const uint16_t*>(scale)[so]);
          hv = tables_f32 ? static_cast<const float*>(shift)[ho]
                          : bf16_bits_to_f32(static_cast<const uint16_t*>(shift)[ho]);
        }
        tab[0][cc] = wv;
        tab[1][cc] = 1.0f + sv;  // the (1 + scale) factor, formed once per column
        tab[2][cc] = hv;
      }
    }
  }
  __syncthreads();
  {
    const int64_t r = r0 + wave;
    if (r >= rp) return;  // whole wave (no barrier follows)
    const bool in_row = r < rows;
    const int64_t table_row = in_row ? indices[r] : 0;
    // the row stays in registers as packed bf16 (kS x 4 VGPRs) and is unpacked where used
    u32x4 raw[kS];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < kS; ++j) {
      const int64_t c0 = (lane + 64 * j) * 8;
      raw[j] = u32x4{0u, 0u, 0u, 0u};
      if (in_row && c0 < k) raw[j] = *reinterpret_cast<const u32x4*>(x + r * stride + c0);
      float f[8];
      unpack_bf16x8(raw[j], f);
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += f[i] * f[i];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
    const float ms = ss / static_cast<float>(k) + eps;
    const float inv_rms = static_cast<float>(1.0 / sqrt(static_cast<double>(ms)));
    // A nonfinite input makes its row's sum of squares nonfinite and so some output of the
    // row nonfinite: testing the outputs covers the inputs.
    bool bad = false;
#pragma unroll
    for (int j = 0; j < kS; ++j) {
      const int64_t sl = lane + 64 * j;
      if (sl >= slices) break;  // slices beyond KP: none of this lane's later ones exist
      const int64_t c0 = sl * 8;
      float v[8];
      if (in_row && c0 < k) {
        float xv[8], w[8], u[8], sh[8];
        unpack_bf16x8(raw[j], xv);
        if (shared_row) {
#pragma unroll
          for (int i = 0; i < 8; i += 4) {
            const f32x4 a = *reinterpret_cast<const f32x4*>(&tab[0][c0 + i]);
            const f32x4 b = *reinterpret_cast<const f32x4*>(&tab[1][c0 + i]);
            const f32x4 c = *reinterpret_cast<const f32x4*>(&tab[2][c0 + i]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              w[i + e] = a[e];
              u[i + e] = b[e];
              sh[i + e] = c[e];
            }
          }
        } else {
          load_table8(weight, weight_f32, c0, w);
          load_table8(scale, tables_f32, table_row * scale_stride + c0, u);
          load_table8(shift, tables_f32, table_row * shift_stride + c0, sh);
#pragma unroll
          for (int i = 0; i < 8; ++i) u[i] = 1.0f + u[i];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float t = (xv[i] * inv_rms) * w[i];
          v[i] = round_bf16(t * u[i] + sh[i]);
          bad |= !(fabsf(v[i]) < INFINITY);
        }
        if (y != nullptr) {
          u32x4 packed;
#pragma unroll
          for (int i = 0; i < 4; ++i) packed[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
          *reinterpret_cast<u32x4*>(y + r * k + c0) = packed;
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = 0.f;
      }
      quantize_store8(v, lane & 15, r, sl >> 4, kp, q, s);
    }
    const bool any_bad = __ballot(bad) != 0;
    if (lane == 0) finite[r] = any_bad ? 0 : 1;
  }
}

template <int kMaxSlices, bool kVec>
__global__ void __launch_bounds__(kThreads)
prenorm_quantize_kernel(const uint16_t* __restrict__ x, int64_t rows, int64_t k, int64_t stride,
                        const void* __restrict__ weight, int weight_f32, float eps,
                        const void* __restrict__ scale, int64_t scale_stride,
                        const void* __restrict__ shift, int64_t shift_stride, int tables_f32,
                        const int64_t* __restrict__ indices, uint16_t* __restrict__ y,
                        uint8_t* __restrict__ q, uint8_t* __restrict__ s,
                        uint8_t* __restrict__ finite, int64_t kp) {
#pragma clang fp contract(off)
  __shared__ float red_sum[kThreads / 64];
  __shared__ int red_bad[kThreads / 64];
  const int tid = threadIdx.x;
  const int lane16 = tid & 15;
  const int64_t r = blockIdx.x;
  const bool in_row = r < rows;
  const int64_t slices = kp >> 3;
  const int64_t table_row = in_row ? indices[r] : 0;
  float v[kMaxSlices][8];
  bool bad = false;
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kMaxSlices; ++j) {
    const int64_t sl = tid + j * kThreads;
    load_row8<kVec>(x, sl < slices ? r : rows, sl * 8, rows, k, stride, v[j], bad);
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += v[j][i] * v[j][i];
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  if ((tid & 63) == 0) red_sum[tid >> 6] = ss;
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int w = 0; w < kThreads / 64; ++w) total += red_sum[w];
  const float ms = total / static_cast<float>(k) + eps;
  const float inv_rms = static_cast<float>(1.0 / sqrt(static_cast<double>(ms)));
#pragma unroll
  for (int j = 0; j < kMaxSlices; ++j) {
    const int64_t sl = tid + j * kThreads;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t c = sl * 8 + i;
      float value = 0.f;
      if (in_row && c < k) {
        const float w = weight_f32 ? static_cast<const float*>(weight)[c]
                                   : bf16_bits_to_f32(static_cast<const uint16_t*>(weight)[c]);
        float sc, sh;
        if (tables_f32) {
          sc = static_cast<const float*>(scale)[table_row * scale_stride + c];
          sh = static_cast<const float*>(shift)[table_row * shift_stride + c];
        } else {
          sc = bf16_bits_to_f32(static_cast<const uint16_t*>(scale)[table_row * scale_stride + c]);
          sh = bf16_bits_to_f32(static_cast<const uint16_t*>(shift)[table_row * shift_stride + c]);
        }
        const float t = (v[j][i] * inv_rms) * w;
        const float u = 1.0f + sc;
        value = round_bf16(t * u + sh);
        bad |= !(fabsf(value) < INFINITY);
      }
      v[j][i] = value;
    }
    if (y != nullptr && in_row && sl < slices) {
      if (kVec && sl * 8 < k) {
        u32x4 packed;
#pragma unroll
        for (int i = 0; i < 4; ++i) packed[i] = pack_bf16x2(v[j][2 * i], v[j][2 * i + 1]);
        *reinterpret_cast<u32x4*>(y + r * k + sl * 8) = packed;
      } else if (!kVec) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
          if (sl * 8 + i < k) y[r * k + sl * 8 + i] = f32_to_bf16_bits(v[j][i]);
      }
    }
    if (sl < slices) quantize_store8(v[j], lane16, r, sl >> 4, kp, q, s);
  }
  const int any_bad = __ballot(bad) != 0;
  if ((tid & 63) == 0) red_bad[tid >> 6] = any_bad;
  __syncthreads();
  if (tid == 0) {
    int b = 0;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) b |= red_bad[w];
    finite[r] = b ? 0 : 1;
  }
}

int64_t pad128(int64_t n) { return (n + 127) / 128 * 128; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <int kAct>
int launch_quantize(const void* x, int64_t rows, int64_t k, int64_t stride, void* q, void* s,
                    uint32_t* nonfinite, uint8_t* finite_tiles, hipStream_t stream,
                    const char* name) {
  if (rows < 0 || k <= 0) return set_error(kInvalidArgument, "%s: rows must be >= 0 and K > 0", name);
  if (stride < k * (kAct == kActSwiGLU ? 2 : 1))
    return set_error(kInvalidArgument, "%s: row stride %lld smaller than row width", name,
                     static_cast<long long>(stride));
  if (x == nullptr || q == nullptr || s == nullptr || nonfinite == nullptr)
    return set_error(kInvalidArgument, "%s: null pointer argument", name);
  const int64_t rp = pad128(rows), kp = pad128(k);
  if (rp == 0) return kOk;
  const int64_t items = rp * (kp / 128);
  const int64_t per_block = (kThreads / 16) * kItemsPerGroup;
  const int64_t blocks = (items + per_block - 1) / per_block;
  if (items + per_block * 2 > (1ll << 31))  // item indices (plus a grid of slack) fit in 31 bits
    return set_error(kUnsupported, "%s: %lld x %lld is too large (2^31 128-column items)", name,
                     static_cast<long long>(rows), static_cast<long long>(k));
  const bool vec = (k % 8 == 0) && (stride % 8 == 0) && aligned16(x) &&
                   (kAct != kActSwiGLU || k % 8 == 0);
  auto* xp = static_cast<const uint16_t*>(x);
  auto* qp = static_cast<uint8_t*>(q);
  auto* sp = static_cast<uint8_t*>(s);
  // the 32-bit form: plain quantize, byte offsets of x over the padded rows and of the codes
  // below 2^31
  if (kAct == kActNone && vec && finite_tiles == nullptr && rp * stride * 2 + 16 < (1ll << 31) &&
      rp * kp < (1ll << 31)) {
    const int64_t per32 = (kQ32Threads / 16) * kQ32Items;
    hipLaunchKernelGGL(mxfp8_quantize32_kernel, dim3((items + per32 - 1) / per32),
                       dim3(kQ32Threads), 0, stream, xp,
                       static_cast<int>(rows), static_cast<int>(k), static_cast<int>(stride), qp,
                       sp, static_cast<int>(kp), static_cast<uint32_t>(items), nonfinite);
    return check_launch(name);
  }
  if (vec) {
    hipLaunchKernelGGL((mxfp8_quantize_kernel<kAct, true>), dim3(blocks), dim3(kThreads), 0, stream,
                       xp, rows, k, stride, qp, sp, kp, items, nonfinite, finite_tiles);
  } else {
    hipLaunchKernelGGL((mxfp8_quantize_kernel<kAct, false>), dim3(blocks), dim3(kThreads), 0, stream,
                       xp, rows, k, stride, qp, sp, kp, items, nonfinite, finite_tiles);
  }
  return check_launch(name);
}

}  // namespace
}  // namespace vdn

using namespace vdn;

// Reference: src/models/ops/mxfp8_kernels.py:31-58 (_quantize / launch_quantize).
VDN_API int vdn_mxfp8_quantize(const void* x, int64_t rows, int64_t k, int64_t row_stride,
                               void* q, void* scales, uint32_t* nonfinite, void* stream) {
  return launch_quantize<kActNone>(x, rows, k, row_stride, q, scales, nonfinite, nullptr,
                                   static_cast<hipStream_t>(stream), "vdn_mxfp8_quantize");
}

// Reference: src/models/ops/mxfp8_kernels.py:62-84, 113-124 (_swiglu_mx) and the block's
// GELU-tanh FFN activation. act: 1 = GELU-tanh over [R,K]; 2 = SwiGLU a*silu(g) over [R,2K].
// finite_tiles (nullable, caller-initialised to 1): byte (r / 16) * ceil(KP / 256) + c / 256
// is cleared when tile (16 rows, 256 output columns) holds a nonfinite input or activation,
// the FINITE output of _swiglu_mx (mxfp8_kernels.py:73-75).
VDN_API int vdn_mxfp8_act_quantize(const void* x, int64_t rows, int64_t k, int64_t row_stride,
                                   int act, void* q, void* scales, uint32_t* nonfinite,
                                   uint8_t* finite_tiles, void* stream) {
  auto st = static_cast<hipStream_t>(stream);
  if (act == kActGeluTanh)
    return launch_quantize<kActGeluTanh>(x, rows, k, row_stride, q, scales, nonfinite,
                                         finite_tiles, st, "vdn_mxfp8_act_quantize");
  if (act == kActSwiGLU)
    return launch_quantize<kActSwiGLU>(x, rows, k, row_stride, q, scales, nonfinite,
                                       finite_tiles, st, "vdn_mxfp8_act_quantize");
  return set_error(kInvalidArgument, "vdn_mxfp8_act_quantize: unknown activation %d", act);
}

// Reference: src/models/ops/mxfp8_kernels.py:87-110, 127-139 (_prenorm_mx /
// launch_prenorm_quantize). flags: bit0 weight is fp32, bit1 scale/shift tables are fp32.
VDN_API int vdn_mxfp8_prenorm_quantize(const void* x, int64_t rows, int64_t k, int64_t row_stride,
                                       const void* weight, float eps, const void* scale,
                                       int64_t scale_stride, const void* shift,
                                       int64_t shift_stride, const int64_t* indices, int flags,
                                       void* y, void* q, void* scales, uint8_t* finite,
                                       void* stream) {
  const char* name = "vdn_mxfp8_prenorm_quantize";
  if (rows < 0 || k <= 0) return set_error(kInvalidArgument, "%s: rows must be >= 0 and K > 0", name);
  if (row_stride < k) return set_error(kInvalidArgument, "%s: row stride smaller than K", name);
  if (x == nullptr || weight == nullptr || scale == nullptr || shift == nullptr ||
      indices == nullptr || q == nullptr || scales == nullptr || finite == nullptr)
    return set_error(kInvalidArgument, "%s: null pointer argument", name);
  const int64_t rp = pad128(rows), kp = pad128(k);
  if (rp == 0) return kOk;
  const int64_t slices = kp / 8;
  const bool vec = (k % 8 == 0) && (row_stride % 8 == 0) && aligned16(x) &&
                   (y == nullptr || aligned16(y));
  auto st = static_cast<hipStream_t>(stream);
  auto* xp = static_cast<const uint16_t*>(x);
  auto* yp = static_cast<uint16_t*>(y);
  auto* qp = static_cast<uint8_t*>(q);
  auto* sp = static_cast<uint8_t*>(scales);
  const int wf = flags & 1, tf = (flags >> 1) & 1;
#define VDN_PRENORM(MS)                                                                        \
  if (vec)                                                                                     \
    hipLaunchKernelGGL((prenorm_quantize_kernel<MS, true>), dim3(rp), dim3(kThreads), 0, st,  \
                       xp, rows, k, row_stride, weight, wf, eps, scale, scale_stride, shift,   \
                       shift_stride, tf, indices, yp, qp, sp, finite, kp);                     \
  else                                                                                         \
    hipLaunchKernelGGL((prenorm_quantize_kernel<MS, false>), dim3(rp), dim3(kThreads), 0, st, \
                       xp, rows, k, row_stride, weight, wf, eps, scale, scale_stride, shift,   \
                       shift_stride, tf, indices, yp, qp, sp, finite, kp);
  const int64_t tab_align = tf ? 4 : 8;
  const bool wave_ok = vec && aligned16(weight) && aligned16(scale) && aligned16(shift) &&
                       scale_stride % tab_align == 0 && shift_stride % tab_align == 0;
  if (wave_ok && slices <= 64 * 10) {
    const dim3 grid(static_cast<unsigned>((rp + kPrenormRows - 1) / kPrenormRows));
#define VDN_PRENORM_FULL(S)                                                                    \
    if (k == 512 * (S)) {                                                                      \
      hipLaunchKernelGGL((prenorm_quantize_full_rows_kernel<S>),                             \
                         dim3(static_cast<unsigned>((rp + kFullRows - 1) / kFullRows)),        \
                         dim3(kFullThreads), 0, st, xp, rows, row_stride, weight, wf, eps,     \
                         scale, scale_stride,                                                  \
                         shift, shift_stride, tf, indices, yp, qp, sp, finite, rp);            \
      return check_launch(name);                                                               \
    }
    VDN_PRENORM_FULL(2)
    VDN_PRENORM_FULL(4)
    VDN_PRENORM_FULL(8)
    VDN_PRENORM_FULL(10)
#undef VDN_PRENORM_FULL
#define VDN_PRENORM_WAVE(S)                                                                   \
    hipLaunchKernelGGL((prenorm_quantize_rows_kernel<S>), grid, dim3(kPrenormThreads), 0, st, xp, rows, \
                       k, row_stride, weight, wf, eps, scale, scale_stride, shift,              \
                       shift_stride, tf, indices, yp, qp, sp, finite, kp, rp);
    if (slices <= 64 * 2) {
      VDN_PRENORM_WAVE(2)
    } else if (slices <= 64 * 4) {
      VDN_PRENORM_WAVE(4)
    } else if (slices <= 64 * 8) {
      VDN_PRENORM_WAVE(8)
    } else {
      VDN_PRENORM_WAVE(10)
    }
#undef VDN_PRENORM_WAVE
    return check_launch(name);
  }
  if (slices <= kThreads * 1) {
    VDN_PRENORM(1)
  } else if (slices <= kThreads * 3) {
    VDN_PRENORM(3)
  } else if (slices <= kThreads * 8) {
    VDN_PRENORM(8)
  } else {
    return set_error(kUnsupported, "%s: K=%lld exceeds the register-resident row limit 16384",
                     name, static_cast<long long>(k));
  }
#undef VDN_PRENORM
  return check_launch(name);
}
