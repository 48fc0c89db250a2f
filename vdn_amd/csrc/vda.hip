// VDA frame-wise delta-rule linear attention ("vdn_solve", bridge = alpha) for gfx950.
//
// Per frame f and head h (S tokens, D = 128):
//   k' = bf16(L2(SiLU(k))), v' = bf16(SiLU(v)), q' = bf16(L2(SiLU(q)))   (paper_prepare)
//   A = 1/2 (Kᵀ diag(β) K + its transpose)  fp32-grade;  B = bf16(bf16(v'·β)ᵀ k')  (paper_statistics)
//   T = diag(α) (I + A)⁻¹,  J = B (I + A)⁻¹                                (paper_delta_factors)
//   forward/reverse affine scans over frames (or frame chunks)             (paper_boundary_scan)
//   state = α-bridged sum of the states just outside each frame's window  (paper_gather)
//   out = RMSNorm(bf16(q'·stateᵀ))·w·gate                                  (readout + vdn_linear_epilogue)
// Reference: src/models/linear_attention/paper_stack.py, paper_sglang.py, paper_factor.py,
// scan.py, delta_rule.py:45-60.
//
// MI355X design notes:
//   * the statistics read raw token-major q/k/v straight from the QKV projection output (any
//     row/head stride) and apply SiLU/L2 in registers, so no frame-major copy is written;
//   * A needs fp32-grade accuracy (I + A is inverted). With bf16 k' and bf16 β the product
//     p = β k' has at most 16 significant bits, so p = hi + lo with hi, lo bf16 is exact and
//     A = Kᵀ·P_hi + Kᵀ·P_lo runs on bf16 MFMA with fp32 accumulation (3 terms for fp32 β);
//   * token-contiguous MFMA operands come from token-major LDS tiles through
//     ds_read_tr16_b64: within a 16-lane group, lane L reading 8 bytes at
//     (row r0 + L/4, column c0 + 4 (L % 4)) delivers to lane l the 4 values
//     M[r0 .. r0+3][c0 + l] (measured on gfx950);
//   * the scans keep a 16-row block of the 128x128 fp32 state per workgroup (rows evolve
//     independently) and use fp32 MFMA for state @ T.
#include "mxfp8_common.h"

#include <math.h>

#include <algorithm>
#include <type_traits>

namespace vdn {
namespace {

constexpr int kD = 128;

typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4_t;

__device__ __forceinline__ bf16x4_t lds_read_tr(const uint16_t* lds_elem_ptr) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
      (lds_bf16x4_t*)((__attribute__((address_space(3))) char*)(lds_elem_ptr)));
}

// SiLU(x) = x / (1 + exp(-x)) with the hardware exp2 and reciprocal: a few fp32 ulp from
// the libm form, far below the bf16 rounding that follows every use.
__device__ __forceinline__ float silu(float x) {
  constexpr float kMinusLog2e = -1.4426950408889634f;
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * kMinusLog2e));
}

__device__ __forceinline__ void unpack8(const u32x4 w, float* v) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = bf16_bits_to_f32(static_cast<uint16_t>(w[i] & 0xffff));
    v[2 * i + 1] = bf16_bits_to_f32(static_cast<uint16_t>(w[i] >> 16));
  }
}

__device__ __forceinline__ u32x4 pack8(const float* v) {
  u32x4 w;
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
  return w;
}

// SiLU (+ L2 over the 16-lane group's 128 channels) of 8 values, not rounded: the caller
// rounds through the packing conversion. paper_sglang.py:235-238: y = silu(x);
// y / sqrt(max(sum y^2, 1e-12)).
__device__ __forceinline__ void activate8_f32(float* v, bool l2) {
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    v[i] = silu(v[i]);
    ss += v[i] * v[i];
  }
  if (l2) {
    ss = sum16(ss);
    const float inv = __builtin_amdgcn_rsqf(fmaxf(ss, 1e-12f));
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] *= inv;
  }
}

// Dispatch id -> logical id such that each XCD (dispatch is round-robin over 8) runs one
// contiguous range of logical ids.
__device__ __forceinline__ int xcd_contiguous(int b, int n) {
  const int xcd = b & 7, local = b >> 3;
  const int per = n >> 3, rem = n & 7;
  return xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
}

// Strided 3-D view of a bf16 [frames, heads, tokens, channel] operand; channels contiguous.
struct View {
  const uint16_t* base;
  int64_t sf, sh, ss;
  __device__ __forceinline__ const uint16_t* at(int f, int h, int s) const {
    return base + f * sf + h * sh + s * ss;
  }
};

// ------------------------------------------------------------------- prepare ----
// tokens [N, H, D] (row stride sn, head stride sh) -> frame-major out [F, H, S, D]
template <bool kF32>
__global__ void __launch_bounds__(256)
vda_prepare_kernel(const void* __restrict__ x, int64_t n, int heads, int64_t sn, int64_t sh,
                   int spatial, int l2, void* __restrict__ out) {
  const int lane16 = threadIdx.x & 15;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 16 + (threadIdx.x >> 4);
  const int64_t items = n * heads;
  if (item >= items) return;  // uniform per 16-lane group
  const int64_t row = item / heads;
  const int h = static_cast<int>(item % heads);
  const int64_t f = row / spatial, s = row % spatial;
  float v[8];
  if (kF32) {
    const float* src = static_cast<const float*>(x) + row * sn + h * sh + lane16 * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = src[i];
  } else {
    const uint16_t* src = static_cast<const uint16_t*>(x) + row * sn + h * sh + lane16 * 8;
    unpack8(*reinterpret_cast<const u32x4*>(src), v);
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    v[i] = silu(v[i]);
    ss += v[i] * v[i];
  }
  if (l2) {
    ss = sum16(ss);
    const float inv = __builtin_amdgcn_rsqf(fmaxf(ss, 1e-12f));
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] *= inv;
  }
  const int64_t dst = ((f * heads + h) * spatial + s) * kD + lane16 * 8;
  if (kF32) {
    float* o = static_cast<float*>(out) + dst;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = v[i];
  } else {
    *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(out) + dst) = pack8(v);
  }
}

// ---------------------------------------------------------------- statistics ----
constexpr int kTS = 32;          // tokens per step
constexpr int kRow = 144;        // padded LDS row (bf16 elements): 288 bytes
constexpr int kTile = kTS * kRow;
constexpr int kStWaves = 8;
constexpr int kStThreads = 64 * kStWaves;

// One workgroup per (frame, head); 8 waves, wave w owns rows [64 (w / 4), +64) x columns
// [32 (w % 4), +32) of both A' = Kᵀ P and B' = Vbᵀ K. Each step thread t loads token t / 16
// of the step's 32, channels 8 (t % 16) .. +8, applies the activation and writes k', the
// split products and vb to the step's LDS tiles. With bf16 beta (kSplit = 2) two
// workgroups share a CU (16 waves): at most 128 VGPRs.
template <int kSplit>
__global__ void __launch_bounds__(kStThreads)
__attribute__((amdgpu_waves_per_eu(kSplit == 2 ? 4 : 2)))
vda_statistics_kernel(View kv, View vv, const void* __restrict__ beta, int64_t b_sf,
                      int64_t b_sh, int64_t b_ss, int beta_f32, int spatial, int heads,
                      int activate, float* __restrict__ A, float* __restrict__ B) {
  constexpr int kTiles = 2 + kSplit;
  __shared__ __attribute__((aligned(16))) uint16_t lds[2][kTiles][kTile];
  const int fh = blockIdx.x;
  const int f = fh / heads, h = fh % heads;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;
  const int lane16 = tid & 15;
  const int c8 = lane16 * 8;
  const int r = tid >> 4;
  const int steps = (spatial + kTS - 1) / kTS;

  // Raw rows of one step in registers: activated and stored to the other LDS buffer at the
  // end of the step before the one that reads them.
  // beta's raw bits (fp32 for kSplit 3, the beta_f32 launch; else bf16 in the low half), turned
  // into a float only when the step is activated, so no wait follows the loads
  (void)beta_f32;
  u32x4 kraw, vraw;
  uint32_t braw;
  auto load_step = [&](int step, u32x4& kr, u32x4& vr, uint32_t& br) __attribute__((always_inline)) {
    const int s = step * kTS + r;
    if (s < spatial) {
      kr = *reinterpret_cast<const u32x4*>(kv.at(f, h, s) + c8);
      vr = *reinterpret_cast<const u32x4*>(vv.at(f, h, s) + c8);
      const int64_t bo = f * b_sf + h * b_sh + s * b_ss;
      if constexpr (kSplit == 3)
        br = static_cast<const uint32_t*>(beta)[bo];
      else
        br = static_cast<const uint16_t*>(beta)[bo];
    } else {
      kr = u32x4{0, 0, 0, 0};
      vr = u32x4{0, 0, 0, 0};
      br = 0u;
    }
  };
  // Each rounding to bf16 is the packing conversion (RNE); the packed words are the LDS
  // tiles and, unpacked, the exact bf16 values the next step of the arithmetic uses.
  auto store_step = [&](int buf) __attribute__((always_inline)) {
    float kf[8], vf[8];
    unpack8(kraw, kf);
    unpack8(vraw, vf);
    if (activate) {
      activate8_f32(kf, true);
      activate8_f32(vf, false);
    }
    // The packed words are made opaque so that the values are taken back out of them (one
    // shift or mask each) rather than rounded again one by one.
    u32x4 kw = pack8(kf);  // k' (bf16)
    asm volatile("" : "+v"(kw));
    unpack8(kw, kf);
    const float b = __uint_as_float(kSplit == 3 ? braw : braw << 16);
    const float b16 = round_bf16(b);
    float prod[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) prod[i] = b * kf[i];  // exact for bf16 beta
    u32x4 hw = pack8(prod);                             // hi = bf16(prod)
    asm volatile("" : "+v"(hw));
    float hi[8];
    unpack8(hw, hi);
#pragma unroll
    for (int i = 0; i < 8; ++i) prod[i] -= hi[i];       // remainder, exact
    uint16_t* row = &lds[buf][0][r * kRow + c8];
    *reinterpret_cast<u32x4*>(row) = kw;
    *reinterpret_cast<u32x4*>(row + kTile) = hw;
    if constexpr (kSplit == 2) {
      *reinterpret_cast<u32x4*>(row + 2 * kTile) = pack8(prod);  // representable for bf16 beta
    } else {
      const u32x4 mw = pack8(prod);
      float mid[8];
      unpack8(mw, mid);
#pragma unroll
      for (int i = 0; i < 8; ++i) prod[i] -= mid[i];
      *reinterpret_cast<u32x4*>(row + 2 * kTile) = mw;
      *reinterpret_cast<u32x4*>(row + 3 * kTile) = pack8(prod);
    }
    u32x4 vw = pack8(vf);  // v' (bf16)
    asm volatile("" : "+v"(vw));
    unpack8(vw, vf);
#pragma unroll
    for (int i = 0; i < 8; ++i) vf[i] *= b16;
    *reinterpret_cast<u32x4*>(row + (1 + kSplit) * kTile) = pack8(vf);  // bf16(v'·bf16(beta))
  };

  f32x4 accA[4][2], accB[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      accA[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
      accB[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

  // transpose-read fragment: lane (g = lane/16, l = lane%16) gets tokens 8g..8g+7 of channel
  // c0 + l. Both MFMA operands use this same token assignment, so every token pairs with
  // itself whatever order the instruction consumes its K slots in.
  const int g = lane >> 4;
  const int tr_row = 8 * g + (lane16 >> 2);
  const int tr_col = 4 * (lane16 & 3);
  auto frag = [&](const uint16_t* tile, int c0) {
    const bf16x4_t lo = lds_read_tr(tile + tr_row * kRow + c0 + tr_col);
    const bf16x4_t hi = lds_read_tr(tile + (tr_row + 4) * kRow + c0 + tr_col);
    return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  };

  // The raw rows of step s + 1 were loaded at the end of step s - 1 (right after step s's rows
  // were activated), so their latency is covered by a whole step, not only its MFMAs.
  load_step(0, kraw, vraw, braw);
  store_step(0);
  if (steps > 1) load_step(1, kraw, vraw, braw);
  __syncthreads();
  for (int step = 0; step < steps; ++step) {
    const int buf = step & 1;
    const bool more = step + 1 < steps;
    const uint16_t* tk = lds[buf][0];
    const uint16_t* tv = lds[buf][1 + kSplit];
    bf16x8 kn[2], pn[kSplit][2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      kn[nt] = frag(tk, wn * 32 + nt * 16);
#pragma unroll
      for (int t = 0; t < kSplit; ++t) pn[t][nt] = frag(lds[buf][1 + t], wn * 32 + nt * 16);
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const bf16x8 km = frag(tk, wm * 64 + mt * 16);
      const bf16x8 vm = frag(tv, wm * 64 + mt * 16);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
        for (int t = 0; t < kSplit; ++t)
          accA[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(km, pn[t][nt], accA[mt][nt], 0, 0, 0);
        accB[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vm, kn[nt], accB[mt][nt], 0, 0, 0);
      }
    }
    if (more) store_step(buf ^ 1);
    if (step + 2 < steps) load_step(step + 2, kraw, vraw, braw);
    __syncthreads();
  }

  // ---- epilogue: A = (A' + A'ᵀ) / 2 through LDS; B rounded to bf16 ----
  float* sA = reinterpret_cast<float*>(&lds[0][0][0]);  // [128][129] fp32 (66 KB, fits)
  constexpr int kLd = 129;
  const int row_base = (lane >> 4) * 4;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = wm * 64 + mt * 16 + row_base + v;
        const int j = wn * 32 + nt * 16 + lane16;
        sA[i * kLd + j] = accA[mt][nt][v];
      }
  __syncthreads();
  float* An = A + static_cast<int64_t>(fh) * kD * kD;
  for (int idx = tid; idx < kD * kD; idx += kStThreads) {
    const int i = idx >> 7, j = idx & 127;
    An[idx] = (sA[i * kLd + j] + sA[j * kLd + i]) * 0.5f;
  }
  __syncthreads();
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = wm * 64 + mt * 16 + row_base + v;
        const int j = wn * 32 + nt * 16 + lane16;
        sA[i * kLd + j] = round_bf16(accB[mt][nt][v]);
      }
  __syncthreads();
  float* Bn = B + static_cast<int64_t>(fh) * kD * kD;
  for (int idx = tid; idx < kD * kD; idx += kStThreads) Bn[idx] = sA[(idx >> 7) * kLd + (idx & 127)];
}

// ------------------------------------------------------------------- factors ----
// One workgroup per matrix. Thread (ti, tj) = (tid / 16, tid % 16) keeps the 8x8 block
// rows 8ti.., cols 8tj.. of M = I + A in registers; Gauss-Jordan without pivoting (I + A is
// SPD, every pivot is >= 1), one pivot per step, pivot row/column broadcast through a
// double-buffered LDS line so each step needs a single barrier (a thread writes the line
// of step k + 1 only after the barrier of step k, by which time every thread has read the
// line of step k - 1 that it overwrites).
// J = B M^-1 then runs on v_mfma_f32_16x16x4_f32 (lane l: A = B[i = l % 16][k slot l / 16],
// B = M^-1[k slot l / 16][j = l % 16], accumulator rows 4 (l / 16) + v, column l % 16), M^-1
// staged in LDS. Wave w computes J rows [32 w, 32 w + 32) as two 16-row tiles mt by eight
// 16-column tiles nt, where MFMA column c of tile nt is J column 8 c + nt: a lane's eight
// B operands of one k are the 8 consecutive floats M^-1[k][8 c .. 8 c + 8) (two 16-byte LDS
// reads) and its results for one row are 8 consecutive J columns (two 16-byte stores). K runs
// in the order k = 16 q + 4 g + s (chunk q < 8, lane group g, element s < 4), so lane (i, g)
// takes its A operands of chunk q from one 16-byte load B[i][16 q + 4 g .. + 4).
__global__ void __launch_bounds__(256, 2)
vda_factors_kernel(const float* __restrict__ A, const float* __restrict__ B,
                   const float* __restrict__ alpha, float* __restrict__ T,
                   float* __restrict__ J) {
  __shared__ float prow[2][kD], pcol[2][kD];
  __shared__ __attribute__((aligned(16))) float minv[kD * (kD + 4)];
  constexpr int kLd = kD + 4;
  const int64_t mat = static_cast<int64_t>(blockIdx.x) * kD * kD;
  const int tid = threadIdx.x, ti = tid >> 4, tj = tid & 15;
  const int i0 = ti * 8, j0 = tj * 8;
  // the lane's A operands of J = B M^-1 (rows 32 w + 16 mt + li, chunks q), loaded now so
  // that their latency passes under the elimination
  const int wave = tid >> 6, li = tid & 15, lg = (tid >> 4) & 3;
  f32x4 bq[2][8];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int q = 0; q < 8; ++q)
      bq[mt][q] = *reinterpret_cast<const f32x4*>(B + mat + (32 * wave + 16 * mt + li) * kD +
                                                  16 * q + 4 * lg);
  float m[8][8];
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(A + mat + (i0 + r) * kD + j0);
    const f32x4 b = *reinterpret_cast<const f32x4*>(A + mat + (i0 + r) * kD + j0 + 4);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      m[r][c] = a[c];
      m[r][c + 4] = b[c];
    }
  }
  if (ti == tj) {
#pragma unroll
    for (int r = 0; r < 8; ++r) m[r][r] += 1.0f;
  }
  // Pivot k = 8 kb + kr: kb is the runtime loop, kr is unrolled, so the pivot row / column
  // inside a thread's 8 x 8 block are compile-time rows / columns and only those 8 + 8
  // elements need a select; the rest is one fma each.
#pragma unroll 1
  for (int kb = 0; kb < kD / 8; ++kb) {
    const bool row_owner = ti == kb, col_owner = tj == kb;
#pragma unroll
    for (int kr = 0; kr < 8; ++kr) {
      const int k = kb * 8 + kr;
      const int buf = kr & 1;
      if (row_owner) {
#pragma unroll
        for (int c = 0; c < 8; ++c) prow[buf][j0 + c] = m[kr][c];
      }
      if (col_owner) {
#pragma unroll
        for (int r = 0; r < 8; ++r) pcol[buf][i0 + r] = m[r][kr];
      }
      __syncthreads();
      const float rp = 1.0f / prow[buf][k];
      float pr[8], pc[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) pr[c] = prow[buf][j0 + c] * rp;
#pragma unroll
      for (int r = 0; r < 8; ++r) pc[r] = pcol[buf][i0 + r];
#pragma unroll
      for (int r = 0; r < 8; ++r) {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const float upd = m[r][c] - pc[r] * pr[c];
          if (r == kr && c == kr) {
            m[r][c] = row_owner && col_owner ? rp : (row_owner ? pr[c] : (col_owner ? -pc[r] * rp : upd));
          } else if (r == kr) {
            m[r][c] = row_owner ? pr[c] : upd;
          } else if (c == kr) {
            m[r][c] = col_owner ? -pc[r] * rp : upd;
          } else {
            m[r][c] = upd;
          }
        }
      }
    }
  }
  // T = diag(alpha) M^-1 (row i scaled by alpha[i]); M^-1 staged in LDS for J = B M^-1.
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const float a = alpha != nullptr ? alpha[static_cast<int64_t>(blockIdx.x) * kD + i0 + r] : 1.0f;
    f32x4 lo, hi;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      lo[c] = a * m[r][c];
      hi[c] = a * m[r][c + 4];
    }
    *reinterpret_cast<f32x4*>(T + mat + (i0 + r) * kD + j0) = lo;
    *reinterpret_cast<f32x4*>(T + mat + (i0 + r) * kD + j0 + 4) = hi;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      lo[c] = m[r][c];
      hi[c] = m[r][c + 4];
    }
    *reinterpret_cast<f32x4*>(&minv[(i0 + r) * kLd + j0]) = lo;
    *reinterpret_cast<f32x4*>(&minv[(i0 + r) * kLd + j0 + 4]) = hi;
  }
  __syncthreads();
  f32x4 acc[2][8];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < 8; ++q) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const float* xr = &minv[(16 * q + 4 * lg + s) * kLd + 8 * li];
      const f32x4 x0 = *reinterpret_cast<const f32x4*>(xr);
      const f32x4 x1 = *reinterpret_cast<const f32x4*>(xr + 4);
#pragma unroll
      for (int nt = 0; nt < 8; ++nt)
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(bq[mt][q][s], nt < 4 ? x0[nt] : x1[nt - 4],
                                                             acc[mt][nt], 0, 0, 0);
    }
  }
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float* dst = J + mat + (32 * wave + 16 * mt + 4 * lg + v) * kD + 8 * li;
      *reinterpret_cast<f32x4*>(dst) = f32x4{acc[mt][0][v], acc[mt][1][v], acc[mt][2][v], acc[mt][3][v]};
      *reinterpret_cast<f32x4*>(dst + 4) = f32x4{acc[mt][4][v], acc[mt][5][v], acc[mt][6][v], acc[mt][7][v]};
    }
}

// --------------------------------------------------------- affine recurrence ----
// state[16 x 128] <- state @ T + J over a sequence of frames. Workgroup = (row block of 16
// state rows, head, direction[, chunk]); 8 waves, wave w owns output columns [16w, 16w+16).
// state @ T runs on v_mfma_f32_16x16x4_f32: lane l feeds A = state[l%16][4k + l/16] and
// B = T[4k + l/16][n0 + l%16]; the accumulator holds rows (l/16)*4 + v, column n0 + l%16.
// The B operands of a step (the wave's 128 x 16 slice of T, 32 values per lane) and the
// lane's 4 injection values are loaded straight into registers one step ahead: T and J do
// not depend on the state, so only the MFMA chain and the state exchange through LDS are
// serial. With 8 KB of LDS and at most 96 VGPRs, five waves share a SIMD and every row
// block, head and direction of a 40-head launch runs at once.
enum RecurMode : int { kScan = 0, kCompose = 1 };

constexpr int kRecWaves = 8;
constexpr int kRecThreads = 64 * kRecWaves;

template <int kMode>
__global__ void __launch_bounds__(kRecThreads) __attribute__((amdgpu_waves_per_eu(5)))
vda_recur_kernel(const float* __restrict__ Tm, const float* __restrict__ Jm, int heads,
                 const int* __restrict__ starts, const int* __restrict__ ends, int chunks,
                 const float* __restrict__ seed, int per_direction, float* __restrict__ out0,
                 float* __restrict__ out1) {
  // state rows; compose keeps a second state (the accumulated injection b)
  __shared__ __attribute__((aligned(16))) float sS[kMode == kCompose ? 2 : 1][16 * 132];
  // 1-D grid of (row block, head[, chunk], direction), row block fastest: the 8 row blocks
  // that read one T run on one XCD, so its L2 fetches each T once per step.
  const int logical = xcd_contiguous(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
  const int rb = logical % (kD / 16);  // 16-row block
  const int ys = logical / (kD / 16);
  const int ny = kMode == kScan ? heads : static_cast<int>(gridDim.x) / (kD / 16) / 2;
  const int by = ys % ny;
  const int dir = ys / ny;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r0 = rb * 16;
  int h, c = 0;
  if (kMode == kScan) {
    h = by;
  } else {
    h = by % heads;
    c = by / heads;
  }
  const int64_t mat = kD * kD;
  // number of frames in the sequence and the frame index of step t
  int n_steps, lo = 0, hi = 0;
  if (kMode == kScan) {
    n_steps = chunks;
  } else {
    lo = starts[c];
    hi = ends[c];
    n_steps = hi - lo;
  }
  auto frame_of = [&](int t) {
    if (kMode == kScan) return dir == 0 ? t : chunks - 1 - t;
    return dir == 0 ? lo + t : hi - 1 - t;
  };
  // input matrix of frame/chunk x for head h: per-direction composed maps [2, C, H] or
  // per-frame factors [F, H] shared by both directions; scan outputs are always [2, C, H].
  auto in_index = [&](int x) -> int64_t {
    if (kMode == kScan && per_direction) return (static_cast<int64_t>(dir) * chunks + x) * heads + h;
    return static_cast<int64_t>(x) * heads + h;
  };
  auto out_index = [&](int x) -> int64_t {
    return (static_cast<int64_t>(dir) * chunks + x) * heads + h;
  };
  // initial state: scan -> seed or zero; compose -> m = I (sS[0]), b = 0 (sS[1])
  for (int idx = tid; idx < 16 * kD; idx += kRecThreads) {
    const int i = idx >> 7, j = idx & 127;
    float s0;
    if (kMode == kScan) {
      s0 = seed != nullptr ? seed[(static_cast<int64_t>(h) * kD + r0 + i) * kD + j] : 0.f;
    } else {
      s0 = (r0 + i) == j ? 1.f : 0.f;
      sS[kMode == kCompose ? 1 : 0][i * 132 + j] = 0.f;
    }
    sS[0][i * 132 + j] = s0;
  }
  const int n0 = wave * 16;
  const int frow = lane & 15, fk = lane >> 4;
  const int row_base = (lane >> 4) * 4;
  constexpr int kStates = kMode == kCompose ? 2 : 1;
  const int inj = kMode == kCompose ? 1 : 0;  // the state that receives the injection
  float tcur[32], tnext[32], jcur[4], jnext[4];
  // Buffer loads: the lane's offset is one VGPR, the matrix base and the row step are
  // uniform (SGPRs), so the 36 loads of a step need no 64-bit address registers.
  const int t_off = (fk * kD + n0 + frow) * 4;
  const int j_off = ((r0 + row_base) * kD + n0 + frow) * 4;
  auto load_step = [&](int t, float (&tb)[32], float (&jb)[4]) __attribute__((always_inline)) {
    const int64_t m = in_index(frame_of(t)) * mat;
    const __amdgpu_buffer_rsrc_t tr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(Tm + m), 0, kD * kD * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t jr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(Jm + m), 0, kD * kD * 4, 0x00020000);
#pragma unroll
    for (int kk = 0; kk < kD / 4; ++kk)
      tb[kk] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(tr, t_off, kk * 4 * kD * 4, 0));
#pragma unroll
    for (int v = 0; v < 4; ++v)
      jb[v] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(jr, j_off, v * kD * 4, 0));
  };
  if (n_steps > 0) load_step(0, tcur, jcur);
  __syncthreads();  // initial state written
  for (int t = 0; t < n_steps; ++t) {
    const int x = frame_of(t);
    if (t + 1 < n_steps) load_step(t + 1, tnext, jnext);
    f32x4 acc[2];  // [state m / b]
#pragma unroll
    for (int a = 0; a < 2; ++a) acc[a] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < kD / 4; ++kk) {
      const int krow = 4 * kk + fk;
#pragma unroll
      for (int a = 0; a < kStates; ++a)
        acc[a] = __builtin_amdgcn_mfma_f32_16x16x4f32(sS[a][frow * 132 + krow], tcur[kk], acc[a],
                                                      0, 0, 0);
    }
    __syncthreads();  // all waves done reading sS before it is overwritten
#pragma unroll
    for (int a = 0; a < kStates; ++a)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int i = row_base + v;
        const int j = n0 + frow;
        float y = acc[a][v];
        if (a == inj) y += jcur[v];
        sS[a][i * 132 + j] = y;
        if (kMode == kScan) out0[out_index(x) * mat + (r0 + i) * kD + j] = y;
      }
    __syncthreads();  // the new state is complete
#pragma unroll
    for (int kk = 0; kk < kD / 4; ++kk) tcur[kk] = tnext[kk];
#pragma unroll
    for (int v = 0; v < 4; ++v) jcur[v] = jnext[v];
  }
  if constexpr (kMode == kCompose) {
    __syncthreads();
    const int64_t o = ((static_cast<int64_t>(dir) * chunks + c) * heads + h) * mat;
    for (int idx = tid; idx < 16 * kD; idx += kRecThreads) {
      const int i = idx >> 7, j = idx & 127;
      out0[o + (r0 + i) * kD + j] = sS[0][i * 132 + j];
      out1[o + (r0 + i) * kD + j] = sS[1][i * 132 + j];
    }
  }
}

// ---------------------------------------------------------------- short conv ----
// paper_prepare with the linear branch's separable short conv: depthwise 5x5 spatial conv
// per frame (zero padding 2, no bias; LinearAttentionSepConv.spatial, features.py:175-196),
// its output rounded to bf16 as the reference's bf16 conv2d returns it, then the depthwise
// 5-tap temporal conv across frames (zero padding 2) in fp32, SiLU, L2 over the head's 128
// channels, one rounding and the frame-major [F, H, S, 128] store (vdn_temporal_conv_act,
// paper_sglang.py:165-203).
// One workgroup per (head, 8 x 8 spatial tile) walks the frames in order. A frame's 12 x 12
// input positions (the tile and its 2-position halo) x 128 channels come into LDS by
// buffer-resource DMA, double-buffered; positions outside the frame read as zero. Wave w
// computes the 4 x 4 position block (w / 2, w % 2) of the tile and lane l holds channels
// 2l, 2l + 1, so the LDS reads of one position are 256 contiguous bytes. The rounded
// spatial output of the last five frames stays in registers: when frame t is done, frame
// t - 2 gets its temporal taps, SiLU and L2 (one wave reduction per position) and is
// stored, 256 contiguous bytes per position.
constexpr int kCvTile = 8;
constexpr int kCvHalo = kCvTile + 4;
constexpr int kCvPos = kCvHalo * kCvHalo;       // 144 staged positions
constexpr int kCvBuf = kCvPos * kD * 2;         // 36864 bytes per frame

// LDS DMA through a buffer resource as inline asm: lane l's 16 bytes at voffset land at LDS
// byte lds_base + 16 l. The compiler does not see it as an LDS write, so the reads of the
// current frame's buffer do not wait for the next frame's DMA into the other buffer (with the
// builtin they would); the kernel waits on vmcnt itself before its barrier. M0 is an input
// operand ("{m0}"): the compiler writes it and knows it is live; the s_nop is the wait state
// between an M0 write and an LDS DMA that reads it.
__device__ __forceinline__ void cv_buffer_to_lds16(__amdgpu_buffer_rsrc_t r, uint32_t voffset,
                                                   uint32_t lds_base) {
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               ::"v"(voffset), "s"(r), "{m0}"(lds_base) : "memory");
}

// Sum over the 64 lanes of a wave (every lane gets the same bits).
// Total over the wave, the same bits in every lane: the 16-lane row sums r0..r3 (sum16),
// then DPP row_bcast:15 (rows 1-3 add lane 15 of the row before them; row 0 has no source
// row) and row_bcast:31 (rows 2 and 3 add lane 31). Lane 63 then holds (r3 + r2) + (r1 + r0):
// row 3 added lane 47 (r2) and then lane 31 (r1 + r0, row 1 having added lane 15).
// v_readlane makes it wave-uniform; the other lanes' partial sums are never read. The same sum as sum_quad_rows(sum16(x))
// (addition commutes), without the register copies that the permlane swaps need.
__device__ __forceinline__ float wave_sum(float x) {
  x = sum16(x);
  x += dpp_f32<0x142>(x);
  x += dpp_f32<0x143>(x);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 63));
}

__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
vda_conv_prepare_kernel(const uint16_t* __restrict__ tokens, int64_t row_stride,
                        int64_t head_stride, int frames, int fh, int fw, int heads, int tiles_x,
                        const void* __restrict__ w_sp, const void* __restrict__ w_tm, int l2norm,
                        uint16_t* __restrict__ out) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[2][kCvBuf];
  const int h = blockIdx.x % heads;
  const int tile = blockIdx.x / heads;
  const int ty = tile / tiles_x, tx = tile % tiles_x;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: LDS bases go in M0
  const int spatial = fh * fw;

  // ---- DMA: 36 wave instructions per frame, 9 per wave; instruction i loads staged
  // positions 4i .. 4i + 3 (16 lanes each) into LDS bytes [1024 i, 1024 i + 1024) ----
  uint32_t voff[9];
#pragma unroll
  for (int j = 0; j < 9; ++j) {
    const int q = (wave * 9 + j) * 4 + (lane >> 4);
    const int y = ty * kCvTile + q / kCvHalo - 2, x = tx * kCvTile + q % kCvHalo - 2;
    const bool in = y >= 0 && y < fh && x >= 0 && x < fw;
    voff[j] = in ? static_cast<uint32_t>(((y * fw + x) * row_stride + h * head_stride) * 2 +
                                         (lane & 15) * 16)
                 : 0x80000000u;   // past the resource's end: reads as zero
  }
  const uint32_t frame_bytes = static_cast<uint32_t>(spatial * row_stride * 2);
  auto dma_frame = [&](int f, int buf) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(tokens + static_cast<int64_t>(f) * spatial * row_stride), 0,
        static_cast<int>(frame_bytes), 0x00020000);
    const uint32_t base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
        (__attribute__((address_space(3))) void*)(&lds[buf][0])));
#pragma unroll
    for (int j = 0; j < 9; ++j) cv_buffer_to_lds16(r, voff[j], base + (wave * 9 + j) * 1024);
  };

  // ---- bf16 weights of channels c0 = 128 h + 2 lane (ch 0) and c0 + 1 (ch 1). Taps go in
  // pairs through v_dot2c_f32_bf16 (two bf16 products added to an fp32 sum): per channel and
  // tap row i, the words (w[i][0], w[i][1]) and (w[i][2], w[i][3]) and tap 4 as a float; the
  // temporal taps as (w[0], w[1]), (w[2], w[3]) and w[4]. ----
  const int c0 = h * kD + 2 * lane;
  const uint16_t* wsp16 = static_cast<const uint16_t*>(w_sp);
  const uint16_t* wtm16 = static_cast<const uint16_t*>(w_tm);
  auto word = [](const uint16_t* p) {
    return static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 16);
  };
  uint32_t wsp2[2][5][2], wtm2[2][2];
  float wsp4[2][5], wtm4[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const uint16_t* ws = wsp16 + (c0 + c) * 25;
#pragma unroll
    for (int i = 0; i < 5; ++i) {
      wsp2[c][i][0] = word(ws + 5 * i);
      wsp2[c][i][1] = word(ws + 5 * i + 2);
      wsp4[c][i] = bf16_bits_to_f32(ws[5 * i + 4]);
    }
    const uint16_t* wt = wtm16 + (c0 + c) * 5;
    wtm2[c][0] = word(wt);
    wtm2[c][1] = word(wt + 2);
    wtm4[c] = bf16_bits_to_f32(wt[4]);
  }
  // (x.ch c of word a, x.ch c of word b) as one bf16 pair: v_perm_b32 byte selects
  auto pair = [](uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_perm(b, a, c ? 0x07060302u : 0x05040100u);
  };
  auto dot2 = [](uint32_t x, uint32_t w, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x),
                                           __builtin_bit_cast(bf16x2, w), acc, false);
  };
  auto chan = [](uint32_t w, int c) {
    return __uint_as_float(c ? w & 0xffff0000u : w << 16);
  };

  const int by = wave >> 1, bx = wave & 1;
  // Byte offsets of the lane's 16 output words in a (frame, head) slice of `out` (32-bit: a
  // slice spans spatial * 256 bytes); a position outside the frame gets an offset past the
  // slice, where the buffer store is dropped.
  uint32_t out_off[16];
#pragma unroll
  for (int p = 0; p < 16; ++p) {
    const int yy = ty * kCvTile + by * 4 + (p >> 2), xx = tx * kCvTile + bx * 4 + (p & 3);
    out_off[p] = yy < fh && xx < fw
                     ? static_cast<uint32_t>(((yy * fw + xx) * kD + 2 * lane) * 2)
                     : 0x80000000u;
  }
  // spatial outputs (bf16 channel pairs) of the last five frames, frame t in slot t % 5
  uint32_t win[5][16];
#pragma unroll
  for (int k = 0; k < 5; ++k)
#pragma unroll
    for (int p = 0; p < 16; ++p) win[k][p] = 0u;

  // Frame t's spatial output goes to slot t % 5 of win; the frame loop is unrolled five
  // times so that every slot index is a constant (no register rotation per frame).
  auto step = [&](int t, auto phase_tag) __attribute__((always_inline)) {
    constexpr int P = decltype(phase_tag)::value;   // t % 5
    const int buf = t & 1;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();   // frame t is in LDS; every wave is done with frame t - 1's buffer
    if (t + 1 < frames) dma_frame(t + 1, buf ^ 1);
    if (t < frames) {
      float acc[4][4][2];   // set by each output's first tap row (i == 0)
      const uint8_t* src = &lds[buf][((by * 4) * kCvHalo + bx * 4) * 256 + lane * 4];
#pragma unroll
      for (int ir = 0; ir < 8; ++ir) {
        // one input row in flight at a time: the scheduler would otherwise hoist all 64 LDS
        // reads (and their pairs) ahead of the arithmetic
        __builtin_amdgcn_sched_barrier(0);
        uint32_t xw[8];
#pragma unroll
        for (int ic = 0; ic < 8; ++ic)
          xw[ic] = *reinterpret_cast<const uint32_t*>(src + (ir * kCvHalo + ic) * 256);
        // per channel: horizontally adjacent positions (ic, ic + 1) as one bf16 pair, and
        // positions 4..7 (tap 4 of the four outputs) as floats
        uint32_t xp[2][7];
        float x4[2][4];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
#pragma unroll
          for (int ic = 0; ic < 7; ++ic) xp[c][ic] = pair(xw[ic], xw[ic + 1], c);
#pragma unroll
          for (int ox = 0; ox < 4; ++ox) x4[c][ox] = chan(xw[ox + 4], c);
        }
#pragma unroll
        for (int oy = 0; oy < 4; ++oy) {
          const int i = ir - oy;
          if (i < 0 || i > 4) continue;
#pragma unroll
          for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int ox = 0; ox < 4; ++ox) {
              if (i == 0) {
                // the first row starts the sum with its tap-4 product (exact in fp32: two
                // bf16 factors), so no dot starts from a zeroed register
                float a = x4[c][ox] * wsp4[c][i];
                a = dot2(xp[c][ox], wsp2[c][i][0], a);
                acc[oy][ox][c] = dot2(xp[c][ox + 2], wsp2[c][i][1], a);
              } else {
                float a = dot2(xp[c][ox], wsp2[c][i][0], acc[oy][ox][c]);
                a = dot2(xp[c][ox + 2], wsp2[c][i][1], a);
                acc[oy][ox][c] = __builtin_fmaf(x4[c][ox], wsp4[c][i], a);
              }
            }
        }
      }
#pragma unroll
      for (int oy = 0; oy < 4; ++oy)
#pragma unroll
        for (int ox = 0; ox < 4; ++ox) win[P][oy * 4 + ox] = pack_bf16x2(acc[oy][ox][0], acc[oy][ox][1]);
    } else {
#pragma unroll
      for (int p = 0; p < 16; ++p) win[P][p] = 0u;
    }
    if (t < 2) return;
    // ---- frame o = t - 2: temporal taps, SiLU, L2, store ----
    const int o = t - 2;
    uint16_t* out_f = out + (static_cast<int64_t>(o) * heads + h) * spatial * kD;
    float y[16][2];
#pragma unroll
    for (int p = 0; p < 16; ++p)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        // frame o + 4's product (exact in fp32), then frames o .. o + 3 in pairs (o, o + 1),
        // (o + 2, o + 3)
        float a = chan(win[P][p], c) * wtm4[c];
        a = dot2(pair(win[(P + 1) % 5][p], win[(P + 2) % 5][p], c), wtm2[c][0], a);
        a = dot2(pair(win[(P + 3) % 5][p], win[(P + 4) % 5][p], c), wtm2[c][1], a);
        y[p][c] = silu(a);
      }
    if (l2norm) {
      // the 16 positions' sums over the head's 128 channels, reduced side by side so that
      // their cross-lane steps fill each other's wait states
      float ss[16];
#pragma unroll
      for (int p = 0; p < 16; ++p) ss[p] = y[p][0] * y[p][0] + y[p][1] * y[p][1];
#pragma unroll
      for (int p = 0; p < 16; ++p) ss[p] = wave_sum(ss[p]);
#pragma unroll
      for (int p = 0; p < 16; ++p) {
        const float inv = __builtin_amdgcn_rsqf(fmaxf(ss[p], 1e-12f));
        y[p][0] *= inv;
        y[p][1] *= inv;
      }
    }
    const __amdgpu_buffer_rsrc_t orsrc =
        __builtin_amdgcn_make_buffer_rsrc(out_f, 0, spatial * kD * 2, 0x00020000);
#pragma unroll
    for (int p = 0; p < 16; ++p)
      __builtin_amdgcn_raw_buffer_store_b32(pack_bf16x2(y[p][0], y[p][1]), orsrc, out_off[p], 0, 0);
  };
  if (frames > 0) dma_frame(0, 0);
  for (int t0 = 0; t0 < frames + 2; t0 += 5) {
    step(t0, std::integral_constant<int, 0>{});
    if (t0 + 1 >= frames + 2) break;
    step(t0 + 1, std::integral_constant<int, 1>{});
    if (t0 + 2 >= frames + 2) break;
    step(t0 + 2, std::integral_constant<int, 2>{});
    if (t0 + 3 >= frames + 2) break;
    step(t0 + 3, std::integral_constant<int, 3>{});
    if (t0 + 4 >= frames + 2) break;
    step(t0 + 4, std::integral_constant<int, 4>{});
  }
}

// ----------------------------------------------------------------- log prefix ----
// logp[n, h, j] = sum_{u < n} log(max(alpha[u, h, j], 1e-12)), summed in frame order.
__global__ void vda_log_prefix_kernel(const float* __restrict__ alpha, int frames, int hd,
                                      float* __restrict__ logp) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= hd) return;
  float acc = 0.f;
  logp[idx] = 0.f;
  for (int n = 0; n < frames; ++n) {
    acc += logf(fmaxf(alpha[static_cast<int64_t>(n) * hd + idx], 1e-12f));
    logp[static_cast<int64_t>(n + 1) * hd + idx] = acc;
  }
}

// -------------------------------------------------------------------- gather ----
// out[f, h, i, j] = P[before f][h][i][j] * exp(lp[f+1] - lp[bb f])[j]
//                 + R[after f][h][i][j]  * exp(lp[ba f] - lp[f])[j]
// with out-of-range sides reading the text seed (or zero). paper_sglang.py:445-501.
__global__ void __launch_bounds__(256)
vda_gather_kernel(const float* __restrict__ prefix, const float* __restrict__ suffix,
                  const float* __restrict__ logp, const float* __restrict__ text,
                  const int* __restrict__ before, const int* __restrict__ after,
                  const int* __restrict__ has_b, const int* __restrict__ has_a,
                  const int* __restrict__ bridge_b, const int* __restrict__ bridge_a, int heads,
                  int bridge, int out_f32, void* __restrict__ out) {
  const int f = blockIdx.x, h = blockIdx.y;
  const int64_t mat = kD * kD;
  const int fb = before[f], fa = after[f];
  const bool hb = has_b[f] != 0, ha = has_a[f] != 0;
  const int64_t hd = static_cast<int64_t>(heads) * kD;
  for (int idx = threadIdx.x + blockIdx.z * 256; idx < kD * kD; idx += 256 * gridDim.z) {
    const int j = idx & 127;
    float sb, sa;
    const float ts = text != nullptr ? text[h * mat + idx] : 0.f;
    sb = hb ? prefix[(static_cast<int64_t>(fb) * heads + h) * mat + idx] : ts;
    sa = ha ? suffix[(static_cast<int64_t>(fa) * heads + h) * mat + idx] : ts;
    if (bridge) {
      const float lt1 = logp[(f + 1) * hd + h * kD + j];
      const float lt = logp[f * hd + h * kD + j];
      const float lbb = logp[bridge_b[f] * hd + h * kD + j];
      const float lba = logp[bridge_a[f] * hd + h * kD + j];
      sb = sb * expf(lt1 - lbb);
      sa = sa * expf(lba - lt);
    }
    const float y = sb + sa;
    const int64_t o = (static_cast<int64_t>(f) * heads + h) * mat + idx;
    if (out_f32)
      static_cast<float*>(out)[o] = y;
    else
      static_cast<uint16_t*>(out)[o] = f32_to_bf16_bits(y);
  }
}

// ------------------------------------------------------------ readout + norm ----
// RMSNorm(d)·w·gate of 8 channels held by one lane of a 16-lane token group
// (paper_sglang.py:398-403): y * (1 / sqrt(mean(y^2) + eps)) * w * g, fp32, one rounding.
// MXFP8 destination of the readout (instead of bf16 rows): token row n = f * S + s, head h
// fills 128-column chunk chunk0 + h of codes [rows, kp] and its SWIZZLE_32_4_4 scales.
struct MxDst {
  uint8_t* codes;
  uint8_t* scales;
  int64_t kp;
  int chunk0;
};

// RMSNorm(y)·w·gate of one lane's 8 values, rounded to bf16 (as stored by the bf16 form).
// inv_dim = 1 / head_dim, a power of two: rows are 128 wide, channels past head_dim hold
// zeros, and the mean of squares is over head_dim channels.
__device__ __forceinline__ void norm_gate8(const float* y, const float* w, const u32x4 graw,
                                           float eps, float inv_dim, float* o) {
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss += y[i] * y[i];
  ss = sum16(ss);
  const float inv = 1.0f / sqrtf(ss * inv_dim + eps);
  float gv[8];
  unpack8(graw, gv);
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = round_bf16(y[i] * inv * w[i] * gv[i]);
}

__device__ __forceinline__ void norm_gate_store8(float* y, const float* w, const uint16_t* gsrc,
                                                 uint16_t* dst, float eps, float inv_dim) {
  float o[8];
  norm_gate8(y, w, *reinterpret_cast<const u32x4*>(gsrc), eps, inv_dim, o);
  *reinterpret_cast<u32x4*>(dst) = pack8(o);
}

// Readout, transposed: Y' = state · q'ᵀ, i.e. Y'[c][t] = y[t][c] = q'[t] · state[c].
// A workgroup of kRoWaves waves takes one (frame, head) and a range of the frame's 16-token
// groups. It stages the 128 x 128 state (and, for a formed gate, head h's 128 x 128 up
// weights) in LDS once; then each wave walks its token groups without barriers.
// For a group, lane l (t = l % 16, g = l / 16) loads channels 32 ks + 8 g .. +8 (ks = 0..3)
// of token t, which is exactly its B operand of v_mfma_f32_16x16x32_bf16 (no LDS round
// trip for q or for the gate's down rows); the A operand is 16 LDS state rows. The LDS rows
// are permuted (ro_row) so that accumulator mt, element v of lane group g holds output
// channel 32 (mt / 2) + 8 g + 4 (mt % 2) + v of token t: a lane's accumulators 2j, 2j + 1
// are the 8 contiguous channels 32 j + 8 g .. +8, read (gate) and written (output) as 16
// bytes, the same footprint as its q loads. The SiLU/L2 of q, the gate's bias and sigmoid,
// RMSNorm·w·gate and the MXFP8 quantization all run in those registers: a per-token sum or
// a per-32-block max needs only the four lanes t, t + 16, t + 32, t + 48 (two permlane
// swaps), and 32-block b is accumulators 2b, 2b + 1.
constexpr int kRoWaves = 8;
constexpr int kRoThreads = 64 * kRoWaves;
constexpr int kQRow = 136;  // padded bf16 row of the LDS matrices (272 bytes)

// LDS row of output channel c (inverse of the accumulator order above).
__device__ __forceinline__ int ro_row(int c) {
  return 16 * (2 * (c >> 5) + ((c >> 2) & 1)) + 4 * ((c >> 3) & 3) + (c & 3);
}

// The low-rank output gate of the linear branch, formed inside the readout instead of read:
// gate[t, h*128 + c] = bf16(sigmoid(bf16(down[t] . up_w[h*128 + c] + up_b[h*128 + c]))), with
// down [F*S, 128] bf16 rows (row stride d_st), up_w [H*128, 128] bf16, up_b [H*128] bf16.
struct GateProj {
  const uint16_t* down;
  int64_t d_st;
  const uint16_t* up_w;
  const uint16_t* up_b;
};

// acc[mt] += rows 16 mt .. 16 mt + 15 of the LDS matrix m ([row][k], row stride kQRow) times
// the B operands b[ks] (this lane's token, K = 128 in 4 steps of 32).
// The A rows are the same for every token group: `base` is made opaque per call, so the
// compiler reads them from LDS each time instead of keeping all 64 fragments (256 VGPRs)
// in registers across the group loop.
__device__ __forceinline__ void rows_times_tokens(const uint16_t* m, const bf16x8 (&b)[4],
                                                  int t16, int g, f32x4 (&acc)[8]) {
  int base = t16 * kQRow + g * 8;
  asm volatile("" : "+v"(base));
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) {
      const bf16x8 a = *reinterpret_cast<const bf16x8*>(&m[base + mt * 16 * kQRow + ks * 32]);
      acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[ks], acc[mt], 0, 0, 0);
    }
}

// The global operands of one 16-token group in this lane: q channels 32 ks + 8 g .. +8 and,
// for a read gate, gate channels 32 j + 8 g .. +8, or, for a formed gate, the same channels
// of the token's down-projection row (its B operands). A token past the frame reads the
// frame's last token instead: every value of a token stays in its own lanes (the B column of
// its MFMAs and the four lanes of its sums and maxima), and nothing of it is stored.
struct RoLoads {
  u32x4 q[4];
  u32x4 gt[4];
};

// Per-lane row bases of one (frame, head): q and gate rows of token s are at q0 + s * qs and
// g0 + s * gs (elements).
struct RoRows {
  const uint16_t* q0;
  const uint16_t* g0;
  int64_t qs, gs;
};

__device__ __forceinline__ void ro_load(const RoRows& rows, int s, RoLoads& L) {
  const uint16_t* qrow = rows.q0 + s * rows.qs;
  const uint16_t* grow = rows.g0 + s * rows.gs;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    L.q[j] = *reinterpret_cast<const u32x4*>(qrow + j * 32);
    L.gt[j] = *reinterpret_cast<const u32x4*>(grow + j * 32);
  }
}

// Fused readout: q' = bf16(L2(SiLU(q_raw))) (optional), y = bf16(q' · stateᵀ), then
// o = bf16(RMSNorm(y)·w·gate) into bf16 out[f*S + s, h*D + c] or, with kMx, MXFP8 codes and
// scales (token row f*S + s, chunk chunk0 + h). kProj forms the gate from GateProj; else it
// is read from gv. Two workgroups per CU (four waves per SIMD): at most 128 VGPRs.
template <bool kMx, bool kProj>
__global__ void __launch_bounds__(kRoThreads) __attribute__((amdgpu_waves_per_eu(4)))
vda_readout_kernel(View qv, int activate_q, const uint16_t* __restrict__ state,
                   const void* __restrict__ weight, int weight_f32, float eps, float inv_dim,
                   View gv,
                   GateProj gp, uint16_t* __restrict__ out, int64_t o_sf, int64_t o_sh,
                   int64_t o_ss, int spatial, int heads, int parts, MxDst mx) {
  __shared__ __attribute__((aligned(16))) uint16_t sState[kD * kQRow];     // [ro_row(c)][k]
  __shared__ __attribute__((aligned(16))) uint16_t sUp[kProj ? kD * kQRow : 8];
  __shared__ __attribute__((aligned(16))) float sW[kD];                    // [ro_row(c)]
  __shared__ __attribute__((aligned(16))) float sB[kD];
  const int logical = xcd_contiguous(static_cast<int>(blockIdx.x), static_cast<int>(gridDim.x));
  const int h = logical % heads;
  const int fp = logical / heads;
  const int part = fp % parts, f = fp / parts;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int t16 = lane & 15, g = lane >> 4;

  const uint16_t* st = state + (static_cast<int64_t>(f) * heads + h) * kD * kD;
  for (int idx = tid * 8; idx < kD * kD; idx += kRoThreads * 8)
    *reinterpret_cast<u32x4*>(&sState[ro_row(idx >> 7) * kQRow + (idx & 127)]) =
        *reinterpret_cast<const u32x4*>(st + idx);
  if constexpr (kProj) {
    const uint16_t* up = gp.up_w + static_cast<int64_t>(h) * kD * kD;
    for (int idx = tid * 8; idx < kD * kD; idx += kRoThreads * 8)
      *reinterpret_cast<u32x4*>(&sUp[ro_row(idx >> 7) * kQRow + (idx & 127)]) =
          *reinterpret_cast<const u32x4*>(up + idx);
    if (tid < kD) sB[ro_row(tid)] = bf16_bits_to_f32(gp.up_b[h * kD + tid]);
  }
  if (tid < kD)
    sW[ro_row(tid)] = weight_f32 ? static_cast<const float*>(weight)[tid]
                                 : bf16_bits_to_f32(static_cast<const uint16_t*>(weight)[tid]);
  __syncthreads();

  const int groups = (spatial + 15) >> 4;
  const int per = (groups + parts - 1) / parts;
  const int g_end = min(groups, (part + 1) * per);
  const int64_t row0 = static_cast<int64_t>(f) * spatial;
  int grp = part * per + wave;
  const RoRows rows{qv.at(f, h, 0) + g * 8,
                    kProj ? gp.down + row0 * gp.d_st + g * 8 : gv.at(f, h, 0) + g * 8, qv.ss,
                    kProj ? gp.d_st : gv.ss};
  RoLoads cur;
  if (grp < g_end) ro_load(rows, min(grp * 16 + t16, spatial - 1), cur);
  for (; grp < g_end; grp += kRoWaves) {
    const int s = grp * 16 + t16;
    const bool valid = s < spatial;
    // ---- gate (bf16 pairs in the accumulator layout) ----
    uint32_t gate_pk[8][2];
    if constexpr (kProj) {
      bf16x8 db[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) db[ks] = __builtin_bit_cast(bf16x8, cur.gt[ks]);
      f32x4 ag[8];
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) ag[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
      rows_times_tokens(sUp, db, t16, g, ag);
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) {
        const f32x4 b = *reinterpret_cast<const f32x4*>(&sB[mt * 16 + g * 4]);
        float gv4[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) gv4[v] = ag[mt][v] + b[v];
        round_bf16_pair(gv4[0], gv4[1]);
        round_bf16_pair(gv4[2], gv4[3]);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          // sigmoid by the hardware exp2 and reciprocal: a few fp32 ulp from 1 / (1 + exp(-z)),
          // below the bf16 rounding that follows
          gv4[v] = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(gv4[v] * -1.4426950408889634f));
        }
        gate_pk[mt][0] = pack_bf16x2(gv4[0], gv4[1]);
        gate_pk[mt][1] = pack_bf16x2(gv4[2], gv4[3]);
      }
    } else {
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) {
        gate_pk[mt][0] = cur.gt[mt >> 1][2 * (mt & 1)];
        gate_pk[mt][1] = cur.gt[mt >> 1][2 * (mt & 1) + 1];
      }
    }
    bf16x8 qb[4];
    {
      float qf[4][8];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) unpack8(cur.q[ks], qf[ks]);
      if (activate_q) {
        // paper_sglang.py:235-238: y = silu(x); y / sqrt(max(sum y^2, 1e-12))
        float ss = 0.f;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            qf[ks][i] = silu(qf[ks][i]);
            ss += qf[ks][i] * qf[ks][i];
          }
        const float inv = __builtin_amdgcn_rsqf(fmaxf(sum_quad_rows(ss), 1e-12f));
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
          for (int i = 0; i < 8; ++i) qf[ks][i] *= inv;
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) qb[ks] = __builtin_bit_cast(bf16x8, pack8(qf[ks]));
    }
    // ---- readout ----
    f32x4 ay[8];
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) ay[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    rows_times_tokens(sState, qb, t16, g, ay);
    // ---- RMSNorm(y)·w·gate (paper_sglang.py:398-403), rounded to bf16 ----
    // (two values per rounding conversion)
    float ss = 0.f;
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) {
      round_bf16_x4(ay[mt]);
#pragma unroll
      for (int v = 0; v < 4; ++v) ss += ay[mt][v] * ay[mt][v];
    }
    const float inv = 1.0f / sqrtf(sum_quad_rows(ss) * inv_dim + eps);
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) {
      const f32x4 w = *reinterpret_cast<const f32x4*>(&sW[mt * 16 + g * 4]);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const uint32_t pk = gate_pk[mt][v >> 1];
        const float gt = __uint_as_float(v & 1 ? pk & 0xffff0000u : pk << 16);
        ay[mt][v] = ay[mt][v] * inv * w[v] * gt;
      }
      round_bf16_x4(ay[mt]);
    }
    if constexpr (kMx) {
      // 32-block b of the head's 128 channels = accumulators 2b, 2b + 1; this lane's 8 codes
      // of it are channels 32 b + 8 g .. +8
      const int64_t row = row0 + s;
      uint8_t* crow = mx.codes + row * mx.kp + (mx.chunk0 + h) * 128 + g * 8;
      uint32_t word = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        float amax = 0.f;
#pragma unroll
        for (int m = 2 * b; m < 2 * b + 2; ++m)
#pragma unroll
          for (int v = 0; v < 4; ++v) amax = fmaxf(amax, fabsf(ay[m][v]));
        amax = max_quad_rows(amax);
        float sinv;
        const uint32_t byte = e8m0_from_amax(amax, &sinv);
        word |= byte << (8 * b);
        const float sf = e8m0_scale(byte);
        u32x2 c2;
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          const f32x4& y4 = ay[2 * b + m];
          c2[m] = e4m3x4_scaled(y4[0], y4[1], y4[2], y4[3], sf);
        }
        if (valid) *reinterpret_cast<u32x2*>(crow + b * 32) = c2;
      }
      if (valid && g == 0)
        *reinterpret_cast<uint32_t*>(
            mx.scales + swizzled_scale_offset(row, (mx.chunk0 + h) * 4, mx.kp >> 7)) = word;
    } else if (valid) {
      uint16_t* orow = out + f * o_sf + h * o_sh + s * o_ss + g * 8;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        u32x4 o4;
        o4[0] = pack_bf16x2(ay[2 * j][0], ay[2 * j][1]);
        o4[1] = pack_bf16x2(ay[2 * j][2], ay[2 * j][3]);
        o4[2] = pack_bf16x2(ay[2 * j + 1][0], ay[2 * j + 1][1]);
        o4[3] = pack_bf16x2(ay[2 * j + 1][2], ay[2 * j + 1][3]);
        *reinterpret_cast<u32x4*>(orow + j * 32) = o4;
      }
    }
    // the next group's loads (a copy into a second register set held across the MFMAs
    // would not fit the 128-VGPR budget)
    if (grp + kRoWaves < g_end) ro_load(rows, min(s + 16 * kRoWaves, spatial - 1), cur);
  }
}

// Epilogue alone (vdn_linear_epilogue): readout [F, H, S, D] bf16 -> out [F*S, H*D].
__global__ void __launch_bounds__(256)
vda_epilogue_kernel(const uint16_t* __restrict__ readout, const void* __restrict__ weight,
                    int weight_f32, float eps, float inv_dim, View gv,
                    uint16_t* __restrict__ out,
                    int64_t o_sf, int64_t o_sh, int64_t o_ss, int frames, int heads,
                    int spatial) {
  const int lane16 = threadIdx.x & 15;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 16 + (threadIdx.x >> 4);
  if (item >= static_cast<int64_t>(frames) * heads * spatial) return;
  const int s = static_cast<int>(item % spatial);
  const int fh = static_cast<int>(item / spatial);
  const int f = fh / heads, h = fh % heads;
  float y[8], w[8];
  unpack8(*reinterpret_cast<const u32x4*>(readout + item * kD + lane16 * 8), y);
#pragma unroll
  for (int i = 0; i < 8; ++i)
    w[i] = weight_f32 ? static_cast<const float*>(weight)[lane16 * 8 + i]
                      : bf16_bits_to_f32(static_cast<const uint16_t*>(weight)[lane16 * 8 + i]);
  norm_gate_store8(y, w, gv.at(f, h, s) + lane16 * 8,
                   out + f * o_sf + h * o_sh + s * o_ss + lane16 * 8, eps, inv_dim);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
bool valid_head_dim(int d) { return d == 16 || d == 32 || d == 64 || d == 128; }
bool stride8(int64_t s) { return s % 8 == 0; }

}  // namespace
}  // namespace vdn

using namespace vdn;

// Reference: paper_stack.py:30-48 -> paper_sglang.py:211-283 (vdn_silu_l2norm, frame-major).
VDN_API int vdn_vda_prepare(const void* tokens, int64_t n, int heads, int64_t row_stride,
                            int64_t head_stride, int frames, int spatial, int l2norm, int is_f32,
                            void* out, void* stream) {
  const char* name = "vdn_vda_prepare";
  if (tokens == nullptr || out == nullptr) return set_error(kInvalidArgument, "%s: null pointer", name);
  if (n != static_cast<int64_t>(frames) * spatial || heads <= 0 || spatial <= 0)
    return set_error(kInvalidArgument, "%s: tokens must be [frames*spatial, heads, 128]", name);
  if (!is_f32 && (!aligned16(tokens) || !stride8(row_stride) || !stride8(head_stride)))
    return set_error(kInvalidArgument, "%s: bf16 rows need 16-byte alignment", name);
  if (n == 0) return kOk;
  const int64_t items = n * heads;
  auto st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>((items + 15) / 16));
  if (is_f32)
    hipLaunchKernelGGL(vda_prepare_kernel<true>, grid, dim3(256), 0, st, tokens, n, heads,
                       row_stride, head_stride, spatial, l2norm, out);
  else
    hipLaunchKernelGGL(vda_prepare_kernel<false>, grid, dim3(256), 0, st, tokens, n, heads,
                       row_stride, head_stride, spatial, l2norm, out);
  return check_launch(name);
}

// Reference: paper_stack.py:30-48 with a short conv -> LinearAttentionSepConv.spatial
// (features.py:175-196, cudnn depthwise 5x5, bf16 output) + vdn_temporal_conv_act
// (paper_sglang.py:165-203, frame_major = True). tokens [F*S, H, 128] bf16 (row / head
// strides in elements, unit channel stride), token f*S + y*W + x; w_sp [H*128, 5, 5] and
// w_tm [H*128, 5] bf16 (the module in the activation dtype, as the reference's conv2d
// requires); out [F, H, S, 128] bf16.
VDN_API int vdn_vda_conv_prepare(const void* tokens, int heads, int64_t row_stride,
                                 int64_t head_stride, int frames, int frame_h, int frame_w,
                                 const void* w_sp, const void* w_tm, int l2norm, void* out,
                                 void* stream) {
  const char* name = "vdn_vda_conv_prepare";
  if (tokens == nullptr || w_sp == nullptr || w_tm == nullptr || out == nullptr)
    return set_error(kInvalidArgument, "%s: null pointer", name);
  if (heads <= 0 || frames <= 0 || frame_h <= 0 || frame_w <= 0)
    return set_error(kInvalidArgument, "%s: positive heads, frames and frame size required", name);
  if (!aligned16(tokens) || !stride8(row_stride) || !stride8(head_stride) || row_stride <= 0 ||
      head_stride < 0)
    return set_error(kInvalidArgument, "%s: bf16 rows need 16-byte alignment", name);
  const int64_t spatial = static_cast<int64_t>(frame_h) * frame_w;
  if (spatial * row_stride * 2 >= (1ll << 31) ||
      (static_cast<int64_t>(heads) - 1) * head_stride + kD > row_stride)
    return set_error(kUnsupported, "%s: one frame of tokens must span < 2 GiB with the heads inside a row",
                     name);
  const int tiles_x = (frame_w + kCvTile - 1) / kCvTile;
  const int64_t wgs = static_cast<int64_t>(heads) * tiles_x * ((frame_h + kCvTile - 1) / kCvTile);
  if (wgs > (1ll << 31) - 1) return set_error(kUnsupported, "%s: grid too large", name);
  hipLaunchKernelGGL(vda_conv_prepare_kernel, dim3(static_cast<unsigned>(wgs)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(tokens),
                     row_stride, head_stride, frames, frame_h, frame_w, heads, tiles_x, w_sp, w_tm,
                     l2norm, static_cast<uint16_t*>(out));
  return check_launch(name);
}

// Reference: paper_stack.py:51-110 (_joint_stats / paper_statistics; BF16 path), fed either
// prepared [F,H,S,D] operands (activate = 0) or raw token-major projections with the
// paper_prepare activation applied in registers (activate = 1).
// Strides are in elements: operand (f, h, s, c) at base + f*sf + h*sh + s*ss + c.
VDN_API int vdn_vda_statistics(const void* k, int64_t k_sf, int64_t k_sh, int64_t k_ss,
                               const void* v, int64_t v_sf, int64_t v_sh, int64_t v_ss,
                               const void* beta, int64_t b_sf, int64_t b_sh, int64_t b_ss,
                               int beta_f32, int frames, int heads, int spatial, int activate,
                               float* A, float* B, void* stream) {
  const char* name = "vdn_vda_statistics";
  if (k == nullptr || v == nullptr || beta == nullptr || A == nullptr || B == nullptr)
    return set_error(kInvalidArgument, "%s: null pointer", name);
  if (frames <= 0 || heads <= 0 || spatial <= 0)
    return set_error(kInvalidArgument, "%s: positive frames/heads/spatial required", name);
  if (!aligned16(k) || !aligned16(v) || !stride8(k_sf) || !stride8(k_sh) || !stride8(k_ss) ||
      !stride8(v_sf) || !stride8(v_sh) || !stride8(v_ss))
    return set_error(kInvalidArgument, "%s: k/v rows need 16-byte alignment", name);
  auto st = static_cast<hipStream_t>(stream);
  const View kv{static_cast<const uint16_t*>(k), k_sf, k_sh, k_ss};
  const View vv{static_cast<const uint16_t*>(v), v_sf, v_sh, v_ss};
  const dim3 grid(frames * heads);
  if (beta_f32)
    hipLaunchKernelGGL(vda_statistics_kernel<3>, grid, dim3(kStThreads), 0, st, kv, vv, beta, b_sf, b_sh,
                       b_ss, 1, spatial, heads, activate, A, B);
  else
    hipLaunchKernelGGL(vda_statistics_kernel<2>, grid, dim3(kStThreads), 0, st, kv, vv, beta, b_sf, b_sh,
                       b_ss, 0, spatial, heads, activate, A, B);
  return check_launch(name);
}

// Reference: paper_factor.py:133-186 -> vdn_delta_factors (T = diag(alpha) (I+A)^-1,
// J = B (I+A)^-1, fp32, no pivoting). alpha may be null (all ones).
VDN_API int vdn_vda_factors(const float* A, const float* B, const float* alpha, int64_t count,
                            float* T, float* J, void* stream) {
  const char* name = "vdn_vda_factors";
  if (A == nullptr || B == nullptr || T == nullptr || J == nullptr)
    return set_error(kInvalidArgument, "%s: null pointer", name);
  if (count < 0 || count > (1ll << 31) - 1) return set_error(kInvalidArgument, "%s: bad count", name);
  if (!aligned16(A) || !aligned16(B) || !aligned16(T) || !aligned16(J))
    return set_error(kInvalidArgument, "%s: matrices need 16-byte alignment", name);
  if (count == 0) return kOk;
  hipLaunchKernelGGL(vda_factors_kernel, dim3(static_cast<unsigned>(count)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), A, B, alpha, T, J);
  return check_launch(name);
}

// Reference: paper_stack.py:162-181 (_compose): per chunk c and direction, CT = ordered
// product of the chunk's transitions, CI = the chunk's accumulated injection.
// T, J: [F, H, 128, 128]; starts/ends: int32 [chunks]; CT, CI: [2, chunks, H, 128, 128].
VDN_API int vdn_vda_compose(const float* T, const float* J, int heads, const int* starts,
                            const int* ends, int chunks, float* CT, float* CI, void* stream) {
  const char* name = "vdn_vda_compose";
  if (T == nullptr || J == nullptr || starts == nullptr || ends == nullptr || CT == nullptr ||
      CI == nullptr)
    return set_error(kInvalidArgument, "%s: null pointer", name);
  if (heads <= 0 || chunks <= 0) return set_error(kInvalidArgument, "%s: bad geometry", name);
  if (static_cast<int64_t>(heads) * chunks * (kD / 16) * 2 > (1ll << 31) - 1)
    return set_error(kUnsupported, "%s: grid too large", name);
  const dim3 grid(kD / 16 * heads * chunks * 2);
  hipLaunchKernelGGL(vda_recur_kernel<kCompose>, grid, dim3(kRecThreads), 0,
                     static_cast<hipStream_t>(stream), T, J, heads, starts, ends, chunks,
                     nullptr, 0, CT, CI);
  return check_launch(name);
}

// Reference: paper_stack.py:184-199 (_scan_both): both directional scans over chunks.
// per_direction = 1: CT, CI are [2, chunks, H, 128, 128] (composed maps); per_direction = 0:
// CT, CI are per-frame factors [chunks, H, 128, 128] used by both directions (one-frame
// chunks). bank: [2, chunks, H, 128, 128] fp32; seed (nullable): [H, 128, 128].
VDN_API int vdn_vda_scan(const float* CT, const float* CI, const float* seed, int chunks,
                         int heads, int per_direction, float* bank, void* stream) {
  const char* name = "vdn_vda_scan";
  if (CT == nullptr || CI == nullptr || bank == nullptr)
    return set_error(kInvalidArgument, "%s: null pointer", name);
  if (heads <= 0 || chunks <= 0) return set_error(kInvalidArgument, "%s: bad geometry", name);
  if (static_cast<int64_t>(heads) * (kD / 16) * 2 > (1ll << 31) - 1)
    return set_error(kUnsupported, "%s: grid too large", name);
  const dim3 grid(kD / 16 * heads * 2);
  hipLaunchKernelGGL(vda_recur_kernel<kScan>, grid, dim3(kRecThreads), 0,
                     static_cast<hipStream_t>(stream), CT, CI, heads, nullptr, nullptr, chunks,
                     seed, per_direction, bank, nullptr);
  return check_launch(name);
}

// Exclusive log-prefix of alpha over frames (paper_stack.py:256): logp [F+1, H, 128].
VDN_API int vdn_vda_log_prefix(const float* alpha, int frames, int heads, float* logp,
                               void* stream) {
  if (alpha == nullptr || logp == nullptr)
    return set_error(kInvalidArgument, "vdn_vda_log_prefix: null pointer");
  const int hd = heads * kD;
  hipLaunchKernelGGL(vda_log_prefix_kernel, dim3((hd + 255) / 256), dim3(256), 0,
                     static_cast<hipStream_t>(stream), alpha, frames, hd, logp);
  return check_launch("vdn_vda_log_prefix");
}

// Reference: paper_stack.py:239-263 -> paper_sglang.py:445-501 (_gather_state_kernel) with
// compact bank indices. prefix/suffix: [chunks, H, 128, 128] views of bank[0]/bank[1];
// index arrays int32 [frames]; text (nullable) [H, 128, 128]; out [F, H, 128, 128].
VDN_API int vdn_vda_gather(const float* prefix, const float* suffix, const float* logp,
                           const float* text, const int* before, const int* after,
                           const int* has_before, const int* has_after, const int* bridge_before,
                           const int* bridge_after, int frames, int heads, int bridge,
                           int out_f32, void* out, void* stream) {
  const char* name = "vdn_vda_gather";
  if (prefix == nullptr || suffix == nullptr || (bridge && logp == nullptr) || before == nullptr ||
      after == nullptr || has_before == nullptr || has_after == nullptr || out == nullptr ||
      (bridge && (bridge_before == nullptr || bridge_after == nullptr)))
    return set_error(kInvalidArgument, "%s: null pointer", name);
  if (frames <= 0 || heads <= 0) return set_error(kInvalidArgument, "%s: bad geometry", name);
  hipLaunchKernelGGL(vda_gather_kernel, dim3(frames, heads, 8), dim3(256), 0,
                     static_cast<hipStream_t>(stream), prefix, suffix, logp, text, before, after,
                     has_before, has_after, bridge_before, bridge_after, heads, bridge, out_f32,
                     out);
  return check_launch(name);
}

// Fused readout (paper_stack.py:317 torch.matmul + paper_sglang.py:377-437 epilogue), with
// the q activation of paper_prepare applied in registers when activate_q = 1.
// q: (f, h, s, c) at q + f*q_sf + h*q_sh + s*q_ss + c; gate likewise; out likewise.
// state: bf16 [F, H, 128, 128] ([v][k]); weight [128] bf16 or fp32. head_dim < 128 (16, 32,
// 64): rows stay 128 wide with zeros past head_dim in q and state (and in the weight, so
// those output channels are zero), and the norm's mean is over head_dim channels.
namespace vdn {
namespace {

int launch_readout(const char* name, const void* q, int64_t q_sf, int64_t q_sh, int64_t q_ss,
                   int activate_q, const void* state, const void* weight, int weight_f32,
                   float eps, const void* gate, int64_t g_sf, int64_t g_sh, int64_t g_ss,
                   const GateProj* gp, void* out, int64_t o_sf, int64_t o_sh, int64_t o_ss,
                   const MxDst* mx, int head_dim, int frames, int heads, int spatial,
                   void* stream) {
  if (q == nullptr || state == nullptr || weight == nullptr ||
      (gp == nullptr && gate == nullptr) || (mx == nullptr && out == nullptr))
    return set_error(kInvalidArgument, "%s: null pointer", name);
  if (frames <= 0 || heads <= 0 || spatial <= 0)
    return set_error(kInvalidArgument, "%s: bad geometry", name);
  if (!valid_head_dim(head_dim) || ((gp != nullptr || mx != nullptr) && head_dim != kD))
    return set_error(kInvalidArgument,
                     "%s: head_dim must be 16, 32, 64 or 128 (128 with an MXFP8 destination "
                     "or a formed gate)", name);
  if (!aligned16(q) || !aligned16(state) || !stride8(q_sf) || !stride8(q_sh) ||
      !stride8(q_ss) ||
      (gp == nullptr &&
       (!aligned16(gate) || !stride8(g_sf) || !stride8(g_sh) || !stride8(g_ss))) ||
      (mx == nullptr && (!aligned16(out) || !stride8(o_sf) || !stride8(o_sh) || !stride8(o_ss))))
    return set_error(kInvalidArgument, "%s: operands need 16-byte aligned rows", name);
  if (gp != nullptr) {
    if (gp->down == nullptr || gp->up_w == nullptr || gp->up_b == nullptr)
      return set_error(kInvalidArgument, "%s: null pointer", name);
    if (!aligned16(gp->down) || !aligned16(gp->up_w) || !stride8(gp->d_st) || gp->d_st < kD)
      return set_error(kInvalidArgument,
                       "%s: gate down rows and up weights need 16-byte aligned rows of 128", name);
  }
  if (mx != nullptr) {
    if (mx->codes == nullptr || mx->scales == nullptr)
      return set_error(kInvalidArgument, "%s: null pointer", name);
    if (!aligned16(mx->codes) || (reinterpret_cast<uintptr_t>(mx->scales) & 3) != 0 ||
        mx->kp <= 0 || mx->kp % 128 != 0 || mx->chunk0 < 0 ||
        static_cast<int64_t>(mx->chunk0 + heads) * 128 > mx->kp)
      return set_error(kInvalidArgument,
                       "%s: codes need 16-byte alignment, a multiple-of-128 row length holding "
                       "chunks [chunk0, chunk0 + heads), scales 4-byte alignment", name);
  }
  // Token-group ranges per (frame, head): enough workgroups to fill the GPU a few times
  // over, each range at least one group per wave.
  const int groups = (spatial + 15) / 16;
  const int64_t fh = static_cast<int64_t>(frames) * heads;
  int parts = static_cast<int>((4096 + fh - 1) / fh);
  parts = std::max(1, std::min(parts, groups / kRoWaves));
  if (fh * parts > (1ll << 31) - 1) return set_error(kUnsupported, "%s: grid too large", name);
  const View qv{static_cast<const uint16_t*>(q), q_sf, q_sh, q_ss};
  const View gv{static_cast<const uint16_t*>(gate), g_sf, g_sh, g_ss};
  const GateProj g = gp != nullptr ? *gp : GateProj{nullptr, 0, nullptr, nullptr};
  const MxDst m = mx != nullptr ? *mx : MxDst{nullptr, nullptr, 0, 0};
  const dim3 grid(static_cast<unsigned>(fh * parts)), block(kRoThreads);
  const auto st = static_cast<hipStream_t>(stream);
  const auto* sp = static_cast<const uint16_t*>(state);
  auto* op = static_cast<uint16_t*>(out);
#define VDN_READOUT(MX, PROJ)                                                                  \
  hipLaunchKernelGGL((vda_readout_kernel<MX, PROJ>), grid, block, 0, st, qv, activate_q, sp,   \
                     weight, weight_f32, eps, 1.0f / head_dim, gv, g, op, o_sf, o_sh, o_ss,     \
                     spatial, heads,                                                            \
                     parts, m)
  if (mx != nullptr && gp != nullptr)
    VDN_READOUT(true, true);
  else if (mx != nullptr)
    VDN_READOUT(true, false);
  else if (gp != nullptr)
    VDN_READOUT(false, true);
  else
    VDN_READOUT(false, false);
#undef VDN_READOUT
  return check_launch(name);
}

}  // namespace
}  // namespace vdn

VDN_API int vdn_vda_readout(const void* q, int64_t q_sf, int64_t q_sh, int64_t q_ss,
                            int activate_q, const void* state, const void* weight, int weight_f32,
                            float eps, const void* gate, int64_t g_sf, int64_t g_sh, int64_t g_ss,
                            void* out, int64_t o_sf, int64_t o_sh, int64_t o_ss, int head_dim,
                            int frames, int heads, int spatial, void* stream) {
  return launch_readout("vdn_vda_readout", q, q_sf, q_sh, q_ss, activate_q, state, weight,
                        weight_f32, eps, gate, g_sf, g_sh, g_ss, nullptr, out, o_sf, o_sh, o_ss,
                        nullptr, head_dim, frames, heads, spatial, stream);
}

// The same readout with the output quantized in the epilogue: token row f * S + s, head h ->
// MXFP8 codes[row, 128 (chunk0 + h) ..] (row length kp) and the swizzled scales of its four
// 32-blocks, bit-identical to vdn_mxfp8_quantize of the bf16 output. Reference: the
// projection's producer, quantize_activation (src/models/ops/mxfp8_quant.py:77-90), applied
// to the readout of paper_readout (src/models/linear_attention/paper_stack.py:266-318).
VDN_API int vdn_vda_readout_mxfp8(const void* q, int64_t q_sf, int64_t q_sh, int64_t q_ss,
                                  int activate_q, const void* state, const void* weight,
                                  int weight_f32, float eps, const void* gate, int64_t g_sf,
                                  int64_t g_sh, int64_t g_ss, void* codes, void* scales,
                                  int64_t kp, int chunk0, int frames, int heads, int spatial,
                                  void* stream) {
  const MxDst mx{static_cast<uint8_t*>(codes), static_cast<uint8_t*>(scales), kp, chunk0};
  return launch_readout("vdn_vda_readout_mxfp8", q, q_sf, q_sh, q_ss, activate_q, state,
                        weight, weight_f32, eps, gate, g_sf, g_sh, g_ss, nullptr, nullptr, 0, 0,
                        0, &mx, kD, frames, heads, spatial, stream);
}

// The readout with the linear branch's low-rank output gate formed in the kernel:
// gate = bf16(sigmoid(bf16(down · up_wᵀ + up_b))) per (token, head, channel), the
// OutputGate of the linear branch (src/models/attention_gates.py:52-55, up(down(x)) then
// sigmoid), from down [F*S, 128] bf16 rows (row stride d_st), up_w [H*128, 128] bf16 and
// up_b [H*128] bf16. Exactly one destination: bf16 `out` (strides as vdn_vda_readout) or,
// with out = NULL, MXFP8 `codes` / `scales` (as vdn_vda_readout_mxfp8). Replaces the pair
// output_gate(xv) + paper_readout (src/models/linear_attention/paper_stack.py:315-318).
VDN_API int vdn_vda_readout_gated(const void* q, int64_t q_sf, int64_t q_sh, int64_t q_ss,
                                  int activate_q, const void* state, const void* weight,
                                  int weight_f32, float eps, const void* down, int64_t d_st,
                                  const void* up_w, const void* up_b, void* out, int64_t o_sf,
                                  int64_t o_sh, int64_t o_ss, void* codes, void* scales,
                                  int64_t kp, int chunk0, int frames, int heads, int spatial,
                                  void* stream) {
  const GateProj gp{static_cast<const uint16_t*>(down), d_st,
                    static_cast<const uint16_t*>(up_w), static_cast<const uint16_t*>(up_b)};
  if ((out == nullptr) == (codes == nullptr))
    return set_error(kInvalidArgument,
                     "vdn_vda_readout_gated: give exactly one of out and codes");
  const MxDst mx{static_cast<uint8_t*>(codes), static_cast<uint8_t*>(scales), kp, chunk0};
  return launch_readout("vdn_vda_readout_gated", q, q_sf, q_sh, q_ss, activate_q, state,
                        weight, weight_f32, eps, nullptr, 0, 0, 0, &gp, out, o_sf, o_sh, o_ss,
                        codes != nullptr ? &mx : nullptr, kD, frames, heads, spatial, stream);
}

// Reference: paper_sglang.py:377-437 (_linear_epilogue_kernel / vdn_linear_epilogue):
// readout [F, H, S, 128] bf16 contiguous -> RMSNorm(d)·w·gate -> out.
VDN_API int vdn_vda_epilogue(const void* readout, const void* weight, int weight_f32, float eps,
                             const void* gate, int64_t g_sf, int64_t g_sh, int64_t g_ss,
                             void* out, int64_t o_sf, int64_t o_sh, int64_t o_ss, int head_dim,
                             int frames, int heads, int spatial, void* stream) {
  const char* name = "vdn_vda_epilogue";
  if (readout == nullptr || weight == nullptr || gate == nullptr || out == nullptr)
    return set_error(kInvalidArgument, "%s: null pointer", name);
  if (frames <= 0 || heads <= 0 || spatial <= 0)
    return set_error(kInvalidArgument, "%s: bad geometry", name);
  if (!valid_head_dim(head_dim))
    return set_error(kInvalidArgument, "%s: head_dim must be 16, 32, 64 or 128", name);
  const int64_t items = static_cast<int64_t>(frames) * heads * spatial;
  const View gv{static_cast<const uint16_t*>(gate), g_sf, g_sh, g_ss};
  hipLaunchKernelGGL(vda_epilogue_kernel, dim3(static_cast<unsigned>((items + 15) / 16)),
                     dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(readout), weight, weight_f32, eps,
                     1.0f / head_dim, gv,
                     static_cast<uint16_t*>(out), o_sf, o_sh, o_ss, frames, heads, spatial);
  return check_launch(name);
}
