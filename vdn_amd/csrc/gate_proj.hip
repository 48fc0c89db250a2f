// The hybrid block's small projections of the attention input and its two GEMVs, for gfx950.
//
// vdn_gate_projection: one bf16 MFMA pass over x1 [T, K] (T = frames x spatial rows) against
//   W = [W_gate (heads rows, zero-padded to 64) | W_beta (same) | W_down (128) | W_alpha (128)]
//   (384 rows), with the epilogue of each column group fused:
//     soft_gate = bf16(sigmoid(bf16(acc + b)))   OutputGate: sigmoid(Linear(x1, W, b)), the
//     beta      = bf16(sigmoid(bf16(acc)))       bias added before the one bf16 rounding
//     gate_down = bf16(acc)                      (attention_gates.py:52-55,
//                                                 tensor_parallel.py:194-198)
//     per-frame fp32 sums of acc over the alpha-down columns, one partial row per 128-row
//     block of a frame (the FrameKDAAlpha MLP starts with Linear(mean over the frame's rows of
//     x1), layers.py:36-69, and Linear(mean(x)) = mean(Linear(x)), so the frame mean costs
//     no pass over x1 of its own).
// vdn_frame_alpha: mean of those partial sums, then alpha = exp(-exp(A_log) softplus(up(.) +
//   dt_bias)) in fp32 (layers.py:29-34, 69).
// vdn_adaln_tables: the AdaLN projection Linear(bf16(SiLU(temb in fp32))) (paper_adaln.py:
//   174-188), a GEMV streaming the [6H, H] weight once.
#include "common.h"

#include <math.h>

namespace vdn {
namespace {

typedef __attribute__((address_space(3))) void lds_void_t;
typedef const __attribute__((address_space(1))) void global_void_t;

constexpr int kGK = 32;          // K per LDS stage (two 16-deep MFMA steps)
constexpr int kGRows = 128;      // rows per workgroup (2 x 64: two waves along M)
constexpr int kGCols = 384;      // W rows = output columns (4 x 96: four waves along N)
constexpr int kGGroup = 64;      // gate / beta column group (heads <= 64)
constexpr int kGRank = 128;      // output-gate down and alpha-down widths
constexpr int kARing = 6;        // x1 stages in LDS (issued 5 stages ahead)
constexpr int kWRing = 4;        // W stages in LDS (issued 3 stages ahead)

// global -> LDS DMA of 16 bytes per lane (lane l's bytes land at LDS byte M0 + 16 l), as
// inline asm: the compiler does not see it as an LDS write, so it never makes a fragment read
// wait for a DMA into another ring slot; the kernel orders the DMAs itself (vmcnt waits before
// its barriers; no other vector memory access is in flight in the K loop). With either LDS
// DMA builtin (global or buffer form) the compiler puts a vmcnt(0) before every stage's
// fragment reads, which serializes the rings. M0 is an input operand ("{m0}"): the compiler
// writes it and knows it is live; the s_nop is the wait state between an M0 write and an
// LDS DMA that reads it.
__device__ __forceinline__ void g_load_lds16(const void* src, void* lds_wave_base) {
  const uint32_t lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_t*)lds_wave_base));
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(lds) : "memory");
}

// 16-byte chunk c (0..3) of a 64-byte tile row r is stored at c ^ ((r >> 2) & 3): the 16 lanes
// an LDS read serves together read one chunk of 16 consecutive rows, which then covers all
// 64 banks.
__device__ __forceinline__ int gswz(int r) { return (r >> 2) & 3; }

__device__ __forceinline__ float sigmoid_f32(float x) { return 1.0f / (1.0f + expf(-x)); }

// 8 waves, two per SIMD: wave (wm, wn) owns rows 64 wm .. +64 (two 32-row MFMA blocks) and
// columns 96 wn .. +96 (three 32-column blocks); one wave's DMA issue and fragment reads
// overlap the other's MFMAs on each SIMD.
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2)))
gate_projection_kernel(const uint16_t* __restrict__ x, int64_t x_st, int k,
                       const uint16_t* __restrict__ w, int heads, int spatial, int bpf,
                       const uint16_t* __restrict__ gate_bias, uint16_t* __restrict__ soft_gate,
                       uint16_t* __restrict__ beta, uint16_t* __restrict__ gate_down,
                       float* __restrict__ partial) {
  // Two rings of LDS stages: kARing (6) of x1 (its HBM stream needs many bytes in flight)
  // and kWRing (4) of W (read by every workgroup, mostly from L2). After the K loop the W
  // ring stages the outputs: softmax gate [128][64], beta [128][64], down [128][128] bf16.
  __shared__ __attribute__((aligned(1024))) uint16_t sA[kARing * kGRows * kGK];
  __shared__ __attribute__((aligned(1024))) uint16_t sW[kWRing * kGCols * kGK];
  __shared__ float s_alpha[2][kGRank];
  static_assert(kWRing * kGCols * kGK >= kGRows * (2 * kGGroup + kGRank), "output staging");

  const int f = blockIdx.x / bpf, jb = blockIdx.x % bpf;
  const int row0 = jb * kGRows;                     // first row of the block within the frame
  const int nrows = min(kGRows, spatial - row0);    // rows of the block that belong to frame f
  const int64_t grow0 = static_cast<int64_t>(f) * spatial + row0;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int g = lane >> 5, col = lane & 31;

  // ---- DMA: the x1 tile is 512 16-byte chunks, the W tile 1536; chunk q of a tile is LDS
  // chunk q, i.e. row q / 4, stored chunk q % 4. Waves 0-3 load x1 (2 chunks per lane), waves
  // 4-7 load W (6 per lane): vmcnt retires in order, so with each stream in waves of its own a
  // wait for W from L2 never waits for x1 loads from HBM issued after it (and x1 keeps its
  // full prefetch distance). Rows past the block's last row repeat it (their results are
  // dropped). ----
  const bool a_loader = wave < 4;   // wave-uniform
  const int lw = a_loader ? wave : wave - 4;
  const char* src[6];
  if (a_loader) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int q = 64 * (2 * lw + i) + lane, r = q >> 2, c = q & 3;
      src[i] = reinterpret_cast<const char*>(x + (grow0 + min(r, nrows - 1)) * x_st) +
               16 * (c ^ gswz(r));
    }
#pragma unroll
    for (int i = 2; i < 6; ++i) src[i] = src[1];
  } else {
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      const int q = 64 * (6 * lw + i) + lane, r = q >> 2, c = q & 3;
      src[i] = reinterpret_cast<const char*>(w + static_cast<int64_t>(r) * k) + 16 * (c ^ gswz(r));
    }
  }
  // DMA i (0-1 for x1 waves, 0-5 for W waves) of stage s into ring slot `slot`
  auto issue_one = [&](int i, int s, int slot) __attribute__((always_inline)) {
    const int64_t off = static_cast<int64_t>(s) * kGK * 2;
    if (a_loader)
      g_load_lds16(src[i] + off, sA + slot * (kGRows * kGK) + 64 * (2 * lw + i) * 8);
    else
      g_load_lds16(src[i] + off, sW + slot * (kGCols * kGK) + 64 * (6 * lw + i) * 8);
  };
  auto issue_a = [&](int s, int slot) __attribute__((always_inline)) {
    if (a_loader) {
      issue_one(0, s, slot);
      issue_one(1, s, slot);
    }
  };
  auto issue_w = [&](int s, int slot) __attribute__((always_inline)) {
    if (!a_loader) {
#pragma unroll
      for (int i = 0; i < 6; ++i) issue_one(i, s, slot);
    }
  };

  f32x16 acc[2][3];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int nb = 0; nb < 3; ++nb)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mb][nb][v] = 0.f;

  // fragment offsets (elements): row, then the stored chunk of logical chunk 2 j + g
  int a_off[2][2], w_off[3][2];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
    const int r = 64 * wm + 32 * mb + col;
#pragma unroll
    for (int j = 0; j < 2; ++j) a_off[mb][j] = r * kGK + 8 * ((2 * j + g) ^ gswz(r));
  }
#pragma unroll
  for (int nb = 0; nb < 3; ++nb) {
    const int r = 96 * wn + 32 * nb + col;
#pragma unroll
    for (int j = 0; j < 2; ++j) w_off[nb][j] = r * kGK + 8 * ((2 * j + g) ^ gswz(r));
  }
  // Fragments of one stage: 4 x1 and 6 W 16-byte reads per lane.
  struct Frags {
    bf16x8 a[2][2], w[2][3];
  };
  auto read_frags = [&](Frags& fr, const uint16_t* tA, const uint16_t* tW) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) fr.a[j][mb] = *reinterpret_cast<const bf16x8*>(tA + a_off[mb][j]);
#pragma unroll
      for (int nb = 0; nb < 3; ++nb) fr.w[j][nb] = *reinterpret_cast<const bf16x8*>(tW + w_off[nb][j]);
    }
  };
  // The 12 MFMAs of one stage, with the wave's DMAs of one batch (x1 stage sa into slot sla
  // after MFMAs 0 and 6, or W stage sw into slot slw after MFMAs 0, 2, .., 10): a DMA issue
  // can stall while the CU's address unit is busy, and in the shadow of queued MFMAs the
  // stall costs less than a burst.
  auto mfmas = [&](const Frags& fr, int sa, int sla, int sw, int slw) __attribute__((always_inline)) {
    int n = 0;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int nb = 0; nb < 3; ++nb)
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
          acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fr.a[j][mb], fr.w[j][nb], acc[mb][nb], 0, 0, 0);
          if (n % 2 == 0) {
            asm volatile("" ::"v"(acc[mb][nb]) : "memory");
            __builtin_amdgcn_sched_barrier(0);
            if (a_loader) {
              if (n % 6 == 0) issue_one(n / 6, sa, sla);
            } else {
              issue_one(n / 2, sw, slw);
            }
            __builtin_amdgcn_sched_barrier(0);
          }
          ++n;
        }
  };

  // ---- K loop. Stage s lives in x1 slot s % 6 and W slot s % 4. The prologue issues x1
  // stages 0-4 (x1 waves) and W stages 0-2 (W waves); iteration s (after its barrier) reads
  // the fragments of stage s + 1 into registers, then runs the MFMAs of stage s from the
  // registers read one iteration earlier and, among them, issues x1 stage s + 5 (x1 waves) or
  // W stage s + 3 (W waves) into the slots of stage s - 1 (whose fragments every wave read
  // in iteration s - 2 and consumed in iteration s - 1), so the LDS reads of one stage
  // overlap the MFMAs of the previous. Past the last stage a batch loads the last stage again
  // (into those free slots), so every batch is 2 (x1) or 6 (W) DMAs per wave and the waits
  // are exact: stage s + 1 must have landed before the barrier of iteration s, which leaves
  // x1 stages s + 2 .. s + 4 (6 DMAs) or W stage s + 2 (6 DMAs) in flight. ----
  static_assert(kARing >= kWRing, "x1 runs at least as far ahead as W");
  const int stages = k / kGK;
#pragma unroll
  for (int a = 0; a < kARing - 1; ++a) issue_a(min(a, stages - 1), a);
#pragma unroll
  for (int b = 0; b < kWRing - 1; ++b) issue_w(min(b, stages - 1), b);
  // stage 0 must have landed: x1 stages 1-4 (8 DMAs) or W stages 1-2 (12) may be in flight
  if (a_loader)
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  else
    asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
  __syncthreads();
  Frags fr[2];
  read_frags(fr[0], sA, sW);
  int aslot = 0, wslot = 0;  // slots of stage s
  for (int s = 0; s < stages; s += 2) {
    // two iterations per trip, so the fragment sets alternate at compile time
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int si = s + h;
      if (si >= stages) break;
      // stage si + 1 must have landed: x1 waves may have stages si + 2 .. si + 4 in flight (3
      // batches of 2), W waves stage si + 2 (one batch of 6)
      asm volatile("s_waitcnt vmcnt(6)\n\ts_barrier" ::: "memory");
      const int an = aslot == kARing - 1 ? 0 : aslot + 1;
      const int wn2 = wslot == kWRing - 1 ? 0 : wslot + 1;
      // unconditional (past the last stage the values are unused): with a path that skipped
      // the reads, the merged LDS wait before the first MFMA would be lgkmcnt(0), i.e. for the
      // reads just issued, instead of only those of the fragments the MFMAs use
      read_frags(fr[1 - h], sA + an * (kGRows * kGK), sW + wn2 * (kGCols * kGK));
      mfmas(fr[h], min(si + kARing - 1, stages - 1), aslot == 0 ? kARing - 1 : aslot - 1,
            min(si + kWRing - 1, stages - 1), wslot == 0 ? kWRing - 1 : wslot - 1);
      aslot = an;
      wslot = wn2;
    }
  }
  // the batches issued past the last stage must land before the ring is reused
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  // ---- epilogue: lane (g, col) of block (mb, nb) holds column col of block 3 wn + nb
  // (0-1 softmax gate, 2-3 beta, 4-7 down, 8-11 alpha down) for rows
  // 64 wm + 32 mb + 8 (v / 4) + 4 g + v % 4. Gate, beta and down go to the staging tiles,
  // the alpha columns are summed over the block's rows. ----
  uint16_t* st_gate = sW;
  uint16_t* st_beta = sW + kGRows * kGGroup;
  uint16_t* st_down = sW + 2 * kGRows * kGGroup;
#pragma unroll
  for (int nb = 0; nb < 3; ++nb) {
    const int gb = 3 * wn + nb;  // uniform per wave
    if (gb < 8) {
      const int c = 32 * (gb & 1) + col;
      const float b = gb < 2 && c < heads ? bf16_bits_to_f32(gate_bias[c]) : 0.f;
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int r = 64 * wm + 32 * mb + 8 * (v >> 2) + 4 * g + (v & 3);
          const float a = acc[mb][nb][v];
          if (gb < 2)
            st_gate[r * kGGroup + c] = f32_to_bf16_bits(sigmoid_f32(round_bf16(a + b)));
          else if (gb < 4)
            st_beta[r * kGGroup + c] = f32_to_bf16_bits(sigmoid_f32(round_bf16(a)));
          else
            st_down[r * kGRank + 32 * (gb - 4) + col] = f32_to_bf16_bits(a);
        }
    } else {
      float t = 0.f;
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          if (64 * wm + 32 * mb + 8 * (v >> 2) + 4 * g + (v & 3) < nrows) t += acc[mb][nb][v];
      const uint32_t u = __float_as_uint(t);
      const auto sw = __builtin_amdgcn_permlane32_swap(u, u, false, false);
      if (g == 0) s_alpha[wm][32 * (gb - 8) + col] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
  }
  __syncthreads();
  // ---- stores: each output's rows of the block are one contiguous range ----
  {
    const int words = nrows * heads / 2;  // heads is even: a word never crosses a row
    uint32_t* dg = reinterpret_cast<uint32_t*>(soft_gate + grow0 * heads);
    uint32_t* db = reinterpret_cast<uint32_t*>(beta + grow0 * heads);
    for (int i = tid; i < words; i += 512) {
      const int r = (2 * i) / heads, c = 2 * i - r * heads;
      dg[i] = *reinterpret_cast<const uint32_t*>(st_gate + r * kGGroup + c);
      db[i] = *reinterpret_cast<const uint32_t*>(st_beta + r * kGGroup + c);
    }
    u32x4* dd = reinterpret_cast<u32x4*>(gate_down + grow0 * kGRank);
    for (int i = tid; i < nrows * (kGRank / 8); i += 512)
      dd[i] = *reinterpret_cast<const u32x4*>(st_down + 8 * i);
    if (tid < kGRank)
      partial[static_cast<int64_t>(blockIdx.x) * kGRank + tid] = s_alpha[0][tid] + s_alpha[1][tid];
  }
}

// alpha[f, i] = exp(-exp(a_log[i / d]) * softplus(delta)), delta = sum_j mean[f, j] up_w[i, j]
// + dt_bias[i], mean[f, j] = (sum over the frame's blocks of partial[., j]) / spatial.
__global__ void __launch_bounds__(256)
frame_alpha_kernel(const float* __restrict__ partial, int bpf, int spatial,
                   const uint16_t* __restrict__ up_w, const float* __restrict__ dt_bias,
                   const float* __restrict__ a_log, int d, int inner, float* __restrict__ alpha) {
  __shared__ float mean[kGRank];
  const int f = blockIdx.x;
  const int tid = threadIdx.x;
  if (tid < kGRank) {
    float t = 0.f;
    for (int b = 0; b < bpf; ++b) t += partial[(static_cast<int64_t>(f) * bpf + b) * kGRank + tid];
    mean[tid] = t / static_cast<float>(spatial);
  }
  __syncthreads();
  const int i = blockIdx.y * 256 + tid;
  if (i >= inner) return;
  const u32x4* wr = reinterpret_cast<const u32x4*>(up_w + static_cast<int64_t>(i) * kGRank);
  float acc = 0.f;
#pragma unroll 4
  for (int q = 0; q < kGRank / 8; ++q) {
    const u32x4 w8 = wr[q];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc = fmaf(mean[8 * q + 2 * e], bf16_bits_to_f32(static_cast<uint16_t>(w8[e] & 0xffff)), acc);
      acc = fmaf(mean[8 * q + 2 * e + 1], bf16_bits_to_f32(static_cast<uint16_t>(w8[e] >> 16)), acc);
    }
  }
  const float delta = acc + dt_bias[i];
  // softplus with torch's threshold: x for x > 20, log1p(exp(x)) otherwise
  const float sp = delta > 20.f ? delta : log1pf(expf(delta));
  alpha[static_cast<int64_t>(f) * inner + i] = expf(-expf(a_log[i / d]) * sp);
}

// out[m, n] = bf16(sum_k s[m, k] w[n, k] + b[n]) with s = bf16(SiLU(temb[m, k])) in fp32;
// temb is bf16 or fp32 (temb_f32). 256 threads, 8 output rows per workgroup (two per wave,
// whose weight loads go out together); lane l covers k = 8 l + 512 i (K a multiple of 8).
constexpr int kAdaRows = 8;
__device__ __forceinline__ float dot8(const u32x4& s8, const u32x4& w8, float acc) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    acc = fmaf(bf16_bits_to_f32(static_cast<uint16_t>(s8[e] & 0xffff)),
               bf16_bits_to_f32(static_cast<uint16_t>(w8[e] & 0xffff)), acc);
    acc = fmaf(bf16_bits_to_f32(static_cast<uint16_t>(s8[e] >> 16)),
               bf16_bits_to_f32(static_cast<uint16_t>(w8[e] >> 16)), acc);
  }
  return acc;
}

__device__ __forceinline__ float wave_sum(float acc) {
  acc += __shfl_xor(acc, 32);
  acc += __shfl_xor(acc, 16);
  acc += __shfl_xor(acc, 8);
  acc += __shfl_xor(acc, 4);
  acc += __shfl_xor(acc, 2);
  acc += __shfl_xor(acc, 1);
  return acc;
}

__global__ void __launch_bounds__(256)
adaln_gemv_kernel(const void* __restrict__ temb, int temb_f32, int64_t t_st, int m, int k,
                  const uint16_t* __restrict__ w, const uint16_t* __restrict__ b, int n,
                  uint16_t* __restrict__ out, int64_t o_st) {
  extern __shared__ uint16_t s_act[];  // [k] bf16 of one temb row
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int chunks = (k + 511) / 512;  // 16-byte pieces per lane (the last one partial)
  const int r0 = blockIdx.x * kAdaRows + 2 * wave;
  // rows past n read row n - 1 and store nothing
  const uint16_t* w0 = w + static_cast<int64_t>(min(r0, n - 1)) * k;
  const uint16_t* w1 = w + static_cast<int64_t>(min(r0 + 1, n - 1)) * k;
  for (int mi = 0; mi < m; ++mi) {
    __syncthreads();
    for (int e = tid; e < k; e += 256) {
      const int64_t ti = mi * t_st + e;
      const float t = temb_f32 ? static_cast<const float*>(temb)[ti]
                               : bf16_bits_to_f32(static_cast<const uint16_t*>(temb)[ti]);
      s_act[e] = f32_to_bf16_bits(t / (1.0f + expf(-t)));
    }
    __syncthreads();
    float a0 = 0.f, a1 = 0.f;
    for (int i = 0; i < chunks; ++i) {
      const int e0 = 512 * i + 8 * lane;
      if (e0 >= k) break;
      const u32x4 x0 = *reinterpret_cast<const u32x4*>(w0 + e0);
      const u32x4 x1 = *reinterpret_cast<const u32x4*>(w1 + e0);
      const u32x4 s8 = *reinterpret_cast<const u32x4*>(s_act + e0);
      a0 = dot8(s8, x0, a0);
      a1 = dot8(s8, x1, a1);
    }
    a0 = wave_sum(a0);
    a1 = wave_sum(a1);
    if (lane == 0) {
      if (r0 < n)
        out[mi * o_st + r0] = f32_to_bf16_bits(a0 + (b != nullptr ? bf16_bits_to_f32(b[r0]) : 0.f));
      if (r0 + 1 < n)
        out[mi * o_st + r0 + 1] =
            f32_to_bf16_bits(a1 + (b != nullptr ? bf16_bits_to_f32(b[r0 + 1]) : 0.f));
    }
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace vdn

using namespace vdn;

VDN_API int vdn_gate_projection(const void* x, int64_t x_st, int64_t k, const void* w, int heads,
                                int frames, int spatial, const void* gate_bias, void* soft_gate,
                                void* beta, void* gate_down, float* partial, void* stream) {
  const char* name = "vdn_gate_projection";
  if (x == nullptr || w == nullptr || gate_bias == nullptr || soft_gate == nullptr ||
      beta == nullptr || gate_down == nullptr || partial == nullptr)
    return set_error(kInvalidArgument, "%s: null pointer", name);
  if (heads <= 0 || heads > kGGroup || heads % 2 != 0)
    return set_error(kUnsupported, "%s: heads must be even, in [2, %d]", name, kGGroup);
  if (frames <= 0 || spatial <= 0 || k <= 0 || k % kGK != 0 || k > (1 << 20))
    return set_error(kInvalidArgument, "%s: bad geometry (K a multiple of %d)", name, kGK);
  if (!aligned16(x) || !aligned16(w) || x_st < k || x_st % 8 != 0 || !aligned16(gate_down) ||
      (reinterpret_cast<uintptr_t>(soft_gate) & 3) != 0 || (reinterpret_cast<uintptr_t>(beta) & 3) != 0)
    return set_error(kInvalidArgument,
                     "%s: x, w and gate_down need 16-byte alignment, soft_gate and beta 4-byte",
                     name);
  const int bpf = (spatial + kGRows - 1) / kGRows;
  const int64_t blocks = static_cast<int64_t>(frames) * bpf;
  if (blocks > (1ll << 31) - 1) return set_error(kUnsupported, "%s: too many rows", name);
  hipLaunchKernelGGL(gate_projection_kernel, dim3(static_cast<unsigned>(blocks)), dim3(512), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(x), x_st,
                     static_cast<int>(k), static_cast<const uint16_t*>(w), heads, spatial, bpf,
                     static_cast<const uint16_t*>(gate_bias), static_cast<uint16_t*>(soft_gate),
                     static_cast<uint16_t*>(beta), static_cast<uint16_t*>(gate_down), partial);
  return check_launch(name);
}

VDN_API int vdn_frame_alpha(const float* partial, int frames, int spatial, const void* up_w,
                            const float* dt_bias, const float* a_log, int heads, int head_dim,
                            float* alpha, void* stream) {
  const char* name = "vdn_frame_alpha";
  if (partial == nullptr || up_w == nullptr || dt_bias == nullptr || a_log == nullptr ||
      alpha == nullptr)
    return set_error(kInvalidArgument, "%s: null pointer", name);
  if (frames <= 0 || spatial <= 0 || heads <= 0 || head_dim <= 0)
    return set_error(kInvalidArgument, "%s: bad geometry", name);
  if (!aligned16(up_w)) return set_error(kInvalidArgument, "%s: up_w needs 16-byte alignment", name);
  const int bpf = (spatial + kGRows - 1) / kGRows;
  const int inner = heads * head_dim;
  hipLaunchKernelGGL(frame_alpha_kernel, dim3(frames, (inner + 255) / 256), dim3(256), 0,
                     static_cast<hipStream_t>(stream), partial, bpf, spatial,
                     static_cast<const uint16_t*>(up_w), dt_bias, a_log, head_dim, inner, alpha);
  return check_launch(name);
}

VDN_API int vdn_adaln_tables(const void* temb, int temb_f32, int64_t t_st, int m, int64_t k,
                             const void* w, const void* b, int64_t n, void* out, int64_t o_st,
                             void* stream) {
  const char* name = "vdn_adaln_tables";
  if (temb == nullptr || w == nullptr || out == nullptr)
    return set_error(kInvalidArgument, "%s: null pointer", name);
  if (m <= 0 || k <= 0 || n <= 0 || k % 8 != 0 || k > (1 << 14) || t_st < k || o_st < n ||
      n > (1ll << 31) - 1)
    return set_error(kInvalidArgument, "%s: bad geometry (K a multiple of 8, at most 16384)",
                     name);
  if (!aligned16(w) || (reinterpret_cast<uintptr_t>(temb) & (temb_f32 ? 3 : 1)) != 0)
    return set_error(kInvalidArgument, "%s: w needs 16-byte alignment, temb element alignment",
                     name);
  const int64_t blocks = (n + kAdaRows - 1) / kAdaRows;
  hipLaunchKernelGGL(adaln_gemv_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256),
                     static_cast<size_t>(k) * 2, static_cast<hipStream_t>(stream),
                     temb, temb_f32 != 0, t_st, m, static_cast<int>(k),
                     static_cast<const uint16_t*>(w), static_cast<const uint16_t*>(b),
                     static_cast<int>(n), static_cast<uint16_t*>(out), o_st);
  return check_launch(name);
}
