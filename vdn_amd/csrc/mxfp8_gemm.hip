// Block-scaled MXFP8 GEMM for gfx950:  C[m, n] = sum_k A[m, k] * W[n, k]  (both K-major),
// E4M3FN codes with one E8M0 scale per 32 K values, fp32 accumulation, bf16 output.
//
// Replaces the reference's F.scaled_mm(BlockWise1x32, SWIZZLE_32_4_4) call in
// MXFP8Linear.forward_quantized (src/models/ops/mxfp8_linear.py:61-93).
//
// Design:
//   * one workgroup computes a BM x BN tile; its waves form a WGM x WGN grid and each
//     wave owns a (BM/WGM) x (BN/WGN) sub-tile made of 16x16 outputs;
//   * the inner product is v_mfma_scale_f32_16x16x128_f8f6f4. For 8-bit operands its K
//     layout is split: lane l (group g = l / 16) holds row (l % 16), K [16g, 16g+16) in
//     bytes 0-15 and K [64+16g, 64+16g+16) in bytes 16-31, and the E8M0 byte of lane l
//     scales K-block g (K [32g, 32g+32)) of row l % 16 (measured on gfx950);
//   * A and W tiles (128 K bytes per row) are streamed global -> LDS with
//     global_load_lds_dwordx4 (no VGPR staging), double-buffered; each 16-byte chunk c of
//     tile row r lives at chunk c ^ ((r >> 1) & 7) so the fragment reads of 16 consecutive
//     rows touch 16 distinct 16-byte bank groups;
//   * scale bytes are read straight from the caller's SWIZZLE_32_4_4 buffer: one dword
//     holds a row's 4 K-blocks of one 128-K step, and each lane shifts its own block's
//     byte into byte 0 (the instruction ignores OPSEL and always reads byte 0);
//   * workgroup ids are remapped so consecutive tiles land on the same XCD (dispatch is
//     round-robin over the 8 XCDs) and tiles are walked in GROUP_M-row groups, which keeps
//     each XCD's L2 working set to a few A row-panels and W column-panels.
#include "mxfp8_common.h"

#include <type_traits>

namespace vdn {
namespace {

constexpr int kBK = 128;

typedef __attribute__((address_space(3))) void lds_void_t;
typedef const __attribute__((address_space(1))) void global_void_t;

__device__ __forceinline__ void load_to_lds16(const void* src, void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds((global_void_t*)src, (lds_void_t*)lds_wave_base, 16, 0, 0);
}

__device__ __forceinline__ void load_to_lds4(const void* src, void* lds_wave_base) {
  __builtin_amdgcn_global_load_lds((global_void_t*)src, (lds_void_t*)lds_wave_base, 4, 0, 0);
}

// SWIZZLE_32_4_4 keeps the scale dwords (4 K-blocks of one 128-K step) of a 128-row block
// in one contiguous 512-byte run: row r's dword sits at 16 (r % 32) + 4 ((r % 128) / 32)
// of it. The run of block b for K step ks starts at (b * col_tiles + ks) * 512.
__device__ __forceinline__ int scale_in_block(int r) { return (r & 31) * 16 + ((r & 127) >> 5) * 4; }

// Epilogue of one output element y (the bf16-rounded accumulator), in this order:
//   y = bf16(y + bias[c])                    (bias: nullable, [n])
//   y = bf16(addend[r, c] + y)               (addend: nullable)
//   y = bf16(residual[r, c] + bf16(gate[c] * y))   (residual: nullable; gate nullable = 1)
// `out` may alias `addend` or `residual`: every element is read and written by one lane.
struct Epilogue {
  const uint16_t* bias;
  const uint16_t* addend;
  int64_t ld_add;
  const uint16_t* residual;
  int64_t ld_res;
  const uint16_t* gate;
  uint16_t* out;
  int64_t ldc;
  uint32_t* nonfinite;
  int vec;  // 16-byte accesses: n, every leading dimension and pointer 8-element aligned
  // Producer mode (q_out non-null): instead of bf16 `out`, y = bf16(bf16(acc) + bias) goes
  // through `act` (0 none, 1 GELU-tanh, rounded to bf16) and is stored as MXFP8 codes
  // q_out [mp, kp_out] + swizzled scales s_out, exactly what the producer kernels write
  // for that bf16 matrix. Rows >= out_rows and columns >= n are stored as zero.
  uint8_t* q_out;
  uint8_t* s_out;
  int64_t kp_out;
  int act;
};

// Epilogue arithmetic of one element (see Epilogue).
__device__ __forceinline__ float epilogue_value(float y, float b, float addend, float res, float gt,
                                                const Epilogue& ep) {
  if (ep.bias != nullptr) y = round_bf16(y + b);
  if (ep.addend != nullptr) y = round_bf16(addend + y);
  if (ep.residual != nullptr) {
    const float t = ep.gate != nullptr ? round_bf16(gt * y) : y;
    y = round_bf16(res + t);
  }
  return y;
}

__device__ __forceinline__ void unpack4(const u32x2 w, float* f) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ void unpack8(const u32x4 w, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_bits_to_f32(static_cast<uint16_t>(w[i] & 0xffff));
    f[2 * i + 1] = bf16_bits_to_f32(static_cast<uint16_t>(w[i] >> 16));
  }
}

template <int BM, int BN, int WGM, int WGN>
__global__ void __launch_bounds__(WGM * WGN * 64) __attribute__((amdgpu_waves_per_eu(1, 1)))
mxfp8_gemm_kernel(const uint8_t* __restrict__ A, const uint8_t* __restrict__ As,
                  const uint8_t* __restrict__ W, const uint8_t* __restrict__ Ws, int64_t mp,
                  int64_t np, int64_t kp, Epilogue ep, int64_t out_rows, int64_t n,
                  int tiles_m, int tiles_n, int group_m) {
  constexpr int kWaves = WGM * WGN;
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int kASegs = BM / 8 / kWaves;  // 1 KB (8-row) segments per wave per K step
  constexpr int kBSegs = BN / 8 / kWaves;
  static_assert(kASegs * kWaves * 8 == BM && kBSegs * kWaves * 8 == BN, "tile/wave mismatch");
  // Two K-step buffers for the main loop; after it the same memory stages the bf16 tile
  // (row stride BN * 2 + 32 bytes: the 16-row x 32-byte writes of one instruction then
  // touch every bank exactly twice).
  // step buffer: A tile (BM x 128 B), W tile (BN x 128 B), then the step's scale runs
  // (BM / 128 A blocks, then BN / 128 W blocks, 512 B each)
  constexpr int kScaleOff = (BM + BN) * kBK;
  constexpr int kStepBytes = kScaleOff + (BM + BN) * 4;
  constexpr int kStageStride = BN * 2 + 32;
  constexpr int kLdsBytes = 2 * kStepBytes > BM * kStageStride ? 2 * kStepBytes : BM * kStageStride;
  __shared__ __attribute__((aligned(1024))) uint8_t lds_raw[kLdsBytes];
  uint8_t (*lds)[kStepBytes] = reinterpret_cast<uint8_t (*)[kStepBytes]>(lds_raw);

  // ---- tile selection: XCD-contiguous ids, then GROUP_M-row grouping ----
  const int num_wg = tiles_m * tiles_n;
  int pid = blockIdx.x;
  {
    const int xcd = pid & 7, local = pid >> 3;
    const int per = num_wg >> 3, rem = num_wg & 7;
    pid = xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
  }
  const int in_group = group_m * tiles_n;
  const int first_m = (pid / in_group) * group_m;
  const int gm = min(tiles_m - first_m, group_m);
  const int tm = first_m + (pid % in_group) % gm;
  const int tn = (pid % in_group) / gm;
  const int64_t m0 = static_cast<int64_t>(tm) * BM;
  const int64_t n0 = static_cast<int64_t>(tn) * BN;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int wm = wave / WGN, wn = wave % WGN;
  const int64_t col_tiles = kp >> 7;
  const int nk = static_cast<int>(kp / kBK);

  // ---- per-lane source offsets for the LDS-direct loads ----
  // Segment g of a tile holds tile rows [8g, 8g+8); lane l writes 16 bytes at LDS offset
  // 16 l of that segment, i.e. row 8g + l/8, physical chunk l%8, so it must fetch
  // logical chunk (l%8) ^ ((row >> 1) & 7). Offsets are 32-bit and relative to the tile's
  // first row (the host guarantees BM * kp < 2^31); rows past the padded end are clamped.
  const uint8_t* a_tile = A + m0 * kp;
  const uint8_t* w_tile = W + n0 * kp;
  const int seg_row = lane >> 3;
  // With an even wave count every segment a lane loads has the same (row >> 1) & 7.
  static_assert(kWaves % 2 == 0, "chunk swizzle assumes an even wave count");
  const uint32_t logical16 = ((lane & 7) ^ (((wave * 8 + seg_row) >> 1) & 7)) * 16;
  const int a_last = static_cast<int>(min<int64_t>(BM, mp - m0)) - 1;
  const int b_last = static_cast<int>(min<int64_t>(BN, np - n0)) - 1;
  const uint32_t kpu = static_cast<uint32_t>(kp);
  // Scale runs: wave w loads runs w, w + kWaves, ... (two 256-byte dword DMAs each); row
  // blocks past the padded end are clamped (their rows are never stored).
  constexpr int kARuns = BM / 128, kRuns = (BM + BN) / 128;
  const int64_t a_blocks = mp >> 7, w_blocks = np >> 7;
  auto issue_scale_loads = [&](int ks, int buf) {
#pragma unroll
    for (int run = wave; run < kRuns; run += kWaves) {
      const bool is_a = run < kARuns;
      const int blk = is_a ? run : run - kARuns;
      const int64_t row_block = is_a ? min<int64_t>((m0 >> 7) + blk, a_blocks - 1)
                                     : min<int64_t>((n0 >> 7) + blk, w_blocks - 1);
      const uint8_t* src = (is_a ? As : Ws) + (row_block * col_tiles + ks) * 512 + lane * 4;
      uint8_t* dst = &lds[buf][kScaleOff + run * 512];
      load_to_lds4(src, dst);
      load_to_lds4(src + 256, dst + 256);
    }
  };
  // Tile segment `seg` (0 .. kASegs + kBSegs - 1) of K step ks: 8 rows x 128 bytes.
  auto issue_segment = [&](int ks, int buf, int seg) {
    if (seg < kASegs) {
      const uint32_t row = min((seg * kWaves + wave) * 8 + seg_row, a_last);
      load_to_lds16(a_tile + static_cast<int64_t>(ks) * kBK + (row * kpu + logical16),
                    &lds[buf][(seg * kWaves + wave) * 1024]);
    } else {
      const int i = seg - kASegs;
      const uint32_t row = min((i * kWaves + wave) * 8 + seg_row, b_last);
      load_to_lds16(w_tile + static_cast<int64_t>(ks) * kBK + (row * kpu + logical16),
                    &lds[buf][BM * kBK + (i * kWaves + wave) * 1024]);
    }
  };
  auto issue_loads = [&](int ks, int buf) {
    issue_scale_loads(ks, buf);
#pragma unroll
    for (int seg = 0; seg < kASegs + kBSegs; ++seg) issue_segment(ks, buf, seg);
  };

  const int frag_row = lane & 15;
  const int block_shift = 8 * (lane >> 4);
  int a_sidx[TM], b_sidx[TN];  // LDS offsets of this lane's scale dwords within a step buffer
#pragma unroll
  for (int mt = 0; mt < TM; ++mt) {
    const int r = wm * WM + mt * 16 + frag_row;
    a_sidx[mt] = kScaleOff + (r >> 7) * 512 + scale_in_block(r);
  }
#pragma unroll
  for (int nt = 0; nt < TN; ++nt) {
    const int r = wn * WN + nt * 16 + frag_row;
    b_sidx[nt] = kScaleOff + (kARuns + (r >> 7)) * 512 + scale_in_block(r);
  }

  f32x4 acc[TM][TN];
#pragma unroll
  for (int mt = 0; mt < TM; ++mt)
#pragma unroll
    for (int nt = 0; nt < TN; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

  issue_loads(0, 0);

  // Step ks: wait for tile ks (issued one step earlier) and for every wave to have finished
  // reading the other buffer, then prefetch tile ks + 1 into it and run the MFMAs of tile ks.
  // The wait sits at the top of the step so the MFMAs are the last instructions of the
  // loop body: nothing can sink them below the wait, and the prefetch overlaps them.
  const int c_lo = lane >> 4;  // 16-byte chunks g and g + 4 of the 128-byte K step
  auto step = [&](int ks, auto more_tag) {
    constexpr bool more = decltype(more_tag)::value;
    const int buf = ks & 1;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if constexpr (more) issue_scale_loads(ks + 1, buf ^ 1);
    uint32_t sa[TM], sb[TN];
    if constexpr (WM == 128 && WN == 128) {
      // Rows 16 mt + frag_row of a 128-row wave tile: the even-mt words are the 16 bytes at
      // a_sidx[0] and the odd-mt words the 16 bytes at a_sidx[1], so four 16-byte reads
      // fetch every scale word of the step before any fragment read.
      const u32x4 ae = *reinterpret_cast<const u32x4*>(&lds[buf][a_sidx[0]]);
      const u32x4 ao = *reinterpret_cast<const u32x4*>(&lds[buf][a_sidx[1]]);
      const u32x4 be = *reinterpret_cast<const u32x4*>(&lds[buf][b_sidx[0]]);
      const u32x4 bo = *reinterpret_cast<const u32x4*>(&lds[buf][b_sidx[1]]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sa[2 * i] = ae[i] >> block_shift;
        sa[2 * i + 1] = ao[i] >> block_shift;
        sb[2 * i] = be[i] >> block_shift;
        sb[2 * i + 1] = bo[i] >> block_shift;
      }
    } else {
#pragma unroll
      for (int mt = 0; mt < TM; ++mt)
        sa[mt] = *reinterpret_cast<const uint32_t*>(&lds[buf][a_sidx[mt]]) >> block_shift;
#pragma unroll
      for (int nt = 0; nt < TN; ++nt)
        sb[nt] = *reinterpret_cast<const uint32_t*>(&lds[buf][b_sidx[nt]]) >> block_shift;
    }
    const uint8_t* abuf = lds[buf];
    const uint8_t* bbuf = lds[buf] + BM * kBK;
    auto frag = [&](const uint8_t* base, int row) {
      const int sw = (row >> 1) & 7;
      const i32x4 lo = *reinterpret_cast<const i32x4*>(base + row * kBK + ((c_lo ^ sw) << 4));
      const i32x4 hi = *reinterpret_cast<const i32x4*>(base + row * kBK + (((c_lo + 4) ^ sw) << 4));
      return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };
    // All B fragments stay in registers for the step; A fragments are read one ahead, so the
    // first MFMA waits for two fragments only. The next tile's segments are issued between
    // the MFMA groups, which spreads their address work over the step.
    constexpr int kSegs = kASegs + kBSegs;
    constexpr int kSegsPerGroup = (kSegs + TM - 1) / TM;
    i32x8 acur = frag(abuf, wm * WM + frag_row);
    i32x8 bfrag[TN];
#pragma unroll
    for (int nt = 0; nt < TN; ++nt) bfrag[nt] = frag(bbuf, wn * WN + nt * 16 + frag_row);
#pragma unroll
    for (int mt = 0; mt < TM; ++mt) {
      i32x8 anext = acur;
      if (mt + 1 < TM) anext = frag(abuf, wm * WM + (mt + 1) * 16 + frag_row);
      // The next A fragment's reads stay ahead of this group's MFMAs (the scheduler would
      // otherwise sink them below, making the next group wait on their full latency).
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int nt = 0; nt < TN; ++nt) {
        // D = W_frag . A_frag^T: lane l then holds output columns 4(l/16)..+3 of row l%16
        acc[mt][nt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
            bfrag[nt], acur, acc[mt][nt], 0, 0, 0, static_cast<int>(sb[nt]), 0,
            static_cast<int>(sa[mt]));
      }
      if constexpr (more) {
#pragma unroll
        for (int j = 0; j < kSegsPerGroup; ++j)
          if (mt * kSegsPerGroup + j < kSegs) issue_segment(ks + 1, buf ^ 1, mt * kSegsPerGroup + j);
      }
      __builtin_amdgcn_sched_barrier(0);
      acur = anext;
    }
  };
  for (int ks = 0; ks + 1 < nk; ++ks) step(ks, std::true_type{});
  step(nk - 1, std::false_type{});

  // ---- epilogue 1: bf16(acc) staged row-major in LDS ----
  // Lane l holds, for each (mt, nt), tile row wm*WM + mt*16 + l%16 and the four
  // consecutive columns wn*WN + nt*16 + 4(l/16) .. +3.
  __syncthreads();  // every wave is done reading the K-step buffers
#pragma unroll
  for (int mt = 0; mt < TM; ++mt) {
    const int row = wm * WM + mt * 16 + frag_row;
#pragma unroll
    for (int nt = 0; nt < TN; ++nt) {
      const int col = wn * WN + nt * 16 + 4 * (lane >> 4);
      u32x2 packed;
      packed[0] = pack_bf16x2(round_bf16(acc[mt][nt][0]), round_bf16(acc[mt][nt][1]));
      packed[1] = pack_bf16x2(round_bf16(acc[mt][nt][2]), round_bf16(acc[mt][nt][3]));
      *reinterpret_cast<u32x2*>(lds_raw + row * kStageStride + col * 2) = packed;
    }
  }
  __syncthreads();

  // ---- epilogue 2: each lane finishes 8 consecutive outputs of a row per pass ----
  constexpr int kThreads = kWaves * 64;
  constexpr int kChunksPerRow = BN / 8;
  constexpr int kRowsPerPass = kThreads / kChunksPerRow;
  static_assert(kThreads % kChunksPerRow == 0 && BM % kRowsPerPass == 0, "epilogue mapping");
  const int chunk = tid % kChunksPerRow;
  const int64_t col = n0 + chunk * 8;
  bool bad = false;
  float bias8[8], gate8[8];
  if (ep.vec && col + 8 <= n) {
    if (ep.bias != nullptr) unpack8(*reinterpret_cast<const u32x4*>(ep.bias + col), bias8);
    if (ep.gate != nullptr) unpack8(*reinterpret_cast<const u32x4*>(ep.gate + col), gate8);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bool in = col + e < n;
      bias8[e] = ep.bias != nullptr && in ? bf16_bits_to_f32(ep.bias[col + e]) : 0.f;
      gate8[e] = ep.gate != nullptr && in ? bf16_bits_to_f32(ep.gate[col + e]) : 1.f;
    }
  }
  constexpr int kPasses = BM / kRowsPerPass;
  constexpr int kBatch = kPasses < 8 ? kPasses : 8;
  static_assert(kPasses % kBatch == 0, "epilogue batching");
  if (ep.q_out != nullptr) {
    // Eight consecutive columns per lane; the four lanes of a 32-column block and the
    // sixteen of a 128-column chunk are consecutive lanes of one row (kChunksPerRow is a
    // multiple of 16), which is the lane layout quantize_store8 expects.
    static_assert(kChunksPerRow % 16 == 0, "producer epilogue lane layout");
    const int64_t chunk128 = (n0 >> 7) + (chunk >> 4);
    // a 256-wide tile can reach past the padded output (rows >= mp, chunks >= kp_out / 128);
    // both tests are uniform over the 16 lanes of a chunk
    const bool chunk_in = chunk128 < (ep.kp_out >> 7);
    for (int pass = 0; pass < kPasses; ++pass) {
      const int r = pass * kRowsPerPass + tid / kChunksPerRow;
      const int64_t row = m0 + r;
      if (row >= mp || !chunk_in) continue;
      float y[8];
      unpack8(*reinterpret_cast<const u32x4*>(lds_raw + r * kStageStride + chunk * 16), y);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float v = 0.f;
        if (row < out_rows && col + e < n) {
          v = ep.bias != nullptr ? round_bf16(y[e] + bias8[e]) : y[e];
          if (ep.act == 1) v = round_bf16(gelu_tanh(v));
          bad = bad || !(fabsf(v) < INFINITY);
        }
        y[e] = v;
      }
      quantize_store8(y, tid & 15, row, chunk128, ep.kp_out, ep.q_out, ep.s_out);
    }
  } else if (ep.vec && col + 8 <= n) {
    // Batches of kBatch rows: every load of a batch is issued before any arithmetic, so
    // the addend/residual latency is paid once per batch rather than once per row.
    for (int b0 = 0; b0 < kPasses; b0 += kBatch) {
      u32x4 yv[kBatch], av[kBatch], rv[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int r = (b0 + j) * kRowsPerPass + tid / kChunksPerRow;
        const int64_t row = m0 + r;
        yv[j] = *reinterpret_cast<const u32x4*>(lds_raw + r * kStageStride + chunk * 16);
        if (row < out_rows) {
          if (ep.addend != nullptr)
            av[j] = *reinterpret_cast<const u32x4*>(ep.addend + row * ep.ld_add + col);
          if (ep.residual != nullptr)
            rv[j] = *reinterpret_cast<const u32x4*>(ep.residual + row * ep.ld_res + col);
        }
      }
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int r = (b0 + j) * kRowsPerPass + tid / kChunksPerRow;
        const int64_t row = m0 + r;
        if (row >= out_rows) continue;
        float y[8], add[8], res[8];
        unpack8(yv[j], y);
        if (ep.addend != nullptr) unpack8(av[j], add);
        if (ep.residual != nullptr) unpack8(rv[j], res);
        u32x4 packed;
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          const float y0 = epilogue_value(y[e], bias8[e], add[e], res[e], gate8[e], ep);
          const float y1 = epilogue_value(y[e + 1], bias8[e + 1], add[e + 1], res[e + 1],
                                          gate8[e + 1], ep);
          bad = bad || !(fabsf(y0) < INFINITY) || !(fabsf(y1) < INFINITY);
          packed[e / 2] = pack_bf16x2(y0, y1);
        }
        *reinterpret_cast<u32x4*>(ep.out + row * ep.ldc + col) = packed;
      }
    }
  } else if (col < n) {
    for (int pass = 0; pass < kPasses; ++pass) {
      const int r = pass * kRowsPerPass + tid / kChunksPerRow;
      const int64_t row = m0 + r;
      if (row >= out_rows) continue;
      float y[8];
      unpack8(*reinterpret_cast<const u32x4*>(lds_raw + r * kStageStride + chunk * 16), y);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (col + e >= n) continue;
        const float a = ep.addend != nullptr ? bf16_bits_to_f32(ep.addend[row * ep.ld_add + col + e]) : 0.f;
        const float rs = ep.residual != nullptr ? bf16_bits_to_f32(ep.residual[row * ep.ld_res + col + e]) : 0.f;
        const float v = epilogue_value(y[e], bias8[e], a, rs, gate8[e], ep);
        bad = bad || !(fabsf(v) < INFINITY);
        ep.out[row * ep.ldc + col + e] = f32_to_bf16_bits(v);
      }
    }
  }
  if (ep.nonfinite != nullptr && __ballot(bad) != 0 && lane == 0) atomicOr(ep.nonfinite, 1u);
}

// ---------------------------------------------------------------------------------------
// Persistent 256 x 256 kernel (the large-problem path).
//
// One workgroup per CU walks its tiles (XCD-contiguous order as above) with one K-step
// pipeline that runs across tile boundaries: step s of the workgroup's (tile, K step)
// sequence lives in LDS buffer s % 2. Each step has one barrier, in the middle:
//   head  A groups mt < kHead: 8 MFMAs each against all 8 B fragments (in registers),
//         reading the remaining A fragments of the step;
//   mid   wait for step s+1's tiles (DMA issued one step earlier) and barrier: every wave
//         is then done reading buffer s % 2 and buffer (s+1) % 2 is complete;
//   tail  A groups mt >= kHead in N order: after the MFMAs of B fragment nt, fragment nt of
//         step s+1 is read into the same registers; step s+2's tiles are DMA'd into buffer
//         s % 2, one segment after the first and one after the third MFMA of each column
//         (a DMA issue stalls while the CU's address unit is busy; issued in the shadow of
//         queued MFMAs it costs less than in bursts).
// So the next step starts with its B fragments and first A fragment already in registers,
// and a tile's epilogue (straight from the accumulators: 8-byte bf16 or 4-byte MXFP8 stores)
// runs while the next tile's first steps are in flight.
// Tiles are fetched with buffer_load ... lds through buffer resources (rows past the padded
// end read as zero; see buffer_to_lds16).
constexpr int kPTile = 256;
constexpr int kPScaleOff = 2 * kPTile * kBK;                 // A tile, then W tile
constexpr int kPStep = kPScaleOff + 2 * kPTile * 4;          // + four 512-byte scale runs
constexpr int kPStageStride = 272;                           // 128 bf16 + 16 pad bytes
constexpr int kPStageBytes = 16 * kPStageStride;             // one wave's 16-row strip

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const int64_t n = bytes < 0x7fffffffll ? bytes : 0x7fffffffll;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(n),
                                           0x00020000);
}

// LDS DMA through a buffer resource: lane l's 16 (4) bytes at voffset land at LDS byte
// lds_base + 16 l (4 l). The compiler sets M0 to the wave's LDS base itself (with the wait
// state an M0 write needs before an LDS DMA) and counts these loads on vmcnt only: the
// fragment reads of the other step buffer keep their exact lgkmcnt waits, and the kernel
// orders the step buffers with its own vmcnt waits before its barriers.
__device__ __forceinline__ void buffer_to_lds16(__amdgpu_buffer_rsrc_t r, uint32_t voffset,
                                                void* lds_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)lds_base, 16, voffset, 0, 0, 0);
}

__device__ __forceinline__ void buffer_to_lds4(__amdgpu_buffer_rsrc_t r, uint32_t voffset,
                                               void* lds_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)lds_base, 4, voffset, 0, 0, 0);
}

// Virtual tile id b (b % 8 is the XCD that runs it) -> (tile row, tile column).
__device__ __forceinline__ void tile_coords(int b, int num_wg, int tiles_m, int tiles_n,
                                            int group_m, int& tm, int& tn) {
  const int xcd = b & 7, local = b >> 3;
  const int per = num_wg >> 3, rem = num_wg & 7;
  const int pid = xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
  const int in_group = group_m * tiles_n;
  const int first_m = (pid / in_group) * group_m;
  const int gm = min(tiles_m - first_m, group_m);
  tm = first_m + (pid % in_group) % gm;
  tn = (pid % in_group) / gm;
}

// Empty asm statements that take accumulators as operands: the MFMAs producing them are
// then issued before the statement, and memory operations stay on their side of it
// ("memory" clobber). This keeps each MFMA group between the LDS reads and the barrier
// it is meant to overlap; without it the pure MFMA calls may be sunk past the barrier.
__device__ __forceinline__ void pin_group(const f32x4 (&g)[8]) {
  asm volatile("" ::"a"(g[0]), "a"(g[1]), "a"(g[2]), "a"(g[3]), "a"(g[4]), "a"(g[5]), "a"(g[6]),
               "a"(g[7]) : "memory");
}

template <int kFirst>
__device__ __forceinline__ void pin_column_from(const f32x4 (&acc)[8][8], int nt) {
#pragma unroll
  for (int mt = kFirst; mt < 8; ++mt) asm volatile("" ::"a"(acc[mt][nt]) : "memory");
}

// kMode: 0 bf16 output, 1 bf16 output with a residual (Epilogue::residual, prefetched one
// row group ahead), 2 the MXFP8 producer epilogue (Epilogue::q_out, act 0 / 1), 3 the SwiGLU
// producer epilogue (act 2, interleaved weight). The bf16 modes need 16-byte accesses
// (Epilogue::vec) and no addend.
template <int kHead, int kMode>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
mxfp8_gemm_persistent_kernel(const uint8_t* __restrict__ A, const uint8_t* __restrict__ As,
                             const uint8_t* __restrict__ W, const uint8_t* __restrict__ Ws,
                             int64_t mp, int64_t np, int64_t kp, Epilogue ep, int64_t out_rows,
                             int64_t n, int tiles_m, int tiles_n, int group_m) {
  constexpr int TM = 8, TN = 8;
  static_assert(kHead >= 1 && kHead + 2 < TM, "head groups");
  // after the two step buffers: the bf16 modes' staging strips, or the producer's SwiGLU
  // hand-over slots (2 wave pairs x 64 lanes x 32 fp32)
  __shared__ __attribute__((aligned(1024))) uint8_t
      lds[2 * kPStep + (kMode == 3 ? 2 * 64 * 32 * 4 : kMode == 2 ? 0 : 4 * kPStageBytes)];

  const int num_wg = tiles_m * tiles_n;
  const int grid = gridDim.x;
  const int my_tiles = (num_wg - static_cast<int>(blockIdx.x) + grid - 1) / grid;
  const int nk = static_cast<int>(kp / kBK);
  const int total_steps = my_tiles * nk;
  const int64_t col_tiles = kp >> 7;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  // ---- DMA side: a cursor over the workgroup's (tile, K step) sequence ----
  // Segment i of a tile (i < 8: A rows, else W rows) is rows 32 (i % 8) + 8 wave + lane / 8;
  // lane l writes 16 bytes at LDS offset 16 l of its 1 KB slot, i.e. physical chunk l % 8,
  // so it fetches logical chunk (l % 8) ^ ((row >> 1) & 7), the same for every segment.
  const int seg_row = lane >> 3;
  const uint32_t kpu = static_cast<uint32_t>(kp);
  const uint32_t dma_voff =
      (wave * 8 + seg_row) * kpu + ((lane & 7) ^ (((wave * 8 + seg_row) >> 1) & 7)) * 16;
  const __amdgpu_buffer_rsrc_t as_rsrc = make_rsrc(As, mp * kp / 32);
  const __amdgpu_buffer_rsrc_t ws_rsrc = make_rsrc(Ws, np * kp / 32);
  int d_step = 0, d_tile = 0, d_ks = 0;
  int64_t d_m0 = 0, d_n0 = 0;
  __amdgpu_buffer_rsrc_t d_a, d_w;
  auto dma_tile = [&](int j) __attribute__((always_inline)) {
    int tm, tn;
    tile_coords(static_cast<int>(blockIdx.x) + j * grid, num_wg, tiles_m, tiles_n, group_m, tm, tn);
    d_m0 = static_cast<int64_t>(tm) * kPTile;
    d_n0 = static_cast<int64_t>(tn) * kPTile;
    d_a = make_rsrc(A + d_m0 * kp, (mp - d_m0) * kp);
    d_w = make_rsrc(W + d_n0 * kp, (np - d_n0) * kp);
  };
  // Past the last step the cursor stays on it: those DMAs rewrite a buffer whose reads are
  // finished with the same bytes, and the workgroup waits for them before it exits.
  auto dma_advance = [&]() __attribute__((always_inline)) {
    if (d_step + 1 < total_steps) {
      ++d_step;
      if (++d_ks == nk) {
        d_ks = 0;
        dma_tile(++d_tile);
      }
    }
  };
  auto dma_scales = [&](uint8_t* buf) __attribute__((always_inline)) {
    // wave w loads run w: A 128-row blocks 0, 1, then W blocks 0, 1 (two 256-byte DMAs)
    const bool is_a = wave < 2;
    const int64_t blk = (is_a ? d_m0 : d_n0) / 128 + (wave & 1);
    const uint32_t off = static_cast<uint32_t>((blk * col_tiles + d_ks) * 512) + lane * 4;
    uint8_t* dst = buf + kPScaleOff + wave * 512;
    buffer_to_lds4(is_a ? as_rsrc : ws_rsrc, off, dst);
    buffer_to_lds4(is_a ? as_rsrc : ws_rsrc, off + 256, dst + 256);
  };
  auto dma_segment = [&](uint8_t* buf, int seg) __attribute__((always_inline)) {
    const uint32_t off = dma_voff + static_cast<uint32_t>(d_ks) * kBK + (seg & 7) * 32 * kpu;
    if (seg < 8)
      buffer_to_lds16(d_a, off, buf + ((seg & 7) * 4 + wave) * 1024);
    else
      buffer_to_lds16(d_w, off, buf + kPTile * kBK + ((seg & 7) * 4 + wave) * 1024);
  };

  // ---- consumer side ----
  const int frag_row = lane & 15;
  const int c_lo = lane >> 4;
  const int block_shift = 8 * c_lo;
  auto frag = [&](const uint8_t* base, int row) __attribute__((always_inline)) {
    const int sw = (row >> 1) & 7;
    const i32x4 lo = *reinterpret_cast<const i32x4*>(base + row * kBK + ((c_lo ^ sw) << 4));
    const i32x4 hi = *reinterpret_cast<const i32x4*>(base + row * kBK + (((c_lo + 4) ^ sw) << 4));
    return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  };
  // Scale words of rows 16 mt + frag_row of the wave tile: even mt in the 16 bytes at
  // `ae`, odd mt at `ao` (SWIZZLE_32_4_4 run layout); the same for W.
  const int sa_off = kPScaleOff + wm * 512 + frag_row * 16;
  const int sb_off = kPScaleOff + (2 + wn) * 512 + frag_row * 16;
  u32x4 ae, ao, be, bo;
  auto read_scales = [&](const uint8_t* buf) __attribute__((always_inline)) {
    ae = *reinterpret_cast<const u32x4*>(buf + sa_off);
    ao = *reinterpret_cast<const u32x4*>(buf + sa_off + 256);
    be = *reinterpret_cast<const u32x4*>(buf + sb_off);
    bo = *reinterpret_cast<const u32x4*>(buf + sb_off + 256);
  };
  uint32_t sa[TM], sb[TN];
  auto unpack_scales = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sa[2 * i] = ae[i] >> block_shift;
      sa[2 * i + 1] = ao[i] >> block_shift;
      sb[2 * i] = be[i] >> block_shift;
      sb[2 * i + 1] = bo[i] >> block_shift;
    }
  };

  f32x4 acc[TM][TN];

  bool bad = false;
  u16x2 mag_max = {0, 0};   // bf16 output modes: largest magnitude bit pattern stored

  // ---- producer epilogue of one tile (kMode 2), straight from the accumulators ----
  // acc[mt][nt][v] is C[m0 + 128 wm + 16 mt + r][n0 + 128 wn + 16 nt + 4 g + v] with r = lane % 16
  // and g = lane / 16: each lane holds 4 consecutive columns of one row, and a 4 x 4 lane
  // transpose of the code words gives each of the row's 4 lanes 16 contiguous code bytes (two
  // 16-byte stores per row group), with no LDS staging. A 32-column block is nt = 2b, 2b + 1 of
  // the four lanes g of a row (two permlane swaps give its amax), and the wave's 128 columns
  // are one MXFP8 chunk, whose 4 scale bytes are one dword of the swizzled layout.
  // SwiGLU (ep.act 2) reads W with its a and g halves interleaved in 128-row blocks: block j
  // of a is W rows [256 j, 256 j + 128), block j of g the next 128. A 256-column tile then
  // holds a-block j in wave column wn = 0 and g-block j in wn = 1, for the same rows: the g
  // wave passes g * sigmoid(g) of its values through an 8 KB LDS slot per wave pair (lane
  // l's 32 values at its own offset, the a wave's lane l reads them), and the a wave forms
  // bf16(a * that), quantizes and stores output chunk j. Bias is interleaved the same way.
  constexpr bool swiglu = kMode == 3;
  float* pass_slot = reinterpret_cast<float*>(lds + 2 * kPStep) + (wm * 64 + lane) * 32;
  // kGelu (compile time) applies GELU-tanh: with a runtime test of the activation inside the
  // unrolled value loop, the compiler branched around every pair's GELU, so the exp2 and
  // reciprocal latencies of neighbouring pairs could not overlap.
  auto epilogue_direct = [&](int64_t m0, int64_t n0, auto gelu_tag) __attribute__((always_inline)) {
    constexpr bool kGelu = decltype(gelu_tag)::value;
    const int64_t col0 = n0 + wn * 128 + c_lo * 4;       // + 16 nt (physical columns)
    const int64_t rows0 = m0 + wm * 128 + frag_row;      // + 16 mt
    // the output columns of the lane: physical for GELU / none, block j of a for SwiGLU
    const int64_t ocol0 = swiglu ? (n0 >> 1) + c_lo * 4 : col0;
    const int64_t n_phys = swiglu ? 2 * ep.kp_out : n;
    // bias of the lane's 32 columns; a missing bias is -0: bf16(y + -0) = y exactly
    float bias4[TN][4];
#pragma unroll
    for (int nt = 0; nt < TN; ++nt) {
      const int64_t col = col0 + nt * 16;
#pragma unroll
      for (int v = 0; v < 4; ++v) bias4[nt][v] = -0.f;
      if (ep.bias == nullptr) continue;
      if ((ep.vec || swiglu) && col < n_phys) {   // the lane's 4 columns are all inside
        unpack4(*reinterpret_cast<const u32x2*>(ep.bias + col), bias4[nt]);
      } else if (!ep.vec && !swiglu) {
#pragma unroll
        for (int v = 0; v < 4; ++v)
          if (col + v < n) bias4[nt][v] = bf16_bits_to_f32(ep.bias[col + v]);
      }
    }
    const int64_t chunk128 = swiglu ? n0 >> 8 : (n0 + wn * 128) >> 7;
    const bool chunk_in = chunk128 < (ep.kp_out >> 7);
    // every row and column of the tile inside the output: no per-value bounds selects
    const bool interior = m0 + kPTile <= out_rows && n0 + kPTile <= n;
    // A rolled loop over the 8 row groups keeps one copy of the code; the accumulators
    // (registers) are picked by a uniform branch chain, not indexed.
#pragma nounroll
    for (int mt = 0; mt < TM; ++mt) {
      // y = bf16(acc)
      float y[TN][4];
#pragma unroll
      for (int m = 0; m < TM; ++m) {
        if (m != mt) continue;
#pragma unroll
        for (int nt = 0; nt < TN; ++nt) {
          f32x4 a = acc[m][nt];
          // the copy is opaque: the rounding below stays in this branch instead of being
          // hoisted (for all 256 accumulators at once) out of the loop; so is the packed
          // pair, which is then unpacked rather than each value converted on its own
          asm volatile("" : "+v"(a));
          u32x2 p;
          p[0] = pack_bf16x2(a[0], a[1]);
          p[1] = pack_bf16x2(a[2], a[3]);
          asm volatile("" : "+v"(p));
          unpack4(p, y[nt]);
        }
      }
      const int64_t row = rows0 + mt * 16;
      if constexpr (swiglu) {
        // bf16(acc + bias) of both halves; the g wave hands over g * sigmoid(g)
        if (wn == 1) {
#pragma unroll
          for (int nt = 0; nt < TN; ++nt) {
            f32x4 gs;
#pragma unroll
            for (int v = 0; v < 4; v += 2) {
              float g0 = y[nt][v] + bias4[nt][v], g1 = y[nt][v + 1] + bias4[nt][v + 1];
              round_bf16_pair(g0, g1);
              gs[v] = swiglu_gate(g0);
              gs[v + 1] = swiglu_gate(g1);
            }
            *reinterpret_cast<f32x4*>(pass_slot + nt * 4) = gs;
          }
        }
        __syncthreads();
        if (wn == 0) {
#pragma unroll
          for (int nt = 0; nt < TN; ++nt) {
            const f32x4 gs = *reinterpret_cast<const f32x4*>(pass_slot + nt * 4);
#pragma unroll
            for (int v = 0; v < 4; v += 2) {
              float a0 = y[nt][v] + bias4[nt][v], a1 = y[nt][v + 1] + bias4[nt][v + 1];
              round_bf16_pair(a0, a1);
              a0 *= gs[v];
              a1 *= gs[v + 1];
              round_bf16_pair(a0, a1);
              y[nt][v] = a0;
              y[nt][v + 1] = a1;
            }
          }
          if (ep.nonfinite != nullptr) {
#pragma unroll
            for (int nt = 0; nt < TN; ++nt)
#pragma unroll
              for (int v = 0; v < 4; ++v) bad = bad || !(fabsf(y[nt][v]) < INFINITY);
          }
#pragma unroll
          for (int nt = 0; nt < TN; ++nt)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              const bool in = row < out_rows && ocol0 + nt * 16 + v < n;
              y[nt][v] = in ? y[nt][v] : 0.f;
            }
        }
        __syncthreads();   // the slot is free for the next row group
        if (wn == 1) continue;   // the a wave quantizes and stores the chunk
      } else {
        // bias, activation and bf16 rounding, two values at a time; rows >= out_rows and
        // columns >= n are zero (tested only on tiles that reach past the output)
#pragma unroll
        for (int nt = 0; nt < TN; ++nt)
#pragma unroll
          for (int v = 0; v < 4; v += 2) {
            float a = y[nt][v] + bias4[nt][v], b = y[nt][v + 1] + bias4[nt][v + 1];
            round_bf16_pair(a, b);
            if constexpr (kGelu) {
              a = gelu_tanh(a);
              b = gelu_tanh(b);
              round_bf16_pair(a, b);
            }
            y[nt][v] = a;
            y[nt][v + 1] = b;
          }
        if (ep.nonfinite != nullptr) {
#pragma unroll
          for (int nt = 0; nt < TN; ++nt)
#pragma unroll
            for (int v = 0; v < 4; ++v) bad = bad || !(fabsf(y[nt][v]) < INFINITY);
        }
        if (!interior) {
#pragma unroll
          for (int nt = 0; nt < TN; ++nt)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              const bool in = row < out_rows && col0 + nt * 16 + v < n;
              y[nt][v] = in ? y[nt][v] : 0.f;
            }
        }
      }
      // every lane takes part in the block maxima and the code transposes; only the stores
      // are predicated (uniform over the 4 lanes of a row)
      const bool store = chunk_in && row < mp;
      uint32_t word = 0;
      uint32_t cw[TN];   // codes of columns 16 nt + 4 c_lo .. + 4
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        float amax = 0.f;
#pragma unroll
        for (int nt = 2 * b; nt < 2 * b + 2; ++nt)
#pragma unroll
          for (int v = 0; v < 4; ++v) amax = fmaxf(amax, fabsf(y[nt][v]));
        amax = max_quad_rows(amax);
        float sinv;
        const uint32_t byte = e8m0_from_amax(amax, &sinv);
        word |= byte << (8 * b);
        const float sf = e8m0_scale(byte);
#pragma unroll
        for (int nt = 2 * b; nt < 2 * b + 2; ++nt)
          cw[nt] = e4m3x4_scaled(y[nt][0], y[nt][1], y[nt][2], y[nt][3], sf);
      }
      // 4 x 4 transpose of code words over the row's 4 lanes (c_lo = lane / 16): afterwards
      // lane c_lo holds word c' of column group 4 q + c_lo from lane c', i.e. the 16
      // contiguous code bytes of columns 16 (4 q + c_lo) ..; c_lo bit 1 first (lanes 32
      // apart, v_permlane32_swap), then bit 0 (16 apart, v_permlane16_swap). Each swap
      // gives lane l < 32 (row 2 j) lane l + 32's (row 2 j + 1's) vdst in vsrc and that lane
      // l's vsrc in vdst, so the returned pair is the new words k, k + 2 (k, k + 1).
#pragma unroll
      for (int qg = 0; qg < 2; ++qg) {
        uint32_t* w4 = cw + 4 * qg;
        const auto a02 = __builtin_amdgcn_permlane32_swap(w4[0], w4[2], false, false);
        const auto a13 = __builtin_amdgcn_permlane32_swap(w4[1], w4[3], false, false);
        const auto b01 = __builtin_amdgcn_permlane16_swap(a02[0], a13[0], false, false);
        const auto b23 = __builtin_amdgcn_permlane16_swap(a02[1], a13[1], false, false);
        const u32x4 out16 = {b01[0], b01[1], b23[0], b23[1]};
        if (store)
          *reinterpret_cast<u32x4*>(ep.q_out + row * ep.kp_out + chunk128 * 128 +
                                    16 * (4 * qg + c_lo)) = out16;
      }
      if (store && c_lo == 0)
        *reinterpret_cast<uint32_t*>(
            ep.s_out + swizzled_scale_offset(row, chunk128 * 4, ep.kp_out >> 7)) = word;
    }
  };

  // ---- bf16 epilogue of one tile (kModes 0, 1): per wave, 16 rows at a time through its LDS
  // strip, so that each lane stores 16 contiguous bytes ----
  uint8_t* stage = lds + 2 * kPStep + wave * kPStageBytes;
  auto epilogue_staged = [&](int64_t m0, int64_t n0) __attribute__((always_inline)) {
    const int chunk = lane & 15;                       // 8 columns of the wave's 128
    const int64_t col = n0 + wn * 128 + chunk * 8;
    // Bias and gate of the lane's 8 columns. A missing bias is -0 and a missing gate 1:
    // bf16(y + -0) = y and bf16(1 * y) = y exactly, so the arithmetic below needs no
    // per-element tests.
    float bias8[8], gate8[8];
    if (ep.vec && col + 8 <= n) {
      u32x4 bw = {0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u};
      u32x4 gw = {0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
      if (ep.bias != nullptr) bw = *reinterpret_cast<const u32x4*>(ep.bias + col);
      if (ep.gate != nullptr) gw = *reinterpret_cast<const u32x4*>(ep.gate + col);
      unpack8(bw, bias8);
      unpack8(gw, gate8);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const bool in = col + e < n;
        bias8[e] = ep.bias != nullptr && in ? bf16_bits_to_f32(ep.bias[col + e]) : -0.f;
        gate8[e] = ep.gate != nullptr && in ? bf16_bits_to_f32(ep.gate[col + e]) : 1.f;
      }
    }
    // The residual rows of row group mt+1 are loaded while group mt is finished, so their
    // latency is paid once per tile rather than once per group.
    const int64_t rows0 = m0 + wm * 128 + c_lo;   // + 16 mt + 4 pass
    u32x4 res_next[4];
    auto load_residual = [&](int mt, u32x4 (&r)[4]) __attribute__((always_inline)) {
      if (col >= n) return;
#pragma unroll
      for (int pass = 0; pass < 4; ++pass) {
        const int64_t row = rows0 + mt * 16 + pass * 4;
        if (row < out_rows)   // read once: a streaming load, like the output store
          r[pass] = __builtin_nontemporal_load(
              reinterpret_cast<const u32x4*>(ep.residual + row * ep.ld_res + col));
      }
    };
    if constexpr (kMode == 1) load_residual(0, res_next);
    // A rolled loop over the 8 row groups keeps one copy of the store code; the
    // accumulators (registers) are picked by a uniform branch chain, not indexed.
#pragma nounroll
    for (int mt = 0; mt < TM; ++mt) {
      u32x4 res_cur[4];
      if constexpr (kMode == 1) {
#pragma unroll
        for (int pass = 0; pass < 4; ++pass) res_cur[pass] = res_next[pass];
        if (mt + 1 < TM) load_residual(mt + 1, res_next);
      }
      // lane l holds columns nt * 16 + 4 (l / 16) .. +3 of strip row l % 16
#pragma unroll
      for (int m = 0; m < TM; ++m) {
        if (m != mt) continue;
#pragma unroll
        for (int nt = 0; nt < TN; ++nt) {
          f32x4 v = acc[m][nt];
          // the copy is opaque: the rounding below stays in this branch instead of being
          // hoisted (for all 256 accumulators at once) out of the loop
          asm volatile("" : "+v"(v));
          u32x2 packed;   // RNE to bf16 in the conversion itself
          packed[0] = pack_bf16x2(v[0], v[1]);
          packed[1] = pack_bf16x2(v[2], v[3]);
          *reinterpret_cast<u32x2*>(stage + frag_row * kPStageStride + nt * 32 + c_lo * 8) = packed;
        }
      }
      const int64_t row0 = rows0 + mt * 16;   // + 4 pass
      u32x4 yv[4];
#pragma unroll
      for (int pass = 0; pass < 4; ++pass)
        yv[pass] = *reinterpret_cast<const u32x4*>(stage + (pass * 4 + c_lo) * kPStageStride +
                                                   chunk * 16);
      if (col < n) {
#pragma unroll
        for (int pass = 0; pass < 4; ++pass) {
          const int64_t row = row0 + pass * 4;
          if (row >= out_rows) continue;
          float y[8];
          unpack8(yv[pass], y);
          float r[8];
          if constexpr (kMode == 1) unpack8(res_cur[pass], r);
          u32x4 packed;
#pragma unroll
          for (int e = 0; e < 8; e += 2) {
            // the last rounding of each value is the one of the packing conversion; the
            // residual form r + bf16(gate * bf16(v)) rounds two values at a time
            float v0 = y[e] + bias8[e], v1 = y[e + 1] + bias8[e + 1];
            if constexpr (kMode == 1) {
              round_bf16_pair(v0, v1);
              v0 *= gate8[e];
              v1 *= gate8[e + 1];
              round_bf16_pair(v0, v1);
              v0 += r[e];
              v1 += r[e + 1];
            }
            packed[e / 2] = pack_bf16x2(v0, v1);
          }
          // streaming store: the output is not read again here, and in L2 it would only evict
          // the A / W panels the next tiles need
          __builtin_nontemporal_store(packed, reinterpret_cast<u32x4*>(ep.out + row * ep.ldc + col));
          // nonfinite outputs: bf16 exponent all ones, tested on the packed words with a
          // running 16-bit max of the magnitudes (checked once at the end)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            mag_max = __builtin_elementwise_max(
                mag_max, __builtin_bit_cast(u16x2, packed[i] & 0x7fff7fffu));
        }
      }
    }
  };

  // ---- prologue: steps 0 and 1 in flight, step 0's fragments in registers ----
  dma_tile(0);
  dma_scales(lds);
#pragma unroll
  for (int seg = 0; seg < 16; ++seg) dma_segment(lds, seg);
  dma_advance();
  dma_scales(lds + kPStep);
#pragma unroll
  for (int seg = 0; seg < 16; ++seg) dma_segment(lds + kPStep, seg);
  dma_advance();
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  i32x8 bfrag[TN];
  i32x8 a0;
  // Fragments and scales of the step in buffer `buf`, read at a tile's start.
  auto load_fragments = [&](const uint8_t* buf) __attribute__((always_inline)) {
    read_scales(buf);
    unpack_scales();
#pragma unroll
    for (int nt = 0; nt < TN; ++nt) bfrag[nt] = frag(buf + kPTile * kBK, wn * 128 + nt * 16 + frag_row);
    a0 = frag(buf, wm * 128 + frag_row);
  };

  // The K steps of all the workgroup's tiles as one sequence: the tail of the last step of a
  // tile already reads the next tile's first fragments, but those are read again after the
  // epilogue (load_fragments), so no fragment register is live across the epilogue.
  int s = 0;
  for (int c_tile = 0; c_tile < my_tiles; ++c_tile) {
    load_fragments(lds + (s & 1) * kPStep);
#pragma unroll
    for (int mt = 0; mt < TM; ++mt)
#pragma unroll
      for (int nt = 0; nt < TN; ++nt) acc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int ks = 0; ks < nk; ++ks, ++s) {
      uint8_t* cur = lds + (s & 1) * kPStep;
      uint8_t* nxt = lds + ((s & 1) ^ 1) * kPStep;
      // head: A groups 0 .. kHead-1, each against all B fragments; the A fragments of the
      // tail groups are read with the last head group
      i32x8 af[TM];
      af[0] = a0;
#pragma unroll
      for (int mt = 0; mt < kHead; ++mt) {
        if (mt + 1 < kHead) {
          af[mt + 1] = frag(cur, wm * 128 + (mt + 1) * 16 + frag_row);
        } else {
#pragma unroll
          for (int t = kHead; t < TM; ++t) af[t] = frag(cur, wm * 128 + t * 16 + frag_row);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int nt = 0; nt < TN; ++nt)
          acc[mt][nt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              bfrag[nt], af[mt], acc[mt][nt], 0, 0, 0, static_cast<int>(sb[nt]), 0,
              static_cast<int>(sa[mt]));
        pin_group(acc[mt]);
      }
      // mid: step s+1's tiles have landed (its DMAs went out during step s-1) and every
      // wave is done reading this step's buffer
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      dma_scales(cur);
      a0 = frag(nxt, wm * 128 + frag_row);
      // tail: A groups kHead .. 7 in N order; B fragment nt of step s+1 replaces fragment
      // nt after its last MFMA here; step s+2's segments go out two per N column
#pragma unroll
      for (int nt = 0; nt < TN; ++nt) {
        // step s+1's scale words are read late: the current ones are mostly dead by then
        if (nt == TN - 2) read_scales(nxt);
        __builtin_amdgcn_sched_barrier(0);
        // the column's two DMA segments go out after its first and third MFMA, each in the
        // shadow of the MFMAs that follow it
#pragma unroll
        for (int mt = kHead; mt < TM; ++mt) {
          acc[mt][nt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
              bfrag[nt], af[mt], acc[mt][nt], 0, 0, 0, static_cast<int>(sb[nt]), 0,
              static_cast<int>(sa[mt]));
          if (mt == kHead || mt == kHead + 2) {
            asm volatile("" ::"a"(acc[mt][nt]) : "memory");
            __builtin_amdgcn_sched_barrier(0);
            dma_segment(cur, 2 * nt + (mt == kHead ? 0 : 1));
            __builtin_amdgcn_sched_barrier(0);
          }
        }
        pin_column_from<kHead>(acc, nt);
        bfrag[nt] = frag(nxt + kPTile * kBK, wn * 128 + nt * 16 + frag_row);
      }
      __builtin_amdgcn_sched_barrier(0);
      dma_advance();
      unpack_scales();
    }
    int tm, tn;
    tile_coords(static_cast<int>(blockIdx.x) + c_tile * grid, num_wg, tiles_m, tiles_n, group_m,
                tm, tn);
    const int64_t m0 = static_cast<int64_t>(tm) * kPTile, n0 = static_cast<int64_t>(tn) * kPTile;
    if constexpr (kMode == 2) {
      if (ep.act == 1)
        epilogue_direct(m0, n0, std::true_type{});
      else
        epilogue_direct(m0, n0, std::false_type{});
    } else if constexpr (kMode == 3) {
      epilogue_direct(m0, n0, std::false_type{});
    } else {
      epilogue_staged(m0, n0);
    }
  }
  // the DMAs issued past the last step must land before the workgroup's LDS is released
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  bad = bad || mag_max[0] >= 0x7f80 || mag_max[1] >= 0x7f80;
  if (ep.nonfinite != nullptr && __ballot(bad) != 0 && lane == 0) atomicOr(ep.nonfinite, 1u);
}

// Tile order of the persistent kernel: bands of 4 tile rows, so the 32 tiles an XCD runs
// at once are 4 A row panels x 8 W column panels and the next 32 reuse the same A panels.
// Measured against bands of 2, 6, 8, 16 and 32 rows at the block's shapes: 4 is fastest
// (2-4% over 8 on QKV; 16 and 32 lose 7-25%). The head of a K step takes 2 of the 8 A row
// groups: with the DMA segments spread over the tail's MFMAs, 2 takes 3.5-4.5% fewer cycles
// per K step than 3 with the segments issued in pairs after each column (QKV, [O | O_lin]
// and FFN-down shapes); 3 with the spread segments was in between, and 1 or 2 with paired
// segments no better than 3.
constexpr int kPGroupM = 4;

#ifndef VDN_GEMM_HEAD
#define VDN_GEMM_HEAD 2
#endif

int cu_count() {
  static int cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) dev = 0;
  if (dev >= 0 && dev < 64 && cached[dev] > 0) return cached[dev];
  int cu = 0;
  if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cu <= 0)
    cu = 256;
  if (dev >= 0 && dev < 64) cached[dev] = cu;
  return cu;
}

int launch_persistent(const uint8_t* a, const uint8_t* as, int64_t mp, const uint8_t* w,
                      const uint8_t* ws, int64_t np, int64_t kp, const Epilogue& ep,
                      int64_t out_rows, int64_t n, hipStream_t stream) {
  const int64_t tiles_m = (mp + kPTile - 1) / kPTile, tiles_n = (np + kPTile - 1) / kPTile;
  if (tiles_m * tiles_n > (1ll << 31) - 1 || static_cast<int64_t>(kPTile) * kp >= (1ll << 31) ||
      mp * kp / 32 >= (1ll << 31) || np * kp / 32 >= (1ll << 31))
    return set_error(kUnsupported, "vdn_mxfp8_gemm: problem too large for 32-bit tile offsets");
  const int64_t tiles = tiles_m * tiles_n;
  const int grid = static_cast<int>(tiles < cu_count() ? tiles : cu_count());
  const int tm = static_cast<int>(tiles_m), tn = static_cast<int>(tiles_n);
  if (ep.q_out != nullptr && ep.act == 2)
    hipLaunchKernelGGL((mxfp8_gemm_persistent_kernel<VDN_GEMM_HEAD, 3>), dim3(grid), dim3(256),
                       0, stream, a, as, w, ws, mp, np, kp, ep, out_rows, n, tm, tn, kPGroupM);
  else if (ep.q_out != nullptr)
    hipLaunchKernelGGL((mxfp8_gemm_persistent_kernel<VDN_GEMM_HEAD, 2>), dim3(grid), dim3(256),
                       0, stream, a, as, w, ws, mp, np, kp, ep, out_rows, n, tm, tn, kPGroupM);
  else if (ep.residual != nullptr)
    hipLaunchKernelGGL((mxfp8_gemm_persistent_kernel<VDN_GEMM_HEAD, 1>), dim3(grid), dim3(256),
                       0, stream, a, as, w, ws, mp, np, kp, ep, out_rows, n, tm, tn, kPGroupM);
  else
    hipLaunchKernelGGL((mxfp8_gemm_persistent_kernel<VDN_GEMM_HEAD, 0>), dim3(grid), dim3(256),
                       0, stream, a, as, w, ws, mp, np, kp, ep, out_rows, n, tm, tn, kPGroupM);
  return check_launch("vdn_mxfp8_gemm");
}

template <int BM, int BN, int WGM, int WGN>
int launch_gemm(const uint8_t* a, const uint8_t* as, int64_t mp, const uint8_t* w,
                const uint8_t* ws, int64_t np, int64_t kp, const Epilogue& ep, int64_t out_rows,
                int64_t n, hipStream_t stream) {
  const int64_t tiles_m = (mp + BM - 1) / BM, tiles_n = (np + BN - 1) / BN;
  if (tiles_m * tiles_n > (1ll << 31) - 1 || static_cast<int64_t>(BM) * kp >= (1ll << 31) ||
      mp * kp / 32 >= (1ll << 31) || np * kp / 32 >= (1ll << 31))
    return set_error(kUnsupported, "vdn_mxfp8_gemm: problem too large for 32-bit tile offsets");
  const int group_m = 8;
  hipLaunchKernelGGL((mxfp8_gemm_kernel<BM, BN, WGM, WGN>), dim3(tiles_m * tiles_n),
                     dim3(WGM * WGN * 64), 0, stream, a, as, w, ws, mp, np, kp, ep, out_rows, n,
                     static_cast<int>(tiles_m),
                     static_cast<int>(tiles_n), group_m);
  return check_launch("vdn_mxfp8_gemm");
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace
}  // namespace vdn

using namespace vdn;

// Reference: src/models/ops/mxfp8_linear.py:61-93 (MXFP8Linear.forward_quantized: scaled_mm
// BlockWise1x32 + SWIZZLE_32_4_4, crop to [rows, N], + bias in bf16), with the block's
// following bf16 steps optionally fused into the epilogue: `addend` for
// `out[video] += to_out_linear(...)` (hybrid_attention.py:254) and `residual`/`gate` for the
// gated residual `hidden + gate * branch` (fused_block.py:49-51). `nonfinite` (nullable)
// receives 1 when any stored output is not finite (mxfp8_linear.py:91-92).
VDN_API int vdn_mxfp8_gemm(const void* a, const void* a_scales, int64_t mp, const void* w,
                           const void* w_scales, int64_t np, int64_t kp, const void* bias,
                           const void* addend, int64_t ld_add, const void* residual,
                           int64_t ld_res, const void* gate, void* out, int64_t out_rows,
                           int64_t n, int64_t ldc, uint32_t* nonfinite, void* stream) {
  const char* name = "vdn_mxfp8_gemm";
  if (a == nullptr || a_scales == nullptr || w == nullptr || w_scales == nullptr || out == nullptr)
    return set_error(kInvalidArgument, "%s: null pointer argument", name);
  if (mp <= 0 || np <= 0 || kp <= 0 || mp % 128 || np % 128 || kp % 128)
    return set_error(kInvalidArgument, "%s: padded M/N/K must be positive multiples of 128", name);
  if (n <= 0 || n > np || out_rows < 0 || out_rows > mp || ldc < n ||
      (addend != nullptr && ld_add < n) || (residual != nullptr && ld_res < n))
    return set_error(kInvalidArgument, "%s: invalid output geometry", name);
  if (gate != nullptr && residual == nullptr)
    return set_error(kInvalidArgument, "%s: a gate needs a residual", name);
  if (!aligned(a, 16) || !aligned(w, 16) || !aligned(a_scales, 4) || !aligned(w_scales, 4))
    return set_error(kInvalidArgument, "%s: code buffers need 16-byte, scales 4-byte alignment",
                     name);
  if (out_rows == 0) return kOk;
  auto st = static_cast<hipStream_t>(stream);
  auto* ap = static_cast<const uint8_t*>(a);
  auto* asp = static_cast<const uint8_t*>(a_scales);
  auto* wp = static_cast<const uint8_t*>(w);
  auto* wsp = static_cast<const uint8_t*>(w_scales);
  const bool vec = n % 8 == 0 && ldc % 8 == 0 && aligned(out, 16) &&
                   (bias == nullptr || aligned(bias, 16)) && (gate == nullptr || aligned(gate, 16)) &&
                   (addend == nullptr || (ld_add % 8 == 0 && aligned(addend, 16))) &&
                   (residual == nullptr || (ld_res % 8 == 0 && aligned(residual, 16)));
  const Epilogue ep{static_cast<const uint16_t*>(bias), static_cast<const uint16_t*>(addend),
                    ld_add, static_cast<const uint16_t*>(residual), ld_res,
                    static_cast<const uint16_t*>(gate), static_cast<uint16_t*>(out), ldc,
                    nonfinite, vec ? 1 : 0, nullptr, nullptr, 0, 0};
  if (mp >= 1024 && np >= 1024) {
    if (vec && addend == nullptr)
      return launch_persistent(ap, asp, mp, wp, wsp, np, kp, ep, out_rows, n, st);
    return launch_gemm<256, 256, 2, 2>(ap, asp, mp, wp, wsp, np, kp, ep, out_rows, n, st);
  }
  return launch_gemm<128, 128, 2, 2>(ap, asp, mp, wp, wsp, np, kp, ep, out_rows, n, st);
}

// Fused FFN producer: the GEMM of vdn_mxfp8_gemm (+ bias), then act (0 none, 1 GELU-tanh,
// 2 SwiGLU a * silu(g) over a weight with a and g interleaved in 128-row blocks) rounded to
// bf16 and quantized to MXFP8 in the epilogue, in place of the bf16 output and a separate
// producer pass. Output: codes q [mp, pad128(n)] and swizzled scales s
// (mp * pad128(n) / 32 bytes); rows >= out_rows and columns >= n are zero. nonfinite
// (nullable) receives 1 when an activated value is not finite.
// Reference: MXFP8Linear.forward_quantized (src/models/ops/mxfp8_linear.py:61-93) followed
// by the activation producer (mxfp8_kernels.py:62-84, 113-124) in tp_ff_forward
// (src/inference/utils/tensor_parallel.py:147-161).
VDN_API int vdn_mxfp8_gemm_act_quantize(const void* a, const void* a_scales, int64_t mp,
                                        const void* w, const void* w_scales, int64_t np,
                                        int64_t kp, const void* bias, int act, void* q,
                                        void* scales, int64_t out_rows, int64_t n,
                                        uint32_t* nonfinite, void* stream) {
  const char* name = "vdn_mxfp8_gemm_act_quantize";
  if (a == nullptr || a_scales == nullptr || w == nullptr || w_scales == nullptr || q == nullptr ||
      scales == nullptr)
    return set_error(kInvalidArgument, "%s: null pointer argument", name);
  if (mp <= 0 || np <= 0 || kp <= 0 || mp % 128 || np % 128 || kp % 128)
    return set_error(kInvalidArgument, "%s: padded M/N/K must be positive multiples of 128", name);
  if (n <= 0 || n > np || out_rows < 0 || out_rows > mp)
    return set_error(kInvalidArgument, "%s: invalid output geometry", name);
  if (act != 0 && act != 1 && act != 2)
    return set_error(kInvalidArgument, "%s: unknown activation %d", name, act);
  if (!aligned(a, 16) || !aligned(w, 16) || !aligned(a_scales, 4) || !aligned(w_scales, 4) ||
      !aligned(q, 16) || !aligned(scales, 4) || (bias != nullptr && !aligned(bias, 16)))
    return set_error(kInvalidArgument, "%s: misaligned buffer", name);
  if (out_rows == 0) return kOk;
  const int64_t kp_out = (n + 127) / 128 * 128;
  // Every column chunk up to kp_out must be produced: the padded GEMM width covers it.
  if (kp_out > np) return set_error(kInvalidArgument, "%s: padded N smaller than pad128(n)", name);
  // SwiGLU: W holds a and g interleaved in 128-row blocks (np = 2 pad128(n)); the hand-over
  // between the a and g waves exists in the persistent kernel only.
  if (act == 2 && (np != 2 * kp_out || mp < 1024 || np < 1024))
    return set_error(kUnsupported,
                     "%s: SwiGLU takes the interleaved [a | g] weight (padded N = 2 pad128(n)) "
                     "and M >= 1024, N >= 512", name);
  const Epilogue ep{static_cast<const uint16_t*>(bias), nullptr, 0, nullptr, 0, nullptr, nullptr,
                    0, nonfinite, n % 8 == 0 ? 1 : 0, static_cast<uint8_t*>(q),
                    static_cast<uint8_t*>(scales), kp_out, act};
  auto st = static_cast<hipStream_t>(stream);
  auto* ap = static_cast<const uint8_t*>(a);
  auto* asp = static_cast<const uint8_t*>(a_scales);
  auto* wp = static_cast<const uint8_t*>(w);
  auto* wsp = static_cast<const uint8_t*>(w_scales);
  if (mp >= 1024 && np >= 1024)
    return launch_persistent(ap, asp, mp, wp, wsp, np, kp, ep, out_rows, n, st);
  return launch_gemm<128, 128, 2, 2>(ap, asp, mp, wp, wsp, np, kp, ep, out_rows, n, st);
}
