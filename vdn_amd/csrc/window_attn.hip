// Frame-window softmax attention for gfx950 (bf16 or fp16; head_dim 64, 128, 256), flash style.
//
// Replaces the packed varlen passes of paper_window_attention
// (src/models/softmax_attention/paper_window.py:182-243) and the softmax gate
// (softmax_attention/kernels.py:51-67). Each query block attends to a short list of key
// intervals (the frame window, global rows, anchor frames), so no K/V gather copies exist.
//
// Per workgroup: 256 queries of one head (8 waves x 32), key tiles of 128.
//   Sᵀ[key][q] = K · Qᵀ   on v_mfma_f32_32x32x16_bf16 (A = K rows, B = Q rows; Q fragments for
//                         all 128 channels stay in registers for the whole kernel);
//   online softmax in the exp2 domain, fp32 running max / sum per query;
//   Oᵀ[d][q] += Vᵀ · Pᵀ   where Pᵀ is the Sᵀ accumulator itself: the 32x32 accumulator puts
//                         keys 8(v/4) + 4g + v%4 of query l%32 in lane l (g = l/32), which is
//                         exactly the B-operand K layout of the 16-key MFMA (slots 0-3 = keys
//                         4g.., 4-7 = keys 8+4g..; measured), so P never leaves registers;
//                         Vᵀ fragments come from the token-major V tile via ds_read_tr16_b64.
// K/V tiles stream global -> LDS with buffer_load_dwordx4 ... lds, double-buffered; 16-byte
// chunk c of tile row r is stored at c ^ (r & 15) (K: row reads) or c ^ 4 (r & 3) (V: the
// transpose reads, where the 32 lanes served together touch rows r..r+3 and chunks
// 4j..4j+3 of each, which the XOR spreads over all 16 chunk positions of the bank space),
// which keeps both read patterns free of bank conflicts.
#include "mxfp8_common.h"

#include <math.h>

#include <type_traits>

namespace vdn {
namespace {

constexpr int kMaxIntervals = 8;
constexpr int kBlockWaves = 8;  // queries per block = 32 * kBlockWaves (must match the plan)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

typedef __attribute__((address_space(3))) void lds_void_t;
typedef const __attribute__((address_space(1))) void global_void_t;
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4_t;

// Tile rows go global -> LDS through a buffer resource (buffer_load_dwordx4 ... lds): lane l's
// 16 bytes at voffset + soffset land at lds_wave_base + 16 l. Unlike the flat/global form,
// the compiler counts these on vmcnt only, so the fragment reads of the current tile keep
// exact lgkmcnt waits instead of waiting for every outstanding LDS read before each MFMA.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7fffffff, 0x00020000);
}

__device__ __forceinline__ void load_to_lds16(__amdgpu_buffer_rsrc_t r, uint32_t voffset,
                                              uint32_t soffset, void* lds_wave_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)lds_wave_base, 16, voffset, soffset, 0, 0);
}

__device__ __forceinline__ bf16x4_t lds_read_tr(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
      (lds_bf16x4_t*)((__attribute__((address_space(3))) char*)(p)));
}

// the transpose read's own fp16 vector type (four __fp16), reinterpreted as f16x4
typedef __fp16 fp16x4_raw __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef __attribute__((address_space(3))) fp16x4_raw lds_f16x4_t;

// The 16-bit element type of a kernel instance: bf16 (the block's) or fp16 (the reference's
// other varlen dtype). Both share the storage layout, the LDS swizzles and the transpose
// reads; they differ in the MFMA, the conversions of P and the output's rounding.
template <bool kF16>
struct Elem;

template <>
struct Elem<false> {
  typedef __bf16 type;
  typedef bf16x8 x8;
  typedef bf16x4_t x4;
  static __device__ __forceinline__ x4 read_tr(const uint16_t* p) { return lds_read_tr(p); }
  static __device__ __forceinline__ f32x16 mfma(x8 a, x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float to_f32(uint16_t h) { return bf16_bits_to_f32(h); }
  static __device__ __forceinline__ float round(float f) { return round_bf16(f); }
  static __device__ __forceinline__ uint16_t bits(float f) { return f32_to_bf16_bits(f); }
};

template <>
struct Elem<true> {
  typedef _Float16 type;
  typedef f16x8 x8;
  typedef f16x4 x4;
  static __device__ __forceinline__ x4 read_tr(const uint16_t* p) {
    return __builtin_bit_cast(x4, __builtin_amdgcn_ds_read_tr16_b64_v4f16(
        (lds_f16x4_t*)((__attribute__((address_space(3))) char*)(p))));
  }
  static __device__ __forceinline__ f32x16 mfma(x8 a, x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float to_f32(uint16_t h) { return f16_bits_to_f32(h); }
  static __device__ __forceinline__ float round(float f) { return round_f16(f); }
  static __device__ __forceinline__ uint16_t bits(float f) { return f32_to_f16_bits(f); }
};

// Key tile of each head_dim: 128 keys, 64 for D = 256 (whose Q and O fragments take 192
// registers; the tile buffers then still hold the epilogue's 256 x 256 output block).
template <int D>
constexpr int tile_keys() { return D == 256 ? 64 : 128; }

// 16-byte chunk c of tile row r is stored at c ^ swz(r). K rows are read 16 rows per LDS cycle
// (one chunk each), V rows by the transpose reads 4 rows x 4 chunks per 32 lanes; a 256-byte
// bank window holds 256 / (2 D) rows, and the XOR spreads each read set over all of its 16
// chunk positions (D = 64: two rows per window).
template <int D>
__device__ __forceinline__ int swz_k(int row) { return D == 64 ? (row >> 1) & 7 : row & 15; }
template <int D>
__device__ __forceinline__ int swz_v(int row) { return D == 64 ? 4 * ((row >> 1) & 1) : 4 * (row & 3); }

// MXFP8 destination of the output (instead of bf16 rows): codes [rows, kp] and
// SWIZZLE_32_4_4 scales; head h of query row q fills 128-column chunk chunk0 + h, exactly
// what the MXFP8 producer writes for that bf16 row.
struct MxDst {
  uint8_t* codes;
  uint8_t* scales;
  int64_t kp;
  int chunk0;
};

// RMSNorm of the queries applied as they are loaded (w == nullptr: none): n = bf16((x * (1 /
// sqrt(sum(x^2) / 128 + eps))) * w) per (query, head) row, w [128] bf16.
struct QNorm {
  const uint16_t* w;
  float eps;
};

// The query RMSNorm of qk_rope_row128_kernel (the QK norm of paper_qk_rope.py:82-95, D = 128)
// on this kernel's Q fragments, bit for bit: lane (col, g) holds the 8-channel chunks
// c = 2 ks + g of its query row and lane ^ 32 the chunks of the other parity. Each chunk's sum
// of squares runs in channel order as one lane of the norm kernel does; the pair of chunks
// (2 ks, 2 ks + 1) is added across the two lanes and the pair sums in the same balanced tree
// as that kernel's 16-lane DPP reduction, so the sum, and every output, has the same bits.
__device__ __forceinline__ void rms_norm_q128(bf16x8 (&qf)[8], const QNorm& qn, int g) {
#pragma clang fp contract(off)
  // the lane's weights (channels 16 ks + 8 g .. +8) as 16-byte loads, issued first
  u32x4 wr[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) wr[ks] = *reinterpret_cast<const u32x4*>(qn.w + 16 * ks + 8 * g);
  float part[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    part[ks] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float x = static_cast<float>(qf[ks][i]);
      part[ks] += x * x;
    }
  }
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) part[ks] += __shfl_xor(part[ks], 32);
  const float ss = ((part[0] + part[1]) + (part[2] + part[3])) +
                   ((part[4] + part[5]) + (part[6] + part[7]));
  const float inv = 1.0f / sqrtf(ss / 128.0f + qn.eps);
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    float w[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      w[2 * i] = __uint_as_float(wr[ks][i] << 16);
      w[2 * i + 1] = __uint_as_float(wr[ks][i] & 0xffff0000u);
    }
    u32x4 packed;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      packed[i] = pack_bf16x2((static_cast<float>(qf[ks][2 * i]) * inv) * w[2 * i],
                              (static_cast<float>(qf[ks][2 * i + 1]) * inv) * w[2 * i + 1]);
    qf[ks] = __builtin_bit_cast(bf16x8, packed);
  }
}

struct Layout {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh;  // token / head strides (elements)
};

// kWaves waves of 32 queries each: a workgroup owns kBM = 32 kWaves queries, and every K/V
// tile it loads serves all of them. kD is the head dimension (64, 128 or 256); kF16 selects
// fp16 activations (and gate, output) instead of bf16.
template <int kD, int kWaves, bool kMx, bool kF16 = false>
__global__ void __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
window_attn_kernel(Layout in, const int* __restrict__ blocks, const int* __restrict__ grp_kv,
                   const int* __restrict__ grp_n, int nblocks, int heads, float scale_log2,
                   const uint16_t* __restrict__ gate, int64_t g_st, int64_t g_sh,
                   uint16_t* __restrict__ out, int64_t o_st, int64_t o_sh,
                   float* __restrict__ lse, int64_t l_st, int64_t l_sh, MxDst mx, QNorm qn) {
  constexpr int kBN = tile_keys<kD>();
  constexpr int kKT = kBN / 32;       // 32-key score accumulators per tile
  constexpr int kChunks = kD / 8;     // 16-byte chunks per tile row
  constexpr int kSegRows = 64 / kChunks;  // rows per 1 KB DMA segment (one wave instruction)
  static_assert(!kMx || kD == 128, "the MXFP8 destination holds one head per 128 columns");
  static_assert(!kMx || !kF16, "the MXFP8 destination takes bf16 attention");
  typedef Elem<kF16> E;
  typedef typename E::x8 x8;
  // Separate arrays per buffer: with distinct LDS objects the compiler can tell a tile
  // prefetch into one buffer from reads of the other and does not wait on the prefetch.
  __shared__ __attribute__((aligned(1024))) uint16_t sK0[kBN * kD];
  __shared__ __attribute__((aligned(1024))) uint16_t sK1[kBN * kD];
  __shared__ __attribute__((aligned(1024))) uint16_t sV0[kBN * kD];
  __shared__ __attribute__((aligned(1024))) uint16_t sV1[kBN * kD];
  constexpr int kBM = 32 * kWaves;
  constexpr int kThreads = 64 * kWaves;
  constexpr int kSegs = kBN / kSegRows / kWaves;  // 1 KB segments per tensor per wave
  static_assert(kSegs * kWaves * kSegRows == kBN && kWaves % 4 == 0, "segment mapping");
  static_assert(kBM * kD <= 4 * kBN * kD, "the epilogue stages the block in the tile buffers");

  // ---- work item: (head, query block); consecutive ids of a head land on one XCD ----
  const int total = nblocks * heads;
  int pid = blockIdx.x;
  {
    const int xcd = pid & 7, local = pid >> 3;
    const int per = total >> 3, rem = total & 7;
    pid = xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
  }
  const int h = pid / nblocks;
  const int blk = pid % nblocks;
  // block bounds as wave-uniform scalars, so the per-wave branches below stay scalar
  const int q0 = __builtin_amdgcn_readfirstlane(blocks[3 * blk]);
  const int q1 = __builtin_amdgcn_readfirstlane(blocks[3 * blk + 1]);
  const int grp = __builtin_amdgcn_readfirstlane(blocks[3 * blk + 2]);
  const int nint = __builtin_amdgcn_readfirstlane(grp_n[grp]);
  const int* kv = grp_kv + grp * kMaxIntervals * 2;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, col = lane & 31;

  // ---- Q fragments: query q0 + 32 wave + col, channels 16 ks + 8 g .. +8 ----
  const int my_q = q0 + wave * 32 + col;
  const bool q_live = my_q < q1;
  // A group's last block can hold a few rows only (3600 rows per frame = 14 blocks of 256 + 16):
  // waves without a live query still load their share of every tile and meet every barrier,
  // but skip the arithmetic, so the live waves of their SIMDs run at the full MFMA rate.
  const bool wave_live = q0 + wave * 32 < q1;
  x8 qf[kD / 16];
  {
    const uint16_t* src = in.q + static_cast<int64_t>(q_live ? my_q : q0) * in.q_st + h * in.q_sh;
#pragma unroll
    for (int ks = 0; ks < kD / 16; ++ks) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(src + 16 * ks + 8 * g);
      qf[ks] = __builtin_bit_cast(x8, w);
    }
  }

  // lane's share of a tile load: kSegs 1 KB segments (kSegRows rows each) per tensor per
  // wave. The per-lane byte offsets within a tile are fixed; a tile adds a wave-uniform base,
  // so the loads take the scalar-base + 32-bit-offset form with no per-tile vector address math.
  const int seg_row = lane / kChunks, phys = lane % kChunks;
  uint32_t koff[kSegs], voff[kSegs];
#pragma unroll
  for (int j = 0; j < kSegs; ++j) {
    const int row = (j * kWaves + wave) * kSegRows + seg_row;
    koff[j] = static_cast<uint32_t>(row * in.k_st * 2 + 16 * (phys ^ swz_k<kD>(row)));
    voff[j] = static_cast<uint32_t>(row * in.v_st * 2 + 16 * (phys ^ swz_v<kD>(row)));
  }
  const char* k_head = reinterpret_cast<const char*>(in.k + h * in.k_sh);
  const char* v_head = reinterpret_cast<const char*>(in.v + h * in.v_sh);
  // Buffer resources based at the tile's first key row (wave-uniform); the per-lane offsets
  // stay below kBN rows x stride (the host bounds the strides).
  auto issue_tile = [&](int a, int b, uint16_t* dk, uint16_t* dv) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t k_rsrc = tile_rsrc(k_head + static_cast<int64_t>(a) * in.k_st * 2);
    const __amdgpu_buffer_rsrc_t v_rsrc = tile_rsrc(v_head + static_cast<int64_t>(a) * in.v_st * 2);
    if (b - a == kBN) {
#pragma unroll
      for (int j = 0; j < kSegs; ++j) {
        const int seg = j * kWaves + wave;
        load_to_lds16(k_rsrc, koff[j], 0, dk + seg * kSegRows * kD);
        load_to_lds16(v_rsrc, voff[j], 0, dv + seg * kSegRows * kD);
      }
    } else {  // tail tile: rows past the interval end repeat its last key
#pragma unroll
      for (int j = 0; j < kSegs; ++j) {
        const int seg = j * kWaves + wave;
        const int row = seg * kSegRows + seg_row;
        const int r = min(row, b - a - 1);
        const uint32_t ko = static_cast<uint32_t>(r * in.k_st * 2 + 16 * (phys ^ swz_k<kD>(row)));
        const uint32_t vo = static_cast<uint32_t>(r * in.v_st * 2 + 16 * (phys ^ swz_v<kD>(row)));
        load_to_lds16(k_rsrc, ko, 0, dk + seg * kSegRows * kD);
        load_to_lds16(v_rsrc, vo, 0, dv + seg * kSegRows * kD);
      }
    }
  };

  constexpr int kDB = kD / 32;  // 32-channel output accumulators
  f32x16 o[kDB];
#pragma unroll
  for (int db = 0; db < kDB; ++db)
#pragma unroll
    for (int v = 0; v < 16; ++v) o[db][v] = 0.f;
  float m = -INFINITY, l = 0.f;

  // transpose-read coordinates (16-lane group G = lane/16)
  const int G = lane >> 4, L = lane & 15;
  const int tr_row = 4 * (G >> 1) + (L >> 2);
  const int tr_col = 16 * (G & 1) + 4 * (L & 3);

  // One key tile: tile t is resident in buffer kBuf (sK0/sV0 or sK1/sV1); the next tile is
  // prefetched into the other buffer. Running max m is kept in scaled (exp2) units and may
  // lag the true maximum by up to kLazy: the accumulators are rescaled only when a lane's
  // maximum grows by more than that, so exp2 arguments stay <= kLazy (p <= 2^kLazy) and
  // most tiles skip the rescale.
  constexpr float kLazy = 8.f;
  auto process = [&](int t, int ntiles, int a0, int b0, auto buf_tag) __attribute__((always_inline)) {
    constexpr int kBuf = decltype(buf_tag)::value;
    const uint16_t* tk = kBuf == 0 ? sK0 : sK1;
    const uint16_t* tv = kBuf == 0 ? sV0 : sV1;
    // tile t is resident and every wave is done with the other buffer
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    const int na = a0 + (t + 1) * kBN, nb = min(na + kBN, b0);
    uint16_t* ndk = kBuf == 0 ? sK1 : sK0;
    uint16_t* ndv = kBuf == 0 ? sV1 : sV0;
    // a full next tile of a live wave goes out one segment per channel step of Sᵀ, in the
    // shadow of that step's MFMAs
    const bool spread = kD == 128 && t + 1 < ntiles && wave_live && nb - na == kBN;
    if (t + 1 < ntiles && !spread) issue_tile(na, nb, ndk, ndv);
    const __amdgpu_buffer_rsrc_t nk_rsrc = tile_rsrc(k_head + static_cast<int64_t>(na) * in.k_st * 2);
    const __amdgpu_buffer_rsrc_t nv_rsrc = tile_rsrc(v_head + static_cast<int64_t>(na) * in.v_st * 2);
    const int a = a0 + t * kBN, b = min(a + kBN, b0);
    if (!wave_live) return;

    // ---- Sᵀ = K Qᵀ for the tile's kBN keys (kKT 32-key accumulators) ----
    // channel step major: the kKT K fragments of step ks + 1 are read while the kKT MFMAs of
    // step ks run (each accumulator's chain is in the same order as key block major)
    f32x16 s[kKT];
#pragma unroll
    for (int kt = 0; kt < kKT; ++kt)
#pragma unroll
      for (int v = 0; v < 16; ++v) s[kt][v] = 0.f;
    x8 kf[2][kKT];
    auto kload = [&](int ks, x8 (&dst)[kKT]) __attribute__((always_inline)) {
#pragma unroll
      for (int kt = 0; kt < kKT; ++kt) {
        const int row = kt * 32 + col;
        const int chunk = (2 * ks + g) ^ swz_k<kD>(row);
        dst[kt] = *reinterpret_cast<const x8*>(tk + row * kD + chunk * 8);
      }
    };
    kload(0, kf[0]);
#pragma unroll
    for (int ks = 0; ks < kD / 16; ++ks) {
      if (ks + 1 < kD / 16) kload(ks + 1, kf[(ks + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);   // keep the reads ahead of this step's MFMAs
#pragma unroll
      for (int kt = 0; kt < kKT; ++kt) s[kt] = E::mfma(kf[ks & 1][kt], qf[ks], s[kt]);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (kD == 128 && kD / 16 == 2 * kSegs) {
        if (spread) {
          const int j = ks % kSegs, seg = j * kWaves + wave;
          if (ks < kSegs)
            load_to_lds16(nk_rsrc, koff[j], 0, ndk + seg * kSegRows * kD);
          else
            load_to_lds16(nv_rsrc, voff[j], 0, ndv + seg * kSegRows * kD);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // ---- online softmax (exp2 domain; scores scaled inside the exponent's fma) ----
    if (b - a < kBN) {  // tail tile: keys past the interval end do not exist
#pragma unroll
      for (int kt = 0; kt < kKT; ++kt)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = a + kt * 32 + (v >> 2) * 8 + g * 4 + (v & 3);
          if (key >= b) s[kt][v] = -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < kKT; ++kt)
#pragma unroll
      for (int v = 0; v < 16; ++v) mx = fmaxf(mx, s[kt][v]);
    mx = fmaxf(mx, __shfl_xor(mx, 32)) * scale_log2;
    const bool grow = mx > m + kLazy;
    if (__any(grow)) {
      const float m_new = grow ? mx : m;
      const float corr = __builtin_amdgcn_exp2f(m - m_new);
      l *= corr;
#pragma unroll
      for (int db = 0; db < kDB; ++db)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[db][v] *= corr;
      m = m_new;
    }
    float rs = 0.f;
#pragma unroll
    for (int kt = 0; kt < kKT; ++kt)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][v], scale_log2, -m));
        s[kt][v] = p;
        rs += p;
      }
    rs += __shfl_xor(rs, 32);
    l += rs;

    // ---- Oᵀ += Vᵀ Pᵀ, 16 keys per MFMA; the V fragments of MFMA i + kVA are read before
    // MFMA i (the barriers order only the LDS reads and MFMAs; VALU and transcendental
    // instructions may cross them) ----
    constexpr int kItems = (kBN / 16) * kDB;
    constexpr int kVA = 2;
    x8 vf[kVA + 1];
    auto vload = [&](int i, x8& dst) __attribute__((always_inline)) {
      const int c = i / kDB, db = i % kDB;
      typename E::x4 lo, hi;
      {
        const int row = 16 * c + tr_row;
        const int e = 32 * db + tr_col;
        const int chunk = (e >> 3) ^ swz_v<kD>(row);
        lo = E::read_tr(tv + row * kD + chunk * 8 + (e & 7));
      }
      {
        const int row = 16 * c + 8 + tr_row;
        const int e = 32 * db + tr_col;
        const int chunk = (e >> 3) ^ swz_v<kD>(row);
        hi = E::read_tr(tv + row * kD + chunk * 8 + (e & 7));
      }
      dst = x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };
#pragma unroll
    for (int i = 0; i < kVA; ++i) vload(i, vf[i]);
    x8 pb;
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
      if (i + kVA < kItems) vload(i + kVA, vf[(i + kVA) % (kVA + 1)]);
      __builtin_amdgcn_sched_barrier(0x406);
      const int c = i / kDB, db = i % kDB;
      if (db == 0) {
#pragma unroll
        for (int j = 0; j < 8; ++j) pb[j] = static_cast<typename E::type>(s[c >> 1][(c & 1) * 8 + j]);
      }
      o[db] = E::mfma(vf[i % (kVA + 1)], pb, o[db]);
      __builtin_amdgcn_sched_barrier(0x406);
    }
  };
  // ---- key intervals of the group, one after another ----
  // Each interval is a contiguous key range walked in kBN-key tiles; its bounds are read
  // before its first tile load, so the tile loop itself reads no memory besides the tiles.
  // The online softmax state carries over from one interval to the next.
  // With a query norm, the first non-empty interval's first tile goes out before the norm
  // runs, so that the tile's latency covers it.
  int pre_issued = -1;
  if constexpr (kMx) {
    if (qn.w != nullptr) {
      for (int i = 0; i < nint; ++i) {
        const int a0 = __builtin_amdgcn_readfirstlane(kv[2 * i]);
        const int b0 = __builtin_amdgcn_readfirstlane(kv[2 * i + 1]);
        if (b0 > a0) {
          issue_tile(a0, min(a0 + kBN, b0), sK0, sV0);
          pre_issued = i;
          break;
        }
      }
      rms_norm_q128(qf, qn, g);
    }
  }
  for (int i = 0; i < nint; ++i) {
    const int a0 = __builtin_amdgcn_readfirstlane(kv[2 * i]);
    const int b0 = __builtin_amdgcn_readfirstlane(kv[2 * i + 1]);
    const int ntiles = (b0 - a0 + kBN - 1) / kBN;
    if (ntiles <= 0) continue;
    __syncthreads();  // every wave is done reading the buffers of the previous interval
    if (i != pre_issued) issue_tile(a0, min(a0 + kBN, b0), sK0, sV0);
    for (int t = 0; t < ntiles; t += 2) {
      process(t, ntiles, a0, b0, std::integral_constant<int, 0>{});
      if (t + 1 < ntiles) process(t + 1, ntiles, a0, b0, std::integral_constant<int, 1>{});
    }
  }
  const float inv_l = l > 0.f ? 1.0f / l : 0.f;
  if constexpr (kMx) {
    // ---- MXFP8 epilogue straight from the accumulators ----
    // Lane (col, g) holds channels 32 db + 8 j + 4 g + i (v = 4 j + i) of query my_q: 16 of
    // the 32 channels of MXFP8 block db; lane ^ 32 holds the other 16. y = bf16(bf16(o / l)
    // * gate) as in the bf16 form; the block's amax takes one exchange, and the codes leave
    // as one 16-byte store per lane and block (below).
    float gv = 1.f;
    if (gate != nullptr && q_live) gv = bf16_bits_to_f32(gate[static_cast<int64_t>(my_q) * g_st + h * g_sh]);
    // Lanes l and l + 32 hold the same query row. After two swaps per block each holds 16
    // contiguous code bytes of it (bytes 16 g .. + 16 of the block): one 16-byte store instead
    // of four 4-byte ones scattered over 32 rows.
    uint8_t* crow = mx.codes + static_cast<int64_t>(my_q) * mx.kp + (mx.chunk0 + h) * 128 + 16 * g;
    uint32_t word = 0;
#pragma unroll
    for (int db = 0; db < kDB; ++db) {
      float y[16];
#pragma unroll
      for (int v = 0; v < 16; v += 2) {
        float a = o[db][v] * inv_l, b = o[db][v + 1] * inv_l;
        round_bf16_pair(a, b);
        if (gate != nullptr) {
          a *= gv;
          b *= gv;
          round_bf16_pair(a, b);
        }
        y[v] = a;
        y[v + 1] = b;
      }
      float amax = 0.f;
#pragma unroll
      for (int v = 0; v < 16; ++v) amax = fmaxf(amax, fabsf(y[v]));
      {
        // v_permlane32_swap (vdst, vsrc): lane l < 32 receives lane l + 32's vdst in vsrc and
        // lane l + 32 receives lane l's vsrc in vdst; with one value in both operands the
        // pair holds the lane's own value and its partner's
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(amax),
                                                         __float_as_uint(amax), false, false);
        amax = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
      }
      float sinv;
      const uint32_t byte = e8m0_from_amax(amax, &sinv);
      word |= byte << (8 * db);
      const float sf = e8m0_scale(byte);
      // word j of the lane: code bytes 8 j + 4 g .. + 4 of the block
      uint32_t wv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        wv[j] = e4m3x4_scaled(y[4 * j], y[4 * j + 1], y[4 * j + 2], y[4 * j + 3], sf);
      // lane g = 0 takes words 0 and 1 of lane g = 1 (bytes 4-7, 12-15), lane g = 1 takes
      // words 2 and 3 of lane g = 0 (bytes 16-19, 24-27)
      const auto s02 = __builtin_amdgcn_permlane32_swap(wv[0], wv[2], false, false);
      const auto s13 = __builtin_amdgcn_permlane32_swap(wv[1], wv[3], false, false);
      const u32x4 out16 = g == 0 ? u32x4{wv[0], s02[1], wv[1], s13[1]}
                                 : u32x4{s02[0], wv[2], s13[0], wv[3]};
      if (q_live) *reinterpret_cast<u32x4*>(crow + 32 * db) = out16;
    }
    if (q_live && g == 0)
      *reinterpret_cast<uint32_t*>(
          mx.scales + swizzled_scale_offset(my_q, (mx.chunk0 + h) * 4, mx.kp >> 7)) = word;
    if (lse != nullptr && q_live && g == 0)
      lse[static_cast<int64_t>(my_q) * l_st + h * l_sh] = (m + log2f(l)) * kLn2;
    return;
  }
  __syncthreads();  // the epilogue reuses the K buffers

  // ---- epilogue: O / l, optional gate, through LDS to coalesced rows ----
  // [kBM queries][kD channels] 16-bit values staged across the tile buffers, kBN queries per
  // buffer
  auto stage_rows = [&](int r) -> uint16_t* {
    const int which = r / kBN;  // uniform per wave for both uses below
    return which == 0 ? sK0 : which == 1 ? sK1 : which == 2 ? sV0 : sV1;
  };
  const int qr = wave * 32 + col;
  uint16_t* sO = stage_rows(qr);
  float gv = 1.f;
  if (gate != nullptr && q_live) gv = E::to_f32(gate[static_cast<int64_t>(my_q) * g_st + h * g_sh]);
#pragma unroll
  for (int db = 0; db < kDB; ++db)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int d = 32 * db + (v >> 2) * 8 + g * 4 + (v & 3);
      float y = E::round(o[db][v] * inv_l);
      if (gate != nullptr) y = y * gv;
      sO[(qr % kBN) * kD + d] = E::bits(y);
    }
  if (lse != nullptr && q_live && g == 0)
    lse[static_cast<int64_t>(my_q) * l_st + h * l_sh] = (m + log2f(l)) * kLn2;
  __syncthreads();
  // kChunks lanes write one query row (2 kD bytes, or its 128 MXFP8 codes and 4 scales)
  for (int r = tid / kChunks; r < kBM; r += kThreads / kChunks) {
    const int q = q0 + r;
    if (q >= q1) continue;  // uniform per kChunks-lane group
    const int c8 = (tid % kChunks) * 8;
    const uint16_t* src = stage_rows(r);
    const u32x4 row8 = *reinterpret_cast<const u32x4*>(&src[(r % kBN) * kD + c8]);
    *reinterpret_cast<u32x4*>(out + static_cast<int64_t>(q) * o_st + h * o_sh + c8) = row8;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace vdn

using namespace vdn;

namespace vdn {
namespace {

// Shared validation and launch of both entry points (out / lse for the bf16 form, mx for
// the MXFP8 form).
int launch_window(const char* name, const void* q, int64_t q_st, int64_t q_sh, const void* k,
                  int64_t k_st, int64_t k_sh, const void* v, int64_t v_st, int64_t v_sh,
                  const int* blocks, int nblocks, const int* grp_kv, const int* grp_n, int heads,
                  int head_dim, int dtype, float scale, const void* gate, int64_t g_st,
                  int64_t g_sh, void* out, int64_t o_st, int64_t o_sh, float* lse, int64_t l_st,
                  int64_t l_sh, const MxDst* mx, QNorm qn, void* stream) {
  if (q == nullptr || k == nullptr || v == nullptr || blocks == nullptr || grp_kv == nullptr ||
      grp_n == nullptr || (mx == nullptr && out == nullptr))
    return set_error(kInvalidArgument, "%s: null pointer", name);
  if (heads <= 0 || nblocks < 0) return set_error(kInvalidArgument, "%s: bad geometry", name);
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return set_error(kInvalidArgument, "%s: head_dim must be 64, 128 or 256", name);
  if (mx != nullptr && head_dim != 128)
    return set_error(kUnsupported, "%s: the MXFP8 output takes head_dim 128", name);
  if (dtype != 0 && dtype != 1)
    return set_error(kInvalidArgument, "%s: dtype must be 0 (bf16) or 1 (fp16)", name);
  if (mx != nullptr && dtype != 0)
    return set_error(kUnsupported, "%s: the MXFP8 output takes bf16 attention", name);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || q_st % 8 || q_sh % 8 || k_st % 8 ||
      k_sh % 8 || v_st % 8 || v_sh % 8 ||
      (mx == nullptr && (!aligned16(out) || o_st % 8 || o_sh % 8)))
    return set_error(kInvalidArgument, "%s: rows need 16-byte alignment", name);
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
  if (!(scale > 0.f) || !isfinite(scale)) return set_error(kInvalidArgument, "%s: bad scale", name);
  if (qn.w != nullptr && (mx == nullptr || !(qn.eps > 0.f) || !isfinite(qn.eps)))
    return set_error(kInvalidArgument,
                     "%s: the query norm needs the MXFP8 output and a finite positive eps", name);
  if (qn.w != nullptr && !aligned16(qn.w))
    return set_error(kInvalidArgument, "%s: the query norm weight needs 16-byte alignment",
                     name);
  if (k_st <= 0 || v_st <= 0 || k_st > (1 << 22) || v_st > (1 << 22))
    return set_error(kUnsupported, "%s: K/V token strides must be in (0, 2^22] elements", name);
  if (nblocks == 0) return kOk;
  const Layout in{static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                  static_cast<const uint16_t*>(v), q_st, q_sh, k_st, k_sh, v_st, v_sh};
  const int64_t total = static_cast<int64_t>(nblocks) * heads;
  if (total > (1ll << 31) - 1) return set_error(kUnsupported, "%s: too many blocks", name);
  const dim3 grid(static_cast<unsigned>(total)), block(kBlockWaves * 64);
  const auto st = static_cast<hipStream_t>(stream);
  const auto* g16 = static_cast<const uint16_t*>(gate);
  auto* o16 = static_cast<uint16_t*>(out);
  const MxDst none{nullptr, nullptr, 0, 0};
  if (mx != nullptr)
    hipLaunchKernelGGL((window_attn_kernel<128, kBlockWaves, true>), grid, block, 0, st, in,
                       blocks, grp_kv, grp_n, nblocks, heads, scale * kLog2e, g16, g_st, g_sh,
                       nullptr, 0, 0, nullptr, 0, 0, *mx, qn);
#define VDN_WINDOW(D, F16)                                                                      \
  hipLaunchKernelGGL((window_attn_kernel<D, kBlockWaves, false, F16>), grid, block, 0, st, in,  \
                     blocks, grp_kv, grp_n, nblocks, heads, scale * kLog2e, g16, g_st, g_sh,    \
                     o16, o_st, o_sh, lse, l_st, l_sh, none, QNorm{nullptr, 0.f})
  else if (head_dim == 128 && dtype == 0)
    VDN_WINDOW(128, false);
  else if (head_dim == 64 && dtype == 0)
    VDN_WINDOW(64, false);
  else if (dtype == 0)
    VDN_WINDOW(256, false);
  else if (head_dim == 128)
    VDN_WINDOW(128, true);
  else if (head_dim == 64)
    VDN_WINDOW(64, true);
  else
    VDN_WINDOW(256, true);
#undef VDN_WINDOW
  return check_launch(name);
}

}  // namespace
}  // namespace vdn

// Reference: paper_window_attention (src/models/softmax_attention/paper_window.py:182-243),
// window_softmax_reference (window.py:56-111), apply_softmax_gate (kernels.py:51-67).
// q, k, v: bf16 (dtype 0) or fp16 (dtype 1) [rows, heads, head_dim] (head_dim 64, 128 or
// 256; token / head strides, unit channel stride);
// blocks: int32 [nblocks, 3] = (first query, end of its query group, group index), each
// block at most 256 queries; grp_kv: int32 [groups, 8, 2] key intervals [a, b); grp_n:
// int32 [groups] interval counts. gate (nullable): per (token, head) scalar of the
// activation dtype, multiplied into the output after its rounding. out: rows of head_dim
// channels of the activation dtype; lse (nullable): fp32 natural-log sum of exp of the scaled
// scores.
VDN_API int vdn_window_attention(const void* q, int64_t q_st, int64_t q_sh, const void* k,
                                 int64_t k_st, int64_t k_sh, const void* v, int64_t v_st,
                                 int64_t v_sh, const int* blocks, int nblocks, const int* grp_kv,
                                 const int* grp_n, int heads, int head_dim, int dtype,
                                 float scale, const void* gate, int64_t g_st, int64_t g_sh,
                                 void* out, int64_t o_st, int64_t o_sh, float* lse, int64_t l_st,
                                 int64_t l_sh, void* stream) {
  return launch_window("vdn_window_attention", q, q_st, q_sh, k, k_st, k_sh, v, v_st, v_sh,
                       blocks, nblocks, grp_kv, grp_n, heads, head_dim, dtype, scale, gate,
                       g_st, g_sh,
                       out, o_st, o_sh, lse, l_st, l_sh, nullptr, QNorm{nullptr, 0.f},
                       stream);
}

// The same attention with the output quantized in the epilogue: query row q, head h ->
// MXFP8 codes[q, 128 (chunk0 + h) ..] (row length kp) and the swizzled scales of those four
// 32-blocks, bit-identical to vdn_mxfp8_quantize of the bf16 output. Rows with no query
// are not written. Reference: the output projection's producer, quantize_activation
// (src/models/ops/mxfp8_quant.py:77-90), applied to paper_window_attention's output.
VDN_API int vdn_window_attention_mxfp8(const void* q, int64_t q_st, int64_t q_sh, const void* k,
                                       int64_t k_st, int64_t k_sh, const void* v, int64_t v_st,
                                       int64_t v_sh, const int* blocks, int nblocks,
                                       const int* grp_kv, const int* grp_n, int heads,
                                       float scale, const void* gate, int64_t g_st, int64_t g_sh,
                                       const void* q_norm_w, float q_norm_eps,
                                       void* codes, void* scales, int64_t kp, int chunk0,
                                       void* stream) {
  const MxDst mx{static_cast<uint8_t*>(codes), static_cast<uint8_t*>(scales), kp, chunk0};
  return launch_window("vdn_window_attention_mxfp8", q, q_st, q_sh, k, k_st, k_sh, v, v_st,
                       v_sh, blocks, nblocks, grp_kv, grp_n, heads, 128, 0, scale, gate, g_st,
                       g_sh,
                       nullptr, 0, 0, nullptr, 0, 0, &mx,
                       QNorm{static_cast<const uint16_t*>(q_norm_w), q_norm_eps}, stream);
}
