/*
 * libvdnmi — C ABI of the MI355X (gfx950) kernels for the VDN-H3 hybrid DiT block.
 *
 * Conventions for every entry point:
 *   - arguments are raw device pointers, int64 sizes/strides (in elements unless stated),
 *     scalars and a hipStream_t passed as void* (the caller's current stream);
 *   - the return value is 0 on success, nonzero on failure; vdn_last_error() then holds
 *     a message (thread-local);
 *   - nothing is allocated: the caller owns every buffer; outputs never alias inputs;
 *   - bf16 tensors are passed as 16-bit storage, MXFP8 codes/scales as uint8.
 *
 * MXFP8 layout (reference src/models/ops/mxfp8_quant.py:15-37): rows padded to
 * RP = ceil(R/128)*128 and K to KP = ceil(K/128)*128 with zeros; one E8M0 byte per row
 * and 32-element K block, stored flat in SWIZZLE_32_4_4 order (RP*KP/32 bytes).
 */
#ifndef VDNMI_H_
#define VDNMI_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Message of the last failing call on this thread. */
const char* vdn_last_error(void);

/* ABI revision of this header. */
int vdn_abi_version(void);

/*
 * bf16 x[rows, k] (row stride `row_stride`, unit column stride) -> codes q[RP, KP] and
 * swizzled scales. *nonfinite (a zeroed device uint32) becomes 1 when x holds inf/NaN.
 * Replaces: src/models/ops/mxfp8_kernels.py:31-58 (_quantize / launch_quantize), called by
 * quantize_activation (src/models/ops/mxfp8_quant.py:77-90).
 */
int vdn_mxfp8_quantize(const void* x, int64_t rows, int64_t k, int64_t row_stride, void* q,
                       void* scales, uint32_t* nonfinite, void* stream);

/*
 * Activation + MXFP8 producer: act = 1 quantizes bf16(gelu_tanh(x[rows, k]));
 * act = 2 quantizes bf16(a * silu(g)) for x = [a | g] of width 2k.
 * Replaces: src/models/ops/mxfp8_kernels.py:62-84, 113-124 (_swiglu_mx /
 * launch_swiglu_quantize); GELU-tanh is the same producer for a GELU-tanh FFN.
 */
int vdn_mxfp8_act_quantize(const void* x, int64_t rows, int64_t k, int64_t row_stride, int act,
                           void* q, void* scales, uint32_t* nonfinite, void* stream);

/*
 * Fused RMSNorm + AdaLN + MXFP8 producer:
 *   y = bf16((x * rsqrt(mean(x^2) + eps) * weight) * (1 + scale[idx]) + shift[idx])
 * written to y (nullable) and quantized into q/scales; finite[RP] (uint8) is 1 for rows
 * whose input and output are finite. flags: bit0 weight is fp32 (else bf16), bit1
 * scale/shift tables are fp32 (else bf16). indices: int64 [rows].
 * Replaces: src/models/ops/mxfp8_kernels.py:87-110, 127-139 (_prenorm_mx /
 * launch_prenorm_quantize), called by paper_block_forward (fused_block.py:144-154).
 */
int vdn_mxfp8_prenorm_quantize(const void* x, int64_t rows, int64_t k, int64_t row_stride,
                               const void* weight, float eps, const void* scale,
                               int64_t scale_stride, const void* shift, int64_t shift_stride,
                               const int64_t* indices, int flags, void* y, void* q, void* scales,
                               uint8_t* finite, void* stream);

/*
 * Block-scaled GEMM: out[r, c] = bf16(sum_k dq(a)[r, k] * dq(w)[c, k]) (+ bf16 bias[c]),
 * r < out_rows <= mp, c < n <= np, out row stride ldc. a: codes [mp, kp] + scales,
 * w: codes [np, kp] + scales (mp, np, kp multiples of 128). mode 0 stores, mode 1 adds
 * into out (out = bf16(out + y)). *nonfinite (nullable) becomes 1 on a nonfinite output.
 * Replaces: F.scaled_mm(BlockWise1x32, SWIZZLE_32_4_4) + crop + bias in
 * MXFP8Linear.forward_quantized (src/models/ops/mxfp8_linear.py:61-93).
 */
int vdn_mxfp8_gemm(const void* a, const void* a_scales, int64_t mp, const void* w,
                   const void* w_scales, int64_t np, int64_t kp, const void* bias, void* out,
                   int64_t out_rows, int64_t n, int64_t ldc, int mode, uint32_t* nonfinite,
                   void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VDNMI_H_ */
