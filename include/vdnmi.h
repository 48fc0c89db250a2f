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
 * finite_tiles (nullable; uint8 [ceil(RP/16) * ceil(KP/256)], set to 1 by the caller): the
 * byte of tile (r / 16, c / 256) is cleared when the tile's inputs or activations hold a
 * nonfinite value, the reference's per-program FINITE output.
 * Replaces: src/models/ops/mxfp8_kernels.py:62-84, 113-124 (_swiglu_mx /
 * launch_swiglu_quantize); GELU-tanh is the same producer for a GELU-tanh FFN.
 */
int vdn_mxfp8_act_quantize(const void* x, int64_t rows, int64_t k, int64_t row_stride, int act,
                           void* q, void* scales, uint32_t* nonfinite, uint8_t* finite_tiles,
                           void* stream);

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
 * Block-scaled GEMM: y[r, c] = bf16(sum_k dq(a)[r, k] * dq(w)[c, k]), r < out_rows <= mp,
 * c < n <= np. a: codes [mp, kp] + scales, w: codes [np, kp] + scales (mp, np, kp multiples
 * of 128). Epilogue, each step rounded to bf16 (all operands bf16, nullable):
 *   y = y + bias[c];  y = addend[r, c] + y;  y = residual[r, c] + gate[c] * y
 * (gate requires residual; gate null means 1), stored to out (row stride ldc; out may alias
 * addend or residual). *nonfinite (nullable) becomes 1 on a nonfinite output.
 * Replaces: F.scaled_mm(BlockWise1x32, SWIZZLE_32_4_4) + crop + bias in
 * MXFP8Linear.forward_quantized (src/models/ops/mxfp8_linear.py:61-93); the addend and gated
 * residual are the block's `out[video] += to_out_linear(...)` (hybrid_attention.py:254) and
 * `hidden + gate * branch` (src/models/ops/fused_block.py:49-51).
 */
int vdn_mxfp8_gemm(const void* a, const void* a_scales, int64_t mp, const void* w,
                   const void* w_scales, int64_t np, int64_t kp, const void* bias,
                   const void* addend, int64_t ld_add, const void* residual, int64_t ld_res,
                   const void* gate, void* out, int64_t out_rows, int64_t n, int64_t ldc,
                   uint32_t* nonfinite, void* stream);

/*
 * Block-scaled GEMM feeding the next MXFP8 projection directly: y = bf16(bf16(acc) + bias),
 * act = 1 applies GELU-tanh (rounded to bf16; act = 0: none), and y is stored as MXFP8 codes
 * q [mp, pad128(n)] + swizzled scales (mp * pad128(n) / 32 bytes), exactly what
 * vdn_mxfp8_act_quantize / vdn_mxfp8_quantize write for that bf16 matrix. Rows >= out_rows
 * and columns >= n are zero. *nonfinite (nullable) becomes 1 on a nonfinite activation.
 * Replaces: the FFN up projection + activation producer of tp_ff_forward
 * (src/inference/utils/tensor_parallel.py:147-161: MXFP8Linear.forward_quantized,
 * mxfp8_linear.py:61-93, then the producer of mxfp8_kernels.py:62-84, 113-124).
 */
int vdn_mxfp8_gemm_act_quantize(const void* a, const void* a_scales, int64_t mp, const void* w,
                                const void* w_scales, int64_t np, int64_t kp, const void* bias,
                                int act, void* q, void* scales, int64_t out_rows, int64_t n,
                                uint32_t* nonfinite, void* stream);

/* ---------------------------------------------------------------------------------------
 * VDA linear-attention branch (D = 128). A 4-D operand "(f, h, s, c)" is addressed as
 * base + f*sf + h*sh + s*ss + c (element strides, channels contiguous); raw token-major
 * projections [F*S, H, 128] with row stride R and head stride Hs map to sf = S*R, sh = Hs,
 * ss = R.
 * ------------------------------------------------------------------------------------- */

/*
 * tokens [n = frames*spatial, heads, 128] (row/head strides) -> out [frames, heads, spatial,
 * 128]: SiLU, then L2 over the 128 channels when l2norm (clamp 1e-12 on the sum of squares).
 * is_f32 selects fp32 in/out, else bf16.
 * Replaces: paper_prepare (src/models/linear_attention/paper_stack.py:30-48) ->
 * vdn_silu_l2norm (src/models/linear_attention/paper_sglang.py:251-283).
 */
int vdn_vda_prepare(const void* tokens, int64_t n, int heads, int64_t row_stride,
                    int64_t head_stride, int frames, int spatial, int l2norm, int is_f32,
                    void* out, void* stream);

/*
 * paper_prepare with the linear branch's separable short conv, fused: tokens [frames *
 * frame_h * frame_w, heads, 128] bf16 (row/head strides in elements, token f*S + y*W + x)
 * -> depthwise 5x5 spatial conv per frame (zero padding 2; w_sp [heads*128, 5, 5] bf16),
 * rounded to bf16 -> depthwise 5-tap temporal conv across frames (zero padding 2;
 * w_tm [heads*128, 5] bf16) in fp32 -> SiLU (+ L2 over the 128 channels when l2norm) ->
 * out [frames, heads, S, 128] bf16. One frame of tokens must span < 2 GiB.
 * Replaces: paper_prepare with conv (src/models/linear_attention/paper_stack.py:43-47) ->
 * LinearAttentionSepConv.spatial (src/models/linear_attention/features.py:175-196) +
 * vdn_temporal_conv_act (src/models/linear_attention/paper_sglang.py:165-203).
 */
int vdn_vda_conv_prepare(const void* tokens, int heads, int64_t row_stride, int64_t head_stride,
                         int frames, int frame_h, int frame_w, const void* w_sp,
                         const void* w_tm, int l2norm, void* out, void* stream);

/*
 * Joint statistics per (frame, head): A = (K^T diag(beta) K + transpose) / 2 (fp32-grade),
 * B = bf16(bf16(v * bf16(beta))^T k) (fp32 storage), A, B: [frames, heads, 128, 128] fp32.
 * k, v: bf16 operands; beta: bf16 (beta_f32 = 0) or fp32, addressed (f, h, s). activate = 1
 * applies the paper_prepare activation in registers (k: SiLU + L2, v: SiLU) to raw
 * projections.
 * Replaces: paper_statistics / _joint_stats (src/models/linear_attention/paper_stack.py:51-110).
 */
int vdn_vda_statistics(const void* k, int64_t k_sf, int64_t k_sh, int64_t k_ss, const void* v,
                       int64_t v_sf, int64_t v_sh, int64_t v_ss, const void* beta, int64_t b_sf,
                       int64_t b_sh, int64_t b_ss, int beta_f32, int frames, int heads,
                       int spatial, int activate, float* A, float* B, void* stream);

/*
 * T = diag(alpha) (I + A)^-1 and J = B (I + A)^-1 for `count` 128x128 fp32 matrices
 * (I + A symmetric positive definite; no pivoting). alpha: [count, 128] or null (ones).
 * Replaces: paper_delta_factors (src/models/linear_attention/paper_factor.py:133-186), the
 * reference's pybind11 op delta_factors (src/models/ops/csrc/vdn_delta_factors.cpp:11-14).
 */
int vdn_vda_factors(const float* A, const float* B, const float* alpha, int64_t count, float* T,
                    float* J, void* stream);

/*
 * Per chunk c (frames starts[c] .. ends[c]-1) and direction (0 forward, 1 reverse):
 * CT = ordered product of the chunk's transitions, CI = the injection the chunk adds to a
 * zero state. T, J: [frames, heads, 128, 128]; CT, CI: [2, chunks, heads, 128, 128].
 * Replaces: _compose (src/models/linear_attention/paper_stack.py:162-181).
 */
int vdn_vda_compose(const float* T, const float* J, int heads, const int* starts, const int* ends,
                    int chunks, float* CT, float* CI, void* stream);

/*
 * Both directional scans state <- state @ CT[c] + CI[c] over chunks, starting from seed
 * (nullable: zero), writing bank [2, chunks, heads, 128, 128]. per_direction = 0 takes
 * per-frame factors [chunks, heads, 128, 128] for both directions (one-frame chunks).
 * Replaces: _scan_both / paper_boundary_scan (src/models/linear_attention/paper_stack.py:184-236).
 */
int vdn_vda_scan(const float* CT, const float* CI, const float* seed, int chunks, int heads,
                 int per_direction, float* bank, void* stream);

/*
 * logp [frames + 1, heads, 128]: exclusive prefix sums of log(max(alpha, 1e-12)) over frames.
 * Replaces: the log-prefix of paper_gather (src/models/linear_attention/paper_stack.py:256).
 */
int vdn_vda_log_prefix(const float* alpha, int frames, int heads, float* logp, void* stream);

/*
 * Boundary gather: out[f, h] = prefix[before[f], h] * exp(logp[f+1] - logp[bridge_before[f]])
 * + suffix[after[f], h] * exp(logp[bridge_after[f]] - logp[f]) (per key channel; the exp
 * factors only when bridge), with missing sides (has_* = 0) reading text (nullable: zero).
 * prefix/suffix: [chunks, heads, 128, 128] fp32; index arrays int32 [frames];
 * out: [frames, heads, 128, 128] bf16 (out_f32 = 0) or fp32.
 * Replaces: paper_gather / _gather_state_kernel (src/models/linear_attention/paper_stack.py:239-263,
 * paper_sglang.py:445-501).
 */
int vdn_vda_gather(const float* prefix, const float* suffix, const float* logp, const float* text,
                   const int* before, const int* after, const int* has_before,
                   const int* has_after, const int* bridge_before, const int* bridge_after,
                   int frames, int heads, int bridge, int out_f32, void* out, void* stream);

/*
 * Fused readout: y = bf16(q' . state^T) per (frame, head), q' = bf16(L2(SiLU(q))) when
 * activate_q, then out = bf16(y * (1/sqrt(mean(y^2) + eps)) * weight * gate).
 * q, gate, out: bf16 addressed (f, h, s); state: bf16 [frames, heads, 128, 128] ([v][k]);
 * weight: [128] bf16 or fp32 (weight_f32).
 * head_dim (16, 32, 64 or 128) is the number of channels that carry data: rows are always
 * 128 wide, channels past head_dim are zero in q, state and weight, and the norm's mean is
 * over head_dim channels (the reference's branch body at d < 128, delta_rule.py:45-60).
 * Replaces: the readout matmul and vdn_linear_epilogue of paper_readout
 * (src/models/linear_attention/paper_stack.py:317-318, paper_sglang.py:377-437).
 */
int vdn_vda_readout(const void* q, int64_t q_sf, int64_t q_sh, int64_t q_ss, int activate_q,
                    const void* state, const void* weight, int weight_f32, float eps,
                    const void* gate, int64_t g_sf, int64_t g_sh, int64_t g_ss, void* out,
                    int64_t o_sf, int64_t o_sh, int64_t o_ss, int head_dim, int frames,
                    int heads, int spatial, void* stream);

/* vdn_vda_readout with the output quantized in the epilogue instead of stored as bf16: token
 * row f * spatial + s, head h -> MXFP8 codes[row, 128 (chunk0 + h) .. +128) of a [rows, kp]
 * code matrix and that chunk's four E8M0 scales in its SWIZZLE_32_4_4 scale array; the same
 * bytes vdn_mxfp8_quantize writes for the bf16 output.
 * Replaces: the readout of paper_readout (src/models/linear_attention/paper_stack.py:317-318,
 * paper_sglang.py:377-437) followed by quantize_activation (src/models/ops/mxfp8_quant.py:77-90).
 */
int vdn_vda_readout_mxfp8(const void* q, int64_t q_sf, int64_t q_sh, int64_t q_ss,
                          int activate_q, const void* state, const void* weight, int weight_f32,
                          float eps, const void* gate, int64_t g_sf, int64_t g_sh, int64_t g_ss,
                          void* codes, void* scales, int64_t kp, int chunk0, int frames,
                          int heads, int spatial, void* stream);

/* vdn_vda_readout with the linear branch's low-rank output gate formed in the kernel instead
 * of read: gate[t, h, c] = bf16(sigmoid(bf16(down[t] . up_w[h*128 + c] + up_b[h*128 + c]))),
 * with down [frames*spatial, 128] bf16 rows at row stride d_st (elements), up_w
 * [heads*128, 128] bf16, up_b [heads*128] bf16. Exactly one destination: bf16 `out` (strides
 * as vdn_vda_readout; codes = NULL) or MXFP8 `codes`/`scales`/`kp`/`chunk0` (as
 * vdn_vda_readout_mxfp8; out = NULL).
 * Replaces: output_gate(xv) (OutputGate.forward, src/models/attention_gates.py:52-55) +
 * the readout of paper_readout (src/models/linear_attention/paper_stack.py:315-318).
 */
int vdn_vda_readout_gated(const void* q, int64_t q_sf, int64_t q_sh, int64_t q_ss,
                          int activate_q, const void* state, const void* weight, int weight_f32,
                          float eps, const void* down, int64_t d_st, const void* up_w,
                          const void* up_b, void* out, int64_t o_sf, int64_t o_sh, int64_t o_ss,
                          void* codes, void* scales, int64_t kp, int chunk0, int frames,
                          int heads, int spatial, void* stream);

/*
 * RMSNorm(head_dim) * weight * gate of a frame-major readout [frames, heads, spatial, 128]
 * bf16; head_dim as in vdn_vda_readout (channels past it are zero).
 * Replaces: vdn_linear_epilogue (src/models/linear_attention/paper_sglang.py:406-437).
 */
int vdn_vda_epilogue(const void* readout, const void* weight, int weight_f32, float eps,
                     const void* gate, int64_t g_sf, int64_t g_sh, int64_t g_ss, void* out,
                     int64_t o_sf, int64_t o_sh, int64_t o_ss, int head_dim, int frames,
                     int heads, int spatial, void* stream);

/* ---------------------------------------------------------------------------------------
 * Frame-window softmax branch.
 * ------------------------------------------------------------------------------------- */

/*
 * QK RMSNorm + rotate-half RoPE, with act() the rounding to the activation dtype (flags bits
 * 4-5: 0 bf16, 1 fp16, 2 fp32, which has no rounding): n = act((x * rsqrt(mean(x^2) + eps)) *
 * w); for channel i < rot: out = act(act(n_i * c_i) + act(r_i * s_i)) with r_i = -n_{i+rot/2}
 * (i < rot/2) or n_{i-rot/2}; channels >= rot pass n. q, k: [tokens, heads, head_dim] of the
 * activation dtype with element strides (token, head, channel); weights [head_dim] with
 * stride (flags bit0 / bit1: fp32 q / k weight, else the activation dtype); cos, sin
 * (nullable together): [tokens, rot] with strides, fp32 when flags bit2 else the activation
 * dtype (values rounded to the activation dtype before use). qo, ko: contiguous, activation
 * dtype. flags bit3: q only (k, k's weight and ko may be null).
 * Replaces: paper_qk_rmsnorm_rope (src/models/softmax_attention/paper_qk_rope.py:145-211).
 */
int vdn_qk_rmsnorm_rope(const void* q, int64_t q_st, int64_t q_sh, int64_t q_sd, const void* k,
                        int64_t k_st, int64_t k_sh, int64_t k_sd, const void* q_w, int64_t q_ws,
                        const void* k_w, int64_t k_ws, float eps, const void* cos_t, int64_t c_st,
                        int64_t c_sd, const void* sin_t, int64_t s_st, int64_t s_sd, int rot,
                        int flags, int64_t tokens, int heads, int head_dim, void* qo, void* ko,
                        void* stream);

/*
 * Exact softmax attention of query blocks over key intervals (dtype 0: bf16, 1: fp16; head_dim
 * 64, 128 or 256): blocks int32 [nblocks, 3] = (first query, end of its query range, group),
 * <= 256 queries each; grp_kv int32 [groups, 8, 2] key intervals [a, b); grp_n int32 [groups].
 * q, k, v addressed by (token, head) strides with unit channel stride. gate (nullable): per
 * (token, head) scalar of the activation dtype applied as out = act(act(o) * gate). out:
 * activation dtype, (token, head) strides; lse (nullable): fp32 natural-log sum-exp of the
 * scaled scores.
 * Replaces: paper_window_attention (src/models/softmax_attention/paper_window.py:182-243)
 * and apply_softmax_gate (src/models/softmax_attention/kernels.py:51-67).
 */
int vdn_window_attention(const void* q, int64_t q_st, int64_t q_sh, const void* k, int64_t k_st,
                         int64_t k_sh, const void* v, int64_t v_st, int64_t v_sh,
                         const int* blocks, int nblocks, const int* grp_kv, const int* grp_n,
                         int heads, int head_dim, int dtype, float scale, const void* gate,
                         int64_t g_st, int64_t g_sh, void* out, int64_t o_st, int64_t o_sh,
                         float* lse, int64_t l_st, int64_t l_sh, void* stream);

/* vdn_window_attention with the output quantized in the epilogue instead of stored as bf16:
 * query row q, head h -> MXFP8 codes[q, 128 (chunk0 + h) .. +128) of a [rows, kp] code
 * matrix and the four E8M0 scales of that chunk in its SWIZZLE_32_4_4 scale array; the same
 * bytes vdn_mxfp8_quantize writes for the bf16 output. Rows without a query are not written.
 * codes 16-byte aligned, kp a multiple of 128 with (chunk0 + heads) * 128 <= kp.
 * q_norm_w (nullable, 16-byte aligned): [128] bf16 weight of an RMSNorm applied to each
 * (query, head) row as it is loaded, n = bf16((x * (1 / sqrt(mean(x^2) + q_norm_eps))) * w),
 * bit-identical to vdn_qk_rmsnorm_rope's norm of the queries (the QK norm of
 * src/models/softmax_attention/paper_qk_rope.py:82-95) followed by this entry point.
 * Replaces: paper_window_attention (src/models/softmax_attention/paper_window.py:182-243)
 * followed by quantize_activation (src/models/ops/mxfp8_quant.py:77-90) of its output.
 */
int vdn_window_attention_mxfp8(const void* q, int64_t q_st, int64_t q_sh, const void* k,
                               int64_t k_st, int64_t k_sh, const void* v, int64_t v_st,
                               int64_t v_sh, const int* blocks, int nblocks, const int* grp_kv,
                               const int* grp_n, int heads, float scale, const void* gate,
                               int64_t g_st, int64_t g_sh, const void* q_norm_w,
                               float q_norm_eps, void* codes, void* scales, int64_t kp,
                               int chunk0, void* stream);

/*
 * Gate projections of the hybrid block's attention input x [frames * spatial, k] bf16 (row
 * stride x_st, rows frame-major), one bf16 MFMA pass. w [384, k] bf16 holds the softmax-gate
 * rows (heads of them, zero rows up to 64), the beta rows (same), the output gate's down rows
 * (128) and FrameKDAAlpha's down rows (128). Writes
 *   soft_gate [T, heads] = bf16(sigmoid(bf16(x w_g^T + gate_bias)))   (one Linear with bias),
 *   beta      [T, heads] = bf16(sigmoid(bf16(x w_b^T))),
 *   gate_down [T, 128]   = bf16(x w_down^T)                            (all bf16, contiguous),
 *   partial [frames * ceil(spatial / 128), 128] fp32: sums over each 128-row block of a frame
 *   of x w_alpha^T (vdn_frame_alpha turns them into the frame mean's projection).
 * heads even and <= 64, k a multiple of 32; x, w and gate_down 16-byte aligned, soft_gate and
 * beta 4-byte aligned.
 * Replaces: the softmax gate, beta and output-gate projections of tp_attention_forward
 * (src/inference/utils/tensor_parallel.py:194-198; OutputGate, src/models/attention_gates.py:
 * 52-55) and its frame mean (:198).
 */
int vdn_gate_projection(const void* x, int64_t x_st, int64_t k, const void* w, int heads,
                        int frames, int spatial, const void* gate_bias, void* soft_gate,
                        void* beta, void* gate_down, float* partial, void* stream);

/*
 * FrameKDAAlpha from vdn_gate_projection's partial sums: mean[f] = (sum of the frame's
 * partial rows) / spatial, delta = mean up_w^T + dt_bias, alpha [frames, heads, head_dim] fp32
 * = exp(-exp(a_log[h]) softplus(delta)) (softplus threshold 20). up_w [heads * head_dim, 128]
 * bf16, dt_bias [heads * head_dim] fp32, a_log [heads] fp32.
 * Replaces: FrameKDAAlpha.forward (src/models/linear_attention/layers.py:36-69).
 */
int vdn_frame_alpha(const float* partial, int frames, int spatial, const void* up_w,
                    const float* dt_bias, const float* a_log, int heads, int head_dim,
                    float* alpha, void* stream);

/*
 * AdaLN tables out [m, n] bf16 (row stride o_st) = bf16(s w^T + b), s = bf16(SiLU(temb in
 * fp32)), temb [m, k] bf16 (temb_f32 = 0) or fp32 (row stride t_st), w [n, k] bf16
 * contiguous and 16-byte aligned, b [n] bf16 or null; k a multiple of 8, at most 16384.
 * Replaces: the table projection of _project_schedule (src/inference/utils/paper_adaln.py:
 * 174-188), F.linear(F.silu(temb.float()).to(bf16), weight, bias).
 */
int vdn_adaln_tables(const void* temb, int temb_f32, int64_t t_st, int m, int64_t k,
                     const void* w, const void* b, int64_t n, void* out, int64_t o_st,
                     void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VDNMI_H_ */
