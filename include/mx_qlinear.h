/*
 * mx_qlinear.h -- C ABI of the MI355X (gfx950) quantized DiT linear path.
 *
 * One shared library, libmx_qlinear.so, built by hipcc for gfx950 only. Every entry
 * point takes raw device pointers, element counts and a hipStream_t passed as void*,
 * enqueues its kernels on that stream and returns without synchronising. No entry point
 * allocates device memory: workspaces are the caller's (the INT8 GEMMs' tile-queue counters,
 * mxq_w4a8_codebook_gemm's decode chunk) or a static device array of the library
 * (mxq_w4a8_codebook_gemm_noalloc). Return value: MXQ_OK (0) or a negative error
 * code; mxq_last_error() then describes the failure (thread-local string).
 *
 * Reference paths are relative to the reference tree; CK stands for
 * backends/turbo/vendor/comfy_kitchen. Numerics follow the reference's eager
 * PyTorch path (CK/backends/eager/quantization.py), which is the semantics the
 * parity tests hold these kernels to.
 */
#ifndef MX_QLINEAR_H
#define MX_QLINEAR_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MXQ_ABI_VERSION 5

/* Return codes. */
#define MXQ_OK 0
#define MXQ_ERR_INVALID (-1)     /* bad argument (reference: ValueError / std::runtime_error) */
#define MXQ_ERR_UNSUPPORTED (-2) /* valid request outside this build (reference launchers return false) */
#define MXQ_ERR_HIP (-3)         /* HIP runtime or launch failure */

/* dtype codes: CK/backends/eager/quantization.py:34-42 (DTYPE_CODE_TO_DTYPE). */
#define MXQ_DTYPE_F32 0
#define MXQ_DTYPE_F16 1
#define MXQ_DTYPE_BF16 2
#define MXQ_DTYPE_E4M3 5

/* Pre-quantization activation codes: CK/backends/_activations.py:19-24. */
#define MXQ_ACT_NONE 0
#define MXQ_ACT_GELU_TANH 1
#define MXQ_ACT_SWIGLU 2

/* Thread-local description of the last failure in this thread ("" if none). */
const char* mxq_last_error(void);

/* MXQ_ABI_VERSION of the loaded library. */
int mxq_abi_version(void);

/*
 * Per-row (per-token) symmetric INT8 quantization.
 *   x      [rows, cols] of x_dtype (bf16, fp16 or fp32), row-major, contiguous
 *   q      [rows, cols] int8 out;  scales [rows] fp32 out
 *   input_act  MXQ_ACT_NONE or MXQ_ACT_GELU_TANH (bf16 or fp16): apply tanh-GELU to x first
 * Semantics: CK/backends/eager/quantization.py:857-875.
 * Replaces: launch_quantize_int8_rowwise_kernel, CK/backends/cuda/ops/int8_linear.cu:1035-1084
 * (stochastic rounding: mxq_quantize_int8_rowwise_stochastic).
 */
int mxq_quantize_int8_rowwise(const void* x, int x_dtype, int8_t* q, float* scales,
                              int64_t rows, int64_t cols, int input_act, void* stream);

/*
 * The same quantizer with stochastic rounding: noise [rows, cols] of x_dtype holds the caller's
 * uniform draws in [0, 1) (the reference draws torch.rand(x.shape, dtype=x.dtype) from a
 * generator on x's device seeded with the stochastic_rounding seed); then
 * q = clamp(floor(dt(dt(x / dt(s)) + noise)), -128, 127), dt the input dtype, NaN -> 0.
 * Semantics: quantize_int8_rowwise(x, stochastic_rounding=seed), CK/__init__.py:702-709 and
 * CK/backends/eager/quantization.py:803-826, 857-875.
 */
int mxq_quantize_int8_rowwise_stochastic(const void* x, int x_dtype, const void* noise, int8_t* q,
                                         float* scales, int64_t rows, int64_t cols, void* stream);

/*
 * The same quantizer for bf16 rows whose absmax is already known (row_absmax[r] must
 * equal max |x[r, :]|, e.g. accumulated by mxq_int8_gemm_dequant_gelu_absmax). One
 * streaming pass over x. Second half of the FFN chain's per-token re-quantization.
 */
int mxq_quantize_int8_rowwise_absmax(const void* x_bf16, const float* row_absmax, int8_t* q,
                                     float* scales, int64_t rows, int64_t cols, void* stream);

/*
 * The FFN intermediate's quantizer: h = gelu_tanh(y) in bf16, then the per-token quantizer of h
 * (q, scales as mxq_quantize_int8_rowwise). y bf16 [rows, cols], cols % 8 == 0, cols <= 32768,
 * 16-byte aligned; h_bf16 receives h when not NULL (it may be y itself: the update is in
 * place). Equals mxq_quantize_int8_rowwise(y, ..., MXQ_ACT_GELU_TANH) bit for bit.
 * Replaces: apply_input_act("gelu_tanh") + quantize_int8_rowwise inside fc2's int8_linear,
 * CK/backends/_activations.py:40-53 and CK/backends/eager/quantization.py:857-875.
 */
int mxq_quantize_int8_rowwise_gelu(const void* y_bf16, void* h_bf16, int8_t* q, float* scales,
                                   int64_t rows, int64_t cols, void* stream);

/*
 * adaLN: layer_norm(x, no affine, eps) * (1 + scale) + shift, bf16 in and out.
 *   scale, shift  [rows / scale_group, cols] and [rows / shift_group, cols] bf16: row r uses
 *                 modulation row r / scale_group (r / shift_group); a single [cols] vector
 *                 is scale_group = shift_group = rows.
 * Semantics: CK/backends/eager/adaln.py:11-14 (four bf16 roundings).
 * Replaces: launch_adaln_kernel, CK/backends/cuda/ops/adaln.cu:256-313 (subtract_mean=true).
 */
int mxq_adaln(const void* x, const void* scale, const void* shift, void* out, int64_t rows,
              int64_t cols, int64_t scale_group, int64_t shift_group, float eps, void* stream);

/*
 * adaLN fused with the per-row INT8 quantizer: q, scales = quantize(adaln(x, ...)).
 * y_out (bf16 [rows, cols]) optionally receives the modulated rows; pass NULL to skip.
 * Replaces the launch_adaln_kernel + launch_quantize_int8_rowwise_kernel pair that feeds
 * the QKV projection (CK/backends/cuda/ops/adaln.cu:256-313, int8_linear.cu:1035-1084).
 */
int mxq_adaln_quantize_int8(const void* x, const void* scale, const void* shift,
                            int64_t scale_group, int64_t shift_group, float eps, int8_t* q,
                            float* scales, void* y_out, int64_t rows, int64_t cols,
                            void* stream);

/*
 * adaLN on float16: y = f16(f16(f16(LN(x)) * f16(1 + scale)) + shift) with the LayerNorm
 * statistics in fp32, the reference's adaln evaluated in float16 (CK/backends/eager/adaln.py:
 * 11-14); scale/shift rows per group as mxq_adaln. y_out (float16 [rows, cols]) and q/scales (the
 * row quantizer of y with the float16 rule, CK/backends/eager/quantization.py:857-875) are each
 * optional (NULL), not both. Any cols.
 * Replaces: the reference's adaln and, with q, the quantizer that consumes it, on float16 tensors.
 */
int mxq_adaln_quantize_int8_f16(const void* x, const void* scale, const void* shift, int64_t scale_group,
                                int64_t shift_group, float eps, int8_t* q, float* scales, void* y_out,
                                int64_t rows, int64_t cols, void* stream);

/*
 * Tile-queue workspace of the INT8 GEMMs below (the `workspace, workspace_bytes` pair before the
 * stream). The hardware deals workgroups to the 8 XCDs round-robin, so a static tile order gives
 * every XCD 1/8 of the tiles, and the slowest XCD sets the GEMM's time. With a workspace, the
 * last eighth of each XCD's tiles is claimed at run time by whichever XCD's workgroups get there
 * first (counters in the workspace); the tiles and their outputs are the same, bit for bit.
 * NULL runs the static order. The workspace is MXQ_GEMM_WORKSPACE_BYTES of device memory,
 * 256-byte aligned and zero before its first use; every call leaves it zero again. Calls that
 * share a workspace must be ordered (one workspace per stream): overlapping calls race on it.
 * The reference keeps a per-(device, stream) workspace inside its launchers for the same kind
 * of state (CK/backends/cuda/ops/cutlass_gemm_int8.cu:39-55); here the caller owns it.
 */
#define MXQ_GEMM_WORKSPACE_BYTES ((int64_t)4096)

/*
 * Launch plan the INT8 GEMMs below choose for an M x N x K problem (table_epilogue: 1 for the
 * GELU epilogue, 2 for the SwiGLU one, 0 otherwise) given workspace_bytes of tile-queue workspace (0:
 * none): plan[0] tile rows (256 or 128), plan[1] workgroups, plan[2] tiles, plan[3] tiles per
 * XCD claimed at run time (0: static order), plan[4] workgroups per XCD, plan[5] stages of
 * operands requested ahead of the MFMAs (4 when the 128-tiles all fit on the CUs at once, one
 * workgroup per CU; else 2), plan[6] tile-rows per group of the tile order, plan[7] 1 when
 * the workgroups loop over tiles (one per CU: plan[4] per XCD each take the static positions
 * start + k, start + k + plan[4], ... of their XCD's range, then claim pool positions) and 0 when
 * each runs one tile, plan[8] tile columns (the tile rows, or 96: 128 x 96 tiles when those
 * still fit on the CUs at once and use more of them). plan holds 9 entries. Host only; no
 * reference counterpart (CUTLASS's Gemm::get_workspace_size is the nearest,
 * CK/backends/cuda/ops/cutlass_gemm_int8.cu:318); tests and tuning read it.
 */
int mxq_int8_gemm_plan(int64_t M, int64_t N, int64_t K, int table_epilogue, int64_t workspace_bytes,
                       int64_t* plan);

/*
 * Raw INT8 GEMM: C[m, n] = sum_k A[m, k] * B[n, k] in int32.
 *   a [M, K] int8 row-major; b [N, K] int8 row-major (the checkpoint's [out, in] layout);
 *   c [M, ldc] int32. K must be a multiple of 16.
 * Replaces: torch._int_mm in _int8_matmul_accumulate, CK/backends/eager/quantization.py:749-782.
 */
int mxq_int8_gemm_i32(const int8_t* a, const int8_t* b, int32_t* c, int64_t M, int64_t N,
                      int64_t K, int64_t ldc, void* workspace, int64_t workspace_bytes,
                      void* stream);

/*
 * INT8 GEMM with the fused dequant epilogue:
 *   D[m, n] = out(fp32(acc) * (xs[m] * ws[n]));  D[m, n] = out(D[m, n] + bias[n])
 *   xs [M] fp32; ws [ws_numel] fp32 with ws_numel 1 (tensorwise) or N (per channel);
 *   bias [N] of out_dtype or NULL; d [M, ldd] of out_dtype (fp32, fp16 or bf16).
 * Semantics: CK/backends/eager/quantization.py:1031-1054.
 * Replaces: launch_cutlass_int8_dequant / launch_cutlass_int8_dequant_strided,
 * CK/backends/cuda/ops/cutlass_gemm_int8.cu:613-665 (there bias is fp32 and the bias add is
 * fused before one rounding; here it follows the eager two-rounding recipe).
 */
int mxq_int8_gemm_dequant(const int8_t* a, const int8_t* b, const float* xs, const float* ws,
                          int64_t ws_numel, const void* bias, void* d, int64_t M, int64_t N,
                          int64_t K, int64_t ldd, int out_dtype, void* workspace,
                          int64_t workspace_bytes, void* stream);

/*
 * fc1 of the INT8 FFN chain: the bf16 dequant epilogue above, then tanh-GELU in bf16,
 *   h[m, n] = bf16(gelu(bf16(bf16(acc * (xs*ws)) + bias)))
 * and row_absmax[m] = max(row_absmax[m], max_n |h[m, n]|) by atomics. row_absmax must hold
 * zeros (or earlier partial maxima) on entry; mxq_fill_f32 clears it on the stream.
 * Replaces the reference's fc1 int8_linear + apply_input_act("gelu_tanh") + the absmax half of
 * fc2's quantizer (CK/backends/eager/quantization.py:971-1056, CK/backends/_activations.py:40-53).
 */
int mxq_int8_gemm_dequant_gelu_absmax(const int8_t* a, const int8_t* b, const float* xs,
                                      const float* ws, int64_t ws_numel, const void* bias_bf16,
                                      void* h_bf16, float* row_absmax, int64_t M, int64_t N,
                                      int64_t K, int64_t ldh, void* workspace,
                                      int64_t workspace_bytes, void* stream);

/*
 * SwiGLU fc1: INT8 GEMM + the bf16 dequant epilogue of mxq_int8_gemm_dequant, then
 *   h[m, c] = bf16(bf16(silu(y[m, gate c])) * y[m, up c])        (NaN products -> 0x7FC0)
 * written as h bf16 [M, N / 2] (row stride ldh). b / ws / bias are fc1's [N] rows in the
 * prepared order: for each block of 32 rows, the 16 gate rows 16 b .. 16 b + 15 of the original
 * [gate | up] weight, then the 16 up rows N/2 + 16 b .. N/2 + 16 b + 15. N % 32 == 0.
 * Equals mxq_int8_gemm_dequant (original row order) followed by the SwiGLU input activation of
 * the next quantizer (CK/backends/_activations.py:50-52) bit for bit.
 * Replaces: fc1 + the SwiGLU half of int8_linear(raw, ..., input_act="swiglu")
 * (h3serve/native_engine/model/fused_mlp.py:386-420).
 */
int mxq_int8_gemm_dequant_swiglu(const int8_t* a, const int8_t* b, const float* xs,
                                 const float* ws, int64_t ws_numel, const void* bias_bf16,
                                 void* h_bf16, int64_t M, int64_t N, int64_t K, int64_t ldh,
                                 void* workspace, int64_t workspace_bytes, void* stream);

/*
 * INT8 GEMM + dequant epilogue + gated residual update, in place:
 *   y = the bf16 output of mxq_int8_gemm_dequant (same arguments and roundings)
 *   residual[m, n] = bf16(residual[m, n] + y[m, n] * gate[gate_rows[m], n])
 *   residual  bf16 [M, ldr] (read and written); gate bf16 [gate_count, ldg]; gate_rows int32 [M]
 *   (each row's modulation row; indices outside [0, gate_count) are clamped into it, so a bad
 *   map gives wrong values, never an out-of-bounds read; callers validate it).
 * Semantics: int8_linear followed by residual[a:b].addcmul_(y[a:b], gate[row].to(bf16)) per
 * modulation segment (h3serve/native_engine/model/layers.py:944-960, fused_mlp.py:386-420).
 * Replaces: _fused_down_gated_residual's GEMM + epilogue kernel
 * (h3serve/native_engine/model/fused_mlp.py:63-143, 159-219).
 */
int mxq_int8_gemm_gated_residual(const int8_t* a, const int8_t* b, const float* xs,
                                 const float* ws, int64_t ws_numel, const void* bias_bf16,
                                 void* residual_bf16, int64_t ldr, const void* gate_bf16,
                                 int64_t ldg, int64_t gate_count, const int32_t* gate_rows,
                                 int64_t M, int64_t N, int64_t K, void* workspace,
                                 int64_t workspace_bytes, void* stream);

/*
 * M = 1 INT8 linear: the row quantizer of x (after the optional input activation and ConvRot
 * rotation, exactly as mxq_quantize_int8_rowwise_convrot with rows = 1) into the caller's
 * workspace xq (int8 [K], 16-byte aligned) / xs (fp32 [1]), then a weight-streaming INT8 GEMV
 * against w [N, K] with the dequant epilogue of mxq_int8_gemm_dequant (same roundings, so the
 * result equals the batched path's row). Two launches on `stream`. x bf16 [K] ([2K] for
 * MXQ_ACT_SWIGLU); K % 16 == 0, K <= 16384; group_size 0 or a power of 4 up to 1024 dividing K.
 * Replaces: int8_linear_m1 (CK/backends/cuda/__init__.py:1999-2034; CK/backends/cuda/ops/
 * int8_linear.cu:1490-1590).
 */
int mxq_int8_linear_m1(const void* x_bf16, const int8_t* w, const float* ws, int64_t ws_numel,
                       const void* bias, void* out, int64_t N, int64_t K, int64_t group_size,
                       int input_act, int out_dtype, int8_t* xq, float* xs, void* stream);

/*
 * M = 1 INT8 GEMV + dequant epilogue from an already quantized row (xq int8 [K], xs fp32 [1]);
 * out = the row mxq_int8_gemm_dequant would produce. K % 16 == 0, K <= 16384.
 * Replaces: int8_gemv_dequant (CK/backends/cuda/__init__.py:1587-1610; CK/backends/cuda/ops/
 * int8_linear.cu:411-492).
 */
int mxq_int8_gemv_dequant(const int8_t* xq, const float* xs, const int8_t* w, const float* ws,
                          int64_t ws_numel, const void* bias, void* out, int64_t N, int64_t K,
                          int out_dtype, void* stream);

/*
 * y[i] = gelu_tanh(x[i]) for n bf16 values, bit-identical to torch's CPU
 * gelu(approximate="tanh") on bfloat16 (x and y may alias).
 * Replaces: apply_input_act(x, "gelu_tanh"), CK/backends/_activations.py:40-53.
 */
int mxq_gelu_tanh_bf16(const void* x, void* y, int64_t n, void* stream);

/*
 * RMS adaLN (RMSNorm with weight, then segmented modulation), optionally fused with the ConvRot
 * rotation and the per-row INT8 quantizer:
 *   n = bf16((x * r) * w),  r = 1 / sqrt(fp32(sum x^2) / cols + eps)
 *   y = bf16(bf16(n * bf16(1 + scale[mod_rows[m]])) + shift[mod_rows[m]])
 *   q, scales = the row quantizer of y rotated per group of group_size columns (as
 *   mxq_quantize_int8_rowwise_convrot; group_size 0: no rotation).
 *   x bf16 [rows, cols]; norm_weight bf16 [cols]; scale, shift bf16 [mod_count, ld_mod];
 *   mod_rows int32 [rows] (clamped into [0, mod_count)). y_out (bf16 [rows, cols]) and q/scales
 *   are each optional (NULL), not both. cols % 16 == 0, ld_mod % 8 == 0, 16-byte aligned tensors.
 *   workspace (optional, 16-byte aligned): with q set and at least mod_count * ld_mod * 2 bytes,
 *   bf16(1 + scale) of every modulation row is formed there once per call (one small kernel on
 *   the stream before the main one) and read by the main kernel in place of scale; otherwise each
 *   element forms it. The outputs are the same either way. Calls that share a workspace on two
 *   streams race.
 * Semantics: rms_adaln, h3serve/native_engine/model/kernels.py:7594-7640 (eager branch) with
 * RMSNorm = F.rms_norm(x, weight.to(x.dtype), eps) (h3serve/native_engine/model/layers.py:33-48).
 * Replaces: segmented_rms_adaln / native_rms_one_pass_adaln
 * (backends/original/kernels/fused_norm_rope.py:319-428) and, with q, the quantizer launch of the
 * QKV / fc1 ConvRotInt8Linear that consumes the result.
 */
int mxq_rms_adaln_quantize_int8(const void* x, const void* norm_weight, const void* scale,
                                const void* shift, int64_t ld_mod, int64_t mod_count,
                                const int32_t* mod_rows, float eps, void* y_out, int8_t* q,
                                float* scales, int64_t rows, int64_t cols, int64_t group_size,
                                void* workspace, int64_t workspace_bytes, void* stream);

/*
 * The same on float16: x, norm_weight, scale, shift and y_out float16, every rounding above to
 * float16 instead of bfloat16 (the reference's RMSNorm and modulation evaluated in float16), the
 * rotated values rounded once to float16 and quantized with the float16 rule.
 * Replaces: rms_adaln (kernels.py:7594-7640) and its quantizer on float16 tensors.
 */
int mxq_rms_adaln_quantize_int8_f16(const void* x, const void* norm_weight, const void* scale,
                                    const void* shift, int64_t ld_mod, int64_t mod_count,
                                    const int32_t* mod_rows, float eps, void* y_out, int8_t* q,
                                    float* scales, int64_t rows, int64_t cols, int64_t group_size,
                                    void* stream);

/*
 * ConvRot rotation + per-row INT8 quantization, optionally after an activation:
 *   a = act(x)  (MXQ_ACT_NONE; MXQ_ACT_GELU_TANH; MXQ_ACT_SWIGLU: x is [rows, 2*cols] = [gate | up]
 *               and a = bf16(bf16(silu(gate)) * up), CK/backends/_activations.py:40-53)
 *   r = a @ H_G per group of group_size columns, H_G = kron(h4, ..., h4) / sqrt(G), rounded once
 *       to x's dtype (the exact product; CK/tensor/int8_utils.py:11-74), skipped if group_size == 0
 *   q, scales = the row quantizer of r (CK/backends/eager/quantization.py:857-875).
 *   x_dtype: bf16 or fp16 (any activation; fp16 activations as mxq_input_act_f16) or fp32 (no
 *   activation); cols % 16 == 0; group_size a power of 4 up to 1024 dividing cols (or 0).
 * Replaces: launch_quantize_int8_rowwise_convrot{,64} (CK/backends/cuda/ops/int8_linear.cu:
 * 1086-1157, 1295-1409) and the eager rotation before quantize_int8_rowwise
 * (CK/backends/eager/quantization.py:1012-1025).
 */
int mxq_quantize_int8_rowwise_convrot(const void* x, int x_dtype, int8_t* q, float* scales,
                                      int64_t rows, int64_t cols, int64_t group_size,
                                      int input_act, void* stream);

/*
 * y[r, c] = bf16(bf16(silu(x[r, c])) * x[r, cols + c]) for a [rows, 2*cols] bf16 x (SwiGLU:
 * gate | up halves), bit-identical to torch's CPU silu(gate).mul_(up) on bfloat16.
 * Replaces: apply_input_act(x, "swiglu"), CK/backends/_activations.py:50-52.
 */
int mxq_swiglu_bf16(const void* x, void* y, int64_t rows, int64_t cols, void* stream);

/*
 * The input activation on float16: input_act MXQ_ACT_GELU_TANH gives y[r, c] = gelu_tanh(x[r, c])
 * for x [rows, cols]; MXQ_ACT_SWIGLU gives y[r, c] = fp16(fp16(silu(x[r, c])) * x[r, cols + c])
 * for x [rows, 2*cols]. Bit-identical to torch's CPU routines on float16, NaN patterns included.
 * Replaces: apply_input_act(x, input_act) on a float16 x, CK/backends/_activations.py:40-53.
 */
int mxq_input_act_f16(const void* x, void* y, int64_t rows, int64_t cols, int input_act, void* stream);

/* p[0..n) = value on the stream (a kernel, so it is safe inside captured graphs). */
int mxq_fill_f32(float* p, float value, int64_t n, void* stream);

/*
 * Grouped int4 -> int8 weight decode:
 *   w8[n, k] = clamp(rne(v * s_rel[n, k / G]), -127, 127), v = codebook[c] or c - 8,
 *   c = low nibble of qdata[n, k/2] for even k, high nibble for odd k.
 *   qdata [N, K/2] int8; s_rel [N, K/G] fp32 (s_rel_dtype 0) or float8_e4m3fn bits (5);
 *   codebook [16] fp32 or NULL; out [N, K] int8. K a multiple of 16 and of G, at most 2^30;
 *   G = 4, 8, or a multiple of 16; qdata 8-byte aligned (MXQ_ERR_INVALID / _UNSUPPORTED else).
 * Semantics: CK/backends/eager/w4a8_int8.py:344-363.
 * Replaces: launch_dequant_int4_grouped_to_int8 / _e4m3, CK/backends/cuda/ops/w4a8_gemm.cu:93-121.
 */
int mxq_dequant_int4_grouped_to_int8(const int8_t* qdata, const void* s_rel, int s_rel_dtype,
                                     const float* codebook, int8_t* out, int64_t N, int64_t K,
                                     int64_t group_size, void* stream);

/*
 * Reference-format W4A8 linear on an already quantized activation: decode the packed weight
 * chunk by chunk into `workspace` ([chunk_cols, K] int8) and run the dequant GEMM with
 * ws = s_channel. Arguments as mxq_dequant_int4_grouped_to_int8 and mxq_int8_gemm_dequant;
 * out [M, N] of out_dtype, bias [N] of out_dtype or NULL; gemm_workspace / gemm_workspace_bytes
 * are the chunk GEMMs' tile-queue workspace, as for the INT8 GEMMs (NULL, 0: static order).
 * Replaces: launch_w4a8_codebook_gemm_chunked, CK/backends/cuda/ops/w4a8_gemm.cu:133-164.
 */
int mxq_w4a8_codebook_gemm(const int8_t* xq, const int8_t* qdata, const void* s_rel,
                           int s_rel_dtype, const float* codebook, const float* s_channel,
                           const float* xs, const void* bias, int8_t* workspace, void* out,
                           int64_t M, int64_t N, int64_t K, int64_t group_size,
                           int64_t chunk_cols, int out_dtype, void* gemm_workspace,
                           int64_t gemm_workspace_bytes, void* stream);

/*
 * mxq_w4a8_codebook_gemm without the caller's workspace: the decoded chunk lives in a static
 * device array of the library (32 MiB per GPU, held until the process ends), so the call
 * allocates nothing. No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Same arguments and results (bit for bit) as mxq_w4a8_codebook_gemm, less
 * `workspace` and the GEMM workspace (a second static array, 4 KiB, holds the tile-queue
 * counters); min(chunk_cols, N) * K must not exceed 32 MiB (MXQ_ERR_INVALID otherwise).
 * Calls share the GPU's arrays. Each call makes its stream wait for the previous call on the same
 * GPU (an event the library creates with its first call per device and records after every
 * call), so calls on different streams do not overlap. Under graph capture the wait and the
 * record are left out: a replayed graph that runs beside another call on the same GPU races
 * with it on the arrays.
 */
int mxq_w4a8_codebook_gemm_noalloc(const int8_t* xq, const int8_t* qdata, const void* s_rel,
                                   int s_rel_dtype, const float* codebook, const float* s_channel,
                                   const float* xs, const void* bias, void* out, int64_t M, int64_t N,
                                   int64_t K, int64_t group_size, int64_t chunk_cols, int out_dtype,
                                   void* stream);

/*
 * Grouped-scale W4A8 GEMM (int4 weights with one fp16 scale per K-group and output channel):
 *   P_g[m, n] = sum_{k in group g} A[m, k] * (c[n, k] - 8)      (exact int32)
 *   acc       = fma-accumulated over g = 0, 1, ... of fp32(P_g) * fp32(scale[g, n])
 *   D[m, n]   = out(acc * xs[m]);  then D = out(D + bias[n]) if bias
 *   a [M, K] int8; xs [M] fp32; qdata [N, K/2] int8 (offset-8 nibbles packed as in
 *   CK/backends/eager/w4a8_int8.py:200-202); group_scale [K/G, N] fp16; G = group_size
 *   (a multiple of 128 here); d [M, ldd] of out_dtype.
 * The reference has no kernel for this layout (its W4A8 folds group scales into the int8
 * grid, w4a8_gemm.cu:4-18); unpacking follows CK/backends/eager/w4a8_int8.py:351-355.
 */
int mxq_w4a8_gemm_grouped(const int8_t* a, const float* xs, const int8_t* qdata,
                          const uint16_t* group_scale, const void* bias, void* d, int64_t M,
                          int64_t N, int64_t K, int64_t group_size, int64_t ldd, int out_dtype,
                          void* stream);

/*
 * Left operand of the reference-format W4A8 correction term:
 *   out[m, g] = o(o(sum_{k in group g} xq[m, k]) * o(xs[m])), o = rounding to out_dtype
 *   xq [M, K] int8 (the quantized, rotated activations); xs [M] fp32; out [M, K/G].
 * The caller adds out @ correction ([K/G, N], out_dtype) to the linear's output with a library
 * GEMM (out.addmm_ in the reference).
 * Replaces: the correction branch of CK/backends/cuda/__init__.py:2294-2297 (its group sums).
 */
int mxq_int8_group_sums(const int8_t* xq, const float* xs, void* out, int64_t M, int64_t K,
                        int64_t group_size, int out_dtype, void* stream);

/*
 * Weight preparation for mxq_w4a8_gemm_grouped_prepared (a load-time layout transform, no
 * counterpart in the reference): qdata [N, K/2] as above -> out [N, K/2] (may alias qdata),
 * K % 8 == 0. Each 32-bit word keeps the 8 codes of k = 8w .. 8w + 7; byte j of the result
 * holds (c[8w + j] ^ 8) in its low nibble and (c[8w + 4 + j] ^ 8) in its high nibble (the code
 * as the 4-bit two's complement value c - 8), so the GEMM unpacks a word with one shift and two
 * masks instead of the six instructions the checkpoint layout needs.
 */
int mxq_w4a8_prepare_grouped(const int8_t* qdata, int8_t* out, int64_t N, int64_t K, void* stream);

/*
 * mxq_w4a8_gemm_grouped on weights prepared by mxq_w4a8_prepare_grouped: same arguments and
 * results (bit for bit); group_size must be 128, N a multiple of 8 and group_scale 16-byte
 * aligned (MXQ_ERR_UNSUPPORTED otherwise).
 */
int mxq_w4a8_gemm_grouped_prepared(const int8_t* a, const float* xs, const int8_t* qdata,
                                   const uint16_t* group_scale, const void* bias, void* d, int64_t M,
                                   int64_t N, int64_t K, int64_t group_size, int64_t ldd, int out_dtype,
                                   void* stream);

/* Storage modes of mxq_w4a8_quantize_weight. */
#define MXQ_W4_CODEBOOK 0     /* symmetric, 16-level codebook (the reference's default) */
#define MXQ_W4_SYMMETRIC 1    /* symmetric uniform codes c - 8 */
#define MXQ_W4_ASYMMETRIC 2   /* min/max codes with a correction term */
#define MXQ_W4_ROTATE_ONLY 3  /* only the ConvRot rotation, written to rotated_out */

/*
 * Offline W4A8 weight preparation, one launch: ConvRot rotation of each weight row (group
 * convrot_groupsize, a power of 4, or 0 for none; the exact product rounded once to the weight's
 * dtype) and the grouped int4 storage of the rotated row:
 *   w bf16 or fp32 [N, K] (w_dtype); K % 16 == 0, K <= 16384; group_size >= 4 dividing 16 or a
 *   multiple of 16, at most 128; codebook fp32 [16] (MXQ_W4_CODEBOOK);
 *   packed int8 [N, K/2] (two codes per byte, even k in the low nibble); s_rel [N, K/G] fp32 or
 *   float8_e4m3fn bits (s_rel_dtype 0 or 5); s_channel fp32 [N]; correction [K/G, N] of w_dtype
 *   (MXQ_W4_ASYMMETRIC); rotated_out [N, K] of w_dtype or NULL (the rotated rows).
 * Semantics: _quantize_rotated_w4a8_int8_weight after the weight rotation,
 * CK/backends/eager/w4a8_int8.py:122-209 (group sums in torch's CPU order for groups of <= 32).
 * Replaces: the per-element part of quantize_w4a8_int8_weight (w4a8_int8.py:243-341) and
 * rotate_int8_convrot_weight (CK/backends/eager/quantization.py:909-912); the codebook choice
 * (w4a8_int8.py:24-32, 221-240) stays with the caller.
 */
int mxq_w4a8_quantize_weight(const void* w, int w_dtype, int64_t N, int64_t K, int64_t group_size,
                             int64_t convrot_groupsize, int mode, const float* codebook, int s_rel_dtype,
                             int8_t* packed, void* s_rel, float* s_channel, void* correction, void* rotated_out,
                             void* stream);

/*
 * Measurement helper (no counterpart in the reference; it calibrates the roofline): runs
 * `workgroups` x 256 threads, each lane cycling eight v_mfma_i32_32x32x32_i8 accumulators over
 * four A and two B 16-byte fragments read from a / b (wrapping within a_bytes / b_bytes), for
 * `iters` iterations of 8 MFMAs with no memory traffic. sink int32 [workgroups * 256] receives
 * each lane's accumulator sum; clocks uint64 [workgroups * 2] the shader-clock cycles and the
 * 100 MHz reference-clock ticks of the loop per workgroup. Operands 16-byte aligned.
 * Throughput = 2 * 32768 * 8 * iters * 4 waves * workgroups / elapsed; the clock = cycles /
 * ticks * 100 MHz. With a GEMM's own operands this is the MFMA ceiling for that data: the board
 * power limit lowers the clock as the operand bits toggle more.
 */
int mxq_probe_mfma_i8(const int8_t* a, int64_t a_bytes, const int8_t* b, int64_t b_bytes, int32_t* sink,
                      uint64_t* clocks, int64_t workgroups, int64_t iters, void* stream);

/*
 * Test helper (no counterpart in the reference; it pins the lane pairings the row reductions of
 * the quantizers rely on): one wave64 writes xor4[i] = the value lane_xor4 hands lane i when
 * every lane offers its own index (i ^ 4 by construction), row16[i] = the 16-lane float64 sum of
 * in[] with the pairing i ^ 1, 2, 4, 8 in that order, and wsum[i] = the float32 wave sum of
 * (float)in[] with the pairing i ^ 32, 16, 8, 4, 2, 1. in: 64 doubles; outputs 64 each.
 */
int mxq_probe_lane_exchange(const double* in, uint32_t* xor4, double* row16, float* wsum, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MX_QLINEAR_H */
