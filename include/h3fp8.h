/*
 * libh3fp8 -- C ABI of the MI355X (gfx950) online-FP8 linear path of the MiniMax H3 DiT.
 *
 * Every entry point is `extern "C"`, takes plain device pointers, element strides and sizes, and a HIP stream
 * (`stream` is a `hipStream_t`; NULL = the default stream).  The library never allocates device memory for a call and
 * never keeps a pointer past the call: the caller (the Python shim, which allocates with torch on the current stream)
 * owns every input, output and workspace.  Calls are asynchronous on `stream`; the library launches kernels only.
 *
 * Status: 0 on success, a negative H3FP8_E* code otherwise, with a message in h3fp8_last_error() (thread-local).
 *
 * Layouts (reference: h3_tp2/fp8_gemm.py:362-373, :73; fp8_cutlass.py:93, :111-112):
 *   a   e4m3fn activations [M, K] row-major, row stride lda (elements = bytes)
 *   w   e4m3fn weight [N, K] row-major, row stride ldw (the GEMM's B = w^T: torch's `b` with `b.t()` contiguous)
 *   sa  fp32 per-token scales, element m at sa[m * sa_stride] (sa_stride 0: one scalar scale)
 *   sb  fp32 per-channel scales, element n at sb[n * sb_stride] (sb_stride 0: one scalar scale)
 *   y   [M, N] row-major output, row stride ldy, bf16 or fp16 (out_dtype)
 * Requirements (checked; H3FP8_EINVAL otherwise): K % 16 == 0, N % 16 == 0, 16-byte aligned a/w/y rows
 * (lda, ldw multiples of 16, ldy multiple of 8), M, N, K >= 0.
 */
#ifndef H3FP8_H
#define H3FP8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define H3FP8_ABI_VERSION 1

#define H3FP8_OK 0
#define H3FP8_EINVAL (-22)   /* bad shape, stride, alignment or argument */
#define H3FP8_EHIP (-5)      /* a HIP runtime call failed */

#define H3FP8_DT_BF16 0
#define H3FP8_DT_FP16 1
#define H3FP8_DT_F32 2       /* h3fp8_gemm only: the raw fp32 accumulator, scales ignored (the reference's fused
                                kernel with OUT 0, h3_tp2/fp8_gemm.py:74, :98-99; here also the product of the
                                two-pass form, whose scale pass or fused consumer follows) */

/* ABI version (H3FP8_ABI_VERSION of the build) and the last error of the calling thread. */
int h3fp8_abi_version(void);
const char* h3fp8_last_error(void);

/*
 * One-time set-up of the current device: fills the device-resident SiLU table (65536 bf16 entries) and waits for it.
 * Every entry point calls it on first use of a device; calling it early keeps that wait out of the hot path.
 * No counterpart in the reference (its Triton kernels compute exp inline).
 */
int h3fp8_init(void);

/*
 * Kernel 1 -- per-token dynamic FP8 quant of a bf16 [M, K] tensor:
 *   scale[m] = max(max_k |x[m,k]| / 448, 1/(448*512)),  q[m,k] = e4m3fn_rne(clamp(x[m,k] * (1/scale[m]), +-448)).
 * Replaces QuantFP8.forward (dynamic, per token) as the reference routes it: h3_tp2/fp8_quant_fuse.py:553-576
 * (the forward wrapper), :318-327 (launcher `quant`), :280-290 (`_quant_kernel`); same arithmetic as
 * h3_tp2/ulysses_outq.py:73-93 with one segment.  x rows: stride ldx (elements, multiple of 8); q rows: stride ldq.
 */
int h3fp8_quant_rows(const void* x, int64_t ldx, int64_t M, int64_t K, void* q, int64_t ldq, float* scale,
                     void* stream);

/*
 * The same quant when the row maxima are already known (the tail pass of a GEMM whose epilogue reduced them):
 * scale[m] = max(row_amax[m] / 448, MIN_SCALE), q as above.  x is bf16 [M, K].
 * Replaces the second half of the fused-quant producers (fp8_quant_fuse.py:105-121, :262-278 after the row max).
 */
int h3fp8_quant_rows_amax(const void* x, int64_t ldx, int64_t M, int64_t K, const float* row_amax, void* q,
                          int64_t ldq, float* scale, void* stream);

/*
 * Kernel 1 on rows made of P segments: logical row m (P * seg wide) is x[p * stride_p + m * stride_m .. + seg] for
 * p = 0 .. P-1 (element offsets), e.g. the reverse all-to-all's receive buffer [P, M, seg] (stride_p = M * seg,
 * stride_m = seg) read as the out projection's [M, P * seg] input without unpacking it.  q [M, P * seg] (row stride
 * ldq) and scale [M] as h3fp8_quant_rows.  seg and the strides multiples of 8, P * seg <= 16384, x 16-byte aligned,
 * the source within 2 GiB.  Replaces ulysses_outq.quant_rows / _quant_rows_kernel (h3_tp2/ulysses_outq.py:73-93,
 * :109-124) and fp8_quant_fuse.unpack_quant / _unpack_quant_kernel (h3_tp2/fp8_quant_fuse.py:372-385, :245-260).
 */
int h3fp8_quant_segments(const void* x, int64_t P, int64_t seg, int64_t stride_p, int64_t stride_m, int64_t M,
                         void* q, int64_t ldq, float* scale, void* stream);

/*
 * Kernel 2 -- scaled FP8 GEMM:  y[m,n] = round(sa[m] * (sb[n] * sum_k a[m,k] w[n,k]))  (fp32 accumulation, K
 * ascending per lane, no split-K), or round(fma(sa[m], sb[n]*acc, bias[n])) with a bias ([N], in out_dtype).
 * Replaces ops.cutlass_scaled_mm(a, b=w^T, scale_a, scale_b, out_dtype, bias) as routed by the reference:
 * h3_tp2/fp8_gemm.py:362-382 (`_mm`), :328-341 (`route`), :149-164 (`scaled_mm_tensor32`), :240-248
 * (`scaled_mm_fused`); h3_tp2/fp8_cutlass.py:115-131 (`scaled_mm`), fp8_cutlass_kernel.py:698-733 (epilogue).
 * row_amax: NULL, or an [M] fp32 workspace that receives max_n |y[m,n]| of the rounded outputs (the next layer's
 * per-token quant fused into this epilogue; finish it with h3fp8_quant_rows_amax).  The library zeroes it first.
 */
int h3fp8_gemm(const void* a, int64_t lda, const void* w, int64_t ldw, const float* sa, int64_t sa_stride,
               const float* sb, int64_t sb_stride, const void* bias, void* y, int64_t ldy, int out_dtype, int64_t M,
               int64_t N, int64_t K, float* row_amax, void* stream);

/*
 * Kernel 2 + fused next-layer quant: y as h3fp8_gemm (bf16), then q [M, N] e4m3fn + scale [M] of y.
 * amax_ws: [M] fp32 workspace.  No single counterpart in the reference (its producers fuse the quant instead,
 * fp8_quant_fuse.py:23-28); the arithmetic is kernel 1's on the bf16 output.
 */
int h3fp8_gemm_quant(const void* a, int64_t lda, const void* w, int64_t ldw, const float* sa, int64_t sa_stride,
                     const float* sb, int64_t sb_stride, const void* bias, void* y, int64_t ldy, int64_t M, int64_t N,
                     int64_t K, float* amax_ws, void* q, int64_t ldq, float* scale, void* stream);

/*
 * h3fp8_gemm_quant without the workspace argument: the [M] row maxima go to a buffer the library owns (one static
 * device array of H3FP8_NOALLOC_MAX_ROWS fp32 per device, 1 MiB, held until the process ends), so the call allocates
 * nothing -- no hipMalloc / hipFree, no allocating library routine, no stream or event creation.  The buffer is
 * cleared by a fill kernel on `stream` at every call.  Requirements beyond h3fp8_gemm_quant's: M <= H3FP8_NOALLOC_
 * MAX_ROWS (H3FP8_EINVAL otherwise) and h3fp8_init already run on the current device (H3FP8_EINVAL otherwise).
 * Every call on a device shares that device's buffer: calls that overlap on one device (on different streams, or
 * from different threads) race and must be ordered by the caller.  Outputs y, q and scale equal h3fp8_gemm_quant's.
 * No counterpart in the reference: it is for callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid allocation).
 */
#define H3FP8_NOALLOC_MAX_ROWS 262144
int h3fp8_gemm_quant_noalloc(const void* a, int64_t lda, const void* w, int64_t ldw, const float* sa,
                             int64_t sa_stride, const float* sb, int64_t sb_stride, const void* bias, void* y,
                             int64_t ldy, int64_t M, int64_t N, int64_t K, void* q, int64_t ldq, float* scale,
                             void* stream);

/*
 * Kernel 3 -- gate/up GEMM with the SwiGLU epilogue:  w_gate_up is [2F, K] (gate rows 0..F-1, up rows F..2F-1, vLLM's
 * merged layout), sb and bias are [2F].  For each (m, f):
 *   g = bf16(epi(acc[m, f])), u = bf16(epi(acc[m, F+f])), u = (u == 0 ? +0 : u),
 *   h[m, f] = bf16(bf16(g / (1 + exp(-g))) * u)     (exp correctly rounded; a device table of all 65536 g values)
 * writes h bf16 [M, F] (row stride ldh) and, if row_amax != NULL, max_f |h[m, f]| into row_amax[m] (zeroed first).
 * Replaces fp8_swiglu.gemm_swiglu (h3_tp2/fp8_swiglu.py:230-241, kernel :107-157).
 */
int h3fp8_gemm_swiglu(const void* a, int64_t lda, const void* w_gate_up, int64_t ldw, const float* sa,
                      int64_t sa_stride, const float* sb, int64_t sb_stride, const void* bias, void* h, int64_t ldh,
                      float* row_amax, int64_t M, int64_t F, int64_t K, void* stream);

/*
 * Kernel 3 with the per-token requant: h3fp8_gemm_swiglu into h_ws (bf16 [M, F], row stride F) with the row maxima in
 * amax_ws ([M] fp32), then q [M, F] e4m3fn + scale [M] (h3fp8_quant_rows_amax on h_ws).
 * Replaces fp8_swiglu level 2: scale_swiglu_quant (h3_tp2/fp8_swiglu.py:191-200, kernel :72-103) after the fc1 GEMM.
 */
int h3fp8_gemm_swiglu_quant(const void* a, int64_t lda, const void* w_gate_up, int64_t ldw, const float* sa,
                            int64_t sa_stride, const float* sb, int64_t sb_stride, const void* bias, int64_t M,
                            int64_t F, int64_t K, void* h_ws, float* amax_ws, void* q, int64_t ldq, float* scale,
                            void* stream);

/*
 * Standalone SwiGLU passes (the stash forms of the reference, one wavefront per row):
 *   h3fp8_scale_swiglu        fp32 product x32 [M, 2F] -> bf16 h [M, F]      (h3_tp2/fp8_swiglu.py:180-188, :47-70)
 *   h3fp8_scale_swiglu_quant  fp32 product x32 [M, 2F] -> q [M, F] + scale   (h3_tp2/fp8_swiglu.py:191-200, :72-103)
 *   h3fp8_silu_mul_quant      bf16 [M, 2F] = [gate | up] -> q [M, F] + scale (h3_tp2/fp8_quant_fuse.py:392-402,
 *                                                                             :262-278)
 * x32 rows have stride ldx (elements); sa / sb / bias as in h3fp8_gemm (sb, bias [2F]).
 */
int h3fp8_scale_swiglu(const float* x32, int64_t ldx, const float* sa, int64_t sa_stride, const float* sb,
                       int64_t sb_stride, const void* bias, int64_t M, int64_t F, void* h, int64_t ldh, void* stream);
int h3fp8_scale_swiglu_quant(const float* x32, int64_t ldx, const float* sa, int64_t sa_stride, const float* sb,
                             int64_t sb_stride, const void* bias, int64_t M, int64_t F, void* q, int64_t ldq,
                             float* scale, void* stream);
int h3fp8_silu_mul_quant(const void* x, int64_t ldx, int64_t M, int64_t F, void* q, int64_t ldq, float* scale,
                         void* stream);

/*
 * The per-token quant fused into its producers (one wavefront per row, H % 8 == 0, H <= 8192):
 *   h3fp8_rms_quant       rms_norm_indexed_scale_shift + quant: the qkv site's producer.  Replaces the reference's
 *                         rms_quant / _rms_norm_indexed_scale_shift_quant_kernel (h3_tp2/fp8_quant_fuse.py:330-346,
 *                         :143-188).
 *   h3fp8_gate_rms_quant  indexed_gate_rms_norm_scale_shift + quant: the fc1 site's producer; also writes residual_out.
 *                         Replaces gate_rms_quant / _indexed_gate_rms_norm_scale_shift_quant_kernel
 *                         (h3_tp2/fp8_quant_fuse.py:349-369, :191-243).
 * Per row m, i = indices[m * idx_stride] (int32 if idx_bytes == 4, int64 if 8):
 *   [gate form] u = bf16(residual + gate[i] * branch) -> residual_out[m]; x = u
 *   var = fp32(sum_k x_k^2) / H; r = 1 / sqrt(var + eps)
 *   h = bf16(((x * r) * weight) * (1 + scale[i]) + shift[i]), every fp32 operation rounded on its own
 *   q [M, H] e4m3fn, qscale [M]: h3fp8_quant_rows of h; with h_out != NULL h is stored there too (bf16 [M, H]).
 *   q == NULL (h_out given): h only -- the stock producer itself, with the same arithmetic as the fused form.
 * gate / shift / scale are [n_index, H] bf16 tables with row strides ld_gate / ld_shift / ld_scale (the chunk views
 * of an AdaLN modulation tensor); every bf16 row is 16-byte aligned with a stride that is a multiple of 8 elements.
 * The sum of squares is taken in fp64 and rounded once (exact for rows whose squares span < ~40 binades).  An index
 * outside [0, n_index) is not read through: that row's residual_out, h and codes are NaN and its scale NaN.
 */
int h3fp8_rms_quant(const void* x, int64_t ldx, const void* weight, const void* shift, int64_t ld_shift,
                    const void* scale, int64_t ld_scale, int64_t n_index, const void* indices, int64_t idx_stride,
                    int idx_bytes, int64_t M, int64_t H, float eps, void* q, int64_t ldq, float* qscale, void* h_out,
                    int64_t ldh, void* stream);
int h3fp8_gate_rms_quant(const void* residual, int64_t ldr, const void* gate, int64_t ld_gate, const void* branch,
                         int64_t ld_branch, const void* weight, const void* shift, int64_t ld_shift, const void* scale,
                         int64_t ld_scale, int64_t n_index, const void* indices, int64_t idx_stride, int idx_bytes,
                         int64_t M, int64_t H, float eps, void* residual_out, int64_t ld_res, void* q, int64_t ldq,
                         float* qscale, void* h_out, int64_t ldh, void* stream);

/*
 * The consumers of a two-pass GEMM's fp32 product `acc` [M, N] (row stride ld_acc), with the scale pass fused in:
 * each reads branch[m, n] = bf16(sa[m] * (sb[n] * acc[m, n])) (bias: bf16(fma(sa[m], sb[n] * acc[m, n], bias[n])))
 * where the stock path would read the scale pass's bf16 output.  sa [M] and sb [N] fp32 contiguous, bias bf16 [N] or
 * NULL; product rows 16-byte aligned (8-byte for the qk form).
 *   h3fp8_scale_gate_rms_quant  the out projection's consumer: h3fp8_gate_rms_quant with that branch (q may be NULL:
 *                               residual_out + h only, the stock consumer's outputs; with q the fc1 input's quant as
 *                               well).  Replaces fp8_consumers.gate_rms_fused / _scale_indexed_gate_rms_norm_scale_
 *                               shift_kernel (h3_tp2/fp8_consumers.py:464-485, :242-293).
 *   h3fp8_scale_indexed_gate    the fc2 projection's consumer indexed_gate: out = bf16(x + gate[i] * branch), rows of
 *                               H (H % 8 == 0, H <= 8192).  Replaces gate_fused / _scale_indexed_gate_kernel
 *                               (h3_tp2/fp8_consumers.py:488-504, :204-240).
 *   h3fp8_scale_qk_norm_rope    the qkv projection's consumer for q and k: per token and head (128 dims, q heads
 *                               then k heads in the product's columns), n = bf16((x * r) * w) with
 *                               r = 1 / sqrt(fp32(sum x^2) / 128 + eps), then the half-split rotation of the first 96
 *                               dims by rope[t] (cos | sin, [T, 96] fp32 if rope_f32 else bf16):
 *                               out_d = bf16(n_d cos - n_(d+48) sin) (d < 48), bf16(n_d cos + n_(d-48) sin) (d < 96),
 *                               n_d (d >= 96).  out_q [T, Hq, 128] / out_k [T, Hk, 128] with token / head strides.
 *                               The v columns take h3fp8_scale_bias_cast.  Replaces qk_norm_rope_fused /
 *                               _scale_rms_norm_rope_kernel (h3_tp2/fp8_consumers.py:424-461, :131-193).
 *   h3fp8_scale_qkv_norm_rope   the same with the v columns in the same launch: the Hv heads after the k heads get
 *                               the scale pass alone, out_v [T, Hv, 128] = bf16(sa (sb acc)) (bias: one fma), the
 *                               bytes h3fp8_scale_bias_cast writes (Hv = 0: h3fp8_scale_qk_norm_rope).  Replaces
 *                               qk_norm_rope_fused with its v scale_pass_into (h3_tp2/fp8_consumers.py:424-461,
 *                               :373-380).
 * Sums of squares as in the producers (fp32 squares, fp64 sum, one rounding).
 */
int h3fp8_scale_gate_rms_quant(const float* acc, int64_t ld_acc, const float* sa, const float* sb, const void* bias,
                               const void* residual, int64_t ldr, const void* gate, int64_t ld_gate,
                               const void* weight, const void* shift, int64_t ld_shift, const void* scale,
                               int64_t ld_scale, int64_t n_index, const void* indices, int64_t idx_stride,
                               int idx_bytes, int64_t M, int64_t H, float eps, void* residual_out, int64_t ld_res,
                               void* q, int64_t ldq, float* qscale, void* h_out, int64_t ldh, void* stream);
int h3fp8_scale_indexed_gate(const float* acc, int64_t ld_acc, const float* sa, const float* sb, const void* bias,
                             const void* x, int64_t ldx, const void* gate, int64_t ld_gate, int64_t n_index,
                             const void* indices, int64_t idx_stride, int idx_bytes, int64_t M, int64_t H, void* out,
                             int64_t ldo, void* stream);
int h3fp8_scale_qk_norm_rope(const float* acc, int64_t ld_acc, const float* sa, const float* sb, const void* bias,
                             int64_t T, int Hq, int Hk, const void* q_weight, const void* k_weight, const void* rope,
                             int64_t ld_rope, int rope_f32, float eps, void* out_q, int64_t ldq_t, int64_t ldq_h,
                             void* out_k, int64_t ldk_t, int64_t ldk_h, void* stream);
int h3fp8_scale_qkv_norm_rope(const float* acc, int64_t ld_acc, const float* sa, const float* sb, const void* bias,
                              int64_t T, int Hq, int Hk, int Hv, const void* q_weight, const void* k_weight,
                              const void* rope, int64_t ld_rope, int rope_f32, float eps, void* out_q, int64_t ldq_t,
                              int64_t ldq_h, void* out_k, int64_t ldk_t, int64_t ldk_h, void* out_v, int64_t ldv_t,
                              int64_t ldv_h, void* stream);

/*
 * The two-pass scale pass: y = round(sa[m] * (sb[n] * x32[m, n])) (bias: one fma), bf16 or fp16.
 * Replaces fp8_gemm._scale_bias_cast / _launch (h3_tp2/fp8_gemm.py:37-54, :167-171) and the consumers' stash
 * materialisation (h3_tp2/fp8_consumers.py:373-380).
 */
int h3fp8_scale_bias_cast(const float* x32, int64_t ldx, const float* sa, int64_t sa_stride, const float* sb,
                          int64_t sb_stride, const void* bias, void* y, int64_t ldy, int out_dtype, int64_t M,
                          int64_t N, void* stream);

/*
 * Grouped FP8 GEMM: up to H3FP8_MAX_GROUPS independent h3fp8_gemm problems (bf16 out, no bias) in ONE launch whose
 * tile space is the concatenation of the groups' tile spaces.  No counterpart in the reference (it launches one GEMM
 * per linear, fp8_gemm.py:328-341); each group's result equals h3fp8_gemm's on the same operands.
 */
#define H3FP8_MAX_GROUPS 8
typedef struct h3fp8_group {
    const void* a;
    int64_t lda;
    const void* w;
    int64_t ldw;
    const float* sa;
    int64_t sa_stride;
    const float* sb;
    int64_t sb_stride;
    void* y;
    int64_t ldy;
    int64_t M, N, K;
} h3fp8_group;

int h3fp8_grouped_gemm(const h3fp8_group* groups, int n_groups, void* stream);

/*
 * Self-checks used by the install probe and the tests (no reference counterpart beyond its install probes,
 * h3_tp2/fp8_cutlass.py:196-249):
 *   h3fp8_selfcheck_e4m3   converts every fp32 bit pattern with |x| <= 448 (and the NaNs) with the hardware cvt used
 *                          by the kernels and with the software rule of torch's cast; *mismatches (host pointer)
 *                          receives the count of differing non-NaN results, *nan_bad the NaN inputs not mapped to a
 *                          NaN code.  Synchronous.
 *   h3fp8_copy_silu_table  copies the current device's SiLU table (65536 uint16) to `out` (device memory).
 */
int h3fp8_selfcheck_e4m3(uint64_t* mismatches, uint64_t* nan_bad);
/*   h3fp8_selfcheck_bf16   the same sweep for the hardware fp32 -> bf16 pair conversion used by the GEMM epilogues,
 *                          against the round-to-nearest-even rule of torch's cast (every fp32 pattern).  Synchronous. */
int h3fp8_selfcheck_bf16(uint64_t* mismatches, uint64_t* nan_bad);
int h3fp8_copy_silu_table(void* out, void* stream);

/*
 * Measurement (no counterpart in the reference): the sustained FP8 MFMA rate of the chip with no memory traffic.
 * `blocks` workgroups of 4 waves each run `iters` rounds of 16 independent v_mfma 32x32x64 e4m3 MFMAs on register
 * operands (the GEMM's per-wave accumulator block), 2 * 32 * 32 * 64 * 16 * 4 * iters * blocks FLOP per launch.
 * `out` (device, blocks * 256 floats) receives one sum per thread.  blocks in [1, 65535], iters in [1, 2^30].
 */
int h3fp8_mfma_loop(float* out, int64_t blocks, int64_t iters, uint32_t seed, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* H3FP8_H */
