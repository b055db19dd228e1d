/*
 * CPU oracle for the online-FP8 linear path: TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, in plain C with IEEE fp32 arithmetic, what the reference's eager CPU mirrors compute.  Only the
 * test suite, the smoke check and the CPU-baseline leg of the benchmark may load it, and only as the checker: the
 * product path (the HIP library) never calls into it.  Build: `make -C oracle` (gcc, -ffp-contract=off so that no
 * multiply-add is contracted behind the reference's back).
 *
 * Reference functions restated (paths relative to the reference checkout):
 *   quant_rows        h3_tp2/fp8_quant_fuse.py:302-307 (quant_torch), arithmetic spelled out at :11-13, :92-121;
 *                     h3_tp2/ulysses_outq.py:15-21, :126-135 (same formula)
 *   e4m3fn_from_f32   the `.to(torch.float8_e4m3fn)` of fp8_quant_fuse.py:306: round to nearest even, OCP e4m3fn
 *                     (bias 7, max 448, no infinities, NaN = S.1111.111), non-saturating (>= 480 -> NaN)
 *   bf16_rne          h3_tp2/fp8_swiglu.py:38-45 (_round_bf16) == torch's fp32 -> bf16 cast
 *   epilogue          h3_tp2/fp8_gemm.py:37-54 (_scale_bias_cast), :120-126, :174-185 (epilogue_torch):
 *                     t = sb[n] * acc, y = sa[m] * t, or fma(sa[m], t, bias[n]); one rounding to bf16/fp16
 *   silu_bf16         h3_tp2/fp8_swiglu.py:64-70, :203-212: s = bf16(g / (1 + exp(-g))) in fp32
 *   swiglu_row        h3_tp2/fp8_swiglu.py:64-70, :203-212: u = (u == 0) ? |u| : u; h = bf16(s * u)
 *   scale_swiglu      h3_tp2/fp8_swiglu.py:47-70 (epilogue to bf16, then SwiGLU) and :72-103 (+ quant_rows)
 *   dequant_matmul    h3_tp2/fp8_consumers.py:518-523 (a.float() @ w.float().t()), fp32 accumulation, K ascending
 *
 * exp: the reference's CPU mirror uses torch's exp and its GPU kernels libdevice's expf; neither is correctly rounded.
 * The oracle uses the correctly rounded fp32 exp (computed in long double and rounded once), which makes silu_bf16 a
 * well-defined function of the 65536 bf16 inputs.  The test suite compares that table with torch's CPU exp on every
 * bf16 input.
 *
 * NaN: rows containing NaN produce NaN scales and NaN codes; the sign of a NaN code is not specified by the reference
 * (torch's vectorised clamp may set it), so tests compare NaN positions, not NaN bits.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define FP8_MAX 448.0f

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* vLLM's _FP8_MIN_SCALING_FACTOR = 1/(448*512), rounded to fp32 (fp8_quant_fuse.py:78-79). */
float oracle_min_scale(void) { return (float)(1.0 / (448.0 * 512.0)); }

/* fp32 -> bf16, round to nearest even, NaN kept (quietened) -- torch's cast and _round_bf16 (fp8_swiglu.py:38-45). */
uint16_t oracle_bf16_rne(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float oracle_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* fp32 -> fp16, round to nearest even, overflow -> inf, NaN kept (torch's `.to(torch.float16)`). */
uint16_t oracle_fp16_rne(float f) {
    uint32_t u = f2u(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);          /* rounds to >= 65520: inf */
    if (a < 0x38800000u) {                                              /* below 2^-14: fp16 subnormal or zero */
        /* value * 2^24 rounded to an integer (RNE) is the subnormal code */
        float v = u2f(a) * 16777216.0f;                                 /* exact: power-of-two scaling */
        float r = nearbyintf(v);                                        /* default rounding mode: nearest even */
        return (uint16_t)(sign | (uint16_t)r);
    }
    uint32_t mant_odd = (a >> 13) & 1u;
    a += ((uint32_t)(15 - 127) << 23) + 0xfffu + mant_odd;
    return (uint16_t)(sign | (uint16_t)(a >> 13));
}

/* fp32 -> OCP e4m3fn, round to nearest even; |f| >= 480 (after rounding past 448) and NaN -> 0x7f | sign. */
uint8_t oracle_e4m3fn_from_f32(float f) {
    uint32_t u = f2u(f);
    uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
    uint32_t a = u & 0x7fffffffu;
    if (a >= 0x43f00000u) return (uint8_t)(sign | 0x7fu);               /* >= 480 or inf or NaN */
    if (a < 0x3c800000u) {                                              /* below 2^-6: subnormal grid of 2^-9 */
        float v = u2f(a) * 512.0f;                                      /* exact */
        float r = nearbyintf(v);                                        /* RNE to an integer 0..8 */
        return (uint8_t)(sign | (uint8_t)r);
    }
    uint32_t mant_odd = (a >> 20) & 1u;
    a += ((uint32_t)(7 - 127) << 23) + 0x7ffffu + mant_odd;
    return (uint8_t)(sign | (uint8_t)(a >> 20));
}

float oracle_e4m3fn_to_f32(uint8_t b) {
    uint32_t sign = (uint32_t)(b & 0x80u) << 24;
    uint32_t e = (b >> 3) & 0xfu, m = b & 7u;
    if (e == 0xfu && m == 7u) return u2f(sign | 0x7fc00000u);
    float v = (e == 0) ? ldexpf((float)m, -9) : ldexpf((float)(8u + m), (int)e - 10);
    return sign ? -v : v;
}

/* torch's NaN-propagating maximum/minimum (Inductor triton_helpers, fp8_quant_fuse.py:92-103). */
static inline float nan_max(float a, float b) { return (a > b || a != a) ? a : b; }
static inline float nan_min(float a, float b) { return (a < b || a != a) ? a : b; }

/* Per-token dynamic quant of one bf16 row (fp8_quant_fuse.py:302-307):
 *   amax = max_k |x_k| (NaN propagating); scale = max(amax / 448, MIN_SCALE) (IEEE division);
 *   q_k = e4m3fn_rne(clamp(x_k * (1 / scale), -448, 448)). */
float oracle_quant_row_f32(const float* x, int64_t K, uint8_t* q) {
    float amax = 0.0f;
    for (int64_t k = 0; k < K; ++k) amax = nan_max(amax, fabsf(x[k]));
    volatile float fp8max = FP8_MAX;                                    /* a runtime divisor, as in the reference */
    float scale = nan_max(amax / fp8max, oracle_min_scale());
    volatile float one = 1.0f;
    float inv = one / scale;
    for (int64_t k = 0; k < K; ++k) {
        float y = x[k] * inv;
        y = nan_max(y, -FP8_MAX);
        y = nan_min(y, FP8_MAX);
        q[k] = oracle_e4m3fn_from_f32(y);
    }
    return scale;
}

void oracle_quant_rows(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, uint8_t* q, int64_t ldq, float* scale) {
    float* row = (float*)__builtin_alloca((size_t)K * sizeof(float));
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t k = 0; k < K; ++k) row[k] = oracle_bf16_to_f32(x[m * ldx + k]);
        scale[m] = oracle_quant_row_f32(row, K, q + m * ldq);
    }
}

/* The scaled-mm epilogue on one element: t = sb * acc; y = sa * t, or one fma with the bias (fp8_gemm.py:44-50). */
static inline float epi_f32(float acc, float sa, float sb, const float* bias_n) {
    float t = sb * acc;
    return bias_n ? fmaf(sa, t, *bias_n) : sa * t;
}

/* acc [M,N] fp32 row-major -> y [M,N] (out_fp16 ? fp16 : bf16); bias_bf16 (or NULL) is [N] in the output dtype. */
void oracle_epilogue(const float* acc, int64_t M, int64_t N, const float* sa, const float* sb, const uint16_t* bias,
                     int out_fp16, uint16_t* y) {
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            float b, *bp = NULL;
            if (bias) {
                b = out_fp16 ? 0.0f : oracle_bf16_to_f32(bias[n]);
                if (out_fp16) {                                         /* fp16 -> fp32 (exact) */
                    uint16_t h = bias[n];
                    uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, mm = h & 0x3ffu;
                    if (e == 0x1f) b = u2f(s | 0x7f800000u | (mm << 13));
                    else if (e == 0) b = (s ? -1.0f : 1.0f) * ldexpf((float)mm, -24);
                    else b = u2f(s | ((e + 112u) << 23) | (mm << 13));
                }
                bp = &b;
            }
            float v = epi_f32(acc[m * N + n], sa[m], sb[n], bp);
            y[m * N + n] = out_fp16 ? oracle_fp16_rne(v) : oracle_bf16_rne(v);
        }
}

/* Correctly rounded fp32 exp: long double exp (64-bit significand) rounded once to fp32. */
static inline float exp_cr(float x) { return (float)expl((long double)x); }

/* silu of a bf16 gate value, rounded to bf16 (fp8_swiglu.py:69): s = bf16(g / (1 + exp(-g))), all in fp32. */
uint16_t oracle_silu_bf16(uint16_t g_bits) {
    float g = oracle_bf16_to_f32(g_bits);
    if (g != g) return oracle_bf16_rne(g);
    volatile float e = exp_cr(-g);
    volatile float d = 1.0f + e;
    volatile float s = g / d;
    return oracle_bf16_rne(s);
}

void oracle_silu_table(uint16_t* tab) {
    for (uint32_t i = 0; i < 65536u; ++i) tab[i] = oracle_silu_bf16((uint16_t)i);
}

/* silu_bf16 of every bf16 gate value, computed once (silu_bf16 is a function of the 16 input bits). */
static uint16_t g_silu[65536];
static int g_silu_ready = 0;

static inline uint16_t silu_lookup(uint16_t g) {
    if (!g_silu_ready) {
        oracle_silu_table(g_silu);
        g_silu_ready = 1;
    }
    return g_silu[g];
}

/* One SwiGLU element on bf16 gate/up values (fp8_swiglu.py:64-70): u == +-0 -> +0; h = bf16(silu_bf16(g) * u). */
static inline uint16_t swiglu_elem(uint16_t g, uint16_t u) {
    float uf = oracle_bf16_to_f32(u);
    if (uf == 0.0f) uf = 0.0f;
    float s = oracle_bf16_to_f32(silu_lookup(g));
    return oracle_bf16_rne(s * uf);
}

/* silu_and_mul on bf16 [M, 2F] = [gate | up] -> bf16 h [M, F] (fp8_quant_fuse.py:262-278 before its quant). */
void oracle_swiglu_bf16(const uint16_t* gu, int64_t M, int64_t F, int64_t ldgu, uint16_t* h) {
    for (int64_t m = 0; m < M; ++m)
        for (int64_t f = 0; f < F; ++f) h[m * F + f] = swiglu_elem(gu[m * ldgu + f], gu[m * ldgu + F + f]);
}

/* fp32 product [M, 2F] -> epilogue to bf16 -> SwiGLU -> bf16 h [M, F] (fp8_swiglu.py:47-70, :203-212). */
void oracle_scale_swiglu(const float* acc, int64_t M, int64_t F, const float* sa, const float* sb,
                         const uint16_t* bias, uint16_t* h) {
    for (int64_t m = 0; m < M; ++m)
        for (int64_t f = 0; f < F; ++f) {
            float bg, bu;
            const float *pg = NULL, *pu = NULL;
            if (bias) { bg = oracle_bf16_to_f32(bias[f]); bu = oracle_bf16_to_f32(bias[F + f]); pg = &bg; pu = &bu; }
            uint16_t g = oracle_bf16_rne(epi_f32(acc[m * 2 * F + f], sa[m], sb[f], pg));
            uint16_t u = oracle_bf16_rne(epi_f32(acc[m * 2 * F + F + f], sa[m], sb[F + f], pu));
            h[m * F + f] = swiglu_elem(g, u);
        }
}

/* fp32 product [M, 2F] -> SwiGLU -> per-token quant (fp8_swiglu.py:72-103): q [M, F], scale [M]. */
void oracle_scale_swiglu_quant(const float* acc, int64_t M, int64_t F, const float* sa, const float* sb,
                               const uint16_t* bias, uint8_t* q, float* scale) {
    uint16_t* h = (uint16_t*)__builtin_alloca((size_t)F * 2);
    float* hf = (float*)__builtin_alloca((size_t)F * 4);
    for (int64_t m = 0; m < M; ++m) {
        oracle_scale_swiglu(acc + m * 2 * F, 1, F, sa + m, sb, bias, h);
        for (int64_t f = 0; f < F; ++f) hf[f] = oracle_bf16_to_f32(h[f]);
        scale[m] = oracle_quant_row_f32(hf, F, q + m * F);
    }
}

/* acc[m][n] = sum_k a[m][k] * w[n][k], fp32, K ascending (fp8_consumers.py:518-523 on the CPU). */
void oracle_dequant_matmul(const uint8_t* a, int64_t lda, const uint8_t* w, int64_t ldw, int64_t M, int64_t N,
                           int64_t K, float* acc) {
    float lut[256];
    for (int i = 0; i < 256; ++i) lut[i] = oracle_e4m3fn_to_f32((uint8_t)i);
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            float s = 0.0f;
            for (int64_t k = 0; k < K; ++k) s += lut[a[m * lda + k]] * lut[w[n * ldw + k]];
            acc[m * N + n] = s;
        }
}

/* Array forms of the casts (used by the exhaustive sweeps of the tests). */
void oracle_e4m3fn_from_f32_array(const float* x, int64_t n, uint8_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_e4m3fn_from_f32(x[i]);
}

void oracle_bf16_rne_array(const float* x, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_bf16_rne(x[i]);
}

void oracle_fp16_rne_array(const float* x, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_fp16_rne(x[i]);
}

/* ---- producers with the quant fused in (h3_tp2/fp8_quant_fuse.py:143-243, :330-369) -------------------------------
 *
 * The stock producers, as the reference's CPU stand-ins state them (tests/fake_h3_consumers.py:66-84):
 *   gate form:  u = bf16(residual + gate[i] * branch)                      (fp32 multiply, fp32 add, one rounding)
 *   var = fp32(sum_k x_k * x_k) / H;  r = 1 / sqrt(var + eps)              (torch's CPU rsqrt is 1 / sqrt)
 *   h_k = bf16(((x_k * r) * weight_k) * (1 + scale[i]_k) + shift[i]_k)     (each operation rounded on its own)
 * followed by quant_rows of h.
 *
 * The sum of squares: each x_k * x_k is an fp32 product (exact unless it falls below the normal range), the products
 * are added in fp64 in a fixed order and the total is rounded once to fp32.  For rows whose squares span fewer than
 * about 40 binades the fp64 sum is exact, so the order does not matter and fp32(sum) is the correctly rounded sum the
 * stock kernel's fp32 reduction approximates.  The order fixed here is the HIP kernel's: 64 partial sums, partial l
 * over the 16-byte chunks c = l, l + 64, l + 128, ... of the row (8 elements each, ascending), then an xor butterfly
 * over the partials with distances 32, 16, ..., 1 (p_l <- p_l + p_(l xor d)). */
double oracle_row_sumsq(const float* x, int64_t H) {
    double p[64];
    const int64_t nchunk = H / 8;
    for (int l = 0; l < 64; ++l) {
        double s = 0.0;
        for (int64_t c = l; c < nchunk; c += 64)
            for (int e = 0; e < 8; ++e) {
                const float v = x[8 * c + e];
                s += (double)(v * v);
            }
        p[l] = s;
    }
    for (int d = 32; d >= 1; d >>= 1) {
        double t[64];
        for (int l = 0; l < 64; ++l) t[l] = p[l] + p[l ^ d];
        memcpy(p, t, sizeof(p));
    }
    return p[0];
}

/* One row: x (fp32 values of bf16), weight / shift / scale rows (bf16 bits) -> h (bf16 bits). */
static void rms_mod_row(const float* x, int64_t H, const uint16_t* weight, const uint16_t* shift,
                        const uint16_t* scale, float eps, uint16_t* h) {
    volatile float var = (float)oracle_row_sumsq(x, H);
    volatile float hf = (float)H;
    var = var / hf;
    volatile float t = var + eps;
    volatile float d = sqrtf(t);
    volatile float one = 1.0f;
    const float r = one / d;
    for (int64_t k = 0; k < H; ++k) {
        volatile float n = x[k] * r;
        n = n * oracle_bf16_to_f32(weight[k]);
        volatile float g = 1.0f + oracle_bf16_to_f32(scale[k]);
        volatile float o = n * g;
        o = o + oracle_bf16_to_f32(shift[k]);
        h[k] = oracle_bf16_rne(o);
    }
}

/* rms_norm_indexed_scale_shift + quant (fp8_quant_fuse.py:143-188, :330-346).  x [M, H] bf16 (row stride ldx);
 * weight [H]; shift / scale: row indices[m] of [B, H] tables (row strides ld_shift / ld_scale); indices int64 [M].
 * Outputs: h [M, H] bf16 (row stride H, may be NULL), q [M, H] (row stride H), qscale [M]. */
void oracle_rms_quant(const uint16_t* x, int64_t ldx, const uint16_t* weight, const uint16_t* shift, int64_t ld_shift,
                      const uint16_t* scale, int64_t ld_scale, const int64_t* indices, int64_t M, int64_t H,
                      float eps, uint16_t* h, uint8_t* q, float* qscale) {
    float* xf = (float*)__builtin_alloca((size_t)H * 4);
    uint16_t* hr = (uint16_t*)__builtin_alloca((size_t)H * 2);
    for (int64_t m = 0; m < M; ++m) {
        const int64_t i = indices[m];
        for (int64_t k = 0; k < H; ++k) xf[k] = oracle_bf16_to_f32(x[m * ldx + k]);
        rms_mod_row(xf, H, weight, shift + i * ld_shift, scale + i * ld_scale, eps, hr);
        if (h) memcpy(h + m * H, hr, (size_t)H * 2);
        for (int64_t k = 0; k < H; ++k) xf[k] = oracle_bf16_to_f32(hr[k]);
        qscale[m] = oracle_quant_row_f32(xf, H, q + m * H);
    }
}

/* indexed_gate_rms_norm_scale_shift + quant (fp8_quant_fuse.py:191-243, :349-369): residual_out [M, H] =
 * bf16(residual + gate[i] * branch), then rms_quant's row on residual_out.  gate is a [B, H] table (row stride
 * ld_gate) indexed like shift / scale; branch [M, H] (row stride ld_branch). */
void oracle_gate_rms_quant(const uint16_t* residual, int64_t ldr, const uint16_t* gate, int64_t ld_gate,
                           const uint16_t* branch, int64_t ld_branch, const uint16_t* weight, const uint16_t* shift,
                           int64_t ld_shift, const uint16_t* scale, int64_t ld_scale, const int64_t* indices,
                           int64_t M, int64_t H, float eps, uint16_t* residual_out, uint16_t* h, uint8_t* q,
                           float* qscale) {
    float* xf = (float*)__builtin_alloca((size_t)H * 4);
    uint16_t* hr = (uint16_t*)__builtin_alloca((size_t)H * 2);
    for (int64_t m = 0; m < M; ++m) {
        const int64_t i = indices[m];
        for (int64_t k = 0; k < H; ++k) {
            volatile float p = oracle_bf16_to_f32(gate[i * ld_gate + k]) * oracle_bf16_to_f32(branch[m * ld_branch + k]);
            volatile float u = oracle_bf16_to_f32(residual[m * ldr + k]) + p;
            const uint16_t ub = oracle_bf16_rne(u);
            residual_out[m * H + k] = ub;
            xf[k] = oracle_bf16_to_f32(ub);
        }
        rms_mod_row(xf, H, weight, shift + i * ld_shift, scale + i * ld_scale, eps, hr);
        if (h) memcpy(h + m * H, hr, (size_t)H * 2);
        for (int64_t k = 0; k < H; ++k) xf[k] = oracle_bf16_to_f32(hr[k]);
        qscale[m] = oracle_quant_row_f32(xf, H, q + m * H);
    }
}

/* ---- consumers of the GEMM output (h3_tp2/fp8_consumers.py:131-293) ------------------------------------------------
 *
 * fused_qk_norm_rope's half-split path on one bf16 head of 128 dims (the stock `_rms_norm_rope_kernel` as the
 * reference's CPU stand-in states it, tests/fake_h3_consumers.py:29-48), rotary_half = 48:
 *   var = fp32(sum_d x_d * x_d) / 128;  r = 1 / sqrt(var + eps)
 *   n_d = bf16((x_d * r) * w_d)
 *   pair(d) = d + 48 (d < 48), d - 48 (48 <= d < 96), d;  freq(d) = d (d < 48), d - 48 (48 <= d < 96), 0
 *   c = table[freq(d)], s = table[freq(d) + 48]
 *   out_d = bf16(n_d * c - n_pair * s) (d < 48), bf16(n_d * c + n_pair * s) (48 <= d < 96), n_d (d >= 96)
 * The sum of squares is rounded once to fp32 from an fp64 sum in the HIP kernel's order: lane l of 8 adds the squares
 * of dims 32i + 4l + e in the order i = 0 .. 3, e = 0 .. 3, then an xor butterfly over the 8 lane sums (distances 4,
 * 2, 1). */
static double head_sumsq(const float* x) {
    double p[8];
    for (int l = 0; l < 8; ++l) {
        double s = 0.0;
        for (int i = 0; i < 4; ++i)
            for (int e = 0; e < 4; ++e) s += (double)(x[32 * i + 4 * l + e] * x[32 * i + 4 * l + e]);
        p[l] = s;
    }
    for (int d = 4; d >= 1; d >>= 1) {
        double t[8];
        for (int l = 0; l < 8; ++l) t[l] = p[l] + p[l ^ d];
        memcpy(p, t, sizeof(p));
    }
    return p[0];
}

/* x: bf16 bits [T, heads, 128] (contiguous), weight [128] bf16 bits, table: fp32 [T, 96] (the rope table's values),
 * out: bf16 bits [T, heads, 128]. */
void oracle_qk_norm_rope(const uint16_t* x, int64_t T, int64_t heads, const uint16_t* weight, const float* table,
                         float eps, uint16_t* out) {
    float xf[128];
    uint16_t n[128];
    for (int64_t t = 0; t < T; ++t)
        for (int64_t h = 0; h < heads; ++h) {
            const uint16_t* xr = x + (t * heads + h) * 128;
            for (int d = 0; d < 128; ++d) xf[d] = oracle_bf16_to_f32(xr[d]);
            volatile float var = (float)head_sumsq(xf);
            volatile float hd = 128.0f;
            var = var / hd;
            volatile float dd = sqrtf(var + eps);
            volatile float one = 1.0f;
            const float r = one / dd;
            for (int d = 0; d < 128; ++d) {
                volatile float v = xf[d] * r;
                v = v * oracle_bf16_to_f32(weight[d]);
                n[d] = oracle_bf16_rne(v);
            }
            const float* tb = table + t * 96;
            uint16_t* o = out + (t * heads + h) * 128;
            for (int d = 0; d < 128; ++d) {
                if (d >= 96) { o[d] = n[d]; continue; }
                const int pd = d < 48 ? d + 48 : d - 48, fd = d < 48 ? d : d - 48;
                const float c = tb[fd], s = tb[fd + 48];
                volatile float a = oracle_bf16_to_f32(n[d]) * c;
                volatile float b = oracle_bf16_to_f32(n[pd]) * s;
                volatile float y = d < 48 ? a - b : a + b;
                o[d] = oracle_bf16_rne(y);
            }
        }
}
