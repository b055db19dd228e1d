// Standalone SwiGLU / epilogue passes (kernel 3's stash forms) and the two-pass scale pass.
//
//   h3fp8_scale_bias_cast     fp32 [M, N] -> bf16/fp16: round(sa * (sb * x)), bias by one fma   (fp8_gemm.py:37-54)
//   h3fp8_scale_swiglu        fp32 [M, 2F] -> bf16 h [M, F]                                  (fp8_swiglu.py:47-70)
//   h3fp8_scale_swiglu_quant  fp32 [M, 2F] -> e4m3 q [M, F] + scale [M]                      (fp8_swiglu.py:72-103)
//   h3fp8_silu_mul_quant      bf16 [M, 2F] -> e4m3 q [M, F] + scale [M]              (fp8_quant_fuse.py:262-278)
//
// SwiGLU element (fp8_swiglu.py:64-70): g, u = bf16(epilogue(acc)); u = (u == 0 ? +0 : u);
// h = bf16(silu_bf16(g) * u), silu_bf16 from the device table of all 65536 bf16 gate values.
// The row-quant forms keep a row's bf16 h values in registers: the row maximum is a wave xor-shuffle max plus an LDS
// exchange between the row's waves, and the quant then reuses the registers (the row is read from HBM once).  With
// contiguous sb the fp32 forms take persistent kernels with the compact SiLU table in LDS and the column scales in
// registers (scale_swiglu_seg_kernel, scale_swiglu_quant_lds_kernel); otherwise one thread per 4 columns
// (scale_swiglu_kernel) or one 256-thread workgroup per row (swiglu_quant_rows_kernel).
#include <algorithm>

#include "h3fp8_common.h"

namespace {

using namespace h3;

struct EpiArgs {
    const float* sa;
    int64_t sa_stride;
    const float* sb;
    int64_t sb_stride;
    const uint16_t* bias;      // bf16 (or fp16 for scale_bias_cast with fp16 out), may be null
};

__device__ __forceinline__ float epi(float acc, float sam, float sbn, bool has_bias, float b) {
    const float t = sbn * acc;
    return has_bias ? __builtin_fmaf(sam, t, b) : sam * t;
}

// One SwiGLU element from bf16 gate / up bit patterns.
__device__ __forceinline__ uint32_t swiglu_bits(uint32_t gb, uint32_t ub, const uint16_t* __restrict__ silu) {
    float u = bf16_to_f32(ub);
    u = (u == 0.0f) ? 0.0f : u;
    return bf16_rne(bf16_to_f32(silu[gb]) * u);
}

// The 4 h values of column group c (columns 4c .. 4c+3) of row m.
template <bool SRC_FP32>
__device__ __forceinline__ void swiglu_group(const void* __restrict__ x, int64_t ldx, int64_t m, int64_t c, int64_t F,
                                             const EpiArgs& e, float sam, const uint16_t* __restrict__ silu,
                                             uint32_t h[4]) {
    const int64_t f = 4 * c;
    if (SRC_FP32) {
        const float* xr = reinterpret_cast<const float*>(x) + m * ldx;
        const v4f ga = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(xr + f));
        const v4f ua = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(xr + F + f));
        const float gv[4] = {ga[0], ga[1], ga[2], ga[3]}, uv[4] = {ua[0], ua[1], ua[2], ua[3]};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const bool hb = e.bias != nullptr;
            const float bg = hb ? bf16_to_f32(e.bias[f + r]) : 0.f, bu = hb ? bf16_to_f32(e.bias[F + f + r]) : 0.f;
            const uint32_t gb = bf16_rne(epi(gv[r], sam, e.sb[(f + r) * e.sb_stride], hb, bg));
            const uint32_t ub = bf16_rne(epi(uv[r], sam, e.sb[(F + f + r) * e.sb_stride], hb, bu));
            h[r] = swiglu_bits(gb, ub, silu);
        }
    } else {
        const uint16_t* xr = reinterpret_cast<const uint16_t*>(x) + m * ldx;
        const uint2 gw = *reinterpret_cast<const uint2*>(xr + f), uw = *reinterpret_cast<const uint2*>(xr + F + f);
        h[0] = swiglu_bits(gw.x & 0xffffu, uw.x & 0xffffu, silu);
        h[1] = swiglu_bits(gw.x >> 16, uw.x >> 16, silu);
        h[2] = swiglu_bits(gw.y & 0xffffu, uw.y & 0xffffu, silu);
        h[3] = swiglu_bits(gw.y >> 16, uw.y >> 16, silu);
    }
}

typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
typedef unsigned int v2u __attribute__((ext_vector_type(2)));

// max(m, |lo half|, |hi half|) of a packed bf16 pair, as fp32 bit patterns (NaN patterns order above +inf).
__device__ __forceinline__ uint32_t max_abs_bf16x2_bits(uint32_t m, uint32_t p) {
    const uint32_t lo = (p << 16) & 0x7fff0000u, hi = p & 0x7fff0000u;
    m = m > lo ? m : lo;
    return m > hi ? m : hi;
}

__device__ __forceinline__ uint32_t quant4(const uint32_t h[4], float inv) {
    return e4m3x4(quant_clamp(bf16_to_f32(h[0]), inv), quant_clamp(bf16_to_f32(h[1]), inv),
                  quant_clamp(bf16_to_f32(h[2]), inv), quant_clamp(bf16_to_f32(h[3]), inv));
}

__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, uint32_t* red) {
    v = wave_max_u32(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    uint32_t r = red[0];
#pragma unroll
    for (int i = 1; i < 4; ++i) r = r > red[i] ? r : red[i];
    return r;
}

// One row per workgroup; CPT register-resident column groups per thread (CPT == 0: the row is computed twice).
template <bool SRC_FP32, int CPT>
__global__ void __launch_bounds__(256) swiglu_quant_rows_kernel(const void* __restrict__ x, int64_t ldx, int64_t F,
                                                                EpiArgs e, const uint16_t* __restrict__ silu,
                                                                uint8_t* __restrict__ q, int64_t ldq,
                                                                float* __restrict__ scale) {
    __shared__ uint32_t red[4];
    const int64_t m = blockIdx.x;
    const int64_t ngroups = F >> 2;
    const float sam = SRC_FP32 ? e.sa[m * e.sa_stride] : 1.0f;
    uint32_t* qr = reinterpret_cast<uint32_t*>(q + m * ldq);
    uint32_t mx = 0;
    if (CPT > 0) {
        uint32_t hv[CPT > 0 ? CPT : 1][4];
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int64_t c = threadIdx.x + 256 * j;
            if (c < ngroups) {
                swiglu_group<SRC_FP32>(x, ldx, m, c, F, e, sam, silu, hv[j]);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t a = (hv[j][r] & 0x7fffu) << 16;
                    mx = mx > a ? mx : a;
                }
            }
        }
        const float s = row_scale(u2f(block_max_u32(mx, red)));
        const float inv = inv_scale(s);
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int64_t c = threadIdx.x + 256 * j;
            if (c < ngroups) qr[c] = quant4(hv[j], inv);
        }
        if (threadIdx.x == 0) scale[m] = s;
    } else {
        uint32_t hv[4];
        for (int64_t c = threadIdx.x; c < ngroups; c += 256) {
            swiglu_group<SRC_FP32>(x, ldx, m, c, F, e, sam, silu, hv);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t a = (hv[r] & 0x7fffu) << 16;
                mx = mx > a ? mx : a;
            }
        }
        const float s = row_scale(u2f(block_max_u32(mx, red)));
        const float inv = inv_scale(s);
        for (int64_t c = threadIdx.x; c < ngroups; c += 256) {
            swiglu_group<SRC_FP32>(x, ldx, m, c, F, e, sam, silu, hv);
            qr[c] = quant4(hv, inv);
        }
        if (threadIdx.x == 0) scale[m] = s;
    }
}

// bf16 [gate | up] -> e4m3 q + per-row scale, the HBM-bound form (fp8_quant_fuse.py:262-278): a persistent kernel with
// the SiLU table in LDS (one 128 KiB copy per CU, loaded once), so the 65536-entry lookups are LDS gathers instead of
// scattered global loads.  One 64-lane wave per row, rows wave_id, wave_id + waves, ...: lane l owns the 16-byte column
// chunks l + 64 j of the gate and of the up half (coalesced 1 KiB per load instruction), the row's h values stay in
// VGPRs as packed bf16 pairs, the row maximum is a wave xor-shuffle max (no LDS exchange, no barrier), and every q
// store writes 8 bytes per lane, 512 contiguous bytes per instruction.
constexpr int SMQ_WAVES = 8;                   // waves per workgroup (2 per SIMD; 3 measured slower)
// Quant of one packed bf16 pair: e4m3 bytes of clamp(h * inv, -448, 448).  FINITE: the row maximum is finite, so every
// h * inv is finite and a median-of-three is the clamp exactly; otherwise compare/select, which keeps NaN (the
// reference's clamp, fp8_quant_fuse.py:105-111).
template <bool FINITE>
__device__ __forceinline__ float clamp448(float y) {
    if (FINITE) return __builtin_amdgcn_fmed3f(y, -H3_FP8_MAX, H3_FP8_MAX);
    y = (y < -H3_FP8_MAX) ? -H3_FP8_MAX : y;
    return (y > H3_FP8_MAX) ? H3_FP8_MAX : y;
}

template <bool FINITE>
__device__ __forceinline__ uint32_t quant_pairs(uint32_t p0, uint32_t p1, float inv) {
    return e4m3x4(clamp448<FINITE>(u2f(p0 << 16) * inv), clamp448<FINITE>(u2f(p0 & 0xffff0000u) * inv),
                  clamp448<FINITE>(u2f(p1 << 16) * inv), clamp448<FINITE>(u2f(p1 & 0xffff0000u) * inv));
}

template <int CPL, bool FINITE>
__device__ __forceinline__ void store_q_row(const uint32_t (*h)[4], float inv, __amdgpu_buffer_rsrc_t qr, int lane) {
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const uint32_t lo = quant_pairs<FINITE>(h[j][0], h[j][1], inv);
        const uint32_t hi = quant_pairs<FINITE>(h[j][2], h[j][3], inv);
        const v2u v = {lo, hi};
        // chunks past F fall outside the row's range and are dropped; device-scope (sc1) stores, written through the
        // L2 (measured at 31 248 x 2 x 8192: 222.2 -> 216.6 us against plain stores)
        __builtin_amdgcn_raw_buffer_store_b64(v, qr, (uint32_t)(lane + 64 * j) * 8u, 0, 16);
    }
}

template <int CPL>
__global__ void __launch_bounds__(64 * SMQ_WAVES) silu_mul_quant_lds_kernel(const uint16_t* __restrict__ x,
                                                                          int64_t ldx, int64_t M, int64_t F,
                                                                          const uint16_t* __restrict__ silu,
                                                                          uint8_t* __restrict__ q, int64_t ldq,
                                                                          float* __restrict__ scale) {
    __shared__ __attribute__((aligned(16))) uint16_t tab[65536];
    for (int i = threadIdx.x; i < 65536 / 8; i += 64 * SMQ_WAVES)
        reinterpret_cast<v4u*>(tab)[i] = reinterpret_cast<const v4u*>(silu)[i];
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int64_t waves = (int64_t)gridDim.x * SMQ_WAVES;
    float pz = 0.0f;
    asm volatile("" : "+v"(pz));                        // an opaque +0 (the add below must not be folded away)
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform: row addresses in SGPRs
    for (int64_t m = (int64_t)blockIdx.x * SMQ_WAVES + wv; m < M; m += waves) {
        // per-row buffer ranges: loads past F read zeros, stores past F are dropped (no per-chunk branch)
        const __amdgpu_buffer_rsrc_t gr = make_rsrc(x + m * ldx, (uint32_t)(2 * F));
        const __amdgpu_buffer_rsrc_t ur = make_rsrc(x + m * ldx + F, (uint32_t)(2 * F));
        const __amdgpu_buffer_rsrc_t qr = make_rsrc(q + m * ldq, (uint32_t)F);
        v4u gv[CPL], uv[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const uint32_t off = (uint32_t)(lane + 64 * j) * 16u;
            gv[j] = __builtin_amdgcn_raw_buffer_load_b128(gr, off, 0, 2);   // aux 2: streaming (nt)
            uv[j] = __builtin_amdgcn_raw_buffer_load_b128(ur, off, 0, 2);
        }
        uint32_t h[CPL][4];                             // packed bf16 h pairs
        u16x2_t mx2 = {0, 0};                           // two running maxima of |h| bit patterns
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t g2 = gv[j][k], u2 = uv[j][k];
                // u + (+0): -0 up becomes +0 under round-to-nearest, every other value (NaN included) is unchanged
                // (fp8_swiglu.py:66)
                const float u0 = bf16_to_f32(u2 & 0xffffu) + pz, u1 = u2f(u2 & 0xffff0000u) + pz;
                const float s0 = bf16_to_f32(tab[g2 & 0xffffu]), s1 = bf16_to_f32(tab[g2 >> 16]);
                const uint32_t hp = cvt_bf16x2(s0 * u0, s1 * u1);   // s * u exact in fp32, one RNE to bf16
                h[j][k] = hp;
                // columns past F read zeros (h = +0) and leave the maximum unchanged; |h| bit patterns order like
                // |h| with NaN above +inf, so an unsigned 16-bit max per half is the NaN-propagating row maximum
                mx2 = __builtin_elementwise_max(mx2, __builtin_bit_cast(u16x2_t, hp & 0x7fff7fffu));
            }
        }
        uint32_t mx = mx2[0] > mx2[1] ? (uint32_t)mx2[0] : (uint32_t)mx2[1];
        mx = wave_max_u32(mx << 16);
        const float s = row_scale(u2f(mx));
        const float inv = inv_scale(s);
        if (mx < 0x7f800000u) store_q_row<CPL, true>(h, inv, qr, lane);    // wave-uniform: finite row maximum
        else store_q_row<CPL, false>(h, inv, qr, lane);
        if (lane == 0) scale[m] = s;
    }
}

// The same pass for rows too wide for one wave (8192 < F <= 16 384): 16 waves per row, thread t owns the 16-byte
// chunks t + 1024 j (j < CPL) of the gate and of the up half; the row maximum is a wave shuffle plus an LDS exchange
// behind a bare s_barrier, and the next row's loads are issued before it, so they stay in flight across it and the
// stores.  One workgroup per CU (the 128 KiB table).
constexpr int SMQW_WAVES = 16;
template <int CPL>
__global__ void __launch_bounds__(64 * SMQW_WAVES) silu_mul_quant_wide_kernel(const uint16_t* __restrict__ x,
                                                                             int64_t ldx, int64_t M, int64_t F,
                                                                             const uint16_t* __restrict__ silu,
                                                                             uint8_t* __restrict__ q, int64_t ldq,
                                                                             float* __restrict__ scale) {
    constexpr int THREADS = 64 * SMQW_WAVES;
    __shared__ __attribute__((aligned(16))) uint16_t tab[65536];
    __shared__ uint32_t red[2][SMQW_WAVES];
    for (int i = threadIdx.x; i < 65536 / 8; i += THREADS)
        reinterpret_cast<v4u*>(tab)[i] = reinterpret_cast<const v4u*>(silu)[i];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float pz = 0.0f;
    asm volatile("" : "+v"(pz));                        // an opaque +0 (the add below must not be folded away)
    v4u gv[CPL], uv[CPL];
    auto load_row = [&](int64_t m) {
        // loads past F read zeros: gate 0 looks up silu(0) = 0, so those columns give h = +0
        const __amdgpu_buffer_rsrc_t gr = make_rsrc(x + m * ldx, (uint32_t)(2 * F));
        const __amdgpu_buffer_rsrc_t ur = make_rsrc(x + m * ldx + F, (uint32_t)(2 * F));
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const uint32_t off = (threadIdx.x + THREADS * (uint32_t)j) * 16u;
            gv[j] = __builtin_amdgcn_raw_buffer_load_b128(gr, off, 0, 2);
            uv[j] = __builtin_amdgcn_raw_buffer_load_b128(ur, off, 0, 2);
        }
    };
    int64_t m = blockIdx.x;
    if (m < M) load_row(m);
    __syncthreads();
    for (int par = 0; m < M; m += gridDim.x, par ^= 1) {
        uint32_t h[CPL][4];
        u16x2_t mx2 = {0, 0};
#pragma unroll
        for (int j = 0; j < CPL; ++j)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t g2 = gv[j][k], u2 = uv[j][k];
                const float u0 = bf16_to_f32(u2 & 0xffffu) + pz, u1 = u2f(u2 & 0xffff0000u) + pz;   // -0 up -> +0
                const float s0 = bf16_to_f32(tab[g2 & 0xffffu]), s1 = bf16_to_f32(tab[g2 >> 16]);
                h[j][k] = cvt_bf16x2(s0 * u0, s1 * u1);
                mx2 = __builtin_elementwise_max(mx2, __builtin_bit_cast(u16x2_t, h[j][k] & 0x7fff7fffu));
            }
        if (m + gridDim.x < M) load_row(m + gridDim.x);
        uint32_t mx = mx2[0] > mx2[1] ? (uint32_t)mx2[0] : (uint32_t)mx2[1];
        mx = wave_max_u32(mx << 16);
        if (lane == 0) red[par][wave] = mx;
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");   // no fence: the row loads stay in flight
#pragma unroll
        for (int w = 0; w < SMQW_WAVES; ++w) mx = mx > red[par][w] ? mx : red[par][w];
        const float s = row_scale(u2f(mx));
        const float inv = inv_scale(s);
        const __amdgpu_buffer_rsrc_t qr = make_rsrc(q + m * ldq, (uint32_t)F);
        if (mx < 0x7f800000u) {                          // workgroup-uniform: finite row maximum
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const v2u v = {quant_pairs<true>(h[j][0], h[j][1], inv), quant_pairs<true>(h[j][2], h[j][3], inv)};
                __builtin_amdgcn_raw_buffer_store_b64(v, qr, (threadIdx.x + THREADS * (uint32_t)j) * 8u, 0, 2);
            }
        } else {
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const v2u v = {quant_pairs<false>(h[j][0], h[j][1], inv), quant_pairs<false>(h[j][2], h[j][3], inv)};
                __builtin_amdgcn_raw_buffer_store_b64(v, qr, (threadIdx.x + THREADS * (uint32_t)j) * 8u, 0, 2);
            }
        }
        if (threadIdx.x == 0) scale[m] = s;
    }
}

// fp32 product -> bf16 h, elementwise: one thread per group of 4 columns.
__global__ void __launch_bounds__(256) scale_swiglu_kernel(const float* __restrict__ x, int64_t ldx, int64_t M,
                                                           int64_t F, EpiArgs e, const uint16_t* __restrict__ silu,
                                                           uint16_t* __restrict__ h, int64_t ldh) {
    const int64_t ngroups = F >> 2;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= M * ngroups) return;
    const int64_t m = idx / ngroups, c = idx - m * ngroups;
    uint32_t hv[4];
    swiglu_group<true>(x, ldx, m, c, F, e, e.sa[m * e.sa_stride], silu, hv);
    *reinterpret_cast<uint2*>(h + m * ldh + 4 * c) = make_uint2(hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16));
}

// ---- fp32 forms with the compact SiLU table in LDS (contiguous sb, F < 2^28) -------------------------------------
// A workgroup copies the compact table (17 920 bytes) into LDS once and keeps the sb / bias values of its columns in
// registers (16- and 8-byte loads) across all the rows it covers.  The gate's table key is the bf16 pattern rotated
// left by one (the sign in bit 0), read from a word holding the gate in both halves; a column group whose wave holds
// a key outside the compact range (zeros, |g| < 2.6e-9 or > 88.5, inf, NaN) reads the full table in global memory.

// The compact table into LDS, 16 bytes per load.
__device__ __forceinline__ void load_silu_rot(uint16_t* tab, const uint16_t* __restrict__ rot, int threads) {
    for (int i = threadIdx.x; i < H3_SILU_ROT_LEN / 8; i += threads)
        reinterpret_cast<v4u*>(tab)[i] = reinterpret_cast<const v4u*>(rot)[i];
}

// The sb and bias values of column group g (columns 4g .. 4g+3 of the gate half and of the up half).  Groups past F
// read zeros.
struct ColOps {
    v4u sg, su;
    v2u bg, bu;    // bf16 pairs
};

template <bool HB>
__device__ __forceinline__ ColOps load_cols(const EpiArgs& e, int64_t F, uint32_t g) {
    const uint32_t fb = (uint32_t)F * 4u;
    ColOps c;
    c.sg = __builtin_amdgcn_raw_buffer_load_b128(make_rsrc(e.sb, fb), g * 16u, 0, 0);
    c.su = __builtin_amdgcn_raw_buffer_load_b128(make_rsrc(e.sb + F, fb), g * 16u, 0, 0);
    if (HB) {
        c.bg = __builtin_amdgcn_raw_buffer_load_b64(make_rsrc(e.bias, fb / 2u), g * 8u, 0, 0);
        c.bu = __builtin_amdgcn_raw_buffer_load_b64(make_rsrc(e.bias + F, fb / 2u), g * 8u, 0, 0);
    } else {
        c.bg = v2u{0u, 0u};
        c.bu = v2u{0u, 0u};
    }
    return c;
}

// Keeps the compiler from hoisting the bias conversions out of a row loop, which doubles the registers they take.
template <bool HB, int N>
__device__ __forceinline__ void pin_bias(ColOps (&c)[N]) {
#pragma unroll
    for (int j = 0; j < N; ++j)
        if (HB) asm volatile("" : "+v"(c[j].bg), "+v"(c[j].bu));
}

// Table keys (offsets into the compact table) and bf16-rounded up values (as fp32 bit patterns) of one column group.
// Groups past F (valid false) get key 0, so they never force the full-table path.
template <bool HB>
__device__ __forceinline__ void group_keys(v4u xg, v4u xu, float sam, const ColOps& c, bool valid, uint32_t key[4],
                                           uint32_t uu[4]) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t bgw = c.bg[q >> 1], buw = c.bu[q >> 1];
        const float bgf = (q & 1) ? u2f(bgw & 0xffff0000u) : bf16_to_f32(bgw & 0xffffu);
        const float buf = (q & 1) ? u2f(buw & 0xffff0000u) : bf16_to_f32(buw & 0xffffu);
        const float gy = epi(u2f(xg[q]), sam, u2f(c.sg[q]), HB, bgf);
        const float uy = epi(u2f(xu[q]), sam, u2f(c.su[q]), HB, buf);
        const uint32_t k = ((cvt_bf16x2(gy, gy) >> 15) & 0xffffu) - H3_SILU_ROT_R0;
        key[q] = valid ? k : 0u;
        uu[q] = cvt_bf16x2(0.0f, uy);
    }
}

// bf16(silu(g)) of NG column groups' gates: from LDS when every key of the wave is in the compact range, else from the
// full table (indexed by the gate's bf16 bits, the key rotated back).
template <int NG>
__device__ __forceinline__ void lookup_silu(const uint16_t* tab, const uint16_t* __restrict__ silu,
                                            const uint32_t (*key)[4], uint32_t (*s)[4]) {
    bool out = false;
#pragma unroll
    for (int j = 0; j < NG; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) out |= key[j][q] >= (uint32_t)H3_SILU_ROT_LEN;
    if (__ballot(out) == 0) {
#pragma unroll
        for (int j = 0; j < NG; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) s[j][q] = tab[key[j][q]];
    } else {
#pragma unroll
        for (int j = 0; j < NG; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t rk = (key[j][q] + H3_SILU_ROT_R0) & 0xffffu;
                s[j][q] = silu[(rk >> 1) | ((rk & 1u) << 15)];
            }
    }
}

// The packed bf16 h pairs of one group: h = bf16(silu(g) * u), u + (+0) turning a -0 up into +0 (fp8_swiglu.py:66).
__device__ __forceinline__ v2u group_h(const uint32_t s[4], const uint32_t uu[4], float pz) {
    return v2u{cvt_bf16x2(bf16_to_f32(s[0]) * (u2f(uu[0]) + pz), bf16_to_f32(s[1]) * (u2f(uu[1]) + pz)),
               cvt_bf16x2(bf16_to_f32(s[2]) * (u2f(uu[2]) + pz), bf16_to_f32(s[3]) * (u2f(uu[3]) + pz))};
}

// fp32 product -> bf16 h over row segments: block (s, b) covers the U * 256 column groups of segment s (thread i the
// groups i + 256 u) and the row pairs 2b, 2b + 2 gridDim.y, ...; the two rows of a pair have all their loads in flight
// together.
template <int U, bool HB>
__global__ void __launch_bounds__(256) scale_swiglu_seg_kernel(const float* __restrict__ x, int64_t ldx, int64_t M,
                                                               int64_t F, EpiArgs e, const uint16_t* __restrict__ silu,
                                                               const uint16_t* __restrict__ rot,
                                                               uint16_t* __restrict__ h, int64_t ldh) {
    __shared__ __attribute__((aligned(16))) uint16_t tab[H3_SILU_ROT_LEN];
    load_silu_rot(tab, rot, 256);
    const uint32_t ngroups = (uint32_t)(F >> 2);
    const uint32_t g0 = blockIdx.x * (256u * U) + threadIdx.x;
    const uint32_t fb = (uint32_t)F * 4u;
    ColOps c[U];
#pragma unroll
    for (int u = 0; u < U; ++u) c[u] = load_cols<HB>(e, F, g0 + 256u * u);
    float pz = 0.0f;
    asm volatile("" : "+v"(pz));                        // an opaque +0 (the add in group_h must not be folded away)
    __syncthreads();
    for (int64_t m0 = (int64_t)blockIdx.y * 2; m0 < M; m0 += (int64_t)gridDim.y * 2) {
        v4u xg[2][U], xu[2][U];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const bool in = m0 + r < M;
            const float* xr = x + (in ? m0 + r : m0) * ldx;
            const __amdgpu_buffer_rsrc_t gr = make_rsrc(xr, in ? fb : 0u), ur = make_rsrc(xr + F, in ? fb : 0u);
#pragma unroll
            for (int u = 0; u < U; ++u) {
                xg[r][u] = __builtin_amdgcn_raw_buffer_load_b128(gr, (g0 + 256u * u) * 16u, 0, 2);
                xu[r][u] = __builtin_amdgcn_raw_buffer_load_b128(ur, (g0 + 256u * u) * 16u, 0, 2);
            }
        }
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int64_t m = m0 + r;
            if (m >= M) break;
            const float sam = e.sa[m * e.sa_stride];
            pin_bias<HB>(c);
            uint32_t key[U][4], uu[U][4], s[U][4];
#pragma unroll
            for (int u = 0; u < U; ++u)
                group_keys<HB>(xg[r][u], xu[r][u], sam, c[u], g0 + 256u * u < ngroups, key[u], uu[u]);
            lookup_silu<U>(tab, silu, key, s);
            const __amdgpu_buffer_rsrc_t yr = make_rsrc(h + m * ldh, (uint32_t)F * 2u);
#pragma unroll
            for (int u = 0; u < U; ++u)    // groups past F are dropped by the range; non-temporal: streamed once
                __builtin_amdgcn_raw_buffer_store_b64(group_h(s[u], uu[u], pz), yr, (g0 + 256u * u) * 8u, 0, 2);
        }
    }
}

// fp32 product -> e4m3 q + per-row scale with the row's h in registers: WAVES waves per workgroup, thread t owns the
// column groups t + 64 WAVES j (j < CPT) and their sb / bias values; rows blockIdx.x, + gridDim.x, ....  The next
// row's loads are issued before the row maximum's LDS exchange, so they are in flight across it and the stores.
// At least 4 waves per SIMD (at most 128 VGPRs): the bias form at 4 groups per thread otherwise takes 131 and halves
// the resident workgroups (31 248 x 2 x 8192 with bias: 403 -> 371 us).
template <int CPT, int WAVES, bool HB>
__global__ void __launch_bounds__(64 * WAVES, 4)
    scale_swiglu_quant_lds_kernel(const float* __restrict__ x, int64_t ldx, int64_t M, int64_t F, EpiArgs e,
                                  const uint16_t* __restrict__ silu, const uint16_t* __restrict__ rot,
                                  uint8_t* __restrict__ q, int64_t ldq, float* __restrict__ scale) {
    constexpr int THREADS = 64 * WAVES;
    constexpr int NG = CPT < 2 ? CPT : 2;               // groups per table lookup batch
    __shared__ __attribute__((aligned(16))) uint16_t tab[H3_SILU_ROT_LEN];
    __shared__ uint32_t red[2][WAVES];
    load_silu_rot(tab, rot, THREADS);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t ngroups = (uint32_t)(F >> 2);
    const uint32_t fb = (uint32_t)F * 4u;
    ColOps c[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j) c[j] = load_cols<HB>(e, F, threadIdx.x + THREADS * j);
    float pz = 0.0f;
    asm volatile("" : "+v"(pz));
    v4u xg[CPT], xu[CPT];
    auto load_row = [&](int64_t m) {
        const float* xr = x + m * ldx;
        const __amdgpu_buffer_rsrc_t gr = make_rsrc(xr, fb), ur = make_rsrc(xr + F, fb);
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const uint32_t off = (threadIdx.x + THREADS * (uint32_t)j) * 16u;
            xg[j] = __builtin_amdgcn_raw_buffer_load_b128(gr, off, 0, 2);
            xu[j] = __builtin_amdgcn_raw_buffer_load_b128(ur, off, 0, 2);
        }
    };
    int64_t m = blockIdx.x;
    if (m < M) load_row(m);
    __syncthreads();
    for (int par = 0; m < M; m += gridDim.x, par ^= 1) {
        const float sam = e.sa[m * e.sa_stride];
        pin_bias<HB>(c);
        uint32_t hp[CPT][2];
        uint32_t mx = 0;
#pragma unroll
        for (int j0 = 0; j0 < CPT; j0 += NG) {
            uint32_t key[NG][4], uu[NG][4], s[NG][4];
            bool valid[NG];
#pragma unroll
            for (int j = 0; j < NG; ++j) {
                valid[j] = threadIdx.x + THREADS * (uint32_t)(j0 + j) < ngroups;
                group_keys<HB>(xg[j0 + j], xu[j0 + j], sam, c[j0 + j], valid[j], key[j], uu[j]);
            }
            lookup_silu<NG>(tab, silu, key, s);
#pragma unroll
            for (int j = 0; j < NG; ++j) {
                const v2u hv = group_h(s[j], uu[j], pz);
                hp[j0 + j][0] = hv[0];
                hp[j0 + j][1] = hv[1];
                // |h| bit patterns order like |h| with NaN above +inf; groups past F do not count
                const uint32_t a = valid[j] ? hv[0] & 0x7fff7fffu : 0u, b = valid[j] ? hv[1] & 0x7fff7fffu : 0u;
                const uint32_t am = (a << 16) > (a & 0xffff0000u) ? (a << 16) : (a & 0xffff0000u);
                const uint32_t bm = (b << 16) > (b & 0xffff0000u) ? (b << 16) : (b & 0xffff0000u);
                mx = mx > am ? mx : am;
                mx = mx > bm ? mx : bm;
            }
        }
        if (m + gridDim.x < M) load_row(m + gridDim.x);
        mx = wave_max_u32(mx);
        if (lane == 0) red[par][wave] = mx;
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");   // no fence: the row loads stay in flight
#pragma unroll
        for (int w = 0; w < WAVES; ++w) mx = mx > red[par][w] ? mx : red[par][w];
        const float sc = row_scale(u2f(mx));
        const float inv = inv_scale(sc);
        const __amdgpu_buffer_rsrc_t qr = make_rsrc(q + m * ldq, (uint32_t)F);
        // code stores: device scope (sc1, written through the L2) up to 8 waves per row, non-temporal for the
        // 16-wave rows (measured: 31 248 x 2 x 8192, 8 waves, 369.9 -> 355.8 us with sc1; 4100 x 2 x 14 336,
        // 16 waves, 95.8 -> 100.6 us with sc1)
        constexpr int ST = WAVES <= 8 ? 16 : 2;
        if (mx < 0x7f800000u) {                          // wave-uniform: finite row maximum
#pragma unroll
            for (int j = 0; j < CPT; ++j)
                __builtin_amdgcn_raw_buffer_store_b32(quant_pairs<true>(hp[j][0], hp[j][1], inv), qr,
                                                      (threadIdx.x + THREADS * (uint32_t)j) * 4u, 0, ST);
        } else {
#pragma unroll
            for (int j = 0; j < CPT; ++j)
                __builtin_amdgcn_raw_buffer_store_b32(quant_pairs<false>(hp[j][0], hp[j][1], inv), qr,
                                                      (threadIdx.x + THREADS * (uint32_t)j) * 4u, 0, ST);
        }
        if (threadIdx.x == 0) scale[m] = sc;
    }
}

// The two-pass scale pass, elementwise: one thread per 4 columns.
template <int OUT_DT>
__global__ void __launch_bounds__(256) scale_bias_cast_kernel(const float* __restrict__ x, int64_t ldx, int64_t M,
                                                              int64_t N, EpiArgs e, uint16_t* __restrict__ y,
                                                              int64_t ldy) {
    const int64_t ngroups = N >> 2;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= M * ngroups) return;
    const int64_t m = idx / ngroups, n = 4 * (idx - m * ngroups);
    const v4f v = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(x + m * ldx + n));
    const float xv[4] = {v[0], v[1], v[2], v[3]};
    const float sam = e.sa[m * e.sa_stride];
    uint32_t o[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const bool hb = e.bias != nullptr;
        const float b = hb ? (OUT_DT ? fp16_to_f32(e.bias[n + r]) : bf16_to_f32(e.bias[n + r])) : 0.f;
        const float val = epi(xv[r], sam, e.sb[(n + r) * e.sb_stride], hb, b);
        o[r] = OUT_DT ? fp16_rne(val) : bf16_rne(val);
    }
    *reinterpret_cast<uint2*>(y + m * ldy + n) = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
}

// The scale pass over row segments, for contiguous (16-byte aligned) sb and an 8-byte aligned bias: block (b, s) covers
// the U * 256 column groups of segment s of rows 2b and 2b + 1, thread i the groups i + 256 u (coalesced per u); the
// two rows share the segment's sb / bias loads.  Every load is a range-checked buffer load (groups past the row, and a
// second row past M, read zero; stores past the row are dropped), so all of a thread's loads are in flight before the
// first use; no per-thread division.
template <int OUT_DT, int U>
__global__ void __launch_bounds__(256) scale_bias_cast_seg_kernel(const float* __restrict__ x, int64_t ldx, int64_t N,
                                                                  EpiArgs e, uint16_t* __restrict__ y, int64_t ldy,
                                                                  int64_t M) {
    constexpr int R = 2;
    const int64_t m0 = (int64_t)blockIdx.x * R;
    const uint32_t g0 = blockIdx.y * (256u * U) + threadIdx.x;
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(e.sb, (uint32_t)N * 4u);
    const bool hb = e.bias != nullptr;
    const __amdgpu_buffer_rsrc_t br = make_rsrc(hb ? (const void*)e.bias : (const void*)e.sb, hb ? (uint32_t)N * 2u : 0u);
    v4u xv[R][U], sv[U];
    v2u bv[U];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const bool in = m0 + r < M;
        const __amdgpu_buffer_rsrc_t xr = make_rsrc(x + (in ? m0 + r : m0) * ldx, in ? (uint32_t)N * 4u : 0u);
#pragma unroll
        for (int u = 0; u < U; ++u) xv[r][u] = __builtin_amdgcn_raw_buffer_load_b128(xr, (g0 + 256u * u) * 16u, 0, 2);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t g = g0 + 256u * u;
        sv[u] = __builtin_amdgcn_raw_buffer_load_b128(sr, g * 16u, 0, 0);
        bv[u] = __builtin_amdgcn_raw_buffer_load_b64(br, g * 8u, 0, 0);        // zeros without a bias
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t m = m0 + r;
        if (m >= M) break;
        const float sam = e.sa[m * e.sa_stride];
        const __amdgpu_buffer_rsrc_t yr = make_rsrc(y + m * ldy, (uint32_t)N * 2u);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float val[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t bw = bv[u][q >> 1];
                const uint32_t bh = (q & 1) ? (bw >> 16) : (bw & 0xffffu);
                const float b = OUT_DT ? fp16_to_f32(bh) : bf16_to_f32(bh);
                val[q] = epi(u2f(xv[r][u][q]), sam, u2f(sv[u][q]), hb, b);
            }
            v2u ov;
            if (OUT_DT) {
                ov = v2u{fp16_rne(val[0]) | (fp16_rne(val[1]) << 16), fp16_rne(val[2]) | (fp16_rne(val[3]) << 16)};
            } else {
                ov = v2u{cvt_bf16x2(val[0], val[1]), cvt_bf16x2(val[2], val[3])};
            }
            // non-temporal: the output streams through once (measured at 16 740 x 9216: 181.9 -> 165.8 us)
            __builtin_amdgcn_raw_buffer_store_b64(ov, yr, (g0 + 256u * u) * 8u, 0, 2);
        }
    }
}

template <int OUT_DT>
void launch_scale_bias_cast_seg(const float* x, int64_t ldx, int64_t M, int64_t N, const EpiArgs& e, uint16_t* y,
                                int64_t ldy, hipStream_t st) {
    const int64_t groups = N >> 2;
    const int u = (int)std::min<int64_t>(4, (groups + 255) / 256);
    dim3 grid((unsigned)((M + 1) / 2), (unsigned)((groups + 256 * u - 1) / (256 * u))), block(256);
    if (u <= 1) hipLaunchKernelGGL((scale_bias_cast_seg_kernel<OUT_DT, 1>), grid, block, 0, st, x, ldx, N, e, y, ldy, M);
    else if (u == 2) hipLaunchKernelGGL((scale_bias_cast_seg_kernel<OUT_DT, 2>), grid, block, 0, st, x, ldx, N, e, y, ldy, M);
    else if (u == 3) hipLaunchKernelGGL((scale_bias_cast_seg_kernel<OUT_DT, 3>), grid, block, 0, st, x, ldx, N, e, y, ldy, M);
    else hipLaunchKernelGGL((scale_bias_cast_seg_kernel<OUT_DT, 4>), grid, block, 0, st, x, ldx, N, e, y, ldy, M);
}

// The persistent LDS-table forms of the bf16-source pass, when their 16-byte loads and 8-byte stores are aligned: one
// wave per row for F <= 8192, 16 waves per row for F <= 16 384; returns false to take the one-workgroup-per-row kernel.
bool launch_silu_mul_quant_lds(const void* x, int64_t ldx, int64_t M, int64_t F, const uint16_t* silu, void* q,
                               int64_t ldq, float* scale, hipStream_t st) {
    const int64_t cpl = ((F >> 3) + 63) / 64;
    if (F % 8 != 0 || ldx % 8 != 0 || ldq % 8 != 0 || ((uintptr_t)q & 7) != 0 || F > 2 * 8 * 64 * SMQW_WAVES)
        return false;
    // buffer descriptors need 4-byte aligned bases: every row start is (16-byte x, 8-byte q, even strides)
    const uint16_t* xp = (const uint16_t*)x;
    uint8_t* qp = (uint8_t*)q;
    if (cpl > 16) {                                      // 8192 < F <= 16 384: 16 waves per row, 2 chunks per lane
        const int64_t wgs = std::min<int64_t>(M, h3host::cu_count());
        hipLaunchKernelGGL((silu_mul_quant_wide_kernel<2>), dim3((unsigned)wgs), dim3(64 * SMQW_WAVES), 0, st, xp, ldx,
                           M, F, silu, qp, ldq, scale);
        return true;
    }
    const int64_t wgs = std::min<int64_t>((M + SMQ_WAVES - 1) / SMQ_WAVES, h3host::cu_count());
    dim3 grid((unsigned)std::max<int64_t>(1, wgs)), block(64 * SMQ_WAVES);
#define H3_L(N) hipLaunchKernelGGL((silu_mul_quant_lds_kernel<N>), grid, block, 0, st, xp, ldx, M, F, silu, qp, ldq, scale)
    if (cpl <= 1) H3_L(1);
    else if (cpl <= 2) H3_L(2);
    else if (cpl <= 4) H3_L(4);
    else if (cpl <= 8) H3_L(8);
    else if (cpl <= 12) H3_L(12);
    else H3_L(16);
#undef H3_L
    return true;
}

// Whether the fp32 forms can take the LDS-table kernels: contiguous 16-byte aligned sb, 8-byte aligned bias (rows of
// x are 16-byte aligned by the entry points' checks), and 32-bit buffer ranges.
bool lds_table_ok(const EpiArgs& e, int64_t F) {
    return e.sb_stride == 1 && ((uintptr_t)e.sb & 15) == 0 && ((uintptr_t)e.bias & 7) == 0 &&
           ((uintptr_t)h3host::silu_rot_ptr() & 15) == 0 && F < ((int64_t)1 << 28);
}

// Resident workgroups of a kernel per CU at the given block size (from the occupancy calculator; at least 1).  The
// persistent grids below launch exactly that many per CU, so no workgroup waits for another one's slot.
int resident_per_cu(const void* kernel, int threads) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, 0) != hipSuccess) {
        (void)hipGetLastError();
        n = 1;
    }
    return n < 1 ? 1 : n;
}

template <int U, bool HB>
void launch_scale_swiglu_seg_u(const float* x, int64_t ldx, int64_t M, int64_t F, const EpiArgs& e, uint16_t* h,
                               int64_t ldh, hipStream_t st) {
    static const int per_cu = resident_per_cu((const void*)scale_swiglu_seg_kernel<U, HB>, 256);
    const int64_t groups = F >> 2;
    const int64_t nseg = (groups + 256 * U - 1) / (256 * U);
    const int64_t rows = std::min<int64_t>((M + 1) / 2, std::max<int64_t>(1, h3host::cu_count() * per_cu / nseg));
    hipLaunchKernelGGL((scale_swiglu_seg_kernel<U, HB>), dim3((unsigned)nseg, (unsigned)rows), dim3(256), 0, st, x, ldx,
                       M, F, e, h3host::silu_table_ptr(), h3host::silu_rot_ptr(), h, ldh);
}

void launch_scale_swiglu_seg(const float* x, int64_t ldx, int64_t M, int64_t F, const EpiArgs& e, uint16_t* h,
                             int64_t ldh, hipStream_t st) {
    // 2 groups per thread and row (U = 4 measured the same at 31 248 x 2 x 8192, with twice the registers)
    const bool one = (F >> 2) <= 256;
    if (e.bias) {
        if (one) launch_scale_swiglu_seg_u<1, true>(x, ldx, M, F, e, h, ldh, st);
        else launch_scale_swiglu_seg_u<2, true>(x, ldx, M, F, e, h, ldh, st);
    } else {
        if (one) launch_scale_swiglu_seg_u<1, false>(x, ldx, M, F, e, h, ldh, st);
        else launch_scale_swiglu_seg_u<2, false>(x, ldx, M, F, e, h, ldh, st);
    }
}

template <int CPT, int WAVES, bool HB>
void launch_scale_swiglu_quant_lds_c(const float* x, int64_t ldx, int64_t M, int64_t F, const EpiArgs& e, uint8_t* q,
                                     int64_t ldq, float* scale, hipStream_t st) {
    static const int per_cu = resident_per_cu((const void*)scale_swiglu_quant_lds_kernel<CPT, WAVES, HB>, 64 * WAVES);
    const int64_t wgs = std::min<int64_t>(M, (int64_t)h3host::cu_count() * per_cu);
    hipLaunchKernelGGL((scale_swiglu_quant_lds_kernel<CPT, WAVES, HB>), dim3((unsigned)wgs), dim3(64 * WAVES), 0, st,
                       x, ldx, M, F, e, h3host::silu_table_ptr(), h3host::silu_rot_ptr(), q, ldq, scale);
}

// The quant form with the row in registers, for F <= 16 384 (up to 4 column groups per thread, 4 to 16 waves per row);
// returns false to take the one-workgroup-per-row kernel.  At F = 8192, 8 waves x 4 groups measured 369 us against
// 397 us for 16 waves x 2 groups (31 248 rows).
bool launch_scale_swiglu_quant_lds(const float* x, int64_t ldx, int64_t M, int64_t F, const EpiArgs& e, uint8_t* q,
                                   int64_t ldq, float* scale, hipStream_t st) {
    const int64_t groups = F >> 2;
    if (!lds_table_ok(e, F) || groups > 4 * 1024) return false;
#define H3_Q(C, W, HB) launch_scale_swiglu_quant_lds_c<C, W, HB>(x, ldx, M, F, e, q, ldq, scale, st)
#define H3_QB(HB)                            \
    if (groups <= 256) H3_Q(1, 4, HB);        \
    else if (groups <= 512) H3_Q(2, 4, HB);   \
    else if (groups <= 1024) H3_Q(2, 8, HB);  \
    else if (groups <= 2048) H3_Q(4, 8, HB);  \
    else H3_Q(4, 16, HB);
    if (e.bias) {
        H3_QB(true)
    } else {
        H3_QB(false)
    }
#undef H3_QB
#undef H3_Q
    return true;
}

template <bool SRC_FP32>
int launch_swiglu_quant(const void* x, int64_t ldx, int64_t M, int64_t F, const EpiArgs& e, void* q, int64_t ldq,
                        float* scale, hipStream_t st) {
    if (M == 0 || F == 0) return H3FP8_OK;
    int rc = h3host::ensure_device_init();
    if (rc) return rc;
    const uint16_t* silu = h3host::silu_table_ptr();
    if (!SRC_FP32 && launch_silu_mul_quant_lds(x, ldx, M, F, silu, q, ldq, scale, st)) {
        H3_CHECK_HIP(hipGetLastError());
        return H3FP8_OK;
    }
    if (SRC_FP32 && launch_scale_swiglu_quant_lds((const float*)x, ldx, M, F, e, (uint8_t*)q, ldq, scale, st)) {
        H3_CHECK_HIP(hipGetLastError());
        return H3FP8_OK;
    }
    const int64_t cpt = ((F >> 2) + 255) / 256;
    dim3 grid((unsigned)M), block(256);
    uint8_t* qp = (uint8_t*)q;
#define H3_S(N) hipLaunchKernelGGL((swiglu_quant_rows_kernel<SRC_FP32, N>), grid, block, 0, st, x, ldx, F, e, silu, \
                                   qp, ldq, scale)
    if (cpt <= 1) H3_S(1);
    else if (cpt <= 2) H3_S(2);
    else if (cpt <= 4) H3_S(4);
    else if (cpt <= 8) H3_S(8);
    else if (cpt <= 16) H3_S(16);
    else H3_S(0);
#undef H3_S
    H3_CHECK_HIP(hipGetLastError());
    return H3FP8_OK;
}

int check_common(int64_t M, int64_t W, int64_t ldx, const void* x, const char* who) {
    H3_REQUIRE(M >= 0 && W >= 0, "%s: negative size", who);
    H3_REQUIRE(W % 8 == 0, "%s: width %lld must be a multiple of 8", who, (long long)W);
    H3_REQUIRE(M == 0 || x, "%s: null input", who);
    H3_REQUIRE(ldx >= W && ldx % 4 == 0, "%s: bad row stride %lld", who, (long long)ldx);
    H3_REQUIRE(((uintptr_t)x & 15) == 0, "%s: input must be 16-byte aligned", who);
    return H3FP8_OK;
}

}  // namespace

extern "C" {

int h3fp8_scale_bias_cast(const float* x32, int64_t ldx, const float* sa, int64_t sa_stride, const float* sb,
                          int64_t sb_stride, const void* bias, void* y, int64_t ldy, int out_dtype, int64_t M,
                          int64_t N, void* stream) {
    int rc = check_common(M, N, ldx, x32, "h3fp8_scale_bias_cast");
    if (rc) return rc;
    H3_REQUIRE(out_dtype == H3FP8_DT_BF16 || out_dtype == H3FP8_DT_FP16, "h3fp8_scale_bias_cast: bad out_dtype");
    if (M == 0 || N == 0) return H3FP8_OK;
    H3_REQUIRE(sa && sb && y && ldy >= N && ldy % 4 == 0 && ((uintptr_t)y & 7) == 0,
               "h3fp8_scale_bias_cast: bad scales or output");
    EpiArgs e{sa, sa_stride, sb, sb_stride, (const uint16_t*)bias};
    if (sb_stride == 1 && ((uintptr_t)sb & 15) == 0 && ((uintptr_t)bias & 7) == 0 && N < ((int64_t)1 << 30) &&
        M < ((int64_t)1 << 31)) {
        if (out_dtype == H3FP8_DT_BF16)
            launch_scale_bias_cast_seg<0>(x32, ldx, M, N, e, (uint16_t*)y, ldy, (hipStream_t)stream);
        else
            launch_scale_bias_cast_seg<1>(x32, ldx, M, N, e, (uint16_t*)y, ldy, (hipStream_t)stream);
        H3_CHECK_HIP(hipGetLastError());
        return H3FP8_OK;
    }
    const int64_t total = M * (N >> 2);
    dim3 grid((unsigned)((total + 255) / 256)), block(256);
    if (out_dtype == H3FP8_DT_BF16)
        hipLaunchKernelGGL(scale_bias_cast_kernel<0>, grid, block, 0, (hipStream_t)stream, x32, ldx, M, N, e,
                           (uint16_t*)y, ldy);
    else
        hipLaunchKernelGGL(scale_bias_cast_kernel<1>, grid, block, 0, (hipStream_t)stream, x32, ldx, M, N, e,
                           (uint16_t*)y, ldy);
    H3_CHECK_HIP(hipGetLastError());
    return H3FP8_OK;
}

int h3fp8_scale_swiglu(const float* x32, int64_t ldx, const float* sa, int64_t sa_stride, const float* sb,
                       int64_t sb_stride, const void* bias, int64_t M, int64_t F, void* h, int64_t ldh, void* stream) {
    int rc = check_common(M, 2 * F, ldx, x32, "h3fp8_scale_swiglu");
    if (rc) return rc;
    if (M == 0 || F == 0) return H3FP8_OK;
    H3_REQUIRE(F % 4 == 0 && sa && sb && h && ldh >= F && ldh % 4 == 0 && ((uintptr_t)h & 7) == 0,
               "h3fp8_scale_swiglu: bad scales or output");
    rc = h3host::ensure_device_init();
    if (rc) return rc;
    EpiArgs e{sa, sa_stride, sb, sb_stride, (const uint16_t*)bias};
    if (lds_table_ok(e, F)) {
        launch_scale_swiglu_seg(x32, ldx, M, F, e, (uint16_t*)h, ldh, (hipStream_t)stream);
        H3_CHECK_HIP(hipGetLastError());
        return H3FP8_OK;
    }
    const int64_t total = M * (F >> 2);
    hipLaunchKernelGGL(scale_swiglu_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       x32, ldx, M, F, e, h3host::silu_table_ptr(), (uint16_t*)h, ldh);
    H3_CHECK_HIP(hipGetLastError());
    return H3FP8_OK;
}

int h3fp8_scale_swiglu_quant(const float* x32, int64_t ldx, const float* sa, int64_t sa_stride, const float* sb,
                             int64_t sb_stride, const void* bias, int64_t M, int64_t F, void* q, int64_t ldq,
                             float* scale, void* stream) {
    int rc = check_common(M, 2 * F, ldx, x32, "h3fp8_scale_swiglu_quant");
    if (rc) return rc;
    if (M == 0 || F == 0) return H3FP8_OK;
    H3_REQUIRE(F % 4 == 0 && sa && sb && q && scale && ldq >= F && ldq % 4 == 0 && ((uintptr_t)q & 3) == 0,
               "h3fp8_scale_swiglu_quant: bad scales or output");
    EpiArgs e{sa, sa_stride, sb, sb_stride, (const uint16_t*)bias};
    return launch_swiglu_quant<true>(x32, ldx, M, F, e, q, ldq, scale, (hipStream_t)stream);
}

int h3fp8_silu_mul_quant(const void* x, int64_t ldx, int64_t M, int64_t F, void* q, int64_t ldq, float* scale,
                         void* stream) {
    int rc = check_common(M, 2 * F, ldx, x, "h3fp8_silu_mul_quant");
    if (rc) return rc;
    if (M == 0 || F == 0) return H3FP8_OK;
    H3_REQUIRE(F % 4 == 0 && ldx % 8 == 0 && q && scale && ldq >= F && ldq % 4 == 0 && ((uintptr_t)q & 3) == 0,
               "h3fp8_silu_mul_quant: bad output");
    EpiArgs e{nullptr, 0, nullptr, 0, nullptr};
    return launch_swiglu_quant<false>(x, ldx, M, F, e, q, ldq, scale, (hipStream_t)stream);
}

}  // extern "C"
