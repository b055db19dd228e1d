// Kernel 1: dynamic per-token amax + OCP e4m3fn quant of a bf16 [M, K] tensor (and its "known amax" tail form).
//
// Reference arithmetic (h3_tp2/fp8_quant_fuse.py:11-13, :92-121, :280-290, :302-307):
//   amax = max_k |x_k| (NaN propagating), scale = max(amax / 448, 1/(448*512)),
//   q_k = e4m3fn_rne(clamp(x_k * (1 / scale), -448, 448)).
//
// Design (HBM-bound: 2 bytes read + 1 byte written per element, plus 4 bytes of scale per row):
//   * one 64-lane wavefront per row, or two for rows of 6+ chunks per lane; a lane owns CPL chunks of 8 bf16 (16-byte
//     loads), chunk c = lane + 64 j, so every load instruction of a wave reads 1 KiB of the row contiguously; the row
//     stays in VGPRs (read from HBM once);
//   * range-checked buffer loads and stores (a per-row descriptor): no branch around the row's tail, so all of a
//     row's loads are in flight together (guarded global loads made the compiler wait after every second load);
//   * the row maximum is an integer max over |x| bit patterns (for non-negative floats the integer order is the float
//     order and every NaN pattern is above +inf, so the max propagates NaN exactly like the reference's), reduced
//     across the wave with xor-shuffles (and between the two waves of a split row through LDS);
//   * scale and 1/scale are IEEE fp32 divisions (hipcc's correctly rounded divide), computed once per lane;
//   * the e4m3 conversion is gfx950's v_cvt_pk_fp8_f32 (OCP e4m3fn, RNE), 8-byte stores per chunk.
// Four rows per 256-thread workgroup (two when a row is split over two waves, below); rows beyond M touch no memory.
#include "h3fp8_common.h"

namespace {

using namespace h3;

typedef unsigned int v2u __attribute__((ext_vector_type(2)));

// |x| bit patterns of the 8 bf16 values in a 16-byte chunk, max-reduced to one 16-bit pattern.
__device__ __forceinline__ uint32_t chunk_absmax(uint4 v) {
    uint32_t m = 0;
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t lo = w[i] & 0x7fffu, hi = (w[i] >> 16) & 0x7fffu;
        m = m > lo ? m : lo;
        m = m > hi ? m : hi;
    }
    return m;
}

// x * inv clamped to [-448, 448].  FINITE: the row maximum is finite, so x * inv is finite and a median-of-three is the
// clamp exactly (one instruction); otherwise the reference's compare/select clamp, which keeps NaN.
template <bool FINITE>
__device__ __forceinline__ float scaled_clamp(float x, float inv) {
    if (FINITE) return __builtin_amdgcn_fmed3f(x * inv, -H3_FP8_MAX, H3_FP8_MAX);
    return quant_clamp(x, inv);
}

// 8 bf16 -> 8 e4m3fn bytes with the given inverse scale.
template <bool FINITE>
__device__ __forceinline__ uint2 chunk_quant(uint4 v, float inv) {
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
    float f[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = scaled_clamp<FINITE>(u2f(w[i] << 16), inv);
        f[2 * i + 1] = scaled_clamp<FINITE>(u2f(w[i] & 0xffff0000u), inv);
    }
    return make_uint2(e4m3x4(f[0], f[1], f[2], f[3]), e4m3x4(f[4], f[5], f[6], f[7]));
}

// WPR waves per row, CPL 16-byte chunks per lane held in registers: wave p of a row owns its chunks
// 64 CPL p .. 64 CPL (p + 1) - 1.  KNOWN_AMAX: the row maximum comes from row_amax (fp32 bits) instead of the row, so
// the waves of a row are independent; otherwise two waves of a row exchange their maxima through LDS (one barrier),
// and no wave leaves before it: a wave of a row at or past M reads and writes nothing (empty buffer ranges).
// STORE_AUX: the cache policy of the code stores (the launcher's choice, below).
template <int CPL, bool KNOWN_AMAX, int WPR = 1, int STORE_AUX = 16>
__global__ void __launch_bounds__(256) quant_rows_kernel(const uint16_t* __restrict__ x, int64_t ldx, int64_t M,
                                                         int64_t K, uint8_t* __restrict__ q, int64_t ldq,
                                                         float* __restrict__ scale,
                                                         const float* __restrict__ row_amax) {
    static_assert(WPR == 1 || WPR == 2, "one or two waves per row");
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t row = (int64_t)blockIdx.x * (4 / WPR) + wave / WPR;
    // the lane's first chunk is lane + 64 CPL p; chunk j of the lane is that + 64 j
    const int lane = (threadIdx.x & 63) + 64 * CPL * (wave % WPR);
    constexpr bool SHARED_MAX = WPR == 2 && !KNOWN_AMAX;
    if (!SHARED_MAX && row >= M) return;
    const bool live = row < M;
    // Range-checked buffer accesses: chunks past the row read as zero (|0| does not raise the maximum) and their
    // stores are dropped, with no branch -- every load of the row is in flight at once.
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x + (live ? row : 0) * ldx, live ? (uint32_t)K * 2u : 0u);
    uint4 v[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const v4u t = __builtin_amdgcn_raw_buffer_load_b128(xr, (uint32_t)(lane + 64 * j) * 16u, 0, 2);   // nt
        v[j] = make_uint4(t.x, t.y, t.z, t.w);
    }
    float amax;
    if (KNOWN_AMAX) {
        amax = row_amax[row];
    } else {
        uint32_t m = 0;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            uint32_t c = chunk_absmax(v[j]);
            m = m > c ? m : c;
        }
        m = wave_max_u32(m);
        if (SHARED_MAX) {
            __shared__ uint32_t part[4];
            part[wave] = m;
            __syncthreads();
            const uint32_t o = part[wave ^ 1];
            m = m > o ? m : o;
        }
        amax = u2f(m << 16);
    }
    const float s = row_scale(amax);
    const float inv = inv_scale(s);
    const __amdgpu_buffer_rsrc_t qr = make_rsrc(q + (live ? row : 0) * ldq, live ? (uint32_t)K : 0u);
    if (__builtin_amdgcn_readfirstlane(f2u(amax) & 0x7fffffffu) < 0x7f800000u) {   // wave-uniform: finite maximum
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const uint2 o = chunk_quant<true>(v[j], inv);
            __builtin_amdgcn_raw_buffer_store_b64(v2u{o.x, o.y}, qr, (uint32_t)(lane + 64 * j) * 8u, 0, STORE_AUX);
        }
    } else {
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const uint2 o = chunk_quant<false>(v[j], inv);
            __builtin_amdgcn_raw_buffer_store_b64(v2u{o.x, o.y}, qr, (uint32_t)(lane + 64 * j) * 8u, 0, STORE_AUX);
        }
    }
    if (live && lane == 0) scale[row] = s;
}

// Rows too wide for the register-resident form: the row is read twice (max pass, then quant pass).
template <bool KNOWN_AMAX>
__global__ void __launch_bounds__(256) quant_rows_wide_kernel(const uint16_t* __restrict__ x, int64_t ldx, int64_t M,
                                                              int64_t K, uint8_t* __restrict__ q, int64_t ldq,
                                                              float* __restrict__ scale,
                                                              const float* __restrict__ row_amax) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= M) return;
    const int64_t nchunk = K >> 3;
    const uint4* xr = reinterpret_cast<const uint4*>(x + row * ldx);
    float amax;
    if (KNOWN_AMAX) {
        amax = row_amax[row];
    } else {
        uint32_t m = 0;
        for (int64_t c = lane; c < nchunk; c += 64) {
            uint32_t t = chunk_absmax(xr[c]);
            m = m > t ? m : t;
        }
        amax = u2f(wave_max_u32(m) << 16);
    }
    const float s = row_scale(amax);
    const float inv = inv_scale(s);
    uint2* qr = reinterpret_cast<uint2*>(q + row * ldq);
    for (int64_t c = lane; c < nchunk; c += 64) qr[c] = chunk_quant<false>(xr[c], inv);
    if (lane == 0) scale[row] = s;
}

template <bool KNOWN>
int launch_quant(const void* x, int64_t ldx, int64_t M, int64_t K, void* q, int64_t ldq, float* scale,
                 const float* row_amax, hipStream_t st) {
    if (M == 0) return H3FP8_OK;
    const int64_t nchunk = K >> 3;
    const int64_t cpl = (nchunk + 63) / 64;
    dim3 grid((unsigned)((M + 3) / 4)), block(256);
    const uint16_t* xp = (const uint16_t*)x;
    uint8_t* qp = (uint8_t*)q;
    // Rows of 6 or more chunks per lane go to two waves of half the chunks each: half the registers per wave, twice
    // the waves in flight (measured at M = 91 728: with the maximum given K = 8192 427 -> 383 us, K = 3072
    // 129.7 -> 127.7 us, four waves of a quarter the same as two; the full quant at K = 3072 128.5 -> 125.0 us, and
    // at M = 2048 / 8192 / 16 740 the same as one wave per row or slightly faster)
    //
    // Cache policy of the code stores (the aux operand: bit 0 sc0, bit 1 nt, bit 4 sc1).  Device scope (sc1) writes
    // them through the XCD's L2 instead of leaving dirty lines for the end-of-kernel write-back: measured at K = 3072
    // against plain stores, M = 16 740 27.7 -> 25.9 us, M = 91 728 128.7 -> 123.9 us, the known-maximum form 129.6 ->
    // 124.5 us (non-temporal ones slower at M = 66 960).  Rows of 8 or more chunks per lane and wave (K > 6144) take
    // it while the codes fit the 256 MiB MALL and store non-temporally beyond (the known-maximum form at K = 8192,
    // HIP-graph replays, nt against sc1: M = 15 624 60.8 / 56.9 us, 31 248 120.2 / 111.3, 45 864 177.6 / 183.4,
    // 91 728 362.1 / 374.8).
    const bool codes_fit = M * K <= (256LL << 20);
#define H3_Q(N)                                                                                                        \
    do {                                                                                                               \
        const dim3 g2((unsigned)((M + 1) / 2));                                                                        \
        if constexpr (N >= 16) {                                                                                       \
            if (codes_fit)                                                                                             \
                hipLaunchKernelGGL((quant_rows_kernel<N / 2, KNOWN, 2, 16>), g2, block, 0, st, xp, ldx, M, K, qp, ldq, \
                                   scale, row_amax);                                                                   \
            else                                                                                                       \
                hipLaunchKernelGGL((quant_rows_kernel<N / 2, KNOWN, 2, 2>), g2, block, 0, st, xp, ldx, M, K, qp, ldq,  \
                                   scale, row_amax);                                                                   \
        } else if constexpr (N >= 6) {                                                                                 \
            hipLaunchKernelGGL((quant_rows_kernel<N / 2, KNOWN, 2>), g2, block, 0, st, xp, ldx, M, K, qp, ldq, scale,  \
                               row_amax);                                                                              \
        } else {                                                                                                       \
            hipLaunchKernelGGL((quant_rows_kernel<N, KNOWN>), grid, block, 0, st, xp, ldx, M, K, qp, ldq, scale,       \
                               row_amax);                                                                              \
        }                                                                                                              \
    } while (0)
    if (cpl <= 1) H3_Q(1);
    else if (cpl <= 2) H3_Q(2);
    else if (cpl <= 3) H3_Q(3);
    else if (cpl <= 4) H3_Q(4);
    else if (cpl <= 6) H3_Q(6);
    else if (cpl <= 8) H3_Q(8);
    else if (cpl <= 12) H3_Q(12);
    else if (cpl <= 16) H3_Q(16);
    else if (cpl <= 24) H3_Q(24);
    else if (cpl <= 32) H3_Q(32);
    else hipLaunchKernelGGL((quant_rows_wide_kernel<KNOWN>), grid, block, 0, st, xp, ldx, M, K, qp, ldq, scale, row_amax);
#undef H3_Q
    H3_CHECK_HIP(hipGetLastError());
    return H3FP8_OK;
}

int check_quant_args(const void* x, int64_t ldx, int64_t M, int64_t K, const void* q, int64_t ldq,
                     const float* scale) {
    H3_REQUIRE(M >= 0 && K >= 0, "quant: negative size M=%lld K=%lld", (long long)M, (long long)K);
    H3_REQUIRE(K % 8 == 0, "quant: K=%lld must be a multiple of 8", (long long)K);
    H3_REQUIRE(M == 0 || (x && q && scale), "quant: null pointer");
    H3_REQUIRE(ldx >= K && ldx % 8 == 0, "quant: ldx=%lld must be >= K and a multiple of 8", (long long)ldx);
    H3_REQUIRE(ldq >= K && ldq % 8 == 0, "quant: ldq=%lld must be >= K and a multiple of 8", (long long)ldq);
    H3_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)q & 7) == 0, "quant: x must be 16-byte and q 8-byte aligned");
    return H3FP8_OK;
}

// Rows made of P segments (the Ulysses receive buffer [P, M, seg] read as the out projection's [M, P * seg] input):
// logical row m is x[p * stride_p + m * stride_m .. + seg] for p = 0 .. P-1.  Same arithmetic and layout as
// quant_rows_kernel; 16-byte chunk c of the logical row is chunk c % cps of segment c / cps (cps = seg / 8).  The whole
// source is one buffer descriptor of `bytes`, so chunks past the row read zeros through an out-of-range offset.
template <int CPL>
__global__ void __launch_bounds__(256) quant_segments_kernel(const uint16_t* __restrict__ x, uint32_t bytes,
                                                             int64_t M, int cps, int P, int64_t stride_p,
                                                             int64_t stride_m, uint8_t* __restrict__ q, int64_t ldq,
                                                             float* __restrict__ scale) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (row >= M) return;
    const int nchunk = cps * P;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, bytes);
    uint4 v[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = lane + 64 * j;
        const int p = c / cps;
        const uint32_t off = c < nchunk ? (uint32_t)((p * stride_p + row * stride_m + 8 * (c - p * cps)) * 2) : 0x80000000u;
        const v4u t = __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 2);
        v[j] = make_uint4(t.x, t.y, t.z, t.w);
    }
    uint32_t mx = 0;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const uint32_t c = chunk_absmax(v[j]);
        mx = mx > c ? mx : c;
    }
    const float amax = u2f(wave_max_u32(mx) << 16);
    const float s = row_scale(amax);
    const float inv = inv_scale(s);
    const __amdgpu_buffer_rsrc_t qr = make_rsrc(q + row * ldq, (uint32_t)nchunk * 8u);
    // device-scope (sc1) code stores, as quant_rows_kernel's (measured, HIP-graph replays: [2, 45 864, 12 x 128]
    // 64.2 -> 61.3 us, [4, 22 932, 6 x 128] 35.5 -> 32.9 us, [2, 2050, 28 x 128] 10.5 -> 9.4 us against plain stores)
    if (__builtin_amdgcn_readfirstlane(f2u(amax) & 0x7fffffffu) < 0x7f800000u) {
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const uint2 o = chunk_quant<true>(v[j], inv);
            __builtin_amdgcn_raw_buffer_store_b64(v2u{o.x, o.y}, qr, (uint32_t)(lane + 64 * j) * 8u, 0, 16);
        }
    } else {
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const uint2 o = chunk_quant<false>(v[j], inv);
            __builtin_amdgcn_raw_buffer_store_b64(v2u{o.x, o.y}, qr, (uint32_t)(lane + 64 * j) * 8u, 0, 16);
        }
    }
    if (lane == 0) scale[row] = s;
}

}  // namespace

namespace h3host {
// Used by the fused GEMM paths for their tail pass.
// The quant tail's argument checks alone, for entry points that must refuse a bad call before their first launch.
int quant_args_ok(const void* x, int64_t ldx, int64_t M, int64_t K, const void* q, int64_t ldq, const float* scale) {
    return check_quant_args(x, ldx, M, K, q, ldq, scale);
}

int quant_rows_amax_launch(const void* x, int64_t ldx, int64_t M, int64_t K, const float* row_amax, void* q,
                           int64_t ldq, float* scale, hipStream_t st) {
    int rc = check_quant_args(x, ldx, M, K, q, ldq, scale);
    if (rc) return rc;
    return launch_quant<true>(x, ldx, M, K, q, ldq, scale, row_amax, st);
}
}  // namespace h3host

extern "C" {

int h3fp8_quant_rows(const void* x, int64_t ldx, int64_t M, int64_t K, void* q, int64_t ldq, float* scale,
                     void* stream) {
    int rc = check_quant_args(x, ldx, M, K, q, ldq, scale);
    if (rc) return rc;
    return launch_quant<false>(x, ldx, M, K, q, ldq, scale, nullptr, (hipStream_t)stream);
}

int h3fp8_quant_segments(const void* x, int64_t P, int64_t seg, int64_t stride_p, int64_t stride_m, int64_t M,
                         void* q, int64_t ldq, float* scale, void* stream) {
    H3_REQUIRE(P >= 1 && seg >= 0 && M >= 0 && stride_p >= 0 && stride_m >= 0, "quant_segments: negative size");
    if (M == 0 || seg == 0) {
        H3_REQUIRE(M == 0, "quant_segments: seg = 0 with rows");
        return H3FP8_OK;
    }
    H3_REQUIRE(seg % 8 == 0 && stride_p % 8 == 0 && stride_m % 8 == 0,
               "quant_segments: seg and both strides must be multiples of 8 elements");
    H3_REQUIRE(P * seg <= 64 * 8 * 32, "quant_segments: P * seg = %lld exceeds 16384", (long long)(P * seg));
    H3_REQUIRE(x && q && scale && ((uintptr_t)x & 15) == 0 && ((uintptr_t)q & 7) == 0 && ldq >= P * seg && ldq % 8 == 0,
               "quant_segments: x 16-byte and q 8-byte aligned, ldq >= P * seg and a multiple of 8");
    // bytes of the source that rows 0 .. M-1 reach: the largest element offset + seg
    const int64_t span = (P - 1) * stride_p + (M - 1) * stride_m + seg;
    H3_REQUIRE(span * 2 < 0x80000000ll, "quant_segments: the source spans more than 2 GiB");
    const int64_t cpl = ((P * seg / 8) + 63) / 64;
    dim3 grid((unsigned)((M + 3) / 4)), block(256);
    const uint16_t* xp = (const uint16_t*)x;
    const uint32_t bytes = (uint32_t)(span * 2);
    const int cps = (int)(seg / 8);
    hipStream_t st = (hipStream_t)stream;
#define H3_S(N) hipLaunchKernelGGL((quant_segments_kernel<N>), grid, block, 0, st, xp, bytes, M, cps, (int)P, stride_p, \
                                   stride_m, (uint8_t*)q, ldq, scale)
    if (cpl <= 2) H3_S(2);
    else if (cpl <= 4) H3_S(4);
    else if (cpl <= 6) H3_S(6);
    else if (cpl <= 8) H3_S(8);
    else if (cpl <= 12) H3_S(12);
    else if (cpl <= 16) H3_S(16);
    else if (cpl <= 24) H3_S(24);
    else H3_S(32);
#undef H3_S
    H3_CHECK_HIP(hipGetLastError());
    return H3FP8_OK;
}

int h3fp8_quant_rows_amax(const void* x, int64_t ldx, int64_t M, int64_t K, const float* row_amax, void* q,
                          int64_t ldq, float* scale, void* stream) {
    H3_REQUIRE(M == 0 || row_amax, "quant_rows_amax: null row_amax");
    return h3host::quant_rows_amax_launch(x, ldx, M, K, row_amax, q, ldq, scale, (hipStream_t)stream);
}

}  // extern "C"
