// The per-token FP8 quant fused into its producers: the RMSNorm + AdaLN modulation that produces the qkv input and
// the gated residual + RMSNorm + AdaLN modulation that produces the fc1 input, each writing the e4m3 row and its
// scale instead of the bf16 row (h3_tp2/fp8_quant_fuse.py:143-243; the stock producers' arithmetic as the reference's
// CPU stand-ins state it, tests/fake_h3_consumers.py:66-84).  Per row m of width H, index i = indices[m]:
//
//   gate form only:  u = bf16(residual + gate[i] * branch)   (fp32 multiply, then fp32 add, then RNE to bf16)
//                    residual_out[m] = u, and x = u below
//   var  = fp32(sum_k x_k^2) / H      (x_k^2 is exact in fp32; the sum is taken in fp64 and rounded once to fp32 --
//                                      the stock kernel's fp32 reduction order is its compiler's, this is the sum it
//                                      approximates, and it does not depend on the lane layout)
//   r    = 1 / sqrt(var + eps)        (correctly rounded sqrt, IEEE division: torch's CPU rsqrt)
//   h_k  = bf16(((x_k * r) * weight_k) * (1 + scale[i]_k) + shift[i]_k)   (each fp32 operation rounded, no fma)
//   q, qscale = kernel 1's per-token quant of h (amax, max(amax / 448, 1/(448*512)), clamp, e4m3fn RNE)
//
// One 64-lane wave per row, 4 rows per 256-thread workgroup; lane l owns the 16-byte chunks l + 64 j of the row
// (coalesced 1 KiB per load instruction), the row stays in VGPRs, both reductions are wave shuffles.  HBM-bound:
// 3H + 4 bytes per row (7H + 4 for the gate form); weight, shift and scale rows are re-read from the caches.
//
// An index outside [0, n_index) reads table row 0 instead (no access out of bounds) and poisons the row: residual_out
// and h are NaN, the scale NaN, the codes NaN -- torch's index_select would raise; a kernel cannot.
#include <algorithm>

#include "h3fp8_common.h"

namespace {

using namespace h3;

struct RmsArgs {
    const uint16_t* x;          // x (or the residual of the gate form) bf16 [M, H]
    int64_t ldx;
    const uint16_t* gate;       // gate form: bf16 [B, H] indexed by indices
    int64_t ld_gate;
    const uint16_t* branch;     // gate form: bf16 [M, H]
    int64_t ld_branch;
    uint16_t* residual_out;     // gate form: bf16 [M, H]
    int64_t ld_res;
    const uint16_t* weight;     // bf16 [H]
    const uint16_t* shift;      // bf16 [B, H]
    int64_t ld_shift;
    const uint16_t* scale;      // bf16 [B, H]
    int64_t ld_scale;
    const void* indices;        // int32 or int64 [M], element stride idx_stride
    int64_t idx_stride;
    int64_t n_index;            // rows of the gate / shift / scale tables
    int idx64;
    int64_t M, H;
    float eps;
    uint8_t* q;                 // e4m3 [M, H]
    int64_t ldq;
    float* qscale;              // fp32 [M]
    uint16_t* h_out;            // optional bf16 [M, H]: the modulated row (the stock producer's output)
    int64_t ldh;
};

__device__ __forceinline__ v4u load16(const uint16_t* row, int64_t c) {
    return *reinterpret_cast<const v4u*>(row + 8 * c);
}

// Wave-wide fp64 sum (xor butterfly; exact for the sums of squares of a bf16 row in all practical cases).
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const int lo = __shfl_xor(__double2loint(v), o, 64), hi = __shfl_xor(__double2hiint(v), o, 64);
        v += __hiloint2double(hi, lo);
    }
    return v;
}

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
__device__ __forceinline__ void store_q(const v4u h[CPL], float inv, uint8_t* qrow, int lane, int64_t nchunk) {
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int64_t c = lane + 64 * j;
        if (c < nchunk)
            reinterpret_cast<uint2*>(qrow)[c] = make_uint2(quant_pairs<FINITE>(h[j][0], h[j][1], inv),
                                                           quant_pairs<FINITE>(h[j][2], h[j][3], inv));
    }
}

template <bool GATE, bool WRITE_H, int CPL>
__global__ void __launch_bounds__(256) rms_mod_quant_kernel(RmsArgs a) {
    const int lane = threadIdx.x & 63;
    const int64_t m = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (m >= a.M) return;
    const int64_t nchunk = a.H >> 3;                   // 16-byte chunks per row
    int64_t i = a.idx64 ? reinterpret_cast<const int64_t*>(a.indices)[m * a.idx_stride]
                        : (int64_t)reinterpret_cast<const int32_t*>(a.indices)[m * a.idx_stride];
    const bool bad = (uint64_t)i >= (uint64_t)a.n_index;
    i = bad ? 0 : i;
    const uint32_t poison = bad ? 0x7fc07fc0u : 0u;     // OR-ed into bf16 pairs: NaN if the index is out of range
    const uint16_t* xr = a.x + m * a.ldx;
    v4u xv[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int64_t c = lane + 64 * j;
        xv[j] = (c < nchunk) ? load16(xr, c) : v4u{0u, 0u, 0u, 0u};
    }
    if (GATE) {
        // u = bf16(residual + gate[i] * branch); residual_out = u; the norm below runs on u
        const uint16_t* gr = a.gate + i * a.ld_gate;
        const uint16_t* br = a.branch + m * a.ld_branch;
        uint16_t* ro = a.residual_out + m * a.ld_res;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int64_t c = lane + 64 * j;
            if (c < nchunk) {
                const v4u gv = load16(gr, c), bv = load16(br, c);
                v4u u;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float r0 = u2f(xv[j][k] << 16), r1 = u2f(xv[j][k] & 0xffff0000u);
                    const float p0 = u2f(gv[k] << 16) * u2f(bv[k] << 16);
                    const float p1 = u2f(gv[k] & 0xffff0000u) * u2f(bv[k] & 0xffff0000u);
                    u[k] = cvt_bf16x2(r0 + p0, r1 + p1) | poison;
                }
                xv[j] = u;
                *reinterpret_cast<v4u*>(ro + 8 * c) = u;
            }
        }
    }
    // sum of squares: each square is exact in fp32, the fp64 sum rounds once to fp32
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < CPL; ++j)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float f0 = u2f(xv[j][k] << 16), f1 = u2f(xv[j][k] & 0xffff0000u);
            ss += (double)(f0 * f0);
            ss += (double)(f1 * f1);
        }
    ss = wave_sum_f64(ss);
    const float hf = (float)a.H;
    float var = (float)ss;
    asm volatile("" : "+v"(var));                       // the division by H stays a division
    var = var / hf;
    const float d = __builtin_sqrtf(var + a.eps);     // correctly rounded (HIP's default fp32 sqrt)
    float one = 1.0f;
    asm volatile("" : "+v"(one));
    const float r = bad ? u2f(0x7fc00000u) : one / d;  // IEEE division (torch's CPU rsqrt: 1 / sqrt)
    // modulation, bf16 rounding, row maximum
    const uint16_t* shr = a.shift + i * a.ld_shift;
    const uint16_t* scr = a.scale + i * a.ld_scale;
    v4u h[CPL];
    uint32_t mx = 0;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int64_t c = lane + 64 * j;
        const bool in = c < nchunk;
        const v4u wv = in ? load16(a.weight, c) : v4u{0u, 0u, 0u, 0u};
        const v4u sh = in ? load16(shr, c) : v4u{0u, 0u, 0u, 0u};
        const v4u sc = in ? load16(scr, c) : v4u{0u, 0u, 0u, 0u};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float o[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const float xe = u2f(e ? (xv[j][k] & 0xffff0000u) : (xv[j][k] << 16));
                const float we = u2f(e ? (wv[k] & 0xffff0000u) : (wv[k] << 16));
                const float se = u2f(e ? (sc[k] & 0xffff0000u) : (sc[k] << 16));
                const float be = u2f(e ? (sh[k] & 0xffff0000u) : (sh[k] << 16));
                const float n = (xe * r) * we;
                const float g = one + se;
                o[e] = n * g + be;
            }
            h[j][k] = in ? cvt_bf16x2(o[0], o[1]) : 0u;   // columns past H: +0, the maximum is unchanged
            const uint32_t lo = (h[j][k] << 16) & 0x7fff0000u, hi = h[j][k] & 0x7fff0000u;
            mx = mx > lo ? mx : lo;
            mx = mx > hi ? mx : hi;
        }
    }
    mx = wave_max_u32(mx);
    const float s = row_scale(u2f(mx));
    const float inv = inv_scale(s);
    uint8_t* qrow = a.q + m * a.ldq;
    if (__builtin_amdgcn_readfirstlane(mx) < 0x7f800000u) store_q<CPL, true>(h, inv, qrow, lane, nchunk);
    else store_q<CPL, false>(h, inv, qrow, lane, nchunk);
    if (WRITE_H) {
        uint16_t* hr = a.h_out + m * a.ldh;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int64_t c = lane + 64 * j;
            if (c < nchunk) *reinterpret_cast<v4u*>(hr + 8 * c) = h[j];
        }
    }
    if (lane == 0) a.qscale[m] = s;
}

template <bool GATE, bool WRITE_H>
int launch_rms(const RmsArgs& a, hipStream_t st) {
    const int64_t cpl = ((a.H >> 3) + 63) / 64;
    dim3 grid((unsigned)((a.M + 3) / 4)), block(256);
#define H3_R(N) hipLaunchKernelGGL((rms_mod_quant_kernel<GATE, WRITE_H, N>), grid, block, 0, st, a)
    if (cpl <= 2) H3_R(2);
    else if (cpl <= 4) H3_R(4);
    else if (cpl <= 6) H3_R(6);
    else if (cpl <= 8) H3_R(8);
    else if (cpl <= 12) H3_R(12);
    else H3_R(16);
#undef H3_R
    H3_CHECK_HIP(hipGetLastError());
    return H3FP8_OK;
}

int check_rows(const void* p, int64_t ld, int64_t H, const char* what, const char* who) {
    H3_REQUIRE(p != nullptr, "%s: null %s", who, what);
    H3_REQUIRE(ld >= H && ld % 8 == 0 && ((uintptr_t)p & 15) == 0,
               "%s: %s rows must be 16-byte aligned with a stride >= H and a multiple of 8", who, what);
    return H3FP8_OK;
}

int check_rms(const RmsArgs& a, bool gate, const char* who) {
    H3_REQUIRE(a.M >= 0 && a.H >= 0, "%s: negative size", who);
    H3_REQUIRE(a.H % 8 == 0 && a.H <= 8192, "%s: H=%lld must be a multiple of 8 and <= 8192", who, (long long)a.H);
    if (a.M == 0 || a.H == 0) return H3FP8_OK;
    int rc = check_rows(a.x, a.ldx, a.H, gate ? "residual" : "x", who);
    if (!rc && gate) rc = check_rows(a.gate, a.ld_gate, a.H, "gate", who);
    if (!rc && gate) rc = check_rows(a.branch, a.ld_branch, a.H, "branch", who);
    if (!rc && gate) rc = check_rows(a.residual_out, a.ld_res, a.H, "residual_out", who);
    if (!rc) rc = check_rows(a.weight, a.H, a.H, "weight", who);
    if (!rc) rc = check_rows(a.shift, a.ld_shift, a.H, "shift", who);
    if (!rc) rc = check_rows(a.scale, a.ld_scale, a.H, "scale", who);
    if (!rc && a.h_out) rc = check_rows(a.h_out, a.ldh, a.H, "h_out", who);
    if (rc) return rc;
    H3_REQUIRE(a.indices && a.idx_stride >= 0 && a.n_index > 0, "%s: bad indices or empty tables", who);
    H3_REQUIRE(a.q && a.qscale && a.ldq >= a.H && a.ldq % 8 == 0 && ((uintptr_t)a.q & 7) == 0,
               "%s: q must be 8-byte aligned with a row stride >= H and a multiple of 8", who);
    return H3FP8_OK;
}

}  // namespace

extern "C" {

int h3fp8_rms_quant(const void* x, int64_t ldx, const void* weight, const void* shift, int64_t ld_shift,
                    const void* scale, int64_t ld_scale, int64_t n_index, const void* indices, int64_t idx_stride,
                    int idx_bytes, int64_t M, int64_t H, float eps, void* q, int64_t ldq, float* qscale, void* h_out,
                    int64_t ldh, void* stream) {
    RmsArgs a{};
    a.x = (const uint16_t*)x; a.ldx = ldx;
    a.weight = (const uint16_t*)weight;
    a.shift = (const uint16_t*)shift; a.ld_shift = ld_shift;
    a.scale = (const uint16_t*)scale; a.ld_scale = ld_scale;
    a.indices = indices; a.idx_stride = idx_stride; a.n_index = n_index; a.idx64 = idx_bytes == 8;
    a.M = M; a.H = H; a.eps = eps;
    a.q = (uint8_t*)q; a.ldq = ldq; a.qscale = qscale;
    a.h_out = (uint16_t*)h_out; a.ldh = ldh;
    H3_REQUIRE(idx_bytes == 4 || idx_bytes == 8, "h3fp8_rms_quant: indices must be int32 or int64");
    int rc = check_rms(a, false, "h3fp8_rms_quant");
    if (rc || M == 0 || H == 0) return rc;
    hipStream_t st = (hipStream_t)stream;
    return h_out ? launch_rms<false, true>(a, st) : launch_rms<false, false>(a, st);
}

int h3fp8_gate_rms_quant(const void* residual, int64_t ldr, const void* gate, int64_t ld_gate, const void* branch,
                         int64_t ld_branch, const void* weight, const void* shift, int64_t ld_shift, const void* scale,
                         int64_t ld_scale, int64_t n_index, const void* indices, int64_t idx_stride, int idx_bytes,
                         int64_t M, int64_t H, float eps, void* residual_out, int64_t ld_res, void* q, int64_t ldq,
                         float* qscale, void* h_out, int64_t ldh, void* stream) {
    RmsArgs a{};
    a.x = (const uint16_t*)residual; a.ldx = ldr;
    a.gate = (const uint16_t*)gate; a.ld_gate = ld_gate;
    a.branch = (const uint16_t*)branch; a.ld_branch = ld_branch;
    a.residual_out = (uint16_t*)residual_out; a.ld_res = ld_res;
    a.weight = (const uint16_t*)weight;
    a.shift = (const uint16_t*)shift; a.ld_shift = ld_shift;
    a.scale = (const uint16_t*)scale; a.ld_scale = ld_scale;
    a.indices = indices; a.idx_stride = idx_stride; a.n_index = n_index; a.idx64 = idx_bytes == 8;
    a.M = M; a.H = H; a.eps = eps;
    a.q = (uint8_t*)q; a.ldq = ldq; a.qscale = qscale;
    a.h_out = (uint16_t*)h_out; a.ldh = ldh;
    H3_REQUIRE(idx_bytes == 4 || idx_bytes == 8, "h3fp8_gate_rms_quant: indices must be int32 or int64");
    int rc = check_rms(a, true, "h3fp8_gate_rms_quant");
    if (rc || M == 0 || H == 0) return rc;
    hipStream_t st = (hipStream_t)stream;
    return h_out ? launch_rms<true, true>(a, st) : launch_rms<true, false>(a, st);
}

}  // extern "C"
