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
// (coalesced 1 KiB per load instruction), the row stays in VGPRs, both reductions are wave shuffles.  Every load is a
// range-checked buffer load (no branches, so all of a row's loads are in flight together): the row's own loads go
// out first, then the index and, up to 8 chunks per lane, every weight / shift / scale chunk before the reduction.
// HBM traffic is 3H + 4 bytes per row (7H + 4 for the gate form); the weight and table rows (3 x 2H bytes per row)
// come from L2.  Staging the tables in LDS per persistent workgroup was measured slower (fewer rows in flight); the
// qkv-site form with 4-8 chunks per lane instead stages them once per 8-row workgroup as fp32 values
// (rms_mod_quant_staged_kernel below).
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
    // the consumer forms: the branch (gate form's third operand) is the scaled-GEMM epilogue of an fp32 product,
    // branch = bf16(sa[m] * (sb[n] * acc[m, n])) or bf16(fma(sa[m], sb[n] * acc[m, n], bias[n]))
    const float* acc;           // fp32 [M, H]
    int64_t ld_acc;
    const float* sa;            // fp32 [M], contiguous
    const float* sb;            // fp32 [H], contiguous
    const uint16_t* bias;       // bf16 [H] or null
};

typedef unsigned int v2u __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// Range-checked 16-byte chunk c of a row described by `r` (chunks past the row's end read as zero, stores there are
// dropped): branch-free, so every load of a wave is in flight at once.
template <int AUX = 0>
__device__ __forceinline__ v4u ld16(__amdgpu_buffer_rsrc_t r, int c) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (uint32_t)c * 16u, 0, AUX);
}
// Row stores are non-temporal: the rows stream through once (measured: the out consumer 178 -> 168 us, the qkv
// producer's bf16 h form unchanged).
__device__ __forceinline__ void st16(v4u v, __amdgpu_buffer_rsrc_t r, int c) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, (uint32_t)c * 16u, 0, 2);
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

// The value lane l + D holds, delivered to lane l for l < D (lanes l >= D receive values of no use): D = 32 and 16
// through gfx950's permlane swaps, 8 and 4 through DPP row shifts, 2 and 1 through DPP quad permutations.
template <int D>
__device__ __forceinline__ uint32_t from_lane_plus(uint32_t x) {
    if constexpr (D == 32) return __builtin_amdgcn_permlane32_swap(x, x, false, false)[1];
    else if constexpr (D == 16) return __builtin_amdgcn_permlane16_swap(x, x, false, false)[1];
    else if constexpr (D == 8) return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x108, 0xf, 0xf, false);
    else if constexpr (D == 4) return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x104, 0xf, 0xf, false);
    else if constexpr (D == 2) return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x4e, 0xf, 0xf, false);
    else return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0xb1, 0xf, 0xf, false);
}
template <int D>
__device__ __forceinline__ double add_from_lane_plus(double v) {
    const uint32_t lo = from_lane_plus<D>((uint32_t)__double2loint(v));
    const uint32_t hi = from_lane_plus<D>((uint32_t)__double2hiint(v));
    return v + __hiloint2double((int)hi, (int)lo);
}
// wave_sum_f64's total as lane 0 computes it, returned wave-uniform: in the xor butterfly with distances 32, 16, ..., 1
// lane 0's result depends at each step only on lanes l < d, whose partner l xor d is l + d, so the lane moves above
// reproduce it bit for bit (register moves instead of LDS permutes: a shorter chain).
__device__ __forceinline__ double wave_sum_f64_l0(double v) {
    v = add_from_lane_plus<32>(v);
    v = add_from_lane_plus<16>(v);
    v = add_from_lane_plus<8>(v);
    v = add_from_lane_plus<4>(v);
    v = add_from_lane_plus<2>(v);
    v = add_from_lane_plus<1>(v);
    return __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(v), 0),
                            __builtin_amdgcn_readlane(__double2loint(v), 0));
}
// Wave-wide unsigned maximum through the same lane moves, returned wave-uniform.
__device__ __forceinline__ uint32_t wave_max_u32_l0(uint32_t v) {
    uint32_t w;
    w = from_lane_plus<32>(v); v = v > w ? v : w;
    w = from_lane_plus<16>(v); v = v > w ? v : w;
    w = from_lane_plus<8>(v); v = v > w ? v : w;
    w = from_lane_plus<4>(v); v = v > w ? v : w;
    w = from_lane_plus<2>(v); v = v > w ? v : w;
    w = from_lane_plus<1>(v); v = v > w ? v : w;
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
}
// max(m, |a|, |b|), NaN-propagating (IEEE maximum): one v_maximum3_f32 per pair (as a builtin the compiler rebuilds
// the chain as a tree of more instructions).
__device__ __forceinline__ float max_abs3(float m, float a, float b) {
    float r;
    asm("v_maximum3_f32 %0, %1, |%2|, |%3|" : "=v"(r) : "v"(m), "v"(a), "v"(b));
    return r;
}

// The clamp to [-448, 448].  On a row whose maximum is finite it never changes the code: |h| <= amax, scale =
// RNE(amax / 448) (or the floor, which only makes it larger), inv = RNE(1 / scale), so |h * inv| <= 448 (1 + 2^-24)^3
// < 448.0001, and the conversion rounds everything below 464 (the midpoint to the next binade's 480, which e4m3fn
// lacks) to 448 -- so the finite path converts without it.  Rows with inf or NaN keep the compare / select form
// (NaN propagates, +-inf saturates).
template <bool FINITE>
__device__ __forceinline__ float clamp448(float y) {
    if (FINITE) return y;
    y = (y < -H3_FP8_MAX) ? -H3_FP8_MAX : y;
    return (y > H3_FP8_MAX) ? H3_FP8_MAX : y;
}

template <bool FINITE>
__device__ __forceinline__ uint32_t quant_pairs(uint32_t p0, uint32_t p1, float inv) {
    return e4m3x4(clamp448<FINITE>(u2f(p0 << 16) * inv), clamp448<FINITE>(u2f(p0 & 0xffff0000u) * inv),
                  clamp448<FINITE>(u2f(p1 << 16) * inv), clamp448<FINITE>(u2f(p1 & 0xffff0000u) * inv));
}

template <int CPL, bool FINITE>
__device__ __forceinline__ void store_q(const v4u h[CPL], float inv, __amdgpu_buffer_rsrc_t qr, int lane) {
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const v2u v = {quant_pairs<FINITE>(h[j][0], h[j][1], inv), quant_pairs<FINITE>(h[j][2], h[j][3], inv)};
        __builtin_amdgcn_raw_buffer_store_b64(v, qr, (uint32_t)(lane + 64 * j) * 8u, 0, 0);
    }
}

// Where the weight / shift / scale / gate chunks of a row come from: range-checked buffer loads of the table rows
// (L2-resident after first use).
struct GlobalTables {
    __amdgpu_buffer_rsrc_t w, sh, sc, g;
};
__device__ __forceinline__ v4u tab16(const GlobalTables& t, int which, int c) {
    return ld16(which == 0 ? t.w : which == 1 ? t.sh : which == 2 ? t.sc : t.g, c);
}
// One row m processed by one wave.  OUT: bit 0 = the e4m3 row and its scale, bit 1 = the bf16 modulated row (h only:
// the stock producer itself).  EARLY: every table chunk is fetched together with the row (their latency overlaps the
// row's instead of following the reduction); above 8 chunks per lane (6 for the fp32-branch form) the registers do
// not allow it.
// `tables(bad)` returns the row's table source and sets `bad` (index out of range); it is called after the row's own
// loads are issued, so the table loads that depend on the index overlap the row's latency.
//
// B32 (gate form only): the branch is the scaled-GEMM epilogue of the fp32 product `acc` (the consumer of the out
// projection reading the accumulator instead of a bf16 output).
//
// FULL: H == 512 CPL, every chunk of every lane lies in the row (no masking of the chunks past its end).
template <bool GATE, int OUT, int CPL, bool EARLY, bool B32, bool FULL, class MakeTables>
__device__ __forceinline__ void rms_mod_quant_row(const RmsArgs& a, int64_t m, int lane, MakeTables tables) {
    constexpr bool QUANT = (OUT & 1) != 0, WRITE_H = (OUT & 2) != 0;
    const uint32_t rb = (uint32_t)a.H * 2u;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x + m * a.ldx, rb);
    v4u xv[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) xv[j] = ld16<2>(xr, lane + 64 * j);     // streamed once: non-temporal
    v4u gv[GATE ? CPL : 1], bv[GATE ? CPL : 1];
    constexpr int NB = B32 ? CPL : 1;
    v4u a_lo[NB], a_hi[NB], s_lo[NB], s_hi[NB], b_e[NB];
    if (GATE && !B32) {
        const __amdgpu_buffer_rsrc_t br = make_rsrc(a.branch + m * a.ld_branch, rb);
#pragma unroll
        for (int j = 0; j < (GATE ? CPL : 1); ++j) bv[j] = ld16<2>(br, lane + 64 * j);
    }
    if (GATE && B32) {
        const __amdgpu_buffer_rsrc_t ar = make_rsrc(a.acc + m * a.ld_acc, 2u * rb);
        const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.sb, 2u * rb);
        const __amdgpu_buffer_rsrc_t bsr = make_rsrc(a.bias ? a.bias : a.weight, a.bias ? rb : 0u);
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const uint32_t c = (uint32_t)(lane + 64 * j);
            a_lo[j] = __builtin_amdgcn_raw_buffer_load_b128(ar, c * 32u, 0, 2);
            a_hi[j] = __builtin_amdgcn_raw_buffer_load_b128(ar, c * 32u + 16u, 0, 2);
            s_lo[j] = __builtin_amdgcn_raw_buffer_load_b128(sr, c * 32u, 0, 0);
            s_hi[j] = __builtin_amdgcn_raw_buffer_load_b128(sr, c * 32u + 16u, 0, 0);
            b_e[j] = __builtin_amdgcn_raw_buffer_load_b128(bsr, c * 16u, 0, 0);   // zeros without a bias
        }
    }
    __builtin_amdgcn_sched_barrier(0);                  // the row's loads go out before the index load
    bool bad;
    const auto t = tables(bad);
    const uint32_t poison = bad ? 0x7fc07fc0u : 0u;     // OR-ed into bf16 pairs: NaN if the index is out of range
    if (GATE) {
#pragma unroll
        for (int j = 0; j < (GATE ? CPL : 1); ++j) gv[j] = tab16(t, 3, lane + 64 * j);
    }
    constexpr int NE = EARLY ? CPL : 1;
    v4u wv_e[NE], sh_e[NE], sc_e[NE];
    if (EARLY) {
#pragma unroll
        for (int j = 0; j < NE; ++j) {
            wv_e[j] = tab16(t, 0, lane + 64 * j);
            sh_e[j] = tab16(t, 1, lane + 64 * j);
            sc_e[j] = tab16(t, 2, lane + 64 * j);
        }
    }
    __builtin_amdgcn_sched_barrier(0);                  // keep every load above the reduction
    const int nchunk = (int)(a.H >> 3);
    if (GATE && B32) {
        // branch = bf16(epilogue(acc)): t = sb * acc, then sa * t or fma(sa, t, bias), one rounding (the scale pass)
        const float sam = a.sa[m];
        const bool hb = a.bias != nullptr;
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            float y[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float acc = u2f(e < 4 ? a_lo[j][e] : a_hi[j][e - 4]);
                const float sbn = u2f(e < 4 ? s_lo[j][e] : s_hi[j][e - 4]);
                const uint32_t bw = b_e[j][e >> 1];
                const float b = u2f((e & 1) ? (bw & 0xffff0000u) : (bw << 16));
                const float t = sbn * acc;
                y[e] = hb ? __builtin_fmaf(sam, t, b) : sam * t;
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) bv[j][k] = cvt_bf16x2(y[2 * k], y[2 * k + 1]);
        }
    }
    if (GATE) {
        // u = bf16(residual + gate[i] * branch); residual_out = u; the norm below runs on u.  Chunks past the row are
        // forced to +0 (their stores are dropped).
        const __amdgpu_buffer_rsrc_t ro = make_rsrc(a.residual_out + m * a.ld_res, rb);
#pragma unroll
        for (int j = 0; j < (GATE ? CPL : 1); ++j) {
            const bool in = FULL || lane + 64 * j < nchunk;
            v4u u;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float r0 = u2f(xv[j][k] << 16), r1 = u2f(xv[j][k] & 0xffff0000u);
                const float p0 = u2f(gv[j][k] << 16) * u2f(bv[j][k] << 16);
                const float p1 = u2f(gv[j][k] & 0xffff0000u) * u2f(bv[j][k] & 0xffff0000u);
                u[k] = in ? (cvt_bf16x2(r0 + p0, r1 + p1) | poison) : 0u;
            }
            xv[j] = u;
            st16(u, ro, lane + 64 * j);
        }
    }
    // sum of squares: each square is exact in fp32, the fp64 sum rounds once to fp32 (chunks past the row add +0;
    // a poisoned row's NaN makes the sum NaN)
    double ss = 0.0;
    float xf[CPL][8];                                   // the row in fp32, kept for the modulation
#pragma unroll
    for (int j = 0; j < CPL; ++j)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float f0 = u2f(xv[j][k] << 16), f1 = u2f(xv[j][k] & 0xffff0000u);
            xf[j][2 * k] = f0;
            xf[j][2 * k + 1] = f1;
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
    // modulation, bf16 rounding, row maximum (of the packed |h| pairs, two 16-bit lanes at a time; NaN patterns order
    // above +inf)
    v4u h[CPL];
    u16x2 mx2 = {0, 0};
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const bool in = FULL || lane + 64 * j < nchunk;
        const v4u wv = EARLY ? wv_e[EARLY ? j : 0] : tab16(t, 0, lane + 64 * j);
        const v4u sh = EARLY ? sh_e[EARLY ? j : 0] : tab16(t, 1, lane + 64 * j);
        const v4u sc = EARLY ? sc_e[EARLY ? j : 0] : tab16(t, 2, lane + 64 * j);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float o[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const float xe = xf[j][2 * k + e];
                const float we = u2f(e ? (wv[k] & 0xffff0000u) : (wv[k] << 16));
                const float se = u2f(e ? (sc[k] & 0xffff0000u) : (sc[k] << 16));
                const float be = u2f(e ? (sh[k] & 0xffff0000u) : (sh[k] << 16));
                const float n = (xe * r) * we;
                const float g = one + se;
                o[e] = n * g + be;
            }
            h[j][k] = in ? cvt_bf16x2(o[0], o[1]) : 0u;   // chunks past the row: +0, the maximum is unchanged
            mx2 = __builtin_elementwise_max(mx2, __builtin_bit_cast(u16x2, h[j][k] & 0x7fff7fffu));
        }
    }
    uint32_t mx = (uint32_t)(mx2[0] > mx2[1] ? mx2[0] : mx2[1]) << 16;   // as fp32 bits
    float s = 0.0f;
    if (QUANT) {
        mx = wave_max_u32(mx);
        s = row_scale(u2f(mx));
        const float inv = inv_scale(s);
        const __amdgpu_buffer_rsrc_t qr = make_rsrc(a.q + m * a.ldq, (uint32_t)a.H);
        if (__builtin_amdgcn_readfirstlane(mx) < 0x7f800000u) store_q<CPL, true>(h, inv, qr, lane);
        else store_q<CPL, false>(h, inv, qr, lane);
    }
    if (WRITE_H) {
        const __amdgpu_buffer_rsrc_t hr = make_rsrc(a.h_out + m * a.ldh, rb);
#pragma unroll
        for (int j = 0; j < CPL; ++j) st16(h[j], hr, lane + 64 * j);
    }
    if (QUANT && lane == 0) a.qscale[m] = s;
}

__device__ __forceinline__ int64_t row_index(const RmsArgs& a, int64_t m, bool& bad) {
    int64_t i = a.idx64 ? reinterpret_cast<const int64_t*>(a.indices)[m * a.idx_stride]
                        : (int64_t)reinterpret_cast<const int32_t*>(a.indices)[m * a.idx_stride];
    bad = (uint64_t)i >= (uint64_t)a.n_index;
    return bad ? 0 : i;
}

// Tables read from global memory: one wave per row, 4 rows per 256-thread workgroup.
template <bool GATE, int OUT, int CPL, bool B32, bool FULL>
__global__ void __launch_bounds__(256) rms_mod_quant_kernel(RmsArgs a) {
    const int lane = threadIdx.x & 63;
    const int64_t m = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (m >= a.M) return;
    // the row's index is read first (a scalar load): its latency then overlaps the issue of the row's own loads
    bool bad0;
    const int64_t i0 = row_index(a, m, bad0);
    rms_mod_quant_row<GATE, OUT, CPL, (CPL <= 6 || (CPL <= 8 && !B32)), B32, FULL>(a, m, lane, [&](bool& bad) {
        bad = bad0;
        const int64_t i = i0;
        const uint32_t rb = (uint32_t)a.H * 2u;
        GlobalTables t;
        t.w = make_rsrc(a.weight, rb);
        t.sh = make_rsrc(a.shift + i * a.ld_shift, rb);
        t.sc = make_rsrc(a.scale + i * a.ld_scale, rb);
        t.g = make_rsrc(GATE ? a.gate + i * a.ld_gate : a.weight, rb);
        return t;
    });
}

// The producers and the out consumer with their tables staged in LDS as fp32: one wave per row, eight rows per
// workgroup for the gated forms and four for the qkv producer (measured: with eight rows its index-run case took
// 2 % and its random-index case 14 % longer, and the out consumer 14 % longer with four).  The modulation tables
// have one row per sample, so nearly every workgroup's rows share one index: the workgroup converts once into fp32
// LDS tables the weight row, 1 + scale and shift of its first row's index, and for the gated forms gate of that
// index, for the fp32-branch form sb and the bias (the same fp32 values the per-element arithmetic forms: bf16 ->
// fp32 is exact, 1 + scale the same fp32 add).  A wave whose row has that index reads every table there at the point
// of use -- unpacks and an add fewer per element, and no table chunk held in registers.  A wave whose row has another
// index (a sample boundary inside the workgroup, or an index outside the tables) reads the index-dependent tables
// (gate, scale, shift) from global memory a few chunks at a time.  Arithmetic and order otherwise as
// rms_mod_quant_row, so the outputs are bitwise the same; the two wave reductions run on lane moves (permlane swaps
// and DPP, lane 0's butterfly) and the row maximum on v_maximum3_f32 of the fp32 values before their bf16 rounding
// (measured at the qkv site, M = 16 740: 33.4 -> 32.2 us; the register form above measured 1 % slower with them).
// LDS: table t, half s (elements 0-3 / 4-7 of a chunk), chunk c: tabs[t][s][c] (float4), so a wave's 16-byte reads
// of one half are contiguous (no bank conflicts).  Tables: T_W weight, T_G 1 + scale, T_B shift, T_GATE gate,
// T_SB sb, T_BIAS bias (zeros without one).
template <bool GATE>
constexpr int staged_rows() { return GATE ? 8 : 4; }

template <bool GATE, bool B32, int OUT, int CPL, bool FULL>
__global__ void __launch_bounds__(64 * staged_rows<GATE>()) rms_mod_quant_staged_kernel(RmsArgs a) {
    constexpr bool QUANT = (OUT & 1) != 0, WRITE_H = (OUT & 2) != 0;
    constexpr int ROWS = staged_rows<GATE>(), THREADS = 64 * ROWS;
    constexpr int NC = 64 * CPL;                        // 16-byte bf16 chunks per table row (past H: zeros)
    static_assert(NC <= 2 * THREADS, "at most two staging loads per thread and table");
    static_assert(GATE || !B32, "the fp32 branch belongs to the gated form");
    constexpr int T_W = 0, T_G = 1, T_B = 2, T_GATE = 3, T_SB = GATE ? 4 : 3, T_BIAS = T_SB + 1;
    // a wave off the staged index loads its tables in groups of FB_GROUP chunks (one chunk at a time for the qkv
    // form: grouped, its index-run case measured 3 % slower; the out consumer gains 2-3 % with groups of 3)
    constexpr int FB_GROUP = GATE ? 3 : 1;
    constexpr int NT = 3 + (GATE ? 1 : 0) + (B32 ? 2 : 0);
    __shared__ v4f tabs[NT][2][NC];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t m0 = (int64_t)blockIdx.x * ROWS, m = m0 + wave;
    const bool live = m < a.M;
    const int64_t mr = live ? m : m0;                   // a row past M reads and writes nothing (empty ranges)
    // the indices first (scalar loads), then the row's own loads, then the staging loads
    bool bad, bad0;
    const int64_t i = row_index(a, mr, bad);
    const int64_t i0 = row_index(a, m0, bad0);
    const uint32_t rb = (uint32_t)a.H * 2u;
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x + mr * a.ldx, live ? rb : 0u);
    v4u xv[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) xv[j] = ld16<2>(xr, lane + 64 * j);     // streamed once: non-temporal
    v4u bv[GATE ? CPL : 1];
    constexpr int NB = B32 ? CPL : 1;
    v4u a_lo[NB], a_hi[NB];
    if (GATE && !B32) {
        const __amdgpu_buffer_rsrc_t br = make_rsrc(a.branch + mr * a.ld_branch, live ? rb : 0u);
#pragma unroll
        for (int j = 0; j < (GATE ? CPL : 1); ++j) bv[j] = ld16<2>(br, lane + 64 * j);
    }
    if (B32) {
        const __amdgpu_buffer_rsrc_t ar = make_rsrc(a.acc + mr * a.ld_acc, live ? 2u * rb : 0u);
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const uint32_t c = (uint32_t)(lane + 64 * j);
            a_lo[j] = __builtin_amdgcn_raw_buffer_load_b128(ar, c * 32u, 0, 2);
            a_hi[j] = __builtin_amdgcn_raw_buffer_load_b128(ar, c * 32u + 16u, 0, 2);
        }
    }
    for (int t0 = tid; t0 < NC; t0 += THREADS) {         // wave-uniform (NC is a multiple of 64)
        auto put = [&](int t, v4u v, bool one_plus) {   // a bf16 chunk as two fp32 halves
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                v4f f;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t w = v[2 * s + (e >> 1)];
                    const float x = u2f((e & 1) ? (w & 0xffff0000u) : (w << 16));
                    f[e] = one_plus ? 1.0f + x : x;
                }
                tabs[t][s][t0] = f;
            }
        };
        const v4u w = ld16(make_rsrc(a.weight, rb), t0);
        const v4u sc = ld16(make_rsrc(a.scale + i0 * a.ld_scale, rb), t0);
        const v4u sh = ld16(make_rsrc(a.shift + i0 * a.ld_shift, rb), t0);
        v4u gt = {0, 0, 0, 0}, sbl = {0, 0, 0, 0}, sbh = {0, 0, 0, 0}, bs = {0, 0, 0, 0};
        if (GATE) gt = ld16(make_rsrc(a.gate + i0 * a.ld_gate, rb), t0);
        if (B32) {
            const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.sb, 2u * rb);
            sbl = __builtin_amdgcn_raw_buffer_load_b128(sr, (uint32_t)t0 * 32u, 0, 0);
            sbh = __builtin_amdgcn_raw_buffer_load_b128(sr, (uint32_t)t0 * 32u + 16u, 0, 0);
            bs = ld16(make_rsrc(a.bias ? (const void*)a.bias : (const void*)a.weight, a.bias ? rb : 0u), t0);
        }
        put(T_W, w, false);
        put(T_G, sc, true);
        put(T_B, sh, false);
        if (GATE) put(T_GATE, gt, false);
        if (B32) {
            tabs[T_SB][0][t0] = __builtin_bit_cast(v4f, sbl);
            tabs[T_SB][1][t0] = __builtin_bit_cast(v4f, sbh);
            put(T_BIAS, bs, false);
        }
    }
    __syncthreads();
    if (!live) return;
    const bool staged = !bad && i == i0;                // wave-uniform
    const int nchunk = (int)(a.H >> 3);
    // the index-dependent tables of a wave off the staged index
    const __amdgpu_buffer_rsrc_t gsc = make_rsrc(a.scale + i * a.ld_scale, rb);
    const __amdgpu_buffer_rsrc_t gsh = make_rsrc(a.shift + i * a.ld_shift, rb);
    const __amdgpu_buffer_rsrc_t ggt = make_rsrc(GATE ? a.gate + i * a.ld_gate : a.weight, rb);
    if (GATE) {
        // branch: the bf16 input, or bf16(epilogue(acc)) (t = sb * acc, then sa * t or fma(sa, t, bias), one
        // rounding); u = bf16(residual + gate[i] * branch); residual_out = u; the norm below runs on u.  Chunks past
        // the row are forced to +0 (their stores are dropped); an index outside the tables makes u NaN.
        const uint32_t poison = bad ? 0x7fc07fc0u : 0u;
        const float sam = B32 ? a.sa[m] : 0.0f;
        const bool hb = a.bias != nullptr;
        const __amdgpu_buffer_rsrc_t ro = make_rsrc(a.residual_out + m * a.ld_res, rb);
        v4u gtg[FB_GROUP] = {};
#pragma unroll
        for (int j = 0; j < (GATE ? CPL : 1); ++j) {
            const int c = lane + 64 * j;
            const bool in = FULL || c < nchunk;
            if (B32) {
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    const v4f sbn = tabs[T_SB][s][c], bn = tabs[T_BIAS][s][c];
                    float y[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float acc = u2f(s ? a_hi[B32 ? j : 0][e] : a_lo[B32 ? j : 0][e]);
                        const float t = sbn[e] * acc;
                        y[e] = hb ? __builtin_fmaf(sam, t, bn[e]) : sam * t;
                    }
                    bv[j][2 * s] = cvt_bf16x2(y[0], y[1]);
                    bv[j][2 * s + 1] = cvt_bf16x2(y[2], y[3]);
                }
            }
            if (!staged && j % FB_GROUP == 0) {
                asm volatile("" ::: "memory");        // a group's gate loads are not hoisted above here
#pragma unroll
                for (int u = 0; u < FB_GROUP; ++u)
                    if (j + u < CPL) gtg[u] = ld16(ggt, c + 64 * u);
            }
            const v4u gchunk = gtg[j % FB_GROUP];
            v4u u;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                float g0, g1;
                if (staged) {
                    const v4f gf = tabs[T_GATE][k >> 1][c];
                    g0 = gf[2 * (k & 1)];
                    g1 = gf[2 * (k & 1) + 1];
                } else {
                    g0 = u2f(gchunk[k] << 16);
                    g1 = u2f(gchunk[k] & 0xffff0000u);
                }
                const float r0 = u2f(xv[j][k] << 16), r1 = u2f(xv[j][k] & 0xffff0000u);
                const float p0 = g0 * u2f(bv[j][k] << 16);
                const float p1 = g1 * u2f(bv[j][k] & 0xffff0000u);
                u[k] = in ? (cvt_bf16x2(r0 + p0, r1 + p1) | poison) : 0u;
            }
            xv[j] = u;
            st16(u, ro, c);
        }
    }
    // sum of squares: each square exact in fp32, the fp64 sum in lane order, rounded once to fp32
    double ss = 0.0;
    float xf[CPL][8];
#pragma unroll
    for (int j = 0; j < CPL; ++j)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float f0 = u2f(xv[j][k] << 16), f1 = u2f(xv[j][k] & 0xffff0000u);
            xf[j][2 * k] = f0;
            xf[j][2 * k + 1] = f1;
            ss += (double)(f0 * f0);
            ss += (double)(f1 * f1);
        }
    ss = wave_sum_f64_l0(ss);
    const float hf = (float)a.H;
    float var = (float)ss;
    asm volatile("" : "+v"(var));                       // the division by H stays a division
    var = var / hf;
    const float d = __builtin_sqrtf(var + a.eps);
    float one = 1.0f;
    asm volatile("" : "+v"(one));
    const float r = bad ? u2f(0x7fc00000u) : one / d;
    v4u h[CPL];
    float am = 0.0f;                                    // max |o| of the lane (NaN-propagating)
    if (staged) {
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = lane + 64 * j;
            const bool in = FULL || c < nchunk;
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const v4f wf = tabs[T_W][s][c], gf = tabs[T_G][s][c], bf = tabs[T_B][s][c];
                float o[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float n = (xf[j][4 * s + e] * r) * wf[e];
                    o[e] = n * gf[e] + bf[e];
                }
                h[j][2 * s] = in ? cvt_bf16x2(o[0], o[1]) : 0u;
                h[j][2 * s + 1] = in ? cvt_bf16x2(o[2], o[3]) : 0u;
                am = in ? max_abs3(max_abs3(am, o[0], o[1]), o[2], o[3]) : am;
            }
        }
    } else {
        v4u scg[FB_GROUP], shg[FB_GROUP];
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int c = lane + 64 * j;
            const bool in = FULL || c < nchunk;
            if (j % FB_GROUP == 0) {
                asm volatile("" ::: "memory");        // a group's table loads are not hoisted above here
#pragma unroll
                for (int u = 0; u < FB_GROUP; ++u)
                    if (j + u < CPL) {
                        scg[u] = ld16(gsc, c + 64 * u);
                        shg[u] = ld16(gsh, c + 64 * u);
                    }
            }
            const v4u sc = scg[j % FB_GROUP], sh = shg[j % FB_GROUP];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const v4f wf = tabs[T_W][k >> 1][c];
                float o[2];
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const float we = wf[2 * (k & 1) + e];
                    const float se = u2f(e ? (sc[k] & 0xffff0000u) : (sc[k] << 16));
                    const float be = u2f(e ? (sh[k] & 0xffff0000u) : (sh[k] << 16));
                    const float n = (xf[j][2 * k + e] * r) * we;
                    const float g = one + se;
                    o[e] = n * g + be;
                }
                h[j][k] = in ? cvt_bf16x2(o[0], o[1]) : 0u;
                am = in ? max_abs3(am, o[0], o[1]) : am;
            }
        }
    }
    // the row maximum of |h| = bf16(max |o|) (the bf16 rounding is monotone; NaN stays NaN), as fp32 bits
    uint32_t mx = f2u(am) & 0x7fffffffu;
    float s = 0.0f;
    if (QUANT) {
        mx = (cvt_bf16x2(u2f(wave_max_u32_l0(mx)), 0.0f) & 0xffffu) << 16;
        s = row_scale(u2f(mx));
        const float inv = inv_scale(s);
        const __amdgpu_buffer_rsrc_t qr = make_rsrc(a.q + m * a.ldq, (uint32_t)a.H);
        if (__builtin_amdgcn_readfirstlane(mx) < 0x7f800000u) store_q<CPL, true>(h, inv, qr, lane);
        else store_q<CPL, false>(h, inv, qr, lane);
    }
    if (WRITE_H) {
        const __amdgpu_buffer_rsrc_t hr = make_rsrc(a.h_out + m * a.ldh, rb);
#pragma unroll
        for (int j = 0; j < CPL; ++j) st16(h[j], hr, lane + 64 * j);
    }
    if (QUANT && lane == 0) a.qscale[m] = s;
}

template <bool GATE, int OUT, int CPL, bool B32>
int launch_rms_cpl(const RmsArgs& a, hipStream_t st) {
    const dim3 grid((unsigned)((a.M + 3) / 4)), block(256);
    if (a.H == 512 * CPL)
        hipLaunchKernelGGL((rms_mod_quant_kernel<GATE, OUT, CPL, B32, true>), grid, block, 0, st, a);
    else
        hipLaunchKernelGGL((rms_mod_quant_kernel<GATE, OUT, CPL, B32, false>), grid, block, 0, st, a);
    H3_CHECK_HIP(hipGetLastError());
    return H3FP8_OK;
}

template <bool GATE, bool B32, int OUT, int CPL>
int launch_rms_staged(const RmsArgs& a, hipStream_t st) {
    constexpr int rows = staged_rows<GATE>();
    const dim3 grid((unsigned)((a.M + rows - 1) / rows)), block(64 * rows);
    if (a.H == 512 * CPL)
        hipLaunchKernelGGL((rms_mod_quant_staged_kernel<GATE, B32, OUT, CPL, true>), grid, block, 0, st, a);
    else
        hipLaunchKernelGGL((rms_mod_quant_staged_kernel<GATE, B32, OUT, CPL, false>), grid, block, 0, st, a);
    H3_CHECK_HIP(hipGetLastError());
    return H3FP8_OK;
}

template <bool GATE, int OUT, bool B32 = false>
int launch_rms(const RmsArgs& a, hipStream_t st) {
    const int64_t cpl = ((a.H >> 3) + 63) / 64;
    // the staged form for the qkv producer and the out consumer; the fc1 producer (bf16 branch) measured slower
    // with it (109 -> 121 us at 1344x768: its own HBM stream already fills the time)
    if constexpr (!GATE || B32) {
        if (cpl > 2 && cpl <= 4) return launch_rms_staged<GATE, B32, OUT, 4>(a, st);
        if (cpl > 4 && cpl <= 6) return launch_rms_staged<GATE, B32, OUT, 6>(a, st);
        if (cpl > 6 && cpl <= 8) return launch_rms_staged<GATE, B32, OUT, 8>(a, st);
    }
    if (cpl <= 2) return launch_rms_cpl<GATE, OUT, 2, B32>(a, st);
    if (cpl <= 4) return launch_rms_cpl<GATE, OUT, 4, B32>(a, st);
    if (cpl <= 6) return launch_rms_cpl<GATE, OUT, 6, B32>(a, st);
    if (cpl <= 8) return launch_rms_cpl<GATE, OUT, 8, B32>(a, st);
    if (cpl <= 12) return launch_rms_cpl<GATE, OUT, 12, B32>(a, st);
    return launch_rms_cpl<GATE, OUT, 16, B32>(a, st);
}

int check_rows(const void* p, int64_t ld, int64_t H, const char* what, const char* who) {
    H3_REQUIRE(p != nullptr, "%s: null %s", who, what);
    H3_REQUIRE(ld >= H && ld % 8 == 0 && ((uintptr_t)p & 15) == 0,
               "%s: %s rows must be 16-byte aligned with a stride >= H and a multiple of 8", who, what);
    return H3FP8_OK;
}

// gate: the gated forms; b32: the branch is an fp32 product; norm: the RMSNorm + modulation (+ quant) follows.
int check_rms(const RmsArgs& a, bool gate, bool b32, bool norm, const char* who) {
    H3_REQUIRE(a.M >= 0 && a.H >= 0, "%s: negative size", who);
    H3_REQUIRE(a.H % 8 == 0 && a.H <= 8192, "%s: H=%lld must be a multiple of 8 and <= 8192", who, (long long)a.H);
    if (a.M == 0 || a.H == 0) return H3FP8_OK;
    int rc = check_rows(a.x, a.ldx, a.H, gate ? "residual" : "x", who);
    if (!rc && gate) rc = check_rows(a.gate, a.ld_gate, a.H, "gate", who);
    if (!rc && gate && !b32) rc = check_rows(a.branch, a.ld_branch, a.H, "branch", who);
    if (!rc && gate) rc = check_rows(a.residual_out, a.ld_res, a.H, gate && norm ? "residual_out" : "out", who);
    if (!rc && norm) rc = check_rows(a.weight, a.H, a.H, "weight", who);
    if (!rc && norm) rc = check_rows(a.shift, a.ld_shift, a.H, "shift", who);
    if (!rc && norm) rc = check_rows(a.scale, a.ld_scale, a.H, "scale", who);
    if (!rc && a.h_out) rc = check_rows(a.h_out, a.ldh, a.H, "h_out", who);
    if (rc) return rc;
    if (b32) {
        H3_REQUIRE(a.acc && a.sa && a.sb && a.ld_acc >= a.H && a.ld_acc % 4 == 0 && ((uintptr_t)a.acc & 15) == 0 &&
                       ((uintptr_t)a.sb & 15) == 0 && ((uintptr_t)a.bias & 15) == 0,
                   "%s: the fp32 product rows and sb must be 16-byte aligned (row stride a multiple of 4 >= H), "
                   "bias 16-byte aligned, sa / sb given", who);
        H3_REQUIRE((uint64_t)a.H * 4 <= 0xffffffffull, "%s: row too wide", who);
    }
    H3_REQUIRE(a.indices && a.idx_stride >= 0 && a.n_index > 0, "%s: bad indices or empty tables", who);
    if (!norm) return H3FP8_OK;
    H3_REQUIRE(a.q || a.h_out, "%s: neither q nor h_out given", who);
    if (a.q)
        H3_REQUIRE(a.qscale && a.ldq >= a.H && a.ldq % 8 == 0 && ((uintptr_t)a.q & 7) == 0,
                   "%s: q must be 8-byte aligned with a row stride >= H and a multiple of 8, with a scale vector", who);
    return H3FP8_OK;
}

// indexed_gate of the fc2 site reading the fp32 product: out = bf16(x + gate[i] * branch), branch = the scale pass's
// bf16(sa * (sb * acc)) (or its fma with the bias) -- elementwise, so no row needs to stay in registers.  Block (b, s)
// covers U * 256 groups of 4 columns of rows 2b and 2b + 1, thread t the groups t + 256 u (coalesced per u); the two
// rows share the segment's sb / bias loads.  Every access is a range-checked buffer load or store (groups past the
// row, and a second row past M, read zero; stores past the row are dropped); the two indices are read first, the gate
// rows' loads go out after the rows' own.  An index outside the table reads gate row 0 and writes NaN.
template <int U>
__global__ void __launch_bounds__(256) scale_indexed_gate_seg_kernel(RmsArgs a) {
    constexpr int R = 2;
    const int64_t m0 = (int64_t)blockIdx.x * R;
    const uint32_t g0 = blockIdx.y * (256u * U) + threadIdx.x;
    const uint32_t H = (uint32_t)a.H;
    bool bad[R];
    int64_t idx[R];
#pragma unroll
    for (int r = 0; r < R; ++r) idx[r] = row_index(a, m0 + r < a.M ? m0 + r : m0, bad[r]);   // scalar loads first
    const __amdgpu_buffer_rsrc_t sr = make_rsrc(a.sb, H * 4u);
    const bool hb = a.bias != nullptr;
    const __amdgpu_buffer_rsrc_t br = make_rsrc(hb ? (const void*)a.bias : (const void*)a.sb, hb ? H * 2u : 0u);
    v4u av[R][U], sv[U];
    v2u bv[U], xv[R][U], gv[R][U];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const bool in = m0 + r < a.M;
        const int64_t m = in ? m0 + r : m0;
        const __amdgpu_buffer_rsrc_t ar = make_rsrc(a.acc + m * a.ld_acc, in ? H * 4u : 0u);
        const __amdgpu_buffer_rsrc_t xr = make_rsrc(a.x + m * a.ldx, in ? H * 2u : 0u);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t g = g0 + 256u * u;
            av[r][u] = __builtin_amdgcn_raw_buffer_load_b128(ar, g * 16u, 0, 2);    // streamed once: non-temporal
            xv[r][u] = __builtin_amdgcn_raw_buffer_load_b64(xr, g * 8u, 0, 2);
        }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t g = g0 + 256u * u;
        sv[u] = __builtin_amdgcn_raw_buffer_load_b128(sr, g * 16u, 0, 0);
        bv[u] = __builtin_amdgcn_raw_buffer_load_b64(br, g * 8u, 0, 0);       // zeros without a bias
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const __amdgpu_buffer_rsrc_t gr = make_rsrc(a.gate + idx[r] * a.ld_gate, H * 2u);
#pragma unroll
        for (int u = 0; u < U; ++u) gv[r][u] = __builtin_amdgcn_raw_buffer_load_b64(gr, (g0 + 256u * u) * 8u, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t m = m0 + r;
        if (m >= a.M) break;
        const uint32_t poison = bad[r] ? 0x7fc07fc0u : 0u;
        const float sam = a.sa[m];
        const __amdgpu_buffer_rsrc_t orr = make_rsrc(a.residual_out + m * a.ld_res, H * 2u);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            v2u o;
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                float y[2];
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const float t = u2f(sv[u][2 * k + e]) * u2f(av[r][u][2 * k + e]);
                    const float b = u2f(e ? (bv[u][k] & 0xffff0000u) : (bv[u][k] << 16));
                    y[e] = hb ? __builtin_fmaf(sam, t, b) : sam * t;
                }
                const uint32_t br2 = cvt_bf16x2(y[0], y[1]);                   // the scale pass's rounding
                const float p0 = u2f(gv[r][u][k] << 16) * u2f(br2 << 16);
                const float p1 = u2f(gv[r][u][k] & 0xffff0000u) * u2f(br2 & 0xffff0000u);
                o[k] = cvt_bf16x2(u2f(xv[r][u][k] << 16) + p0, u2f(xv[r][u][k] & 0xffff0000u) + p1) | poison;
            }
            __builtin_amdgcn_raw_buffer_store_b64(o, orr, (g0 + 256u * u) * 8u, 0, 0);
        }
    }
}

int launch_indexed_gate(const RmsArgs& a, hipStream_t st) {
    const int64_t groups = a.H >> 2;
    const int u = (int)std::min<int64_t>(4, (groups + 255) / 256);
    const dim3 grid((unsigned)((a.M + 1) / 2), (unsigned)((groups + 256 * u - 1) / (256 * u))), block(256);
    if (u <= 1) hipLaunchKernelGGL(scale_indexed_gate_seg_kernel<1>, grid, block, 0, st, a);
    else if (u == 2) hipLaunchKernelGGL(scale_indexed_gate_seg_kernel<2>, grid, block, 0, st, a);
    else if (u == 3) hipLaunchKernelGGL(scale_indexed_gate_seg_kernel<3>, grid, block, 0, st, a);
    else hipLaunchKernelGGL(scale_indexed_gate_seg_kernel<4>, grid, block, 0, st, a);
    H3_CHECK_HIP(hipGetLastError());
    return H3FP8_OK;
}

template <bool GATE, bool B32 = false>
int launch_rms_out(const RmsArgs& a, hipStream_t st) {
    if (!a.q) return launch_rms<GATE, 2, B32>(a, st);
    return a.h_out ? launch_rms<GATE, 3, B32>(a, st) : launch_rms<GATE, 1, B32>(a, st);
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
    int rc = check_rms(a, false, false, true, "h3fp8_rms_quant");
    if (rc || M == 0 || H == 0) return rc;
    hipStream_t st = (hipStream_t)stream;
    return launch_rms_out<false>(a, st);
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
    int rc = check_rms(a, true, false, true, "h3fp8_gate_rms_quant");
    if (rc || M == 0 || H == 0) return rc;
    hipStream_t st = (hipStream_t)stream;
    return launch_rms_out<true>(a, st);
}

int h3fp8_scale_gate_rms_quant(const float* acc, int64_t ld_acc, const float* sa, const float* sb, const void* bias,
                               const void* residual, int64_t ldr, const void* gate, int64_t ld_gate,
                               const void* weight, const void* shift, int64_t ld_shift, const void* scale,
                               int64_t ld_scale, int64_t n_index, const void* indices, int64_t idx_stride,
                               int idx_bytes, int64_t M, int64_t H, float eps, void* residual_out, int64_t ld_res,
                               void* q, int64_t ldq, float* qscale, void* h_out, int64_t ldh, void* stream) {
    RmsArgs a{};
    a.x = (const uint16_t*)residual; a.ldx = ldr;
    a.gate = (const uint16_t*)gate; a.ld_gate = ld_gate;
    a.acc = acc; a.ld_acc = ld_acc; a.sa = sa; a.sb = sb; a.bias = (const uint16_t*)bias;
    a.residual_out = (uint16_t*)residual_out; a.ld_res = ld_res;
    a.weight = (const uint16_t*)weight;
    a.shift = (const uint16_t*)shift; a.ld_shift = ld_shift;
    a.scale = (const uint16_t*)scale; a.ld_scale = ld_scale;
    a.indices = indices; a.idx_stride = idx_stride; a.n_index = n_index; a.idx64 = idx_bytes == 8;
    a.M = M; a.H = H; a.eps = eps;
    a.q = (uint8_t*)q; a.ldq = ldq; a.qscale = qscale;
    a.h_out = (uint16_t*)h_out; a.ldh = ldh;
    H3_REQUIRE(idx_bytes == 4 || idx_bytes == 8, "h3fp8_scale_gate_rms_quant: indices must be int32 or int64");
    int rc = check_rms(a, true, true, true, "h3fp8_scale_gate_rms_quant");
    if (rc || M == 0 || H == 0) return rc;
    return launch_rms_out<true, true>(a, (hipStream_t)stream);
}

int h3fp8_scale_indexed_gate(const float* acc, int64_t ld_acc, const float* sa, const float* sb, const void* bias,
                             const void* x, int64_t ldx, const void* gate, int64_t ld_gate, int64_t n_index,
                             const void* indices, int64_t idx_stride, int idx_bytes, int64_t M, int64_t H, void* out,
                             int64_t ldo, void* stream) {
    RmsArgs a{};
    a.x = (const uint16_t*)x; a.ldx = ldx;
    a.gate = (const uint16_t*)gate; a.ld_gate = ld_gate;
    a.acc = acc; a.ld_acc = ld_acc; a.sa = sa; a.sb = sb; a.bias = (const uint16_t*)bias;
    a.residual_out = (uint16_t*)out; a.ld_res = ldo;
    a.indices = indices; a.idx_stride = idx_stride; a.n_index = n_index; a.idx64 = idx_bytes == 8;
    a.M = M; a.H = H;
    H3_REQUIRE(idx_bytes == 4 || idx_bytes == 8, "h3fp8_scale_indexed_gate: indices must be int32 or int64");
    int rc = check_rms(a, true, true, false, "h3fp8_scale_indexed_gate");
    if (rc || M == 0 || H == 0) return rc;
    H3_REQUIRE(M < ((int64_t)1 << 31), "h3fp8_scale_indexed_gate: too many rows");
    return launch_indexed_gate(a, (hipStream_t)stream);
}

}  // extern "C"
