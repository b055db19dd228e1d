// The qkv projection's consumer reading the GEMM accumulator: the scale-pass epilogue fused into
// fused_qk_norm_rope's half-split kernel (h3_tp2/fp8_consumers.py:131-193, the stock kernel's arithmetic as the
// reference's CPU stand-in states it, tests/fake_h3_consumers.py:29-48).  Per token t and q or k head (128 dims,
// rotary 96 = 2 x 48):
//
//   x_d  = bf16(sa[t] * (sb[c] * acc[t, c]))  (or fma(sa, sb * acc, bias[c])), c = head * 128 + d -- the scale pass
//   var  = fp32(sum_d x_d^2) / 128,  r = 1 / sqrt(var + eps)       (squares in fp32, summed in fp64, one rounding:
//                                    lane k of the head sums dims 32i + 4k + e in the order i, e = 0 .. 3, then an
//                                    xor butterfly over 4, 2, 1)
//   n_d  = bf16((x_d * r) * w_d)
//   out_d = bf16(n_d * cos - n_(d+48) * sin)   d < 48,     cos / sin = rope[t, d], rope[t, d + 48]
//           bf16(n_d * cos + n_(d-48) * sin)   48 <= d < 96, cos / sin = rope[t, d - 48], rope[t, d]
//           n_d                                 d >= 96
//
// A 64-lane wave takes a group of 8 heads of two consecutive tokens: lanes 8j .. 8j + 7 hold head 8g + j, lane k of
// the eight dims 32i + 4k .. 32i + 4k + 3 for i = 0 .. 3 (16 dims per lane, so the per-head work -- the butterfly, the
// two divisions, the square root -- is shared by 16 dims), 4 waves per 256-thread workgroup.  The v columns of the
// product (Hv heads after the k heads) take the plain scale pass into the placeholder, where the attention reads them:
// in the same launch (h3fp8_scale_qkv_norm_rope: every token pair's v heads are three more groups of 8, each wave
// x_d = bf16(sa[t] * (sb[c] * acc[t, c])) only, the same lane layout and rounding; 168.5 us against 177-180 us for a
// second launch at 16 740 tokens) or through h3fp8_scale_bias_cast.
#include "h3fp8_common.h"

namespace {

using namespace h3;

typedef unsigned int v2u __attribute__((ext_vector_type(2)));

// An output quad of bf16 pairs, stored non-temporally: the q / k / v rows stream through once (measured: the qkv
// consumer 170.7 -> 165.0 us at 960x576).
__device__ __forceinline__ void st_out8(uint16_t* p, uint32_t lo, uint32_t hi) {
    __builtin_nontemporal_store((v2u){lo, hi}, reinterpret_cast<v2u*>(p));
}

struct QkArgs {
    const float* acc;           // fp32 [T, N], N >= (Hq + Hk) * 128: q heads, then k heads
    int64_t ld_acc;
    const float* sa;            // fp32 [T]
    const float* sb;            // fp32 [N]
    const uint16_t* bias;       // bf16 [N] or null
    int64_t T;
    int Hq, Hk;
    const uint16_t* wq;         // bf16 [128]: the q and k RMSNorm weights
    const uint16_t* wk;
    const void* rope;           // [T, 96] cos | sin, fp32 or bf16
    int64_t ld_rope;
    int rope_f32;
    float eps;
    uint16_t* out_q;            // bf16 [T, Hq, 128], dims contiguous
    int64_t ldq_t, ldq_h;
    uint16_t* out_k;            // bf16 [T, Hk, 128]
    int64_t ldk_t, ldk_h;
    int Hv;                     // v heads after the k heads (0: none): scale pass only
    uint16_t* out_v;            // bf16 [T, Hv, 128]
    int64_t ldv_t, ldv_h;
};

// Sum over the 8 lanes of a head in fp64 (xor butterfly over 4, 2, 1: stays inside each group of 8 lanes).
__device__ __forceinline__ double group8_sum_f64(double v) {
#pragma unroll
    for (int o = 4; o >= 1; o >>= 1) {
        const int lo = __shfl_xor(__double2loint(v), o, 64), hi = __shfl_xor(__double2hiint(v), o, 64);
        v += __hiloint2double(hi, lo);
    }
    return v;
}

__device__ __forceinline__ float lo_bf16(uint32_t w) { return u2f(w << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t w) { return u2f(w & 0xffff0000u); }

// Lane k of a head holds dims 32 i + 4 k + e (chunk i = 0 .. 3, e = 0 .. 3): one 16-byte load instruction covers a
// head's 128 contiguous bytes of the product, so the loads coalesce.  The rotation partner of every rotated dim is lane
// k ^ 4; which of its chunks it is depends on the side of the lane (k < 4 or k >= 4) -- the sender picks it.
// HB: a bias is given; RF: the rope table is fp32 (else bf16).
//
// Everything one token's group of 8 heads reads (the lane's share), loaded before any of it is used.
struct QkIn {
    v4f av[4], sv[4];
    uint2 bw[4], wb[4];
    v4u cr[3], sr[3];
    float sam;
    int64_t t;
    int h;
};

template <bool HB, bool RF>
__device__ __forceinline__ void qk_load(const QkArgs& a, int64_t t, int g, int lane, QkIn& L) {
    const int k = lane & 7;
    const bool up = k >= 4;
    const int heads = a.Hq + a.Hk;
    const int h = 8 * g + (lane >> 3);
    const bool live = h < heads;                                 // the last group of a head count not divisible by 8
    const bool isq = h < a.Hq;
    L.t = t;
    L.h = h;
    const int64_t c = (int64_t)(live ? h : 0) * 128 + 4 * k;     // product column of the lane's dim 4k (chunk 0)
    // every load first: 4 x 16 B of the product and of sb, 4 x 8 B of bias and weight, the rope entries (bf16 operands
    // in 8-byte pieces: they need only 8-byte alignment)
    const float* ap = a.acc + t * a.ld_acc + c;
#pragma unroll
    for (int i = 0; i < 4; ++i) L.av[i] = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(ap + 32 * i));
#pragma unroll
    for (int i = 0; i < 4; ++i) L.sv[i] = *reinterpret_cast<const v4f*>(a.sb + c + 32 * i);
#pragma unroll
    for (int i = 0; i < 4; ++i)
        L.bw[i] = HB ? *reinterpret_cast<const uint2*>(a.bias + c + 32 * i) : make_uint2(0u, 0u);
    const uint16_t* wp = (isq ? a.wq : a.wk) + 4 * k;
#pragma unroll
    for (int i = 0; i < 4; ++i) L.wb[i] = *reinterpret_cast<const uint2*>(wp + 32 * i);
    // rope entries of the rotated chunks 0 .. 2: cos at table index fd, sin at fd + 48
    //   chunk 0: dims 4k + e < 48, fd = 4k;  chunk 1: dims 32 + 4k + e, fd = 32 + 4k (k < 4) or 4k - 16 (k >= 4);
    //   chunk 2: dims 64 + 4k + e >= 48, fd = 16 + 4k
    const int fdi[3] = {4 * k, up ? 4 * k - 16 : 32 + 4 * k, 16 + 4 * k};
    if (RF) {
        const float* rr = reinterpret_cast<const float*>(a.rope) + t * a.ld_rope;
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            L.cr[i] = *reinterpret_cast<const v4u*>(rr + fdi[i]);
            L.sr[i] = *reinterpret_cast<const v4u*>(rr + fdi[i] + 48);
        }
    } else {
        const uint16_t* rr = reinterpret_cast<const uint16_t*>(a.rope) + t * a.ld_rope;
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const uint2 cw = *reinterpret_cast<const uint2*>(rr + fdi[i]);
            const uint2 sw = *reinterpret_cast<const uint2*>(rr + fdi[i] + 48);
            L.cr[i] = v4u{cw.x, cw.y, 0u, 0u};
            L.sr[i] = v4u{sw.x, sw.y, 0u, 0u};
        }
    }
    L.sam = a.sa[t];
}

template <bool HB, bool RF>
__device__ __forceinline__ void qk_compute(const QkArgs& a, const QkIn& L, int lane, bool store) {
    const int k = lane & 7;
    const bool up = k >= 4;
    const int64_t t = L.t;
    const int h = L.h;
    const bool live = h < a.Hq + a.Hk;
    const bool isq = h < a.Hq;
    // the scale pass, rounded once to bf16; x[4i + e] is dim 32i + 4k + e
    float x[16];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float p = L.sv[i][e] * L.av[i][e];
            if (HB) {
                const uint32_t bb = (e >> 1) ? L.bw[i].y : L.bw[i].x;
                x[4 * i + e] = __builtin_fmaf(L.sam, p, (e & 1) ? hi_bf16(bb) : lo_bf16(bb));
            } else {
                x[4 * i + e] = L.sam * p;
            }
        }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t xb = cvt_bf16x2(x[2 * j], x[2 * j + 1]);
        x[2 * j] = lo_bf16(xb);
        x[2 * j + 1] = hi_bf16(xb);
    }
    double ss = 0.0;
#pragma unroll
    for (int d = 0; d < 16; ++d) ss += (double)(x[d] * x[d]);
    ss = group8_sum_f64(ss);
    float var = (float)ss, hd = 128.0f, one = 1.0f;
    asm volatile("" : "+v"(hd), "+v"(one));                       // real divisions, as the stock kernel's
    var = var / hd;
    const float r = one / __builtin_sqrtf(var + a.eps);
    uint32_t nb[8];                                              // packed pairs: nb[2i], nb[2i + 1] = chunk i
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t ww = (j & 1) ? L.wb[j >> 1].y : L.wb[j >> 1].x;
        nb[j] = cvt_bf16x2((x[2 * j] * r) * lo_bf16(ww), (x[2 * j + 1] * r) * hi_bf16(ww));
    }
    // the partner chunk of target chunk i: lanes k < 4 take chunk (i + 1) % 3 of lane k + 4, lanes k >= 4 chunk
    // (i + 2) % 3 of lane k - 4, so lane k sends chunk (i + 1) % 3 if k >= 4 and (i + 2) % 3 if k < 4
    uint32_t ob[8];
    const uint32_t upmask = up ? 0xffffffffu : 0u;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int cu = (i + 1) % 3, cl = (i + 2) % 3;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            // constant indices on both sides, merged by a bit select (a select of the index would become a
            // chain of compares over all eight registers)
            const uint32_t send = (nb[2 * cu + q] & upmask) | (nb[2 * cl + q] & ~upmask);
            const uint32_t pb = (uint32_t)__shfl_xor((int)send, 4, 64);
            float cs[2], sn[2];
            if (RF) {
                cs[0] = u2f(L.cr[i][2 * q]); cs[1] = u2f(L.cr[i][2 * q + 1]);
                sn[0] = u2f(L.sr[i][2 * q]); sn[1] = u2f(L.sr[i][2 * q + 1]);
            } else {
                cs[0] = lo_bf16(L.cr[i][q]); cs[1] = hi_bf16(L.cr[i][q]);
                sn[0] = lo_bf16(L.sr[i][q]); sn[1] = hi_bf16(L.sr[i][q]);
            }
            const uint32_t n = nb[2 * i + q];
            const float u0 = lo_bf16(n) * cs[0], v0 = lo_bf16(pb) * sn[0];
            const float u1 = hi_bf16(n) * cs[1], v1 = hi_bf16(pb) * sn[1];
            const bool minus = i == 0 || (i == 1 && !up);        // dims below 48
            ob[2 * i + q] = minus ? cvt_bf16x2(u0 - v0, u1 - v1) : cvt_bf16x2(u0 + v0, u1 + v1);
        }
    }
    ob[6] = nb[6];                                               // chunk 3: dims 96 + 4k + e, not rotated
    ob[7] = nb[7];
    if (!store || !live) return;
    uint16_t* out = (isq ? a.out_q + t * a.ldq_t + (int64_t)h * a.ldq_h
                         : a.out_k + t * a.ldk_t + (int64_t)(h - a.Hq) * a.ldk_h) + 4 * k;
#pragma unroll
    for (int i = 0; i < 4; ++i) st_out8(out + 32 * i, ob[2 * i], ob[2 * i + 1]);
}

// A wave takes head group g of two consecutive tokens: both tokens' loads are issued before either is computed, and
// the loads that do not depend on the token (sb, bias, norm weights: the same addresses) are issued once.  An odd
// token count leaves the last wave's second token a copy of its first, not stored.
// The v heads of two tokens: the scale pass alone (the same lane layout, the same arithmetic and rounding as the q / k
// heads' scale pass), stored to out_v.
template <bool HB>
__device__ __forceinline__ void v_pass(const QkArgs& a, int64_t t0, int64_t t1, bool st1, int gv, int lane) {
    const int k = lane & 7;
    const int hv = 8 * gv + (lane >> 3);
    if (hv >= a.Hv) return;
    const int64_t c = (int64_t)(a.Hq + a.Hk + hv) * 128 + 4 * k;
    v4f av[2][4], sv[4];
    uint2 bw[4];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const float* ap = a.acc + (u ? t1 : t0) * a.ld_acc + c;
#pragma unroll
        for (int i = 0; i < 4; ++i) av[u][i] = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(ap + 32 * i));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) sv[i] = *reinterpret_cast<const v4f*>(a.sb + c + 32 * i);
#pragma unroll
    for (int i = 0; i < 4; ++i) bw[i] = HB ? *reinterpret_cast<const uint2*>(a.bias + c + 32 * i) : make_uint2(0u, 0u);
    const float sam[2] = {a.sa[t0], a.sa[t1]};
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        if (u == 1 && !st1) break;
        uint16_t* out = a.out_v + (u ? t1 : t0) * a.ldv_t + (int64_t)hv * a.ldv_h + 4 * k;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float x[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float p = sv[i][e] * av[u][i][e];
                if (HB) {
                    const uint32_t bb = (e >> 1) ? bw[i].y : bw[i].x;
                    x[e] = __builtin_fmaf(sam[u], p, (e & 1) ? hi_bf16(bb) : lo_bf16(bb));
                } else {
                    x[e] = sam[u] * p;
                }
            }
            st_out8(out + 32 * i, cvt_bf16x2(x[0], x[1]), cvt_bf16x2(x[2], x[3]));
        }
    }
}

template <bool HB, bool RF>
__global__ void __launch_bounds__(256) scale_qk_norm_rope_kernel(QkArgs a, int64_t units) {
    const int lane = threadIdx.x & 63;
    const int qk_groups = (a.Hq + a.Hk + 7) / 8;
    const int groups = qk_groups + (a.Hv + 7) / 8;
    const int64_t w = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (w >= units) return;
    const int64_t tp = w / groups;
    const int g = (int)(w - tp * groups);
    const int64_t t0 = 2 * tp, t1 = t0 + 1 < a.T ? t0 + 1 : t0;
    if (g >= qk_groups) {
        v_pass<HB>(a, t0, t1, t0 + 1 < a.T, g - qk_groups, lane);
        return;
    }
    QkIn L0, L1;
    qk_load<HB, RF>(a, t0, g, lane, L0);
    qk_load<HB, RF>(a, t1, g, lane, L1);
    qk_compute<HB, RF>(a, L0, lane, true);
    qk_compute<HB, RF>(a, L1, lane, t0 + 1 < a.T);
}

}  // namespace

extern "C" {

int h3fp8_scale_qkv_norm_rope(const float* acc, int64_t ld_acc, const float* sa, const float* sb, const void* bias,
                              int64_t T, int Hq, int Hk, int Hv, const void* q_weight, const void* k_weight,
                              const void* rope, int64_t ld_rope, int rope_f32, float eps, void* out_q, int64_t ldq_t,
                              int64_t ldq_h, void* out_k, int64_t ldk_t, int64_t ldk_h, void* out_v, int64_t ldv_t,
                              int64_t ldv_h, void* stream) {
    H3_REQUIRE(T >= 0 && Hq >= 0 && Hk >= 0 && Hv >= 0, "h3fp8_scale_qk_norm_rope: negative size");
    if (T == 0 || Hq + Hk + Hv == 0) return H3FP8_OK;
    H3_REQUIRE(Hv == 0 || (out_v && ((uintptr_t)out_v & 7) == 0 && ldv_t % 4 == 0 && ldv_h % 4 == 0 && ldv_h >= 128),
               "h3fp8_scale_qkv_norm_rope: the v output needs 8-byte alignment and strides that are multiples of 4, "
               "dims contiguous");
    H3_REQUIRE(acc && sa && sb && q_weight && k_weight && rope && (Hq == 0 || out_q) && (Hk == 0 || out_k),
               "h3fp8_scale_qk_norm_rope: null pointer");
    H3_REQUIRE(ld_acc >= (int64_t)(Hq + Hk + Hv) * 128 && ld_acc % 4 == 0 && ((uintptr_t)acc & 15) == 0 &&
                   ((uintptr_t)sb & 15) == 0 && ((uintptr_t)bias & 7) == 0,
               "h3fp8_scale_qk_norm_rope: the product needs 16-byte aligned rows (stride >= (Hq + Hk) * 128, a "
               "multiple of 4), sb 16-byte and bias 8-byte alignment");
    H3_REQUIRE(((uintptr_t)q_weight & 7) == 0 && ((uintptr_t)k_weight & 7) == 0,
               "h3fp8_scale_qk_norm_rope: norm weights must be 8-byte aligned");
    H3_REQUIRE(ld_rope >= 96 && ld_rope % 4 == 0 && ((uintptr_t)rope & (rope_f32 ? 15 : 7)) == 0,
               "h3fp8_scale_qk_norm_rope: the rope table must be [T, 96] with a row stride that is a multiple of 4, "
               "aligned to 16 (fp32) / 8 (bf16) bytes");
    H3_REQUIRE((Hq == 0 || (((uintptr_t)out_q & 7) == 0 && ldq_t % 4 == 0 && ldq_h % 4 == 0 && ldq_h >= 128)) &&
                   (Hk == 0 || (((uintptr_t)out_k & 7) == 0 && ldk_t % 4 == 0 && ldk_h % 4 == 0 && ldk_h >= 128)),
               "h3fp8_scale_qk_norm_rope: outputs need 8-byte alignment and strides that are multiples of 4, dims "
               "contiguous");
    QkArgs a{};
    a.acc = acc; a.ld_acc = ld_acc; a.sa = sa; a.sb = sb; a.bias = (const uint16_t*)bias;
    a.T = T; a.Hq = Hq; a.Hk = Hk;
    a.wq = (const uint16_t*)q_weight; a.wk = (const uint16_t*)k_weight;
    a.rope = rope; a.ld_rope = ld_rope; a.rope_f32 = rope_f32 ? 1 : 0; a.eps = eps;
    a.out_q = (uint16_t*)out_q; a.ldq_t = ldq_t; a.ldq_h = ldq_h;
    a.out_k = (uint16_t*)out_k; a.ldk_t = ldk_t; a.ldk_h = ldk_h;
    a.Hv = Hv; a.out_v = (uint16_t*)out_v; a.ldv_t = ldv_t; a.ldv_h = ldv_h;
    const int64_t units = ((T + 1) / 2) * ((Hq + Hk + 7) / 8 + (Hv + 7) / 8);
    H3_REQUIRE(units < ((int64_t)1 << 33), "h3fp8_scale_qk_norm_rope: too many tokens");
    const dim3 grid((unsigned)((units + 3) / 4)), block(256);
    hipStream_t st = (hipStream_t)stream;
    if (a.bias && a.rope_f32) hipLaunchKernelGGL((scale_qk_norm_rope_kernel<true, true>), grid, block, 0, st, a, units);
    else if (a.bias) hipLaunchKernelGGL((scale_qk_norm_rope_kernel<true, false>), grid, block, 0, st, a, units);
    else if (a.rope_f32) hipLaunchKernelGGL((scale_qk_norm_rope_kernel<false, true>), grid, block, 0, st, a, units);
    else hipLaunchKernelGGL((scale_qk_norm_rope_kernel<false, false>), grid, block, 0, st, a, units);
    H3_CHECK_HIP(hipGetLastError());
    return H3FP8_OK;
}

int h3fp8_scale_qk_norm_rope(const float* acc, int64_t ld_acc, const float* sa, const float* sb, const void* bias,
                             int64_t T, int Hq, int Hk, const void* q_weight, const void* k_weight, const void* rope,
                             int64_t ld_rope, int rope_f32, float eps, void* out_q, int64_t ldq_t, int64_t ldq_h,
                             void* out_k, int64_t ldk_t, int64_t ldk_h, void* stream) {
    return h3fp8_scale_qkv_norm_rope(acc, ld_acc, sa, sb, bias, T, Hq, Hk, 0, q_weight, k_weight, rope, ld_rope,
                                     rope_f32, eps, out_q, ldq_t, ldq_h, out_k, ldk_t, ldk_h, nullptr, 0, 0, stream);
}

}  // extern "C"
