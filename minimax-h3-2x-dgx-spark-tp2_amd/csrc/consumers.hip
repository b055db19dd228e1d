// The qkv projection's consumer reading the GEMM accumulator: the scale-pass epilogue fused into
// fused_qk_norm_rope's half-split kernel (h3_tp2/fp8_consumers.py:131-193, the stock kernel's arithmetic as the
// reference's CPU stand-in states it, tests/fake_h3_consumers.py:29-48).  Per token t and q or k head (128 dims,
// rotary 96 = 2 x 48):
//
//   x_d  = bf16(sa[t] * (sb[c] * acc[t, c]))  (or fma(sa, sb * acc, bias[c])), c = head * 128 + d -- the scale pass
//   var  = fp32(sum_d x_d^2) / 128,  r = 1 / sqrt(var + eps)       (squares in fp32, summed in fp64, one rounding:
//                                    lane l of the half sums dims 4l .. 4l + 3, then an xor butterfly over 16 .. 1)
//   n_d  = bf16((x_d * r) * w_d)
//   out_d = bf16(n_d * cos - n_(d+48) * sin)   d < 48,     cos / sin = rope[t, d], rope[t, d + 48]
//           bf16(n_d * cos + n_(d-48) * sin)   48 <= d < 96, cos / sin = rope[t, d - 48], rope[t, d]
//           n_d                                 d >= 96
//
// One 64-lane wave per (token, pair of heads), 4 per 256-thread workgroup: each half-wave holds one head, lane l of the
// half dims 4l .. 4l + 3 (16-byte loads of the product and of sb); the rotation partner of lane l is lane l +- 12 of
// the same half (one shuffle per packed pair).  The v columns of the product go through the plain scale pass
// (h3fp8_scale_bias_cast) into the placeholder, where the attention reads them.
#include "h3fp8_common.h"

namespace {

using namespace h3;

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
};

// 32-lane half-wave sum in fp64 (xor butterfly over 16, 8, 4, 2, 1: stays inside each half of the wave).
__device__ __forceinline__ double half_sum_f64(double v) {
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) {
        const int lo = __shfl_xor(__double2loint(v), o, 64), hi = __shfl_xor(__double2hiint(v), o, 64);
        v += __hiloint2double(hi, lo);
    }
    return v;
}

__global__ void __launch_bounds__(256) scale_qk_norm_rope_kernel(QkArgs a) {
    const int lane = threadIdx.x & 63;
    const int hl = lane & 31;                                    // lane within the head: dims 4 hl .. 4 hl + 3
    const int heads = a.Hq + a.Hk;
    const int64_t pairs = (heads + 1) / 2;                       // two heads per wave, one per half
    const int64_t w = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (w >= a.T * pairs) return;
    const int64_t t = w / pairs;
    const int h = 2 * (int)(w - t * pairs) + (lane >> 5);
    const bool live = h < heads;                                 // an odd head count leaves the last half idle
    const bool isq = h < a.Hq;
    const int64_t c = (int64_t)(live ? h : 0) * 128 + 4 * hl;    // product column of dim 4 hl
    const v4f av = *reinterpret_cast<const v4f*>(a.acc + t * a.ld_acc + c);
    const v4f sv = *reinterpret_cast<const v4f*>(a.sb + c);
    const float sam = a.sa[t];
    float x[4];
    if (a.bias) {
        const uint2 bw = *reinterpret_cast<const uint2*>(a.bias + c);
        const uint32_t b2[2] = {bw.x, bw.y};
#pragma unroll
        for (int e = 0; e < 4; ++e)
            x[e] = __builtin_fmaf(sam, sv[e] * av[e], u2f((e & 1) ? (b2[e >> 1] & 0xffff0000u) : (b2[e >> 1] << 16)));
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = sam * (sv[e] * av[e]);
    }
    const uint32_t xb[2] = {cvt_bf16x2(x[0], x[1]), cvt_bf16x2(x[2], x[3])};   // the scale pass's one rounding
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = u2f((e & 1) ? (xb[e >> 1] & 0xffff0000u) : (xb[e >> 1] << 16));
    double ss = 0.0;
#pragma unroll
    for (int e = 0; e < 4; ++e) ss += (double)(x[e] * x[e]);
    ss = half_sum_f64(ss);
    float var = (float)ss, hd = 128.0f, one = 1.0f;
    asm volatile("" : "+v"(hd), "+v"(one));                       // real divisions, as the stock kernel's
    var = var / hd;
    const float r = one / __builtin_sqrtf(var + a.eps);
    const uint2 wb = *reinterpret_cast<const uint2*>((isq ? a.wq : a.wk) + 4 * hl);
    const uint32_t nb[2] = {cvt_bf16x2((x[0] * r) * u2f(wb.x << 16), (x[1] * r) * u2f(wb.x & 0xffff0000u)),
                            cvt_bf16x2((x[2] * r) * u2f(wb.y << 16), (x[3] * r) * u2f(wb.y & 0xffff0000u))};
    // rotation partner: dims d +- 48 live 12 lanes away in the same half
    const int partner = (lane & 32) | (hl < 12 ? hl + 12 : hl < 24 ? hl - 12 : hl);
    const uint32_t pb[2] = {(uint32_t)__shfl((int)nb[0], partner, 64), (uint32_t)__shfl((int)nb[1], partner, 64)};
    uint32_t ob[2] = {nb[0], nb[1]};
    if (hl < 24) {
        const int fd = hl < 12 ? 4 * hl : 4 * hl - 48;
        float cs[4], sn[4];
        if (a.rope_f32) {
            const float* rr = reinterpret_cast<const float*>(a.rope) + t * a.ld_rope;
            const v4f cv = *reinterpret_cast<const v4f*>(rr + fd);
            const v4f sv2 = *reinterpret_cast<const v4f*>(rr + fd + 48);
#pragma unroll
            for (int e = 0; e < 4; ++e) { cs[e] = cv[e]; sn[e] = sv2[e]; }
        } else {
            const uint16_t* rr = reinterpret_cast<const uint16_t*>(a.rope) + t * a.ld_rope;
            const uint2 cw = *reinterpret_cast<const uint2*>(rr + fd);
            const uint2 sw = *reinterpret_cast<const uint2*>(rr + fd + 48);
            const uint32_t c2[2] = {cw.x, cw.y}, s2[2] = {sw.x, sw.y};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                cs[e] = u2f((e & 1) ? (c2[e >> 1] & 0xffff0000u) : (c2[e >> 1] << 16));
                sn[e] = u2f((e & 1) ? (s2[e >> 1] & 0xffff0000u) : (s2[e >> 1] << 16));
            }
        }
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float n = u2f((e & 1) ? (nb[e >> 1] & 0xffff0000u) : (nb[e >> 1] << 16));
            const float p = u2f((e & 1) ? (pb[e >> 1] & 0xffff0000u) : (pb[e >> 1] << 16));
            const float u = n * cs[e], v = p * sn[e];
            o[e] = hl < 12 ? u - v : u + v;
        }
        ob[0] = cvt_bf16x2(o[0], o[1]);
        ob[1] = cvt_bf16x2(o[2], o[3]);
    }
    if (!live) return;
    uint16_t* out = isq ? a.out_q + t * a.ldq_t + (int64_t)h * a.ldq_h
                        : a.out_k + t * a.ldk_t + (int64_t)(h - a.Hq) * a.ldk_h;
    *reinterpret_cast<uint2*>(out + 4 * hl) = make_uint2(ob[0], ob[1]);
}

}  // namespace

extern "C" {

int h3fp8_scale_qk_norm_rope(const float* acc, int64_t ld_acc, const float* sa, const float* sb, const void* bias,
                             int64_t T, int Hq, int Hk, const void* q_weight, const void* k_weight, const void* rope,
                             int64_t ld_rope, int rope_f32, float eps, void* out_q, int64_t ldq_t, int64_t ldq_h,
                             void* out_k, int64_t ldk_t, int64_t ldk_h, void* stream) {
    H3_REQUIRE(T >= 0 && Hq >= 0 && Hk >= 0, "h3fp8_scale_qk_norm_rope: negative size");
    if (T == 0 || Hq + Hk == 0) return H3FP8_OK;
    H3_REQUIRE(acc && sa && sb && q_weight && k_weight && rope && (Hq == 0 || out_q) && (Hk == 0 || out_k),
               "h3fp8_scale_qk_norm_rope: null pointer");
    H3_REQUIRE(ld_acc >= (int64_t)(Hq + Hk) * 128 && ld_acc % 4 == 0 && ((uintptr_t)acc & 15) == 0 &&
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
    const int64_t waves = T * ((Hq + Hk + 1) / 2);
    hipLaunchKernelGGL(scale_qk_norm_rope_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, (hipStream_t)stream,
                       a);
    H3_CHECK_HIP(hipGetLastError());
    return H3FP8_OK;
}

}  // extern "C"
