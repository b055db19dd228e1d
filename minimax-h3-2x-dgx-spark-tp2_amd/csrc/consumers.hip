// The qkv projection's consumer reading the GEMM accumulator: the scale-pass epilogue fused into
// fused_qk_norm_rope's half-split kernel (h3_tp2/fp8_consumers.py:131-193, the stock kernel's arithmetic as the
// reference's CPU stand-in states it, tests/fake_h3_consumers.py:29-48).  Per token t and q or k head (128 dims,
// rotary 96 = 2 x 48):
//
//   x_d  = bf16(sa[t] * (sb[c] * acc[t, c]))  (or fma(sa, sb * acc, bias[c])), c = head * 128 + d -- the scale pass
//   var  = fp32(sum_d x_d^2) / 128,  r = 1 / sqrt(var + eps)       (squares in fp32, summed in fp64, one rounding)
//   n_d  = bf16((x_d * r) * w_d)
//   out_d = bf16(n_d * cos - n_(d+48) * sin)   d < 48,     cos / sin = rope[t, d], rope[t, d + 48]
//           bf16(n_d * cos + n_(d-48) * sin)   48 <= d < 96, cos / sin = rope[t, d - 48], rope[t, d]
//           n_d                                 d >= 96
//
// One 64-lane wave per (token, head), 4 per 256-thread workgroup; lane l holds dims 2l and 2l + 1 (8-byte loads of
// the product and of sb), the rotation partner of lane l is lane l +- 24 (one shuffle).  The v columns of the product
// go through the plain scale pass (h3fp8_scale_bias_cast) into the placeholder, where the attention reads them.
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

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const int lo = __shfl_xor(__double2loint(v), o, 64), hi = __shfl_xor(__double2hiint(v), o, 64);
        v += __hiloint2double(hi, lo);
    }
    return v;
}

__global__ void __launch_bounds__(256) scale_qk_norm_rope_kernel(QkArgs a) {
    const int lane = threadIdx.x & 63;
    const int64_t w = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int heads = a.Hq + a.Hk;
    if (w >= a.T * heads) return;
    const int64_t t = w / heads;
    const int h = (int)(w - t * heads);
    const bool isq = h < a.Hq;
    const int64_t c = (int64_t)h * 128 + 2 * lane;               // product column of dim 2l
    const float2 av = *reinterpret_cast<const float2*>(a.acc + t * a.ld_acc + c);
    const float2 sv = *reinterpret_cast<const float2*>(a.sb + c);
    const float sam = a.sa[t];
    float x[2];
    if (a.bias) {
        const uint32_t bw = *reinterpret_cast<const uint32_t*>(a.bias + c);
        x[0] = __builtin_fmaf(sam, sv.x * av.x, u2f(bw << 16));
        x[1] = __builtin_fmaf(sam, sv.y * av.y, u2f(bw & 0xffff0000u));
    } else {
        x[0] = sam * (sv.x * av.x);
        x[1] = sam * (sv.y * av.y);
    }
    const uint32_t xb = cvt_bf16x2(x[0], x[1]);                  // the scale pass's one rounding to bf16
    x[0] = u2f(xb << 16);
    x[1] = u2f(xb & 0xffff0000u);
    double ss = 0.0;
    ss += (double)(x[0] * x[0]);
    ss += (double)(x[1] * x[1]);
    ss = wave_sum_f64(ss);
    float var = (float)ss, hd = 128.0f, one = 1.0f;
    asm volatile("" : "+v"(hd), "+v"(one));                       // real divisions, as the stock kernel's
    var = var / hd;
    const float r = one / __builtin_sqrtf(var + a.eps);
    const uint32_t wb = *reinterpret_cast<const uint32_t*>((isq ? a.wq : a.wk) + 2 * lane);
    const uint32_t nb = cvt_bf16x2((x[0] * r) * u2f(wb << 16), (x[1] * r) * u2f(wb & 0xffff0000u));
    const int partner = lane < 24 ? lane + 24 : lane < 48 ? lane - 24 : lane;
    const uint32_t pb = (uint32_t)__shfl((int)nb, partner, 64);
    uint32_t ob = nb;
    if (lane < 48) {
        const int fd = lane < 24 ? 2 * lane : 2 * lane - 48;
        float cs[2], sn[2];
        if (a.rope_f32) {
            const float* rr = reinterpret_cast<const float*>(a.rope) + t * a.ld_rope;
            const float2 cv = *reinterpret_cast<const float2*>(rr + fd);
            const float2 sv2 = *reinterpret_cast<const float2*>(rr + fd + 48);
            cs[0] = cv.x; cs[1] = cv.y; sn[0] = sv2.x; sn[1] = sv2.y;
        } else {
            const uint16_t* rr = reinterpret_cast<const uint16_t*>(a.rope) + t * a.ld_rope;
            const uint32_t cw = *reinterpret_cast<const uint32_t*>(rr + fd);
            const uint32_t sw = *reinterpret_cast<const uint32_t*>(rr + fd + 48);
            cs[0] = u2f(cw << 16); cs[1] = u2f(cw & 0xffff0000u);
            sn[0] = u2f(sw << 16); sn[1] = u2f(sw & 0xffff0000u);
        }
        const float n0 = u2f(nb << 16), n1 = u2f(nb & 0xffff0000u);
        const float p0 = u2f(pb << 16), p1 = u2f(pb & 0xffff0000u);
        const float a0 = n0 * cs[0], b0 = p0 * sn[0], a1 = n1 * cs[1], b1 = p1 * sn[1];
        ob = lane < 24 ? cvt_bf16x2(a0 - b0, a1 - b1) : cvt_bf16x2(a0 + b0, a1 + b1);
    }
    uint16_t* o = isq ? a.out_q + t * a.ldq_t + (int64_t)h * a.ldq_h
                      : a.out_k + t * a.ldk_t + (int64_t)(h - a.Hq) * a.ldk_h;
    *reinterpret_cast<uint32_t*>(o + 2 * lane) = ob;
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
    H3_REQUIRE(ld_acc >= (int64_t)(Hq + Hk) * 128 && ld_acc % 2 == 0 && ((uintptr_t)acc & 7) == 0 &&
                   ((uintptr_t)sb & 7) == 0 && ((uintptr_t)bias & 3) == 0,
               "h3fp8_scale_qk_norm_rope: the product needs 8-byte aligned rows (even stride >= (Hq + Hk) * 128), "
               "sb 8-byte and bias 4-byte alignment");
    H3_REQUIRE(((uintptr_t)q_weight & 3) == 0 && ((uintptr_t)k_weight & 3) == 0,
               "h3fp8_scale_qk_norm_rope: norm weights must be 4-byte aligned");
    H3_REQUIRE(ld_rope >= 96 && ld_rope % 2 == 0 && ((uintptr_t)rope & (rope_f32 ? 7 : 3)) == 0,
               "h3fp8_scale_qk_norm_rope: the rope table must be [T, 96] with an even row stride, aligned");
    H3_REQUIRE((Hq == 0 || (((uintptr_t)out_q & 3) == 0 && ldq_t % 2 == 0 && ldq_h % 2 == 0 && ldq_h >= 128)) &&
                   (Hk == 0 || (((uintptr_t)out_k & 3) == 0 && ldk_t % 2 == 0 && ldk_h % 2 == 0 && ldk_h >= 128)),
               "h3fp8_scale_qk_norm_rope: outputs need 4-byte alignment and even strides, dims contiguous");
    QkArgs a{};
    a.acc = acc; a.ld_acc = ld_acc; a.sa = sa; a.sb = sb; a.bias = (const uint16_t*)bias;
    a.T = T; a.Hq = Hq; a.Hk = Hk;
    a.wq = (const uint16_t*)q_weight; a.wk = (const uint16_t*)k_weight;
    a.rope = rope; a.ld_rope = ld_rope; a.rope_f32 = rope_f32 ? 1 : 0; a.eps = eps;
    a.out_q = (uint16_t*)out_q; a.ldq_t = ldq_t; a.ldq_h = ldq_h;
    a.out_k = (uint16_t*)out_k; a.ldk_t = ldk_t; a.ldk_h = ldk_h;
    const int64_t waves = T * (Hq + Hk);
    hipLaunchKernelGGL(scale_qk_norm_rope_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, (hipStream_t)stream,
                       a);
    H3_CHECK_HIP(hipGetLastError());
    return H3FP8_OK;
}

}  // extern "C"
