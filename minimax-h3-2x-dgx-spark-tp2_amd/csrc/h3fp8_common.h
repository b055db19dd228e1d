// Shared device helpers and host plumbing of libh3fp8 (gfx950 / CDNA4 only).
//
// Numerics follow the reference's per-token FP8 path (h3_tp2/fp8_quant_fuse.py:11-13, :92-121, :302-307;
// h3_tp2/fp8_gemm.py:44-50; h3_tp2/fp8_swiglu.py:38-45, :64-70): IEEE fp32 division (hipcc's default correctly
// rounded divide), NaN-propagating max/min, round-to-nearest-even casts to bf16 / fp16 / OCP e4m3fn.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/h3fp8.h"

#define H3_FP8_MAX 448.0f
// vLLM's minimum per-token scale 1/(448*512) as an fp32 constant (fp8_quant_fuse.py:78-79): 0x36924925.
#define H3_MIN_SCALE_BITS 0x36924925u

// The compact SiLU table of kernel 3: entry i holds silu(g) of the bf16 g whose rotated key
// ((bits << 1) & 0xfffe) | (bits >> 15) (the sign moved to the lowest bit) is H3_SILU_ROT_R0 + i.  The keys cover
// |g| in [2.6e-9, 88.5] for both signs (8960 entries, 17920 bytes); every other g (zeros, tinier, larger, inf, NaN)
// is looked up in the full table.
#define H3_SILU_ROT_R0 0x6264u
#define H3_SILU_ROT_LEN 8960

namespace h3 {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }

// torch / Inductor NaN-propagating maximum and minimum (fp8_quant_fuse.py:92-103).
__device__ __forceinline__ float nan_max(float a, float b) { return (a > b || a != a) ? a : b; }
__device__ __forceinline__ float nan_min(float a, float b) { return (a < b || a != a) ? a : b; }

// fp32 -> bf16 bits, round to nearest even, NaN kept (quietened) -- _round_bf16 (fp8_swiglu.py:38-45).
__device__ __forceinline__ uint32_t bf16_rne(float f) {
    uint32_t u = f2u(f);
    uint32_t r = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
    return ((u & 0x7fffffffu) > 0x7f800000u) ? ((u >> 16) | 0x40u) : r;
}

// fp32 -> fp16 bits, round to nearest even (hardware cvt: IEEE RNE, overflow -> inf, denormals kept).  The value is
// first pinned as an fp32 register: otherwise the compiler folds the producing fp32 multiply into v_fma_mix*_f16,
// which rounds the exact product once to fp16 instead of rounding to fp32 and then to fp16 as the reference does.
__device__ __forceinline__ uint32_t fp16_rne(float f) {
    asm("" : "+v"(f));
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return u2f(h << 16); }

// Two fp32 -> packed bf16 (a in the low half), round to nearest even: gfx950's v_cvt_pk_bf16_f32.  It equals bf16_rne
// above on every fp32 input, NaN payloads included (checked over all 2^32 inputs by h3fp8_selfcheck_bf16).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t cvt_bf16x2(float a, float b) {
    const f32x2_t v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ float fp16_to_f32(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

// Software fp32 -> OCP e4m3fn (round to nearest even, >= 480 and NaN -> 0x7f | sign): the bit rule of torch's
// `.to(torch.float8_e4m3fn)`, restated.  Used by the conversion self-check; the kernels use the hardware cvt below.
__device__ __forceinline__ uint32_t e4m3_soft(float f) {
    uint32_t u = f2u(f);
    uint32_t sign = (u >> 24) & 0x80u;
    uint32_t a = u & 0x7fffffffu;
    uint32_t r;
    if (a >= 0x43f00000u) {
        r = 0x7fu;
    } else if (a < 0x3c800000u) {
        r = (uint32_t)__builtin_rintf(u2f(a) * 512.0f);      // subnormal grid 2^-9, RNE (default mode)
    } else {
        a += ((uint32_t)(7 - 127) << 23) + 0x7ffffu + ((a >> 20) & 1u);
        r = (a >> 20) & 0xffu;
    }
    return sign | r;
}

// Two fp32 values (already clamped to [-448, 448] or NaN) -> two e4m3fn bytes in the low half of the result.
// gfx950's v_cvt_pk_fp8_f32 converts to OCP e4m3fn with round-to-nearest-even; the library self-check
// (h3fp8_selfcheck_e4m3) compares it with e4m3_soft over every fp32 bit pattern in [-448, 448] and NaN.
__device__ __forceinline__ uint32_t e4m3x2(float a, float b) {
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xffffu;
}

// Four fp32 -> packed 4 x e4m3fn.
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
    int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
}

// The per-token scale from a row maximum (fp8_quant_fuse.py:108-111): max(amax / 448, MIN_SCALE), IEEE division with
// a runtime divisor; NaN propagates.
__device__ __forceinline__ float row_scale(float amax) {
    float fp8max = H3_FP8_MAX;
    asm volatile("" : "+v"(fp8max));                        // keep it a runtime divisor (no reciprocal folding)
    return nan_max(amax / fp8max, u2f(H3_MIN_SCALE_BITS));
}

__device__ __forceinline__ float inv_scale(float scale) {
    float one = 1.0f;
    asm volatile("" : "+v"(one));
    return one / scale;                                     // IEEE division, as torch's reciprocal on the CPU
}

// x * inv clamped to [-448, 448], NaN propagating (fp8_quant_fuse.py:105-111).
__device__ __forceinline__ float quant_clamp(float x, float inv) {
    float y = x * inv;
    y = (y < -H3_FP8_MAX) ? -H3_FP8_MAX : y;
    y = (y > H3_FP8_MAX) ? H3_FP8_MAX : y;
    return y;
}

// Wave-wide (64-lane) unsigned max.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        uint32_t w = (uint32_t)__shfl_xor((int)v, o, 64);
        v = v > w ? v : w;
    }
    return v;
}

// Buffer resource for raw buffer loads: base, byte size (loads at offsets >= size return 0).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

}  // namespace h3

// ---- host side --------------------------------------------------------------------------------------------------

namespace h3host {
void set_error(const char* fmt, ...);
int hip_fail(hipError_t e, const char* what);
int ensure_device_init();                      // per-device one-time set-up (SiLU table); returns status
bool device_ready(int dev);                    // has ensure_device_init completed on device dev (no side effects)
int gemm_scratch_setup(int dev);               // the device address of gemm.hip's row-maxima buffer (set-up only)
const uint16_t* silu_table_ptr();              // device address of the current device's SiLU table
const uint16_t* silu_rot_ptr();                // ... and of its compact rotated-key copy (kernel 3's LDS table)
int cu_count();                                // compute units of the current device (after ensure_device_init)
}  // namespace h3host

#define H3_CHECK_HIP(call)                                              \
    do {                                                                \
        hipError_t e_ = (call);                                         \
        if (e_ != hipSuccess) return h3host::hip_fail(e_, #call);      \
    } while (0)

#define H3_REQUIRE(cond, ...)                                           \
    do {                                                                \
        if (!(cond)) { h3host::set_error(__VA_ARGS__); return H3FP8_EINVAL; } \
    } while (0)
