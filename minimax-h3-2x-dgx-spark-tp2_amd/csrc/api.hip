// Library plumbing of libh3fp8: error reporting, per-device set-up (the SiLU table) and the self-checks.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>
#include <mutex>

#include "h3fp8_common.h"

// The bf16 SiLU of every bf16 gate value, one table per device (128 KiB), filled once by h3fp8_init.  Both tables
// are 16-byte aligned: the kernels that copy them into LDS read 16 bytes per load.
__device__ __attribute__((aligned(16))) uint16_t g_h3_silu_table[65536];

// The compact rotated-key copy of the table (see h3fp8_common.h), filled from it by h3fp8_init.
__device__ __attribute__((aligned(16))) uint16_t g_h3_silu_rot[H3_SILU_ROT_LEN];

// Counters of the e4m3 conversion self-check.
__device__ unsigned long long g_h3_cvt_counts[4];

namespace {
thread_local char t_err[512] = "";
std::mutex g_init_mu;
constexpr int kMaxDevices = 64;
std::atomic<bool> g_inited[kMaxDevices] = {};
const uint16_t* g_silu_ptr[kMaxDevices] = {};   // device address of each device's copy of g_h3_silu_table
const uint16_t* g_silu_rot_ptr[kMaxDevices] = {};   // ... and of g_h3_silu_rot
int g_cus[kMaxDevices] = {};                    // compute units of each device (persistent GEMM grid size)
}  // namespace

namespace h3host {

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(t_err, sizeof(t_err), fmt, ap);
    va_end(ap);
}

int hip_fail(hipError_t e, const char* what) {
    set_error("%s failed: %s", what, hipGetErrorString(e));
    return H3FP8_EHIP;
}

}  // namespace h3host

// s = bf16(g / (1 + exp(-g))) for every bf16 g (h3_tp2/fp8_swiglu.py:69): exp in float64 rounded once to fp32,
// then IEEE fp32 add and divide, then RNE to bf16.
__global__ void __launch_bounds__(256) h3_build_silu_table_kernel() {
    uint32_t i = blockIdx.x * 256u + threadIdx.x;
    float g = h3::bf16_to_f32(i);
    uint32_t r;
    if (g != g) {
        r = h3::bf16_rne(g);
    } else {
        float e = (float)exp(-(double)g);
        float d = 1.0f + e;
        float s = g / d;
        r = h3::bf16_rne(s);
    }
    g_h3_silu_table[i] = (uint16_t)r;
}

// The chip's sustained FP8 MFMA rate with no memory traffic: each wave keeps the GEMM's 4 x 4 block of 32x32x64 e4m3
// accumulators and issues 16 independent MFMAs per round, two of its eight operand registers changing between rounds
// (finite e4m3 bytes with random signs, so the multipliers toggle as on real data).  One store per thread at the end
// keeps the work.  It runs at the clock the chip holds under FP8 MFMA load, which is what bounds the GEMMs beside
// the published peak.
__global__ void __launch_bounds__(256, 1) h3_mfma_loop_kernel(float* out, int iters, uint32_t seed) {
    typedef float v16f __attribute__((ext_vector_type(16)));
    using h3::v8i;
    const int lane = threadIdx.x & 63;
    v8i af[4], bf[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            uint32_t x = (uint32_t)lane * 2654435761u ^ (uint32_t)(i * 8 + e) * 40503u ^ seed;
            x ^= x >> 13;
            x *= 0x5bd1e995u;
            x ^= x >> 15;
            af[i][e] = (int)(x & 0xbebebebeu);          // bytes below 0x7f in magnitude: finite e4m3
            uint32_t y = x * 0x27d4eb2du;
            y ^= y >> 16;
            bf[i][e] = (int)(y & 0xbebebebeu);
        }
    v16f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = (v16f){};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int t = 0; t < 16; ++t)
            acc[t >> 2][t & 3] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(af[t >> 2], bf[t & 3],
                                                                                 acc[t >> 2][t & 3], 0, 0, 0, 0, 0, 0);
        const int m = (it * 0x01030507) & 0x3e3e3e3e;   // flips low bits of each byte: finite stays finite
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            af[0][e] ^= m;
            bf[1][e] ^= m;
        }
    }
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) s += acc[i][j][r];
    out[blockIdx.x * 256 + threadIdx.x] = s;
}

__global__ void __launch_bounds__(256) h3_build_silu_rot_kernel() {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= H3_SILU_ROT_LEN) return;
    const uint32_t k = H3_SILU_ROT_R0 + i;
    g_h3_silu_rot[i] = g_h3_silu_table[((k & 1u) << 15) | (k >> 1)];
}

__global__ void __launch_bounds__(256) h3_selfcheck_e4m3_kernel() {
    unsigned long long bad = 0, nan_bad = 0;
    const uint64_t total = 1ull << 32;
    const uint64_t step = (uint64_t)gridDim.x * 256u;
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < total; i += step) {
        float x = h3::u2f((uint32_t)i);
        bool nan = x != x;
        if (!nan && !(x >= -H3_FP8_MAX && x <= H3_FP8_MAX)) continue;
        uint32_t hw = h3::e4m3x2(x, 0.0f) & 0xffu;
        if (nan) {
            nan_bad += ((hw & 0x7fu) != 0x7fu);
        } else {
            bad += (hw != h3::e4m3_soft(x));
        }
    }
    if (bad) atomicAdd(&g_h3_cvt_counts[0], bad);
    if (nan_bad) atomicAdd(&g_h3_cvt_counts[1], nan_bad);
}

// The hardware pair conversion to bf16 against bf16_rne (the reference's rounding rule) on every fp32 pattern.
__global__ void __launch_bounds__(256) h3_selfcheck_bf16_kernel() {
    unsigned long long bad = 0, nan_bad = 0;
    const uint64_t total = 1ull << 32;
    const uint64_t step = (uint64_t)gridDim.x * 256u;
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < total; i += step) {
        float x = h3::u2f((uint32_t)i);
        uint32_t hw = h3::cvt_bf16x2(x, 0.0f) & 0xffffu;
        if (x != x) nan_bad += ((hw & 0x7f80u) != 0x7f80u) || !(hw & 0x7fu);
        else bad += (hw != h3::bf16_rne(x));
    }
    if (bad) atomicAdd(&g_h3_cvt_counts[2], bad);
    if (nan_bad) atomicAdd(&g_h3_cvt_counts[3], nan_bad);
}

__global__ void __launch_bounds__(256) h3_copy_table_kernel(uint16_t* out) {
    uint32_t i = blockIdx.x * 256u + threadIdx.x;
    out[i] = g_h3_silu_table[i];
}

namespace h3host {

int ensure_device_init() {
    int dev = 0;
    H3_CHECK_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) {
        set_error("device index %d out of range", dev);
        return H3FP8_EINVAL;
    }
    if (g_inited[dev].load(std::memory_order_acquire)) return H3FP8_OK;
    std::lock_guard<std::mutex> lock(g_init_mu);
    if (g_inited[dev].load(std::memory_order_relaxed)) return H3FP8_OK;
    int cus = 0;
    H3_CHECK_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    hipStream_t s;
    H3_CHECK_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    hipLaunchKernelGGL(h3_build_silu_table_kernel, dim3(65536 / 256), dim3(256), 0, s);
    hipLaunchKernelGGL(h3_build_silu_rot_kernel, dim3((H3_SILU_ROT_LEN + 255) / 256), dim3(256), 0, s);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    (void)hipStreamDestroy(s);
    if (e != hipSuccess) return hip_fail(e, "SiLU table build");
    void* p = nullptr;
    H3_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(g_h3_silu_table)));
    g_silu_ptr[dev] = (const uint16_t*)p;
    H3_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(g_h3_silu_rot)));
    g_silu_rot_ptr[dev] = (const uint16_t*)p;
    const int rc = gemm_scratch_setup(dev);
    if (rc) return rc;
    g_cus[dev] = cus > 0 ? cus : 1;
    g_inited[dev].store(true, std::memory_order_release);
    return H3FP8_OK;
}

bool device_ready(int dev) { return dev >= 0 && dev < kMaxDevices && g_inited[dev].load(std::memory_order_acquire); }

int cu_count() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 1;
    return g_cus[dev] > 0 ? g_cus[dev] : 1;
}

const uint16_t* silu_table_ptr() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    return g_silu_ptr[dev];
}

const uint16_t* silu_rot_ptr() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    return g_silu_rot_ptr[dev];
}

}  // namespace h3host

extern "C" {

int h3fp8_abi_version(void) { return H3FP8_ABI_VERSION; }

const char* h3fp8_last_error(void) { return t_err; }

int h3fp8_init(void) { return h3host::ensure_device_init(); }

int h3fp8_selfcheck_e4m3(uint64_t* mismatches, uint64_t* nan_bad) {
    H3_REQUIRE(mismatches && nan_bad, "h3fp8_selfcheck_e4m3: null output pointer");
    unsigned long long zero[4] = {0, 0, 0, 0};
    H3_CHECK_HIP(hipMemcpyToSymbol(HIP_SYMBOL(g_h3_cvt_counts), zero, sizeof(zero)));
    hipLaunchKernelGGL(h3_selfcheck_e4m3_kernel, dim3(4096), dim3(256), 0, (hipStream_t)0);
    H3_CHECK_HIP(hipGetLastError());
    H3_CHECK_HIP(hipDeviceSynchronize());
    unsigned long long out[4];
    H3_CHECK_HIP(hipMemcpyFromSymbol(out, HIP_SYMBOL(g_h3_cvt_counts), sizeof(out)));
    *mismatches = out[0];
    *nan_bad = out[1];
    return H3FP8_OK;
}

int h3fp8_selfcheck_bf16(uint64_t* mismatches, uint64_t* nan_bad) {
    H3_REQUIRE(mismatches && nan_bad, "h3fp8_selfcheck_bf16: null output pointer");
    unsigned long long zero[4] = {0, 0, 0, 0};
    H3_CHECK_HIP(hipMemcpyToSymbol(HIP_SYMBOL(g_h3_cvt_counts), zero, sizeof(zero)));
    hipLaunchKernelGGL(h3_selfcheck_bf16_kernel, dim3(4096), dim3(256), 0, (hipStream_t)0);
    H3_CHECK_HIP(hipGetLastError());
    H3_CHECK_HIP(hipDeviceSynchronize());
    unsigned long long out[4];
    H3_CHECK_HIP(hipMemcpyFromSymbol(out, HIP_SYMBOL(g_h3_cvt_counts), sizeof(out)));
    *mismatches = out[2];
    *nan_bad = out[3];
    return H3FP8_OK;
}

int h3fp8_mfma_loop(float* out, int64_t blocks, int64_t iters, uint32_t seed, void* stream) {
    H3_REQUIRE(out, "h3fp8_mfma_loop: null output");
    H3_REQUIRE(blocks >= 1 && blocks <= 65535 && iters >= 1 && iters <= (1 << 30),
               "h3fp8_mfma_loop: blocks must be in [1, 65535] and iters in [1, 2^30]");
    hipLaunchKernelGGL(h3_mfma_loop_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, out, (int)iters,
                       seed);
    H3_CHECK_HIP(hipGetLastError());
    return H3FP8_OK;
}

int h3fp8_copy_silu_table(void* out, void* stream) {
    H3_REQUIRE(out, "h3fp8_copy_silu_table: null output");
    int st = h3host::ensure_device_init();
    if (st) return st;
    hipLaunchKernelGGL(h3_copy_table_kernel, dim3(65536 / 256), dim3(256), 0, (hipStream_t)stream, (uint16_t*)out);
    H3_CHECK_HIP(hipGetLastError());
    return H3FP8_OK;
}

}  // extern "C"
