// Kernel 2 (scaled FP8 GEMM, bf16/fp16 out, optional fused row-amax for the next layer's quant) and kernel 3 (the
// gate/up GEMM with the SwiGLU epilogue) on gfx950 MFMA.
//
// Contract (h3_tp2/fp8_gemm.py:44-50, :69-112; fp8_cutlass_kernel.py:698-733; fp8_swiglu.py:107-157):
//   y[m, n] = round(sa[m] * (sb[n] * acc[m, n])), acc = sum_k a[m, k] * w[n, k] in fp32, K ascending per
//   accumulator, no split-K; with a bias: round(fma(sa[m], sb[n] * acc, bias[n])).
//
// Tiling (one workgroup = 4 wavefronts = 256 threads, one workgroup per CU):
//   * block tile 256 (tokens m) x 256 (channels n) x 128 (k); each wave owns a 128 x 128 sub-tile: 8 x 8 MFMA tiles of
//     v_mfma_f32_16x16x128_f8f6f4 (e4m3 x e4m3 -> fp32), 256 fp32 accumulators per lane;
//   * the MFMA's A operand is the weight tile (rows n) and its B operand the activation tile (rows m), so a lane's four
//     accumulators of an MFMA tile are four consecutive channels n of one token m: the epilogue stores 8 bytes per lane;
//   * global -> LDS with buffer_load_dwordx4 ... lds (no VGPR staging): each instruction moves 8 rows x 128 bytes;
//     out-of-range rows and the K tail read as zero through the buffer descriptor's range check;
//   * LDS rows are 128 bytes (one k-step); 16-byte chunk c of row r is stored at chunk c ^ (r & 7), so the eight lanes
//     of an MFMA operand read that share a chunk index hit eight different bank groups;
//   * two LDS stages (2 x 64 KiB): the loads of k-step i+1 are in flight while k-step i is multiplied; one barrier
//     per k-step, after every wave's ds_reads of the stage have completed (lgkmcnt(0)) -- the stage-release rule;
//   * tile order: workgroups are spread over the 8 XCDs round-robin by the hardware, so the block index is remapped to
//     give every XCD a contiguous range of tiles, walked in groups of GROUP_M row tiles (L2 reuse of both operands).
// SwiGLU variant: the weight tile is 128 gate rows f0.. and the 128 matching up rows F+f0..; each wave holds the gate
// and up accumulators of the same (m, f) and applies fp8_swiglu.py:64-70 in registers.
#include <algorithm>

#include "h3fp8_common.h"

namespace {

using namespace h3;

constexpr int BM = 256;          // tokens per block tile
constexpr int BN = 256;          // weight rows per block tile
constexpr int BK = 128;          // k per step = one MFMA's K
constexpr int STAGE_BYTES = (BM + BN) * BK;   // 64 KiB
constexpr int NSTAGE = 2;
constexpr int LDS_BYTES = NSTAGE * STAGE_BYTES;
constexpr uint32_t OOB = 0x80000000u;         // an offset past every buffer's range: the load returns zeros

enum Epi { EPI_PLAIN = 0, EPI_AMAX = 1, EPI_SWIGLU = 2 };

struct GemmParams {
    const uint8_t* a;          // [M, K] e4m3, row stride lda
    const uint8_t* w;          // [Nw, K] e4m3, row stride ldw (Nw = N, or 2F for SwiGLU)
    const float* sa;
    const float* sb;
    const void* bias;
    void* y;                   // [M, N] (SwiGLU: [M, F])
    float* row_amax;           // EPI_AMAX / EPI_SWIGLU (may be null for SwiGLU)
    const uint16_t* silu;      // SwiGLU table
    int64_t lda, ldw, ldy;
    int64_t sa_stride, sb_stride;
    int M, N, K;               // SwiGLU: N = F (output width)
    uint32_t a_bytes, w_bytes; // buffer ranges
    int tiles_m, tiles_n;
    int group_m;
    int tile_offset;           // grouped launches: first block of this problem
};

__device__ __forceinline__ void waitcnt_vm0() { __builtin_amdgcn_s_waitcnt(0x0f70); }     // vmcnt(0)
__device__ __forceinline__ void waitcnt_lgkm0() { __builtin_amdgcn_s_waitcnt(0xc07f); }   // lgkmcnt(0)

// block index -> (tile_m, tile_n): XCD-contiguous ranges, then GROUP_M-row groups (column-major inside a group).
__device__ __forceinline__ void tile_of(int b, int T, int tiles_m, int tiles_n, int group_m, int& tm, int& tn) {
    const int xcd = b & 7, local = b >> 3;
    const int per = T >> 3, rem = T & 7;
    int lid = (xcd < rem) ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
    const int in_group = group_m * tiles_n;
    const int g = lid / in_group;
    const int first = g * group_m;
    const int gsz = min(tiles_m - first, group_m);
    const int r = lid - g * in_group;
    tm = first + r % gsz;
    tn = r / gsz;
}

__device__ __forceinline__ v8i read_frag(const uint8_t* region, int row, int g) {
    const uint8_t* p = region + row * BK;
    const int s = row & 7;
    uint4 lo = *reinterpret_cast<const uint4*>(p + (((2 * g) ^ s) << 4));
    uint4 hi = *reinterpret_cast<const uint4*>(p + (((2 * g + 1) ^ s) << 4));
    v8i f;
    f[0] = (int)lo.x; f[1] = (int)lo.y; f[2] = (int)lo.z; f[3] = (int)lo.w;
    f[4] = (int)hi.x; f[5] = (int)hi.y; f[6] = (int)hi.z; f[7] = (int)hi.w;
    return f;
}

__device__ __forceinline__ float load_bias(const void* bias, int n, int out_dt) {
    uint16_t b = reinterpret_cast<const uint16_t*>(bias)[n];
    return out_dt ? fp16_to_f32(b) : bf16_to_f32(b);
}

template <int OUT_DT, bool HAS_BIAS, int EPI>
__device__ __forceinline__ void gemm_body(const GemmParams& p, int bid, uint8_t* smem) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wn = wave & 1, wm = wave >> 1;

    int tile_m, tile_n;
    tile_of(bid, p.tiles_m * p.tiles_n, p.tiles_m, p.tiles_n, p.group_m, tile_m, tile_n);
    const int m0 = tile_m * BM;

    // ---- global -> LDS addressing ----
    // lane l of an instruction covers row (l >> 3) of an 8-row group and LDS chunk (l & 7), i.e. logical chunk
    // (l & 7) ^ (l >> 3) (the group starts at a multiple of 8 rows, so (row & 7) == (l >> 3)).
    const uint32_t lrow = (uint32_t)(lane >> 3);
    const uint32_t lchunk = (uint32_t)((lane & 7) ^ (lane >> 3));
    int64_t wrow0;   // first global weight row of this wave's 64-row share
    if (EPI == EPI_SWIGLU) {
        const int f0 = tile_n * (BN / 2);
        wrow0 = (wave < 2) ? (int64_t)f0 + 64 * wave : (int64_t)p.N + f0 + 64 * (wave - 2);
    } else {
        wrow0 = (int64_t)tile_n * BN + 64 * wave;
    }
    const int64_t arow0 = (int64_t)m0 + 64 * wave;
    __amdgpu_buffer_rsrc_t rw = make_rsrc(p.w, p.w_bytes);
    __amdgpu_buffer_rsrc_t ra = make_rsrc(p.a, p.a_bytes);
    // SwiGLU gate rows past F would read up rows: their groups are skipped below (F % 16 == 0 keeps groups whole).
    const uint32_t voff_w = (uint32_t)((wrow0 + lrow) * p.ldw) + 16u * lchunk;
    const uint32_t voff_a = (uint32_t)((arow0 + lrow) * p.lda) + 16u * lchunk;
    const uint32_t row8_w = (uint32_t)(8 * p.ldw), row8_a = (uint32_t)(8 * p.lda);
    // A 64-row share wholly past the end of an operand reads zeros; partial shares rely on the descriptor's range
    // check (rows >= M or >= N start past the last valid byte).  The scalar offset is always 0 so that the range
    // check sees the whole offset.
    uint32_t vw = voff_w, va = voff_a;
    const int64_t wlimit_rows = (EPI == EPI_SWIGLU) ? ((wave < 2) ? (int64_t)p.N : 2 * (int64_t)p.N) : (int64_t)p.N;
    const int w_groups = (int)min<int64_t>(8, max<int64_t>(0, (wlimit_rows - wrow0 + 7) / 8));
    if (wrow0 >= wlimit_rows) vw = OOB;
    if (arow0 >= p.M) va = OOB;

    const int nk = (p.K + BK - 1) / BK;

    v4f acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

    auto issue = [&](int ks) {
        uint8_t* stage = smem + (ks & 1) * STAGE_BYTES;
        const uint32_t k0 = (uint32_t)ks * BK;
        uint32_t vwk = vw, vak = va;
        if ((int)k0 + BK > p.K) {                           // K tail: chunks at or past K read zeros
            const bool dead = (k0 + 16u * lchunk) >= (uint32_t)p.K;
            vwk = dead ? OOB : vwk;
            vak = dead ? OOB : vak;
        }
        uint8_t* ldw_base = stage + wave * 64 * BK;
        uint8_t* lda_base = stage + BN * BK + wave * 64 * BK;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (EPI == EPI_SWIGLU && i >= w_groups) {
                // gate/up rows past F: zero-fill so no up row is multiplied as a gate row
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr_t)(ldw_base + i * 8 * BK), 16, OOB, 0, 0, 0);
            } else {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr_t)(ldw_base + i * 8 * BK), 16,
                                                         vwk + k0 + i * row8_w, 0, 0, 0);
            }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)(lda_base + i * 8 * BK), 16,
                                                     vak + k0 + i * row8_a, 0, 0, 0);
    };

    issue(0);
    waitcnt_vm0();
    __syncthreads();

    const int g = lane >> 4;        // k group of the MFMA operand (32 bytes per lane)
    const int r16 = lane & 15;
    for (int ks = 0; ks < nk; ++ks) {
        const uint8_t* stage = smem + (ks & 1) * STAGE_BYTES;
        const uint8_t* wreg = stage;
        const uint8_t* areg = stage + BN * BK;
        // Every ds_read of this stage is issued before the next stage's LDS-DMA loads: a read issued after a DMA
        // would make the compiler wait for that DMA (it cannot tell the two stages apart).
        v8i bf[8], af[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) bf[j] = read_frag(areg, wm * 128 + 16 * j + r16, g);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            int wr;
            if (EPI == EPI_SWIGLU) wr = (i < 4) ? (wn * 64 + 16 * i + r16) : (128 + wn * 64 + 16 * (i - 4) + r16);
            else wr = wn * 128 + 16 * i + r16;
            af[i] = read_frag(wreg, wr, g);
        }
        if (ks + 1 < nk) issue(ks + 1);
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af[i], bf[j], acc[i][j], 0, 0, 0, 0, 0, 0);
        // keep the wait for the next stage behind this stage's MFMAs (the scheduler would hoist it otherwise)
        __builtin_amdgcn_sched_barrier(0);
        waitcnt_vm0();
        waitcnt_lgkm0();
        __syncthreads();
    }

    // ---- epilogue ----
    const int q4 = lane >> 4;       // which 4 consecutive channels of the 16-wide MFMA tile
    if (EPI == EPI_SWIGLU) {
        const int F = p.N;
        const int fbase = tile_n * (BN / 2) + wn * 64;
        uint32_t rmax[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) rmax[j] = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int f = fbase + 16 * i + 4 * q4;
            if (f >= F) continue;
            float sbg[4], sbu[4], bg[4] = {0, 0, 0, 0}, bu[4] = {0, 0, 0, 0};
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                sbg[r] = p.sb[(int64_t)(f + r) * p.sb_stride];
                sbu[r] = p.sb[(int64_t)(F + f + r) * p.sb_stride];
                if (HAS_BIAS) { bg[r] = load_bias(p.bias, f + r, 0); bu[r] = load_bias(p.bias, F + f + r, 0); }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int m = m0 + wm * 128 + 16 * j + r16;
                if (m >= p.M) continue;
                const float sam = p.sa[(int64_t)m * p.sa_stride];
                uint32_t hb[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float tg = sbg[r] * acc[i][j][r];
                    const float tu = sbu[r] * acc[i + 4][j][r];
                    const float gy = HAS_BIAS ? __builtin_fmaf(sam, tg, bg[r]) : sam * tg;
                    const float uy = HAS_BIAS ? __builtin_fmaf(sam, tu, bu[r]) : sam * tu;
                    const uint32_t gb = bf16_rne(gy);
                    float u = bf16_to_f32(bf16_rne(uy));
                    u = (u == 0.0f) ? 0.0f : u;                       // -0 up -> +0 (fp8_swiglu.py:66)
                    const float s = bf16_to_f32(p.silu[gb]);
                    hb[r] = bf16_rne(s * u);
                    const uint32_t ab = (hb[r] & 0x7fffu) << 16;
                    rmax[j] = rmax[j] > ab ? rmax[j] : ab;
                }
                uint2 v = make_uint2(hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16));
                *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(p.y) + (int64_t)m * p.ldy + f) = v;
            }
        }
        if (p.row_amax) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                uint32_t v = rmax[j];
                uint32_t o = (uint32_t)__shfl_xor((int)v, 16, 64); v = v > o ? v : o;
                o = (uint32_t)__shfl_xor((int)v, 32, 64); v = v > o ? v : o;
                const int m = m0 + wm * 128 + 16 * j + r16;
                if (q4 == 0 && m < p.M && v) atomicMax(reinterpret_cast<unsigned int*>(p.row_amax) + m, v);
            }
        }
        return;
    }

    const int nbase = tile_n * BN + wn * 128;
    uint32_t rmax[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) rmax[j] = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int n = nbase + 16 * i + 4 * q4;
        if (n >= p.N) continue;
        float sbn[4], bn[4] = {0, 0, 0, 0};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            sbn[r] = p.sb[(int64_t)(n + r) * p.sb_stride];
            if (HAS_BIAS) bn[r] = load_bias(p.bias, n + r, OUT_DT);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int m = m0 + wm * 128 + 16 * j + r16;
            if (m >= p.M) continue;
            const float sam = p.sa[(int64_t)m * p.sa_stride];
            uint32_t o[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float t = sbn[r] * acc[i][j][r];
                const float v = HAS_BIAS ? __builtin_fmaf(sam, t, bn[r]) : sam * t;
                o[r] = OUT_DT ? fp16_rne(v) : bf16_rne(v);
                if (EPI == EPI_AMAX) {
                    const uint32_t ab = (o[r] & 0x7fffu) << 16;
                    rmax[j] = rmax[j] > ab ? rmax[j] : ab;
                }
            }
            uint2 v = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
            *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(p.y) + (int64_t)m * p.ldy + n) = v;
        }
    }
    if (EPI == EPI_AMAX) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t v = rmax[j];
            uint32_t o = (uint32_t)__shfl_xor((int)v, 16, 64); v = v > o ? v : o;
            o = (uint32_t)__shfl_xor((int)v, 32, 64); v = v > o ? v : o;
            const int m = m0 + wm * 128 + 16 * j + r16;
            if (q4 == 0 && m < p.M && v) atomicMax(reinterpret_cast<unsigned int*>(p.row_amax) + m, v);
        }
    }
}

template <int OUT_DT, bool HAS_BIAS, int EPI>
__global__ void __launch_bounds__(256, 1) gemm_kernel(GemmParams p) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
    gemm_body<OUT_DT, HAS_BIAS, EPI>(p, (int)blockIdx.x, smem);
}

struct GroupedParams {
    GemmParams g[H3FP8_MAX_GROUPS];
    int n;
};

// One launch over the concatenated tile spaces of up to H3FP8_MAX_GROUPS problems (bf16 out, no bias).
__global__ void __launch_bounds__(256, 1) gemm_grouped_kernel(GroupedParams gp) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
    const int b = (int)blockIdx.x;
    int i = 0;
#pragma unroll
    for (int j = 1; j < H3FP8_MAX_GROUPS; ++j)
        if (j < gp.n && b >= gp.g[j].tile_offset) i = j;
    gemm_body<0, false, EPI_PLAIN>(gp.g[i], b - gp.g[i].tile_offset, smem);
}

__global__ void __launch_bounds__(256) fill_zero_kernel(float* p, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0.0f;
}

int zero_rows(float* p, int64_t n, hipStream_t st) {
    if (n <= 0) return H3FP8_OK;
    hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p, n);
    H3_CHECK_HIP(hipGetLastError());
    return H3FP8_OK;
}

// Raises a kernel's dynamic-LDS limit to LDS_BYTES once per device.
int allow_lds(const void* fn, bool* done) {
    int dev = 0;
    H3_CHECK_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return H3FP8_EINVAL;
    if (!done[dev]) {
        H3_CHECK_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, LDS_BYTES));
        done[dev] = true;
    }
    return H3FP8_OK;
}

template <int OUT_DT, bool HAS_BIAS, int EPI>
int launch_one(const GemmParams& p, int blocks, hipStream_t st) {
    static bool done[64] = {};
    int rc = allow_lds((const void*)gemm_kernel<OUT_DT, HAS_BIAS, EPI>, done);
    if (rc) return rc;
    hipLaunchKernelGGL((gemm_kernel<OUT_DT, HAS_BIAS, EPI>), dim3(blocks), dim3(256), LDS_BYTES, st, p);
    H3_CHECK_HIP(hipGetLastError());
    return H3FP8_OK;
}

template <int EPI>
int dispatch(const GemmParams& p, int out_dt, bool has_bias, int blocks, hipStream_t st) {
    if (out_dt == H3FP8_DT_BF16) {
        return has_bias ? launch_one<0, true, EPI>(p, blocks, st) : launch_one<0, false, EPI>(p, blocks, st);
    }
    return has_bias ? launch_one<1, true, EPI>(p, blocks, st) : launch_one<1, false, EPI>(p, blocks, st);
}

constexpr int64_t kMaxBufferBytes = 0x7fff0000LL;   // buffer offsets are 32-bit; keep clear of the OOB marker

// Common argument checks; fills the fields that do not depend on the M range.
int check_gemm(const void* a, int64_t lda, const void* w, int64_t ldw, const float* sa, int64_t sa_stride,
               const float* sb, int64_t sb_stride, const void* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
               int64_t w_rows, const char* who) {
    H3_REQUIRE(M >= 0 && N >= 0 && K >= 0, "%s: negative size", who);
    H3_REQUIRE(K % 16 == 0 && N % 16 == 0, "%s: K=%lld and N=%lld must be multiples of 16", who, (long long)K,
               (long long)N);
    H3_REQUIRE(M <= 0x7fffffff && N <= 0x7fffffff && K <= 0x7fffffff, "%s: size too large", who);
    if (M == 0 || N == 0) return H3FP8_OK;
    H3_REQUIRE(a && w && sa && sb && y, "%s: null pointer", who);
    H3_REQUIRE(lda >= K && lda % 16 == 0 && ldw >= K && ldw % 16 == 0, "%s: lda/ldw must be >= K and multiples of 16",
               who);
    H3_REQUIRE(ldy >= N && ldy % 8 == 0, "%s: ldy must be >= N and a multiple of 8", who);
    H3_REQUIRE(((uintptr_t)a & 15) == 0 && ((uintptr_t)w & 15) == 0 && ((uintptr_t)y & 15) == 0,
               "%s: a, w and y must be 16-byte aligned", who);
    H3_REQUIRE(sa_stride >= 0 && sb_stride >= 0, "%s: negative scale stride", who);
    H3_REQUIRE((w_rows - 1) * ldw + K <= kMaxBufferBytes, "%s: weight too large for one buffer range", who);
    H3_REQUIRE(lda * 512 <= kMaxBufferBytes, "%s: lda too large", who);
    return H3FP8_OK;
}

GemmParams make_params(const uint8_t* a, int64_t lda, const uint8_t* w, int64_t ldw, const float* sa,
                       int64_t sa_stride, const float* sb, int64_t sb_stride, const void* bias, void* y, int64_t ldy,
                       int64_t M, int64_t N, int64_t K, int64_t w_rows, float* row_amax, const uint16_t* silu,
                       bool swiglu) {
    GemmParams p{};
    p.a = a; p.w = w; p.sa = sa; p.sb = sb; p.bias = bias; p.y = y; p.row_amax = row_amax; p.silu = silu;
    p.lda = lda; p.ldw = ldw; p.ldy = ldy;
    p.sa_stride = sa_stride; p.sb_stride = sb_stride;
    p.M = (int)M; p.N = (int)N; p.K = (int)K;
    p.a_bytes = (uint32_t)((M - 1) * lda + K);
    p.w_bytes = (uint32_t)((w_rows - 1) * ldw + K);
    const int64_t n_tile_cols = swiglu ? (BN / 2) : BN;
    p.tiles_m = (int)((M + BM - 1) / BM);
    p.tiles_n = (int)((N + n_tile_cols - 1) / n_tile_cols);
    p.group_m = 4;
    p.tile_offset = 0;
    return p;
}

// Launches one problem, splitting M so that every launch's activation range fits a 32-bit buffer offset.
int run_gemm(int epi, const uint8_t* a, int64_t lda, const uint8_t* w, int64_t ldw, const float* sa,
             int64_t sa_stride, const float* sb, int64_t sb_stride, const void* bias, void* y, int64_t ldy,
             int out_dt, int64_t M, int64_t N, int64_t K, int64_t w_rows, float* row_amax, const uint16_t* silu,
             hipStream_t st) {
    const int64_t rows_per = std::max<int64_t>(BM, ((kMaxBufferBytes - K) / lda + 1) / BM * BM);
    for (int64_t r0 = 0; r0 < M; r0 += rows_per) {
        const int64_t Mi = std::min<int64_t>(rows_per, M - r0);
        GemmParams p = make_params(a + r0 * lda, lda, w, ldw, sa + r0 * sa_stride, sa_stride, sb, sb_stride, bias,
                                   reinterpret_cast<uint16_t*>(y) + r0 * ldy, ldy, Mi, N, K, w_rows,
                                   row_amax ? row_amax + r0 : nullptr, silu, epi == EPI_SWIGLU);
        const int blocks = p.tiles_m * p.tiles_n;
        int rc;
        if (epi == EPI_PLAIN) rc = dispatch<EPI_PLAIN>(p, out_dt, bias != nullptr, blocks, st);
        else if (epi == EPI_AMAX) rc = dispatch<EPI_AMAX>(p, out_dt, bias != nullptr, blocks, st);
        else rc = dispatch<EPI_SWIGLU>(p, H3FP8_DT_BF16, bias != nullptr, blocks, st);
        if (rc) return rc;
    }
    return H3FP8_OK;
}

}  // namespace

namespace h3host {
int quant_rows_amax_launch(const void* x, int64_t ldx, int64_t M, int64_t K, const float* row_amax, void* q,
                           int64_t ldq, float* scale, hipStream_t st);
}

extern "C" {

int h3fp8_gemm(const void* a, int64_t lda, const void* w, int64_t ldw, const float* sa, int64_t sa_stride,
               const float* sb, int64_t sb_stride, const void* bias, void* y, int64_t ldy, int out_dtype, int64_t M,
               int64_t N, int64_t K, float* row_amax, void* stream) {
    int rc = check_gemm(a, lda, w, ldw, sa, sa_stride, sb, sb_stride, y, ldy, M, N, K, N, "h3fp8_gemm");
    if (rc) return rc;
    H3_REQUIRE(out_dtype == H3FP8_DT_BF16 || out_dtype == H3FP8_DT_FP16, "h3fp8_gemm: bad out_dtype %d", out_dtype);
    if (M == 0 || N == 0) return H3FP8_OK;
    hipStream_t st = (hipStream_t)stream;
    if (row_amax) {
        rc = zero_rows(row_amax, M, st);
        if (rc) return rc;
    }
    return run_gemm(row_amax ? EPI_AMAX : EPI_PLAIN, (const uint8_t*)a, lda, (const uint8_t*)w, ldw, sa, sa_stride, sb,
                    sb_stride, bias, y, ldy, out_dtype, M, N, K, N, row_amax, nullptr, st);
}

int h3fp8_gemm_quant(const void* a, int64_t lda, const void* w, int64_t ldw, const float* sa, int64_t sa_stride,
                     const float* sb, int64_t sb_stride, const void* bias, void* y, int64_t ldy, int64_t M, int64_t N,
                     int64_t K, float* amax_ws, void* q, int64_t ldq, float* scale, void* stream) {
    H3_REQUIRE(M == 0 || (amax_ws && q && scale), "h3fp8_gemm_quant: null workspace or output");
    int rc = h3fp8_gemm(a, lda, w, ldw, sa, sa_stride, sb, sb_stride, bias, y, ldy, H3FP8_DT_BF16, M, N, K, amax_ws,
                        stream);
    if (rc) return rc;
    return h3host::quant_rows_amax_launch(y, ldy, M, N, amax_ws, q, ldq, scale, (hipStream_t)stream);
}

int h3fp8_gemm_swiglu(const void* a, int64_t lda, const void* w_gate_up, int64_t ldw, const float* sa,
                      int64_t sa_stride, const float* sb, int64_t sb_stride, const void* bias, void* h, int64_t ldh,
                      float* row_amax, int64_t M, int64_t F, int64_t K, void* stream) {
    int rc = check_gemm(a, lda, w_gate_up, ldw, sa, sa_stride, sb, sb_stride, h, ldh, M, F, K, 2 * F,
                        "h3fp8_gemm_swiglu");
    if (rc) return rc;
    if (M == 0 || F == 0) return H3FP8_OK;
    rc = h3host::ensure_device_init();
    if (rc) return rc;
    hipStream_t st = (hipStream_t)stream;
    if (row_amax) {
        rc = zero_rows(row_amax, M, st);
        if (rc) return rc;
    }
    return run_gemm(EPI_SWIGLU, (const uint8_t*)a, lda, (const uint8_t*)w_gate_up, ldw, sa, sa_stride, sb, sb_stride,
                    bias, h, ldh, H3FP8_DT_BF16, M, F, K, 2 * F, row_amax, h3host::silu_table_ptr(), st);
}

int h3fp8_gemm_swiglu_quant(const void* a, int64_t lda, const void* w_gate_up, int64_t ldw, const float* sa,
                            int64_t sa_stride, const float* sb, int64_t sb_stride, const void* bias, int64_t M,
                            int64_t F, int64_t K, void* h_ws, float* amax_ws, void* q, int64_t ldq, float* scale,
                            void* stream) {
    H3_REQUIRE(M == 0 || (h_ws && amax_ws && q && scale), "h3fp8_gemm_swiglu_quant: null workspace or output");
    int rc = h3fp8_gemm_swiglu(a, lda, w_gate_up, ldw, sa, sa_stride, sb, sb_stride, bias, h_ws, F, amax_ws, M, F, K,
                               stream);
    if (rc) return rc;
    return h3host::quant_rows_amax_launch(h_ws, F, M, F, amax_ws, q, ldq, scale, (hipStream_t)stream);
}

int h3fp8_grouped_gemm(const h3fp8_group* groups, int n_groups, void* stream) {
    H3_REQUIRE(groups && n_groups >= 0 && n_groups <= H3FP8_MAX_GROUPS, "h3fp8_grouped_gemm: bad group list");
    GroupedParams gp{};
    int blocks = 0;
    for (int i = 0; i < n_groups; ++i) {
        const h3fp8_group& g = groups[i];
        int rc = check_gemm(g.a, g.lda, g.w, g.ldw, g.sa, g.sa_stride, g.sb, g.sb_stride, g.y, g.ldy, g.M, g.N, g.K,
                            g.N, "h3fp8_grouped_gemm");
        if (rc) return rc;
        H3_REQUIRE(g.M == 0 || (g.M - 1) * g.lda + g.K <= kMaxBufferBytes,
                   "h3fp8_grouped_gemm: group %d activation too large for one launch", i);
        if (g.M == 0 || g.N == 0) continue;
        GemmParams p = make_params((const uint8_t*)g.a, g.lda, (const uint8_t*)g.w, g.ldw, g.sa, g.sa_stride, g.sb,
                                   g.sb_stride, nullptr, g.y, g.ldy, g.M, g.N, g.K, g.N, nullptr, nullptr, false);
        p.tile_offset = blocks;
        blocks += p.tiles_m * p.tiles_n;
        gp.g[gp.n++] = p;
    }
    if (blocks == 0) return H3FP8_OK;
    static bool done[64] = {};
    int rc = allow_lds((const void*)gemm_grouped_kernel, done);
    if (rc) return rc;
    hipLaunchKernelGGL(gemm_grouped_kernel, dim3(blocks), dim3(256), LDS_BYTES, (hipStream_t)stream, gp);
    H3_CHECK_HIP(hipGetLastError());
    return H3FP8_OK;
}

}  // extern "C"
