// Kernel 2 (scaled FP8 GEMM, bf16/fp16 out, optional fused row-amax for the next layer's quant) and kernel 3 (the
// gate/up GEMM with the SwiGLU epilogue) on gfx950 MFMA.
//
// Contract (h3_tp2/fp8_gemm.py:44-50, :69-112; fp8_cutlass_kernel.py:698-733; fp8_swiglu.py:107-157):
//   y[m, n] = round(sa[m] * (sb[n] * acc[m, n])), acc = sum_k a[m, k] * w[n, k] in fp32, K ascending per
//   accumulator, no split-K; with a bias: round(fma(sa[m], sb[n] * acc, bias[n])).
//
// Tiling (one workgroup = 4 wavefronts = 256 threads, one workgroup per CU):
//   * block tile 256 (tokens m) x 256 (channels n) x 128 (k); each wave owns a 128 x 128 sub-tile: 4 x 4 MFMA tiles of
//     v_mfma_f32_32x32x64_f8f6f4 (e4m3 x e4m3 -> fp32), two k sub-steps per stage, 256 fp32 accumulators per lane (the
//     AGPR file);
//   * the MFMA's A operand is the weight tile (rows n) and its B operand the activation tile (rows m), so each group of
//     four accumulators of a lane holds four consecutive channels n of one token m: the epilogue stores 8 bytes;
//   * global -> LDS with buffer_load_dwordx4 ... lds (no VGPR staging): each instruction moves 8 rows x 128 bytes, i.e.
//     whole 128-byte lines (64-byte row pieces halve the load path's throughput: measured 22 vs 40 bytes/clk/CU);
//     out-of-range rows and the K tail read as zero through the buffer descriptor's range check;
//   * two LDS stages (2 x 64 KiB); a stage is released by a barrier right after the last reads of its k-step (early in
//     the step), so the loads of k-step i+2 run during about 44 MFMAs (about 1.5 k-steps);
//   * LDS rows are 128 bytes; 16-byte chunk c of row r is stored at chunk c ^ swz(r), swz(r) = ((r >> 1) & 7) ^
//     ((r & 1) << 2): eight consecutive rows (32 banks) and sixteen (64 banks) read at one logical chunk never share a
//     bank (conflict-free ds_read_b128);
//   * operand fragments are double-buffered in VGPRs: sub-step 1 is read while sub-step 0 multiplies, and the next
//     stage's sub-step 0 right after the barrier that publishes it, while the last MFMAs of the step run;
//   * stage release: a stage is refilled only after a barrier that every wave reaches with lgkmcnt(0), i.e. after all
//     of its ds_reads have returned;
//   * tile order: workgroups are spread over the 8 XCDs round-robin by the hardware, so the block index is remapped to
//     give every XCD a contiguous range of tiles, walked in groups of GROUP_M row tiles (L2 reuse of both operands).
// SwiGLU variant: the weight tile is 128 gate rows f0.. and the 128 matching up rows F+f0..; each wave holds the gate
// and up accumulators of the same (m, f) and applies fp8_swiglu.py:64-70 in registers.
#include <algorithm>

#include "h3fp8_common.h"

namespace {

using namespace h3;

typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int BM = 256;          // tokens per block tile
constexpr int BN = 256;          // weight rows per block tile
constexpr int BK = 128;          // k per stage: 128-byte row pieces
constexpr int ROWB = BK;         // bytes per LDS row
constexpr int STAGE_BYTES = (BM + BN) * ROWB;   // 64 KiB
constexpr int NSTAGE = 2;
constexpr int A_REGION = BN * ROWB;             // activation rows start after the weight rows
constexpr int MFMA_SPLIT = 12;                  // sub-step-1 MFMAs issued before the stage barrier (of 16)
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

// LDS chunk swizzle (see the header): logical 16-byte chunk c of row r is stored at chunk c ^ swz(r).
__device__ __forceinline__ int swz(int r) { return ((r >> 1) & 7) ^ ((r & 1) << 2); }

// One 32 x 64 MFMA operand of k sub-step `sub`: lane l reads row (l & 31) of the tile, logical chunks 4 sub + 2h and
// 4 sub + 2h + 1 (h = l >> 5).  Tile bases are multiples of 32 rows, so swz of the tile row equals swz of the LDS row.
__device__ __forceinline__ v8i read_frag(const uint8_t* tile, int lane, int sub) {
    const int row = lane & 31, h = lane >> 5;
    const uint8_t* p = tile + row * ROWB;
    const int s = swz(row);
    const int c0 = 4 * sub + 2 * h;
    const uint4 lo = *reinterpret_cast<const uint4*>(p + ((c0 ^ s) << 4));
    const uint4 hi = *reinterpret_cast<const uint4*>(p + (((c0 + 1) ^ s) << 4));
    v8i f;
    f[0] = (int)lo.x; f[1] = (int)lo.y; f[2] = (int)lo.z; f[3] = (int)lo.w;
    f[4] = (int)hi.x; f[5] = (int)hi.y; f[6] = (int)hi.z; f[7] = (int)hi.w;
    return f;
}

__device__ __forceinline__ float load_bias(const void* bias, int n, int out_dt) {
    uint16_t b = reinterpret_cast<const uint16_t*>(bias)[n];
    return out_dt ? fp16_to_f32(b) : bf16_to_f32(b);
}

// s_waitcnt immediate for vmcnt(n) alone (gfx9 encoding: vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14, expcnt
// and lgkmcnt left at their maxima).
constexpr int vmcnt_imm(int n) { return (n & 0xf) | ((n >> 4) << 14) | (0x7 << 4) | (0xf << 8); }

__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt(vmcnt_imm(0)); }

__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xc07f); }

// Workgroup barrier without a memory-model fence: __syncthreads() would add a release fence that waits for every
// in-flight LDS-DMA load (vmcnt(0)), including the k-steps still being prefetched.  The explicit vmcnt/lgkmcnt waits
// before it carry the ordering; the "memory" clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void barrier_nofence() { asm volatile("s_barrier" ::: "memory"); }

// A buffer descriptor as four dwords (base, stride 0, num_records = byte range, gfx9 raw-buffer flags); loads at
// offsets >= num_records return zeros.
__device__ __forceinline__ v4u buffer_desc(const void* base, uint32_t bytes) {
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    v4u d;
    d[0] = __builtin_amdgcn_readfirstlane((uint32_t)b);
    d[1] = __builtin_amdgcn_readfirstlane((uint32_t)(b >> 32) & 0xffffu);
    d[2] = __builtin_amdgcn_readfirstlane(bytes);
    d[3] = 0x00020000u;
    return d;
}

// 16 bytes per lane from a buffer straight into LDS at lds_base + 16 * lane (buffer_load_dwordx4 ... lds).
// Written as inline asm so that the compiler's wait-count pass does not track these loads: it cannot tell one LDS
// stage from another and would wait for every in-flight load before each LDS read.  The kernel therefore places
// every wait on these loads itself (wait_vm before the barrier that publishes a stage).
__device__ __forceinline__ void dma16(v4u desc, uint32_t lds_base, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(lds_base), "v"(voff), "s"(desc)
                 : "memory", "m0");
}

__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) {
    typedef const __attribute__((address_space(3))) uint8_t* lds_u8;
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_u8)(p));
}

// Per-wave state of the mainloop.
struct Loader {
    v4u rw, ra;
    uint32_t vw[2], va[2];      // lane part of the byte offsets for even / odd instructions (OOB: share out of range)
    uint32_t c16[2];            // 16 * logical chunk of this lane for even / odd instructions
    uint32_t row8_w, row8_a;    // byte advance of 8 rows
    int K;
    int w_groups;               // SwiGLU: 8-row groups of this wave's weight share that are in range
};

// One wave's share of a stage: 8 instructions for its 64 weight rows (i = 0..7), 8 for its 64 token rows (i = 8..15).
struct StageIssue {
    uint32_t wdst, adst;        // LDS addresses of the wave's weight / token rows in the stage
    uint32_t vw[2], va[2];      // byte offsets of the lane for even / odd instructions, k0 included
};

template <int EPI>
__device__ __forceinline__ StageIssue stage_issue(uint8_t* stage, const Loader& L, int wave, int ks) {
    StageIssue S;
    const uint32_t k0 = (uint32_t)ks * BK;
    const bool tail = (int)k0 + BK > L.K;                      // K tail: chunks at or past K read zeros
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const bool dead = tail && (k0 + L.c16[e]) >= (uint32_t)L.K;
        S.vw[e] = dead ? OOB : L.vw[e] + k0;
        S.va[e] = dead ? OOB : L.va[e] + k0;
    }
    S.wdst = lds_addr(stage + wave * 64 * ROWB);
    S.adst = lds_addr(stage + A_REGION + wave * 64 * ROWB);
    return S;
}

template <int EPI>
__device__ __forceinline__ void issue_one(const StageIssue& S, const Loader& L, int i) {
    if (i < 8) {
        const uint32_t off = (EPI == EPI_SWIGLU && i >= L.w_groups) ? OOB : S.vw[i & 1] + i * L.row8_w;
        dma16(L.rw, S.wdst + i * 8 * ROWB, off);
    } else {
        dma16(L.ra, S.adst + (i - 8) * 8 * ROWB, S.va[i & 1] + (i - 8) * L.row8_a);
    }
}

template <int EPI>
__device__ __forceinline__ void issue_stage(uint8_t* stage, const Loader& L, int wave, int ks) {
    const StageIssue S = stage_issue<EPI>(stage, L, wave, ks);
#pragma unroll
    for (int i = 0; i < 16; ++i) issue_one<EPI>(S, L, i);
}

// Weight-tile row of MFMA tile tn (0..3) of wave column wn.
template <int EPI>
__device__ __forceinline__ int w_tile_row(int wn, int tn) {
    if (EPI == EPI_SWIGLU) return (tn < 2) ? (wn * 64 + 32 * tn) : (128 + wn * 64 + 32 * (tn - 2));
    return wn * 128 + 32 * tn;
}

template <int EPI>
__device__ __forceinline__ void read_frags(const uint8_t* stage, int wn, int wm, int lane, int sub, v8i af[4],
                                           v8i bf[4]) {
#pragma unroll
    for (int t = 0; t < 4; ++t) af[t] = read_frag(stage + w_tile_row<EPI>(wn, t) * ROWB, lane, sub);
#pragma unroll
    for (int t = 0; t < 4; ++t) bf[t] = read_frag(stage + A_REGION + (wm * 128 + 32 * t) * ROWB, lane, sub);
}

// Fragment f of a sub-step: f = 0..3 weight tiles, 4..7 token tiles.
template <int EPI>
__device__ __forceinline__ void read_one(const uint8_t* stage, int wn, int wm, int lane, int sub, int f, v8i af[4],
                                         v8i bf[4]) {
    if (f < 4) af[f] = read_frag(stage + w_tile_row<EPI>(wn, f) * ROWB, lane, sub);
    else bf[f - 4] = read_frag(stage + A_REGION + (wm * 128 + 32 * (f - 4)) * ROWB, lane, sub);
}

__device__ __forceinline__ void mfma_one(v16f acc[4][4], const v8i af[4], const v8i bf[4], int t) {
    acc[t >> 2][t & 3] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(af[t >> 2], bf[t & 3], acc[t >> 2][t & 3], 0, 0,
                                                                         0, 0, 0, 0);
}

// MFMAs number lo .. hi-1 of the 16 of one sub-step (tile (i, j) = MFMA 4 i + j).
__device__ __forceinline__ void mfma_range(v16f acc[4][4], const v8i af[4], const v8i bf[4], int lo, int hi) {
#pragma unroll
    for (int t = 0; t < 16; ++t)
        if (t >= lo && t < hi)
            acc[t >> 2][t & 3] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(af[t >> 2], bf[t & 3], acc[t >> 2][t & 3],
                                                                                 0, 0, 0, 0, 0, 0);
}

// One k-step.  On entry stage ks & 1 holds k-step ks, its sub-step-0 fragments are in f0, and the loads of k-step
// ks+1 into the other stage are in flight.
//   phase A: the 16 sub-step-0 MFMAs, with the reads of the 8 sub-step-1 fragments issued between the first 8;
//   barrier 1 (after lgkmcnt(0)): every wave's reads of this stage have returned -- the stage is free;
//   phase B: the 16 sub-step-1 MFMAs, with the 16 load instructions of k-step ks+2 into the freed stage issued two per
//   MFMA between the first 8 (loads and reads are spread between MFMAs so that a stalled issue of a memory instruction
//   never holds the matrix core idle), then, once this wave's share of k-step ks+1 has landed (vmcnt(16)), barrier 2
//   publishes it and the sub-step-0 fragments of ks+1 are read between the last MFMA_SPLIT..15 MFMAs.
// The loads of k-step ks+2 therefore have about 1.5 k-steps (about 40 MFMAs) to land.
template <int EPI>
__device__ __forceinline__ void kstep(uint8_t* lds, const Loader& L, int wave, int wn, int wm, int lane, int ks, int nk,
                                      v16f acc[4][4], v8i fa0[4], v8i fb0[4], v8i fa1[4], v8i fb1[4]) {
    uint8_t* cur = lds + (ks & 1) * STAGE_BYTES;
    uint8_t* nxt = lds + ((ks + 1) & 1) * STAGE_BYTES;
#pragma unroll
    for (int t = 0; t < 16; ++t) {
        mfma_one(acc, fa0, fb0, t);
        if (t < 8) read_one<EPI>(cur, wn, wm, lane, 1, t, fa1, fb1);
        __builtin_amdgcn_sched_barrier(0);
    }
    wait_lgkm0();                                       // this wave's reads of stage ks & 1 have returned
    barrier_nofence();                                  // ... and every wave's: the stage is free
    const bool load2 = ks + 2 < nk;
    const StageIssue S = stage_issue<EPI>(cur, L, wave, ks + 2);
#pragma unroll
    for (int t = 0; t < 16; ++t) {
        mfma_one(acc, fa1, fb1, t);
        if (t < 8 && load2) {
            issue_one<EPI>(S, L, 2 * t);
            issue_one<EPI>(S, L, 2 * t + 1);
        }
        if (t == MFMA_SPLIT - 1 && ks + 1 < nk) {
            if (load2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(16));     // k-step ks+1 landed (ks+2 may be in flight)
            else wait_vm0();
            barrier_nofence();
        }
        if (t >= MFMA_SPLIT && ks + 1 < nk) {
            // spread the 8 fragment reads of k-step ks+1 over the MFMAs after barrier 2
            constexpr int PER = (8 + (16 - MFMA_SPLIT) - 1) / (16 - MFMA_SPLIT);
#pragma unroll
            for (int f = (t - MFMA_SPLIT) * PER; f < (t - MFMA_SPLIT + 1) * PER; ++f)
                if (f < 8) read_one<EPI>(nxt, wn, wm, lane, 0, f, fa0, fb0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

template <int OUT_DT, bool HAS_BIAS, int EPI>
__device__ __forceinline__ void gemm_body(const GemmParams& p, int bid) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[NSTAGE * STAGE_BYTES];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wn = wave & 1, wm = wave >> 1;

    int tile_m, tile_n;
    tile_of(bid, p.tiles_m * p.tiles_n, p.tiles_m, p.tiles_n, p.group_m, tile_m, tile_n);
    const int m0 = tile_m * BM;

    // ---- global -> LDS addressing ----
    // lane l of an instruction covers row (l >> 3) of an 8-row group and LDS chunk (l & 7), i.e. logical chunk
    // (l & 7) ^ swz(row); swz depends on the row's bits 0..3, so even and odd groups of 8 rows differ.
    Loader L;
    const uint32_t lrow = (uint32_t)(lane >> 3);
    // LDS chunk of the lane is lane & 7; its row is 8 i + lrow of the share (even i: row & 8 == 0, odd i: 8)
    const uint32_t lch[2] = {(uint32_t)((lane & 7) ^ swz((int)lrow)), (uint32_t)((lane & 7) ^ swz((int)lrow + 8))};
    int64_t wrow0;   // first global weight row of this wave's 64-row share
    int64_t wlimit;  // rows of this share's source range (SwiGLU gate rows stop at F)
    if (EPI == EPI_SWIGLU) {
        const int f0 = tile_n * (BN / 2);
        wrow0 = (wave < 2) ? (int64_t)f0 + 64 * wave : (int64_t)p.N + f0 + 64 * (wave - 2);
        wlimit = (wave < 2) ? (int64_t)p.N : 2 * (int64_t)p.N;
    } else {
        wrow0 = (int64_t)tile_n * BN + 64 * wave;
        wlimit = p.N;
    }
    const int64_t arow0 = (int64_t)m0 + 64 * wave;
    L.rw = buffer_desc(p.w, p.w_bytes);
    L.ra = buffer_desc(p.a, p.a_bytes);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        L.c16[e] = 16u * lch[e];
        L.vw[e] = (wrow0 >= wlimit) ? OOB : (uint32_t)((wrow0 + lrow) * p.ldw) + L.c16[e];
        L.va[e] = (arow0 >= p.M) ? OOB : (uint32_t)((arow0 + lrow) * p.lda) + L.c16[e];
    }
    L.row8_w = (uint32_t)(8 * p.ldw);
    L.row8_a = (uint32_t)(8 * p.lda);
    L.K = p.K;
    // Partial shares rely on the descriptor's range check (rows >= M or >= N start past the last valid byte), except
    // SwiGLU gate rows past F, which would read up rows: those 8-row groups are zero-filled (F % 16 == 0).
    L.w_groups = (int)min<int64_t>(8, max<int64_t>(0, (wlimit - wrow0 + 7) / 8));

    const int nk = (p.K + BK - 1) / BK;             // k-steps of 128

    v16f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // prologue: k-steps 0 and 1 in flight, the sub-step-0 fragments of k-step 0 in registers
    v8i fa0[4], fb0[4], fa1[4], fb1[4];
    issue_stage<EPI>(lds, L, wave, 0);
    if (nk > 1) {
        issue_stage<EPI>(lds + STAGE_BYTES, L, wave, 1);
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(16));
    } else {
        wait_vm0();
    }
    barrier_nofence();
    read_frags<EPI>(lds, wn, wm, lane, 0, fa0, fb0);
    for (int ks = 0; ks < nk; ++ks) kstep<EPI>(lds, L, wave, wn, wm, lane, ks, nk, acc, fa0, fb0, fa1, fb1);

    // ---- epilogue ----
    // The scaled, rounded outputs go through LDS so that global stores are whole 16-byte pieces of contiguous row
    // segments (a wave's 128 x 128 tile leaves the MFMA layout with only 8 contiguous bytes per lane and row).
    // 32x32 MFMA result: lane l, register 4q + r holds D[8q + 4(l >> 5) + r][l & 31], i.e. channel
    // n = tile_n_base + 8q + 4(l >> 5) + r of token m = tile_m_base + (l & 31).
    if (OUT_DT == H3FP8_DT_F32) {
        // probe mode: the raw fp32 accumulators, scales / bias / rounding not applied (16-byte stores per lane)
        float* yf = reinterpret_cast<float*>(p.y);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int n = tile_n * BN + wn * 128 + 32 * i + 8 * q + 4 * (lane >> 5);
                    const int m = m0 + wm * 128 + 32 * j + (lane & 31);
                    if (n < p.N && m < p.M) {
                        const v4f v = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                                       acc[i][j][4 * q + 3]};
                        *reinterpret_cast<v4f*>(yf + (int64_t)m * p.ldy + n) = v;
                    }
                }
        return;
    }
    wait_lgkm0();
    barrier_nofence();                                  // every wave is done with the stages: reuse the LDS
    constexpr int OUT_COLS = (EPI == EPI_SWIGLU) ? 64 : 128;   // output columns per wave
    constexpr int ROW_BYTES = OUT_COLS * 2;
    constexpr int CHUNKS = ROW_BYTES / 16;                       // 16-byte chunks per row: 16 or 8
    uint8_t* tile = lds + wave * (128 * ROW_BYTES);
    // element (ml, cl) of the wave tile: row ml, 16-byte chunk (cl / 8) ^ (ml % CHUNKS), 8-byte half (cl / 4) % 2
    auto put4 = [&](int ml, int cl, uint32_t lo, uint32_t hi2) {
        const int ch = (cl >> 3) ^ (ml & (CHUNKS - 1));
        *reinterpret_cast<uint2*>(tile + ml * ROW_BYTES + ch * 16 + ((cl >> 2) & 1) * 8) = make_uint2(lo, hi2);
    };
    const int hi = lane >> 5;
    const int mj = lane & 31;
    const int mrow0 = m0 + wm * 128;
    uint32_t rmax[4] = {0, 0, 0, 0};
    float sam[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int m = mrow0 + 32 * j + mj;
        sam[j] = (m < p.M) ? p.sa[(int64_t)m * p.sa_stride] : 0.0f;
    }
    int col0, ncols;                                    // first output column of the wave, output width
    if (EPI == EPI_SWIGLU) {
        const int F = p.N;
        col0 = tile_n * (BN / 2) + wn * 64;
        ncols = F;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int cl = 32 * t + 8 * q + 4 * hi;
                const int f = col0 + cl;
                const bool fok = f < F;
                float sbg[4], sbu[4], bg[4] = {0, 0, 0, 0}, bu[4] = {0, 0, 0, 0};
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    sbg[r] = fok ? p.sb[(int64_t)(f + r) * p.sb_stride] : 0.0f;
                    sbu[r] = fok ? p.sb[(int64_t)(F + f + r) * p.sb_stride] : 0.0f;
                    if (HAS_BIAS && fok) { bg[r] = load_bias(p.bias, f + r, 0); bu[r] = load_bias(p.bias, F + f + r, 0); }
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const bool ok = fok && (mrow0 + 32 * j + mj < p.M);
                    uint32_t hb[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float tg = sbg[r] * acc[t][j][4 * q + r];
                        const float tu = sbu[r] * acc[t + 2][j][4 * q + r];
                        const float gy = HAS_BIAS ? __builtin_fmaf(sam[j], tg, bg[r]) : sam[j] * tg;
                        const float uy = HAS_BIAS ? __builtin_fmaf(sam[j], tu, bu[r]) : sam[j] * tu;
                        const uint32_t gb = bf16_rne(gy);
                        float u = bf16_to_f32(bf16_rne(uy));
                        u = (u == 0.0f) ? 0.0f : u;                       // -0 up -> +0 (fp8_swiglu.py:66)
                        const float sl = bf16_to_f32(p.silu[gb]);
                        hb[r] = bf16_rne(sl * u);
                        const uint32_t ab = ok ? ((hb[r] & 0x7fffu) << 16) : 0u;
                        rmax[j] = rmax[j] > ab ? rmax[j] : ab;
                    }
                    put4(32 * j + mj, cl, hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16));
                }
            }
        }
    } else {
        col0 = tile_n * BN + wn * 128;
        ncols = p.N;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int cl = 32 * i + 8 * q + 4 * hi;
                const int n = col0 + cl;
                const bool nok = n < p.N;
                float sbn[4], bn[4] = {0, 0, 0, 0};
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    sbn[r] = nok ? p.sb[(int64_t)(n + r) * p.sb_stride] : 0.0f;
                    if (HAS_BIAS && nok) bn[r] = load_bias(p.bias, n + r, OUT_DT);
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const bool ok = nok && (mrow0 + 32 * j + mj < p.M);
                    uint32_t o[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float t = sbn[r] * acc[i][j][4 * q + r];
                        const float v = HAS_BIAS ? __builtin_fmaf(sam[j], t, bn[r]) : sam[j] * t;
                        o[r] = OUT_DT ? fp16_rne(v) : bf16_rne(v);
                        if (EPI == EPI_AMAX) {
                            const uint32_t ab = ok ? ((o[r] & 0x7fffu) << 16) : 0u;
                            rmax[j] = rmax[j] > ab ? rmax[j] : ab;
                        }
                    }
                    put4(32 * j + mj, cl, o[0] | (o[1] << 16), o[2] | (o[3] << 16));
                }
            }
        }
    }
    if (EPI == EPI_AMAX || (EPI == EPI_SWIGLU && p.row_amax)) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t v = rmax[j];
            const uint32_t o = (uint32_t)__shfl_xor((int)v, 32, 64);
            v = v > o ? v : o;
            const int m = mrow0 + 32 * j + mj;
            if (hi == 0 && m < p.M && v) atomicMax(reinterpret_cast<unsigned int*>(p.row_amax) + m, v);
        }
    }
    // the wave reads back its own tile (LDS accesses of one wave complete in order): 16 bytes per lane, CHUNKS lanes
    // per row, whole row segments per store instruction
    constexpr int ROWS_PER_PASS = 64 / CHUNKS;
    const int c = lane % CHUNKS;
    const int col = col0 + c * 8;
    uint16_t* ybase = reinterpret_cast<uint16_t*>(p.y);
#pragma unroll 4
    for (int it = 0; it < 128 / ROWS_PER_PASS; ++it) {
        const int ml = it * ROWS_PER_PASS + lane / CHUNKS;
        const uint4 v = *reinterpret_cast<const uint4*>(tile + ml * ROW_BYTES + ((c ^ (ml & (CHUNKS - 1))) << 4));
        const int m = mrow0 + ml;
        if (m < p.M && col < ncols) *reinterpret_cast<uint4*>(ybase + (int64_t)m * p.ldy + col) = v;
    }
}

template <int OUT_DT, bool HAS_BIAS, int EPI>
__global__ void __launch_bounds__(256, 1) gemm_kernel(GemmParams p) {
    gemm_body<OUT_DT, HAS_BIAS, EPI>(p, (int)blockIdx.x);
}

struct GroupedParams {
    GemmParams g[H3FP8_MAX_GROUPS];
    int n;
};

// One launch over the concatenated tile spaces of up to H3FP8_MAX_GROUPS problems (bf16 out, no bias).
__global__ void __launch_bounds__(256, 1) gemm_grouped_kernel(GroupedParams gp) {
    const int b = (int)blockIdx.x;
    int i = 0;
#pragma unroll
    for (int j = 1; j < H3FP8_MAX_GROUPS; ++j)
        if (j < gp.n && b >= gp.g[j].tile_offset) i = j;
    gemm_body<0, false, EPI_PLAIN>(gp.g[i], b - gp.g[i].tile_offset);
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

template <int OUT_DT, bool HAS_BIAS, int EPI>
int launch_one(const GemmParams& p, int blocks, hipStream_t st) {
    hipLaunchKernelGGL((gemm_kernel<OUT_DT, HAS_BIAS, EPI>), dim3(blocks), dim3(256), 0, st, p);
    H3_CHECK_HIP(hipGetLastError());
    return H3FP8_OK;
}

template <int EPI>
int dispatch(const GemmParams& p, int out_dt, bool has_bias, int blocks, hipStream_t st) {
    if (out_dt == H3FP8_DT_BF16) {
        return has_bias ? launch_one<0, true, EPI>(p, blocks, st) : launch_one<0, false, EPI>(p, blocks, st);
    }
    if (out_dt == H3FP8_DT_F32) return launch_one<H3FP8_DT_F32, false, EPI_PLAIN>(p, blocks, st);
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
    H3_REQUIRE(out_dtype == H3FP8_DT_BF16 || out_dtype == H3FP8_DT_FP16 || out_dtype == H3FP8_DT_F32,
               "h3fp8_gemm: bad out_dtype %d", out_dtype);
    H3_REQUIRE(out_dtype != H3FP8_DT_F32 || (!bias && !row_amax && ldy % 4 == 0),
               "h3fp8_gemm: the fp32 accumulator probe takes no bias or row_amax and needs ldy %% 4 == 0");
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
    hipLaunchKernelGGL(gemm_grouped_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, gp);
    H3_CHECK_HIP(hipGetLastError());
    return H3FP8_OK;
}

}  // extern "C"
