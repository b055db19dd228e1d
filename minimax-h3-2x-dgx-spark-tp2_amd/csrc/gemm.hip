// Kernel 2 (scaled FP8 GEMM, bf16/fp16 out, optional fused row-amax for the next layer's quant) and kernel 3 (the
// gate/up GEMM with the SwiGLU epilogue) on gfx950 MFMA.
//
// Contract (h3_tp2/fp8_gemm.py:44-50, :69-112; fp8_cutlass_kernel.py:698-733; fp8_swiglu.py:107-157):
//   y[m, n] = round(sa[m] * (sb[n] * acc[m, n])), acc = sum_k a[m, k] * w[n, k] in fp32, K ascending per
//   accumulator, no split-K; with a bias: round(fma(sa[m], sb[n] * acc, bias[n])).
//
// Tiling (one workgroup = 4 wavefronts = 256 threads, one persistent workgroup per CU):
//   * block tile 256 (tokens m) x 256 (channels n) x 128 (k); each wave owns a 128 x 128 sub-tile: 4 x 4 MFMA tiles of
//     v_mfma_f32_32x32x64_f8f6f4 (e4m3 x e4m3 -> fp32), two k sub-steps per stage, 256 fp32 accumulators per lane (the
//     AGPR file);
//   * the MFMA's A operand is the weight tile (rows n) and its B operand the activation tile (rows m), so each group of
//     four accumulators of a lane holds four consecutive channels n of one token m;
//   * global -> LDS with buffer_load_dwordx4 ... lds (no VGPR staging): each instruction moves 8 rows x 128 bytes, i.e.
//     whole 128-byte lines (64-byte row pieces measured at about half the throughput); out-of-range rows and the K
//     tail read as zero through the buffer descriptor's range check;
//   * two LDS stages (2 x 64 KiB); a stage is released by a barrier right after the last reads of its k-step (early in
//     the step), and the loads of k-step i+2 are issued one per MFMA over the following 16 MFMAs (issued in bursts they
//     stall the instruction stream);
//   * persistent tile loop: the load cursor runs two k-steps ahead of the MFMAs across tile boundaries, so the next
//     tile's first stages and its scales (DMA'd into one of three LDS scale sets) load while the current tile's last
//     k-steps and its epilogue run; the epilogue stages its output in a separate area per wave;
//   * LDS rows are 128 bytes; 16-byte chunk c of row r is stored at chunk c ^ swz(r), swz(r) = ((r >> 1) & 7) ^
//     ((r & 1) << 2): eight consecutive rows (32 banks) and sixteen (64 banks) read at one logical chunk never share a
//     bank (conflict-free ds_read_b128);
//   * operand fragments are double-buffered in VGPRs: sub-step 1 is read while sub-step 0 multiplies, and the next
//     stage's sub-step 0 right after the barrier that publishes it, in the order the first MFMAs consume them;
//   * stage release: a stage is refilled only after a barrier that every wave reaches with lgkmcnt(0), i.e. after all
//     of its ds_reads have returned;
//   * every k-step runs the same branch-free instruction stream (no k-step g+2: out-of-range loads; no tile start:
//     the scale loads go to a scratch slot), so the MFMA stream is never broken by a branch;
//   * tile order: workgroups are spread over the 8 XCDs round-robin by the hardware, so the tile index is remapped to
//     give every XCD a contiguous range of tiles, walked in groups of GROUP_M row tiles (L2 reuse of both operands).
// SwiGLU variant: the weight tile is 128 gate rows f0.. and the 128 matching up rows F+f0..; each wave holds the gate
// and up accumulators of the same (m, f) and applies fp8_swiglu.py:64-70 in registers.  Its SiLU lookups go to a
// compact copy of the bf16 SiLU table in LDS (the 8960 gates with 2.6e-9 <= |g| <= 88.5, keyed by the bf16 bits with
// the sign rotated to the lowest bit so that both signs form one contiguous range); a pass of 32 tokens with any gate
// outside that range (zeros, tinier, larger, inf, NaN -- the wave votes) reads the full table in global memory
// instead.  Both give the same table entry, so the output does not depend on the path taken.
// Other forms below, each with the same MFMA sequence per output element (so the same bits): the half-tile kernel
// (256 tokens x 128 channels, three stages) for a problem's last partial round and for problems of fewer tiles than
// CUs, the 128 x 192 tiles (one per CU) for such problems when they occupy more CUs than the half tiles would, and
// the small-M form (M <= 32: one wave per 16 weight rows, the weight streamed once).
#include <algorithm>

#include "h3fp8_common.h"

namespace {

using namespace h3;

typedef float v16f __attribute__((ext_vector_type(16)));
typedef unsigned int v2u32 __attribute__((ext_vector_type(2)));

constexpr int BM = 256;          // tokens per block tile
constexpr int BN = 256;          // weight rows per block tile
constexpr int BK = 128;          // k per stage: 128-byte row pieces
constexpr int ROWB = BK;         // bytes per LDS row
constexpr int STAGE_BYTES = (BM + BN) * ROWB;   // 64 KiB
constexpr int NSTAGE = 2;
constexpr int A_REGION = BN * ROWB;             // activation rows start after the weight rows
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
    const uint16_t* silu_rot;  // its compact rotated-key copy (loaded into LDS)
    int64_t lda, ldw, ldy;
    int64_t sa_stride, sb_stride;
    int M, N, K;               // SwiGLU: N = F (output width)
    int w_rows;                // rows of w and entries of sb (N, or 2F for SwiGLU)
    uint32_t a_bytes, w_bytes; // buffer ranges
    uint32_t y_bytes;          // output range: ((M - 1) * ldy + N) * element size; stores past it are dropped
    int tiles_m, tiles_n;
    int group_m;
    int tile_offset;           // grouped launches: first block of this problem
    int half_first;            // half-tile launches: the first tile (in the full-tile order) they cover
    int y_nt;                  // fp32 outputs: store non-temporally (the whole product is larger than the MALL)
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

// The same load with the non-temporal hint, for operands that stream through once.
__device__ __forceinline__ void dma16_nt(v4u desc, uint32_t lds_base, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds"
                 :
                 : "s"(lds_base), "v"(voff), "s"(desc)
                 : "memory", "m0");
}

__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) {
    typedef const __attribute__((address_space(3))) uint8_t* lds_u8;
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_u8)(p));
}

// 4 bytes per lane straight into LDS at lds_base + 4 * lane (buffer_load_dword ... lds); untracked like dma16.
__device__ __forceinline__ void dma4(v4u desc, uint32_t lds_base, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds"
                 :
                 : "s"(lds_base), "v"(voff), "s"(desc)
                 : "memory", "m0");
}

// ---- LDS layout of a workgroup ----
//   kernel 2 (150.5 KiB of the 160 KiB):
//   [0, 128 KiB)          two operand stages of 64 KiB (weight rows, then token rows, 128 bytes each)
//   [128 KiB, 144 KiB)    epilogue staging, 4 KiB per wave: 32 token rows x 64 channels of bf16
//   [144 KiB, 150 KiB)    three scale sets of 2 KiB: sa of the tile's 256 token rows, then sb of its 256 weight rows
//   [150 KiB, +512)       a scratch slot for the scale loads of k-steps that do not start a tile
//   kernel 3 (160 KiB): the same with 2 KiB of staging per wave (16 token rows per flush), and after the scratch slot
//   the compact SiLU table (17 920 bytes), loaded once per workgroup ahead of the first stage.
// The stages are never used by the epilogue, so the loads of the next tile run under it.
constexpr int SCALE_SET = 2 * 256 * 4;
constexpr int NSCALE = 3;
constexpr int SILU_LDS_BYTES = H3_SILU_ROT_LEN * 2;          // the compact SiLU table (kernel 3)
static_assert(SILU_LDS_BYTES % 256 == 0, "the table loads in 256-byte pieces");

// The layout per epilogue: kernel 3 stages 16 token rows per flush (2 KiB per wave) to make room for the compact SiLU
// table, which brings its workgroup to the 160 KiB of the CU; the other forms stage 32 rows.
template <int EPI>
struct Lds {
    static constexpr int STG_ROWS = (EPI == EPI_SWIGLU) ? 16 : 32;
    static constexpr int STAGING_PER_WAVE = STG_ROWS * 128;
    static constexpr int STAGING_OFF = NSTAGE * STAGE_BYTES;
    static constexpr int SCALES_OFF = STAGING_OFF + 4 * STAGING_PER_WAVE;
    static constexpr int JUNK_OFF = SCALES_OFF + NSCALE * SCALE_SET;   // 512 bytes: target of unneeded scale loads
    static constexpr int SILU_OFF = JUNK_OFF + 512;
    static constexpr int TOTAL = SILU_OFF + ((EPI == EPI_SWIGLU) ? SILU_LDS_BYTES : 0);
};
static_assert(Lds<EPI_SWIGLU>::TOTAL <= 160 * 1024 && Lds<EPI_PLAIN>::TOTAL <= 160 * 1024, "LDS of one CU");

// Per-wave addressing of one tile's global -> LDS loads.
struct Loader {
    v4u rw, ra;                 // weight / activation buffer descriptors
    v4u rsa, rsb;               // scale buffer descriptors
    uint32_t vw[2], va[2];      // lane part of the byte offsets for even / odd instructions (OOB: share out of range)
    uint32_t vw_t[2], va_t[2];  // the same for the tile's last k-step: OOB where the lane's chunk lies at or past K
    uint32_t row8_w, row8_a;    // byte advance of 8 rows
    uint32_t sa_off, sb_off;    // this lane's scale offsets (OOB past the range)
    int w_groups;               // SwiGLU: 8-row groups of this wave's weight share that are in range
};

// One wave's share of a stage: 8 instructions for its 64 weight rows (i = 0..7), 8 for its 64 token rows (i = 8..15).
struct StageIssue {
    uint32_t wdst, adst;        // LDS addresses of the wave's weight / token rows in the stage
    uint32_t vw[2], va[2];      // byte offsets of the lane for even / odd instructions, k0 included
};

template <int EPI>
__device__ __forceinline__ void issue_one(const StageIssue& S, const Loader& L, int i) {
    if (i < 8) {
        const uint32_t off = (EPI == EPI_SWIGLU && i >= L.w_groups) ? OOB : S.vw[i & 1] + i * L.row8_w;
        dma16(L.rw, S.wdst + i * 8 * ROWB, off);
    } else {
        dma16(L.ra, S.adst + (i - 8) * 8 * ROWB, S.va[i & 1] + (i - 8) * L.row8_a);
    }
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

// The first MFMA of an accumulator block in a tile: C is the inline constant 0, so the 256 accumulators of a tile
// are never cleared by moves.
__device__ __forceinline__ void mfma_zero(v16f acc[4][4], const v8i af[4], const v8i bf[4], int t) {
    const v16f z = {};
    acc[t >> 2][t & 3] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(af[t >> 2], bf[t & 3], z, 0, 0, 0, 0, 0, 0);
}

struct GroupedParams {
    GemmParams g[H3FP8_MAX_GROUPS];
    int n;
    int total_tiles;           // tiles of all problems (problem i owns [g[i].tile_offset, + tiles_m * tiles_n))
};

template <bool GROUPED>
__device__ __forceinline__ int problem_of(const GroupedParams& gp, int id) {
    int i = 0;
    if (GROUPED) {
#pragma unroll
        for (int j = 1; j < H3FP8_MAX_GROUPS; ++j)
            if (j < gp.n && id >= gp.g[j].tile_offset) i = j;
    }
    return i;
}

// Global tile id -> problem and tile coordinates.
template <bool GROUPED>
__device__ __forceinline__ int locate(const GroupedParams& gp, int id, int& tm, int& tn) {
    const int pi = problem_of<GROUPED>(gp, id);
    const GemmParams& p = gp.g[pi];
    tile_of(id - p.tile_offset, p.tiles_m * p.tiles_n, p.tiles_m, p.tiles_n, p.group_m, tm, tn);
    return pi;
}

// Addressing of tile (tm, tn) of problem p for this wave.
// lane l of an instruction covers row (l >> 3) of an 8-row group and LDS chunk (l & 7), i.e. logical chunk
// (l & 7) ^ swz(row); swz depends on the row's bits 0..3, so even and odd groups of 8 rows differ.
template <int EPI>
__device__ __forceinline__ void make_loader(const GemmParams& p, int tm, int tn, int wave, int lane, Loader& L) {
    const uint32_t lrow = (uint32_t)(lane >> 3);
    const uint32_t lch[2] = {(uint32_t)((lane & 7) ^ swz((int)lrow)), (uint32_t)((lane & 7) ^ swz((int)lrow + 8))};
    int64_t wrow0;   // first global weight row of this wave's 64-row share
    int64_t wlimit;  // rows of this share's source range (SwiGLU gate rows stop at F)
    if (EPI == EPI_SWIGLU) {
        const int f0 = tn * (BN / 2);
        wrow0 = (wave < 2) ? (int64_t)f0 + 64 * wave : (int64_t)p.N + f0 + 64 * (wave - 2);
        wlimit = (wave < 2) ? (int64_t)p.N : 2 * (int64_t)p.N;
    } else {
        wrow0 = (int64_t)tn * BN + 64 * wave;
        wlimit = p.N;
    }
    const int64_t arow0 = (int64_t)tm * BM + 64 * wave;
    L.rw = buffer_desc(p.w, p.w_bytes);
    L.ra = buffer_desc(p.a, p.a_bytes);
    // bytes of k that the tile's last k-step covers (0: all BK); chunks at or past it read zeros in that k-step
    const uint32_t ktail = (uint32_t)(p.K % BK);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const uint32_t c16 = 16u * lch[e];
        L.vw[e] = (wrow0 >= wlimit) ? OOB : (uint32_t)((wrow0 + lrow) * p.ldw) + c16;
        L.va[e] = (arow0 >= p.M) ? OOB : (uint32_t)((arow0 + lrow) * p.lda) + c16;
        const bool cut = ktail != 0 && c16 >= ktail;
        L.vw_t[e] = cut ? OOB : L.vw[e];
        L.va_t[e] = cut ? OOB : L.va[e];
    }
    L.row8_w = (uint32_t)(8 * p.ldw);
    L.row8_a = (uint32_t)(8 * p.lda);
    // Partial shares rely on the descriptor's range check (rows >= M or >= N start past the last valid byte), except
    // SwiGLU gate rows past F, which would read up rows: those 8-row groups are zero-filled (F % 16 == 0).
    L.w_groups = (int)min<int64_t>(8, max<int64_t>(0, (wlimit - wrow0 + 7) / 8));
    // scales: token row 64 wave + lane of the tile; weight row 64 wave + lane (SwiGLU: gate rows for waves 0-1, the
    // matching up rows for waves 2-3)
    L.rsa = buffer_desc(p.sa, p.sa_stride ? (uint32_t)((p.M - 1) * p.sa_stride * 4 + 4) : 4u);
    L.rsb = buffer_desc(p.sb, p.sb_stride ? (uint32_t)((p.w_rows - 1) * p.sb_stride * 4 + 4) : 4u);
    const int64_t srow = arow0 + lane;
    L.sa_off = (srow < p.M) ? (uint32_t)(srow * p.sa_stride * 4) : OOB;
    const int64_t wr = wrow0 + lane;
    L.sb_off = (wr < wlimit) ? (uint32_t)(wr * p.sb_stride * 4) : OOB;
}

// The load-issue cursor: the (tile, k-step) whose operands are loaded next, two k-steps ahead of the MFMAs.  Everything
// a k-step's loads need is prepared per tile here, so that the k-step itself adds only k0 to four offsets.
struct Cursor {
    Loader L;
    int c;          // workgroup-local tile ordinal (global tile id: round_id(blockIdx.x, c, gridDim.x))
    int ks, nk;
    bool valid;
    uint32_t dsa, dsb;  // LDS addresses of this wave's share of the tile's scale set (set c % NSCALE)
};

// Tile id of workgroup b in its round c of a persistent launch over G workgroups: b + c G; a grouped launch takes the
// workgroups of each XCD (b & 7) in reverse order on odd rounds (a bijection of the round onto itself that keeps every
// id on its XCD), so that the workgroups that drew the longest tiles of one round draw the shortest of the next.  The
// groups' tiles are laid out by descending K, and a round-robin that always starts at workgroup 0 leaves the first
// workgroups with the most k-steps (the four-group workload: 271 against a mean of 252; serpentine 259).
template <bool GROUPED>
__device__ __forceinline__ int round_id(int b, int c, int G) {
    if (!GROUPED || !(c & 1) || (G & 7)) return b + c * G;
    return c * G + ((((G >> 3) - 1 - (b >> 3)) << 3) | (b & 7));
}

template <int EPI, bool GROUPED>
__device__ __forceinline__ void cursor_set(Cursor& I, const GroupedParams& gp, int c, uint32_t lds0, int wave,
                                           int lane) {
    const int id = round_id<GROUPED>((int)blockIdx.x, c, (int)gridDim.x);
    I.c = c;
    I.ks = 0;
    I.valid = id < gp.total_tiles;
    I.dsa = lds0 + Lds<EPI>::SCALES_OFF + (uint32_t)(c % NSCALE) * SCALE_SET + 256u * (uint32_t)wave;
    I.dsb = I.dsa + 1024u;
    if (!I.valid) {
        // past the last tile: the loads still run (every k-step has the same instruction stream and wait counts),
        // read nothing and fill the stage with zeros
#pragma unroll
        for (int e = 0; e < 2; ++e) I.L.vw[e] = I.L.va[e] = I.L.vw_t[e] = I.L.va_t[e] = OOB;
        I.nk = 1;
        return;
    }
    int tm, tn;
    const int pi = locate<GROUPED>(gp, id, tm, tn);
    const GemmParams& p = gp.g[pi];
    I.nk = (p.K + BK - 1) / BK;
    make_loader<EPI>(p, tm, tn, wave, lane, I.L);
}

// The load instructions of the cursor's k-step for this wave (wofs = the wave's 64-row share within a region).
template <int EPI>
__device__ __forceinline__ StageIssue stage_issue(uint32_t stage, const Cursor& I, uint32_t wofs) {
    const Loader& L = I.L;
    StageIssue S;
    const uint32_t k0 = (uint32_t)I.ks * BK;
    const bool last = I.ks == I.nk - 1;                         // uniform: the K tail, if any, is in this k-step
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        S.vw[e] = (last ? L.vw_t[e] : L.vw[e]) + k0;
        S.va[e] = (last ? L.va_t[e] : L.va[e]) + k0;
    }
    S.wdst = stage + wofs;
    S.adst = stage + A_REGION + wofs;
    return S;
}

template <int EPI>
__device__ __forceinline__ void issue_stage(uint32_t stage, const Cursor& I, uint32_t wofs) {
    const StageIssue S = stage_issue<EPI>(stage, I, wofs);
#pragma unroll
    for (int i = 0; i < 16; ++i) issue_one<EPI>(S, I.L, i);
}

// The scales of the cursor's tile when its k-step starts the tile: wave w loads sa of token rows 64 w .. 64 w + 63
// and sb of weight rows 64 w .. 64 w + 63 into scale set c % NSCALE (a scalar scale has stride 0 and fills every
// entry).  At any other k-step the two loads read nothing and land in the scratch slot.
template <int EPI>
__device__ __forceinline__ void issue_scales(uint32_t lds0, const Cursor& I) {
    const bool real = I.valid && I.ks == 0;
    dma4(I.L.rsa, real ? I.dsa : lds0 + Lds<EPI>::JUNK_OFF, real ? I.L.sa_off : OOB);
    dma4(I.L.rsb, real ? I.dsb : lds0 + Lds<EPI>::JUNK_OFF + 256, real ? I.L.sb_off : OOB);
}

template <int EPI, bool GROUPED>
__device__ __forceinline__ void cursor_next(Cursor& I, const GroupedParams& gp, uint32_t lds0, int wave, int lane) {
    if (++I.ks == I.nk) cursor_set<EPI, GROUPED>(I, gp, I.c + 1, lds0, wave, lane);
}

// One k-step g (stage g & 1 holds it, its sub-step-0 fragments are in fa0/fb0, the loads of k-step g+1 are in flight;
// the cursor points at k-step g+2, possibly of the next tile).  The instruction stream is the same for every k-step:
// when there is no k-step g+2 the 16 loads are issued with out-of-range offsets (they fill the freed stage with zeros
// and touch no memory), the two scale loads go to a scratch slot of the LDS unless g+2 starts a tile, and after the
// last k-step the extra fragment reads of the other stage are simply not used.  Loads are issued one per MFMA: issued
// in bursts they stall the wave's instruction stream and with it the matrix core.
// order of the next k-step's sub-step-0 fragment reads (0..3 weight tiles, 4..7 token tiles): MFMA t of phase A uses
// weight tile t / 4 and token tile t % 4, so reading weight tile 0 and then the token tiles lets it start earliest
constexpr int NEXT_READ_ORDER[8] = {0, 4, 5, 6, 7, 1, 2, 3};

// Schedule of one k-step over its 32 MFMAs (u = 0..15: sub-step 0, u = 16..31: sub-step 1):
//   u < 8        the 8 sub-step-1 fragment reads of stage g, one per MFMA;
//   u == REL     lgkmcnt(0) + barrier 1: every wave's reads of stage g have returned -- the stage is free;
//   REL < u      the 16 load instructions of k-step g+2 into the freed stage, one per MFMA, and the two scale loads
//                after the eighth;
//   u == PUB     vmcnt + barrier 2: k-step g+1 has landed (only loads issued in this k-step may be outstanding);
//   u > PUB      the 8 sub-step-0 fragment reads of k-step g+1 (READ_NEXT), in the order its first MFMAs use them.
constexpr int KS_REL = 9;                      // measured best of 9..15 (QKV and K = 8192 shapes)
constexpr int KS_PUB = 26;
static_assert(KS_REL >= 7 && KS_REL + 16 <= 31 && KS_PUB > KS_REL && KS_PUB < 31, "k-step schedule");
constexpr int ks_loads_before_pub() {
    const int stage = (KS_PUB - KS_REL) < 16 ? (KS_PUB - KS_REL) : 16;
    return stage + (KS_REL + 9 <= KS_PUB ? 2 : 0);
}

// FIRST: the tile's first k-step, whose sub-step-0 MFMAs start their accumulator blocks from 0.
template <int EPI, bool READ_NEXT, bool FIRST>
__device__ __forceinline__ void kstep(uint8_t* lds, uint32_t lds0, int g, const Cursor& I, uint32_t wofs, int wn, int wm,
                                      int lane, v16f acc[4][4], v8i fa0[4], v8i fb0[4], v8i fa1[4], v8i fb1[4]) {
    uint8_t* cur = lds + (g & 1) * STAGE_BYTES;
    uint8_t* nxt = lds + ((g + 1) & 1) * STAGE_BYTES;
    const StageIssue S = stage_issue<EPI>(lds0 + (uint32_t)(g & 1) * STAGE_BYTES, I, wofs);
    constexpr int NREAD = 31 - KS_PUB;                  // MFMAs that carry the next k-step's reads
    constexpr int PER = (8 + NREAD - 1) / NREAD;
#pragma unroll
    for (int u = 0; u < 32; ++u) {
        if (u < 16) {
            if (FIRST) mfma_zero(acc, fa0, fb0, u);
            else mfma_one(acc, fa0, fb0, u);
        } else {
            mfma_one(acc, fa1, fb1, u - 16);
        }
        if (u < 8) read_one<EPI>(cur, wn, wm, lane, 1, u, fa1, fb1);
        if (u == KS_REL) {
            wait_lgkm0();                               // this wave's reads of stage g & 1 have returned
            barrier_nofence();                          // ... and every wave's: the stage is free
        }
        if (u > KS_REL && u <= KS_REL + 16) issue_one<EPI>(S, I.L, u - KS_REL - 1);
        if (u == KS_REL + 9) issue_scales<EPI>(lds0, I);
        if (u == KS_PUB) {
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(ks_loads_before_pub()));   // k-step g+1 (and older) has landed
            barrier_nofence();
        }
        if (READ_NEXT && u > KS_PUB) {
#pragma unroll
            for (int f = (u - KS_PUB - 1) * PER; f < (u - KS_PUB) * PER; ++f)
                if (f < 8) read_one<EPI>(nxt, wn, wm, lane, 0, NEXT_READ_ORDER[f], fa0, fb0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Orders one wave's LDS accesses across its lanes: a lane's staging writes become visible to the other lanes' reads
// that follow.  The wave's LDS accesses already complete in order, so this emits no wait; it is there for the compiler,
// which under per-lane semantics may otherwise reorder or tail-duplicate lane-divergent writes past other lanes' reads
// (the barrier is convergent: it cannot be moved into a divergent branch).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// max(m, |lo half|, |hi half|) of a packed bf16 pair, as fp32 bit patterns (the row maximum of the fused quant).
__device__ __forceinline__ uint32_t max_abs_bf16x2(uint32_t m, uint32_t p) {
    const uint32_t lo = (p << 16) & 0x7fff0000u, hi = p & 0x7fff0000u;
    m = m > lo ? m : lo;
    return m > hi ? m : hi;
}

// The same for a packed fp16 pair: each half is widened to fp32 (exact) before its |.| bits are compared, so the row
// maximum is the fp32 value of the largest rounded fp16 output (NaN patterns exceed every finite one, as above).
__device__ __forceinline__ uint32_t max_abs_f16x2(uint32_t m, uint32_t p) {
    const uint32_t lo = f2u(fp16_to_f32(p & 0xffffu)) & 0x7fffffffu, hi = f2u(fp16_to_f32(p >> 16)) & 0x7fffffffu;
    m = m > lo ? m : lo;
    return m > hi ? m : hi;
}

// Running maxima of |x| over packed bf16 pairs, one per 16-bit half: with the sign bit cleared, bf16 magnitudes order
// as their bit patterns (NaN patterns above inf), so a pair costs one mask and one packed u16 max.  pk_max_f32 folds
// the two halves into the fp32 bit pattern of the larger, the value max_abs_bf16x2 accumulates over the same pairs.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u16x2 max_abs_pk(u16x2 m, uint32_t p) {
    return __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, p & 0x7fff7fffu));
}
__device__ __forceinline__ uint32_t pk_max_f32(u16x2 m) {
    const uint32_t a = m[0], b = m[1];
    return (a > b ? a : b) << 16;
}

// A +0 the compiler cannot see through, made once per epilogue: x + z turns -0 into +0 (round to nearest) and leaves
// every other value (NaN included) unchanged, and the add is not folded away.
__device__ __forceinline__ float opaque_zero() {
    float z = 0.0f;
    asm volatile("" : "+v"(z));
    return z;
}

// ---- epilogue ----
// 32x32 MFMA result: lane l, register 4q + r holds D[8q + 4(l >> 5) + r][l & 31], i.e. weight row (channel)
// 8q + 4(l >> 5) + r of the MFMA tile and token l & 31.  The scaled, rounded outputs go through the wave's staging
// area, 32 tokens x 64 channels at a time, so that global stores are 16-byte pieces of 128-byte row segments.
// Scales come from the tile's scale set in LDS (loaded with the tile's first k-step).
template <int OUT_DT, bool HAS_BIAS, int EPI>
__device__ __forceinline__ void epilogue(const GemmParams& p, int tm, int tn, uint8_t* lds, int set, int wave, int wn,
                                         int wm, int lane, v16f acc[4][4]) {
    constexpr int NI = 4;                               // MFMA tiles along the channels per wave
    const int wcol = tn * BN + wn * 128;                // the wave's first output channel
    const int wsb = wn * 128;                           // ... and its first entry in the tile's sb set
    const int hi = lane >> 5;
    const int mj = lane & 31;
    const int mrow0 = tm * BM + wm * 128;               // first token row of the wave
    const float* sa_l = reinterpret_cast<const float*>(lds + Lds<EPI>::SCALES_OFF + set * SCALE_SET);
    const float* sb_l = sa_l + 256;
    uint8_t* stg = lds + Lds<EPI>::STAGING_OFF + wave * Lds<EPI>::STAGING_PER_WAVE;
    if (OUT_DT == H3FP8_DT_F32) {
        // the raw fp32 accumulators (scales / bias / rounding not applied), staged one 32 x 32 MFMA block at a time:
        // lane l writes the 4 x 4 channels of token l & 31 as 16-byte chunks (8q + 4 hi) / 4 of that token's 128-byte
        // row, chunk c stored at c ^ (row % 8); the wave then reads back 8 rows of 128 bytes per instruction and every
        // store writes whole 128-byte row segments (rows past M are out of the descriptor's range, columns past N get
        // an out-of-range offset)
        const __amdgpu_buffer_rsrc_t yr = make_rsrc(p.y, p.y_bytes);
        const uint32_t row4 = (uint32_t)p.ldy * 4u;
        const int c = lane & 7;
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                wave_sync();                            // the previous block's reads before these writes
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const v4f v = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
                    *reinterpret_cast<v4f*>(stg + mj * 128 + (((2 * q + hi) ^ (mj & 7)) << 4)) = v;
                }
                wave_sync();                            // every lane's writes before any lane's reads
                v4u v[4];
#pragma unroll
                for (int it = 0; it < 4; ++it) {
                    const int ml = it * 8 + (lane >> 3);
                    v[it] = *reinterpret_cast<const v4u*>(stg + ml * 128 + ((c ^ (ml & 7)) << 4));
                }
                const int n = wcol + 32 * i + 4 * c;
                const uint32_t off = (n < p.N) ? (uint32_t)(mrow0 + 32 * j + (lane >> 3)) * row4 + (uint32_t)n * 4u : OOB;
                if (p.y_nt) {                           // uniform: whole row segments, not kept in the caches
#pragma unroll
                    for (int it = 0; it < 4; ++it)
                        __builtin_amdgcn_raw_buffer_store_b128(v[it], yr, off + (uint32_t)it * 8u * row4, 0, 2);
                } else {
#pragma unroll
                    for (int it = 0; it < 4; ++it)
                        __builtin_amdgcn_raw_buffer_store_b128(v[it], yr, off + (uint32_t)it * 8u * row4, 0, 0);
                }
            }
        return;
    }
    // element (ml, cl) of the 32 x 64 staging tile: row ml, 16-byte chunk (cl / 8) ^ (ml % 8), 8-byte half (cl / 4) % 2
    auto put4 = [&](int ml, int cl, uint32_t lo, uint32_t h2) {
        const int ch = (cl >> 3) ^ (ml & 7);
        *reinterpret_cast<uint2*>(stg + ml * 128 + ch * 16 + ((cl >> 2) & 1) * 8) = make_uint2(lo, h2);
    };
    // the wave reads back its own staging tile (LDS accesses of one wave complete in order): 16 bytes per lane, 8
    // lanes per 128-byte row segment, 8 rows per store instruction
    // Stores go through a buffer descriptor whose range ends at the last valid element: rows at or past M fall out of
    // range and are dropped by the hardware, columns at or past the output width get an out-of-range offset.  No
    // branch: partial tiles take the same instruction stream as whole ones.
    const __amdgpu_buffer_rsrc_t yr = make_rsrc(p.y, p.y_bytes);
    const uint32_t row2 = (uint32_t)p.ldy * 2u;         // bytes per output row
    auto flush = [&](int m0, int col0, int ncols) {
        const int c = lane & 7;
        const int col = col0 + c * 8;
        v4u v[4];
#pragma unroll
        for (int it = 0; it < 4; ++it) {                // all four reads before the first store
            const int ml = it * 8 + (lane >> 3);
            v[it] = *reinterpret_cast<const v4u*>(stg + ml * 128 + ((c ^ (ml & 7)) << 4));
        }
        const uint32_t off = (col < ncols) ? (uint32_t)(m0 + (lane >> 3)) * row2 + (uint32_t)col * 2u : OOB;
#pragma unroll
        for (int it = 0; it < 4; ++it) __builtin_amdgcn_raw_buffer_store_b128(v[it], yr, off + (uint32_t)it * 8u * row2, 0, 0);
    };
    auto row_amax = [&](uint32_t v, int m) {
        const uint32_t o = (uint32_t)__shfl_xor((int)v, 32, 64);
        v = v > o ? v : o;
        if (hi == 0 && m < p.M && v) atomicMax(reinterpret_cast<unsigned int*>(p.row_amax) + m, v);
    };
    if (EPI == EPI_SWIGLU) {
        const int F = p.N;
        const int col0 = tn * (BN / 2) + wn * 64;
        // every scale the wave needs, read once up front (one LDS round trip instead of one per group of four)
        float sa_j[4];
        v4f sbg_v[2][4], sbu_v[2][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) sa_j[j] = sa_l[wm * 128 + 32 * j + mj];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                sbg_v[t][q] = *reinterpret_cast<const v4f*>(sb_l + wn * 64 + 32 * t + 8 * q + 4 * hi);
                sbu_v[t][q] = *reinterpret_cast<const v4f*>(sb_l + 128 + wn * 64 + 32 * t + 8 * q + 4 * hi);
            }
        const uint16_t* silu_l = reinterpret_cast<const uint16_t*>(lds + Lds<EPI>::SILU_OFF);
        const float zero = opaque_zero();
        // 16 staged token rows to their output rows: 16 bytes per lane, 8 rows per store instruction
        auto flush16 = [&](int m0, int c0, int ncols) {
            const int c = lane & 7;
            const int col = c0 + c * 8;
            v4u v[2];
#pragma unroll
            for (int it = 0; it < 2; ++it) {
                const int ml = it * 8 + (lane >> 3);
                v[it] = *reinterpret_cast<const v4u*>(stg + ml * 128 + ((c ^ (ml & 7)) << 4));
            }
            const uint32_t off = (col < ncols) ? (uint32_t)(m0 + (lane >> 3)) * row2 + (uint32_t)col * 2u : OOB;
#pragma unroll
            for (int it = 0; it < 2; ++it)
                __builtin_amdgcn_raw_buffer_store_b128(v[it], yr, off + (uint32_t)it * 8u * row2, 0, 0);
        };
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int m = mrow0 + 32 * j + mj;
            const float sam = sa_j[j];
            // gate and up of the pass rounded to bf16.  The gate is converted into both halves of a word, so that its
            // table key (the bf16 bits rotated left by one: the sign lands in bit 0 and both signs form one range) is
            // the bit field [15, 31) of that word; the up value goes to the high half over a zero low half, which is
            // its fp32 value.
            uint32_t key[2][4][4], uu[2][4][4], sl[2][4][4];
            uint64_t outside = 0;
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int f = col0 + 32 * t + 8 * q + 4 * hi;
                    float bg[4] = {0, 0, 0, 0}, bu[4] = {0, 0, 0, 0};
                    if (HAS_BIAS) {                     // columns past F read column 0 (not stored)
                        const int fc = f < F ? f : 0;
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            bg[r] = load_bias(p.bias, fc + r, 0);
                            bu[r] = load_bias(p.bias, F + fc + r, 0);
                        }
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float tg = sbg_v[t][q][r] * acc[t][j][4 * q + r];
                        const float tu = sbu_v[t][q][r] * acc[t + 2][j][4 * q + r];
                        const float gy = HAS_BIAS ? __builtin_fmaf(sam, tg, bg[r]) : sam * tg;
                        const float uy = HAS_BIAS ? __builtin_fmaf(sam, tu, bu[r]) : sam * tu;
                        const uint32_t rk = (cvt_bf16x2(gy, gy) >> 15) & 0xffffu;
                        uu[t][q][r] = cvt_bf16x2(0.0f, uy);
                        // the compact table's index; a key outside its range wraps to a large value
                        key[t][q][r] = rk - H3_SILU_ROT_R0;
                        outside |= __ballot(key[t][q][r] >= (uint32_t)H3_SILU_ROT_LEN);
                    }
                }
            // bf16(g/(1+exp(-g))) of every gate of the pass: from the compact table in LDS when every key of the pass
            // lies in its range, else from the full table (indexed by the gate's bf16 bits, the key rotated back)
            if (outside == 0) {
#pragma unroll
                for (int t = 0; t < 2; ++t)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
#pragma unroll
                        for (int r = 0; r < 4; ++r) sl[t][q][r] = silu_l[key[t][q][r]];
            } else {
#pragma unroll
                for (int t = 0; t < 2; ++t)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const uint32_t rk = (key[t][q][r] + H3_SILU_ROT_R0) & 0xffffu;
                            sl[t][q][r] = p.silu[(rk >> 1) | ((rk & 1u) << 15)];
                        }
            }
            uint32_t hp[2][4][2];
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float hv[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r)                    // -0 up -> +0 (fp8_swiglu.py:66)
                        hv[r] = bf16_to_f32(sl[t][q][r]) * (u2f(uu[t][q][r]) + zero);
                    hp[t][q][0] = cvt_bf16x2(hv[0], hv[1]);
                    hp[t][q][1] = cvt_bf16x2(hv[2], hv[3]);
                }
            // the row maximum over the columns before F (rows past M are dropped by row_amax)
            u16x2 mx2 = {0, 0};
            if (col0 + 64 <= F) {
#pragma unroll
                for (int t = 0; t < 2; ++t)
#pragma unroll
                    for (int q = 0; q < 4; ++q) mx2 = max_abs_pk(max_abs_pk(mx2, hp[t][q][0]), hp[t][q][1]);
            } else {
#pragma unroll
                for (int t = 0; t < 2; ++t)
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        if (col0 + 32 * t + 8 * q + 4 * hi < F)
                            mx2 = max_abs_pk(max_abs_pk(mx2, hp[t][q][0]), hp[t][q][1]);
            }
            const uint32_t rmax = pk_max_f32(mx2);
            if (p.row_amax) row_amax(rmax, m);
            // the pass's 32 token rows through the 16-row staging area, one half at a time (this wave's LDS accesses
            // complete in order, so the second half's writes follow the first half's reads)
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                wave_sync();                            // the previous flush's reads before these writes
                if ((mj >> 4) == half) {
#pragma unroll
                    for (int t = 0; t < 2; ++t)
#pragma unroll
                        for (int q = 0; q < 4; ++q) put4(mj & 15, 32 * t + 8 * q + 4 * hi, hp[t][q][0], hp[t][q][1]);
                }
                wave_sync();                            // every lane's writes before any lane's reads
                flush16(mrow0 + 32 * j + 16 * half, col0, F);
            }
        }
    } else {
        const int col0 = wcol;
        // the wave's token scales, and with the row maximum or a bias its channel scales too, read once up front (one
        // LDS round trip instead of one per group of four); the plain epilogue reads each group's channel scales where
        // it uses them, which leaves it the registers to run without scratch
        constexpr bool SB_UPFRONT = EPI == EPI_AMAX || HAS_BIAS;
        float sa_j[4];
        v4f sb_v[4][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) sa_j[j] = sa_l[wm * 128 + 32 * j + mj];
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (SB_UPFRONT) sb_v[i][q] = *reinterpret_cast<const v4f*>(sb_l + wsb + 32 * i + 8 * q + 4 * hi);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int m = mrow0 + 32 * j + mj;
            const float sam = sa_j[j];
            uint32_t rmax = 0;                          // fp16 outputs: the fp32 bits of the largest |y|
            u16x2 mx2 = {0, 0};                         // bf16 outputs: |y| bit patterns, one per half
#pragma unroll
            for (int ip = 0; ip < NI / 2; ++ip) {
                const bool all_cols = col0 + 64 * ip + 64 <= p.N;     // wave-uniform: no column of the pass is past N
                wave_sync();                            // the previous flush's reads before these writes
#pragma unroll
                for (int ii = 0; ii < 2; ++ii) {
                    const int i = 2 * ip + ii;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int cl = 32 * ii + 8 * q + 4 * hi;          // column within the 64-wide pass
                        const int n = col0 + 64 * ip + cl;
                        const bool ok = n < p.N && m < p.M;
                        const v4f sbn = SB_UPFRONT ? sb_v[i][q]
                                                   : *reinterpret_cast<const v4f*>(sb_l + wsb + 32 * i + 8 * q + 4 * hi);
                        float bn[4] = {0, 0, 0, 0};
                        if (HAS_BIAS) {                 // columns past N read column 0 (not stored)
                            const int nc = n < p.N ? n : 0;
#pragma unroll
                            for (int r = 0; r < 4; ++r) bn[r] = load_bias(p.bias, nc + r, OUT_DT);
                        }
                        float v[4];
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const float t = sbn[r] * acc[i][j][4 * q + r];
                            v[r] = HAS_BIAS ? __builtin_fmaf(sam, t, bn[r]) : sam * t;
                        }
                        uint32_t lo, hi2;
                        if (OUT_DT) {
                            lo = fp16_rne(v[0]) | (fp16_rne(v[1]) << 16);
                            hi2 = fp16_rne(v[2]) | (fp16_rne(v[3]) << 16);
                        } else {
                            lo = cvt_bf16x2(v[0], v[1]);
                            hi2 = cvt_bf16x2(v[2], v[3]);
                        }
                        // the row maximum over the columns before N (rows past M are dropped by row_amax)
                        if (EPI == EPI_AMAX && OUT_DT && ok) rmax = max_abs_f16x2(max_abs_f16x2(rmax, lo), hi2);
                        if (EPI == EPI_AMAX && !OUT_DT && (all_cols || n < p.N))
                            mx2 = max_abs_pk(max_abs_pk(mx2, lo), hi2);
                        put4(mj, cl, lo, hi2);
                    }
                }
                wave_sync();                            // every lane's writes before any lane's reads
                flush(mrow0 + 32 * j, col0 + 64 * ip, p.N);
            }
            if (EPI == EPI_AMAX) row_amax(OUT_DT ? rmax : pk_max_f32(mx2), m);
        }
    }
}

// Persistent kernel: workgroup b computes tiles b, b + G, b + 2G, ... (G = gridDim.x <= the CU count, one workgroup per
// CU).  The load cursor runs two k-steps ahead of the MFMAs across tile boundaries, so the first two stages of the
// next tile (and its scales) load while the current tile's last k-steps and epilogue run.
template <int OUT_DT, bool HAS_BIAS, int EPI, bool GROUPED>
__global__ void __launch_bounds__(256, 1) gemm_kernel(GroupedParams gp) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[Lds<EPI>::TOTAL];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: LDS addresses go to SGPRs
    const int wn = wave & 1, wm = wave >> 1;
    const int G = (int)gridDim.x;

    Cursor I;
    const uint32_t lds0 = lds_addr(lds);
    const uint32_t wofs = (uint32_t)wave * 64u * ROWB;  // the wave's 64-row share of a stage region
    cursor_set<EPI, GROUPED>(I, gp, 0, lds0, wave, lane);
    if (!I.valid) return;

    // prologue: k-steps 0 and 1 (and the scales of their tiles) in flight, the sub-step-0 fragments of k-step 0 in
    // registers; every load group is 16 stage loads followed by 2 scale loads
    v8i fa0[4], fb0[4], fa1[4], fb1[4];
    if (EPI == EPI_SWIGLU) {
        // the compact SiLU table into LDS, once per workgroup, ahead of the stage loads: the wait below for the
        // first stage covers it (loads complete in order)
        const v4u td = buffer_desc(gp.g[0].silu_rot, SILU_LDS_BYTES);
        for (int ch = wave; ch < SILU_LDS_BYTES / 256; ch += 4)
            dma4(td, lds0 + Lds<EPI>::SILU_OFF + (uint32_t)ch * 256u, (uint32_t)ch * 256u + 4u * (uint32_t)lane);
    }
    issue_stage<EPI>(lds0, I, wofs);
    issue_scales<EPI>(lds0, I);
    cursor_next<EPI, GROUPED>(I, gp, lds0, wave, lane);
    issue_stage<EPI>(lds0 + STAGE_BYTES, I, wofs);
    issue_scales<EPI>(lds0, I);
    if (I.valid) cursor_next<EPI, GROUPED>(I, gp, lds0, wave, lane);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(18));
    barrier_nofence();
    read_frags<EPI>(lds, wn, wm, lane, 0, fa0, fb0);

    int g = 0;
    for (int c = 0;; ++c) {
        const int id = round_id<GROUPED>((int)blockIdx.x, c, G);
        int tm, tn;
        const int pi = locate<GROUPED>(gp, id, tm, tn);
        const GemmParams& p = gp.g[pi];
        const int nk = (p.K + BK - 1) / BK;

        v16f acc[4][4];
        int ks = 0;
        if (nk > 1) {
            // the first k-step's MFMAs start every accumulator block from 0 (C = the constant 0)
            kstep<EPI, true, true>(lds, lds0, g, I, wofs, wn, wm, lane, acc, fa0, fb0, fa1, fb1);
            if (I.valid) cursor_next<EPI, GROUPED>(I, gp, lds0, wave, lane);
            ++g;
            ++ks;
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
        }
        for (; ks < nk - 1; ++ks, ++g) {
            kstep<EPI, true, false>(lds, lds0, g, I, wofs, wn, wm, lane, acc, fa0, fb0, fa1, fb1);
            if (I.valid) cursor_next<EPI, GROUPED>(I, gp, lds0, wave, lane);
        }
        // the tile's last k-step publishes the next k-step's stage but leaves its fragment registers free for the
        // epilogue; they are read after it
        kstep<EPI, false, false>(lds, lds0, g, I, wofs, wn, wm, lane, acc, fa0, fb0, fa1, fb1);
        if (I.valid) cursor_next<EPI, GROUPED>(I, gp, lds0, wave, lane);
        ++g;
        epilogue<OUT_DT, HAS_BIAS, EPI>(p, tm, tn, lds, c % NSCALE, wave, wn, wm, lane, acc);
        // the next tile's fragment reads stay after the epilogue: hoisted into it they would hold 64 VGPRs across it
        __builtin_amdgcn_sched_barrier(0);
        if ((GROUPED ? round_id<GROUPED>((int)blockIdx.x, c + 1, G) : id + G) >= gp.total_tiles) break;
        read_frags<EPI>(lds + (g & 1) * STAGE_BYTES, wn, wm, lane, 0, fa0, fb0);
    }
    wait_vm0();                                         // the trailing zero-fill loads have landed before the exit
}

// ---- the small-M form: at most 32 token rows ----
// With M <= 32 a GEMM is bound by reading its fp8 weight once (the adaLN modulation: M = 2, 18 432 x 3072 = 56.6 MB),
// and the 256 x 256 tiles above would spend their k-loop on zero token rows with one tile per 256 weight rows.  Here
// one wavefront (a workgroup of its own) owns 16 weight rows and all the token rows (one MFMA B block, rows past M read
// as zeros) and streams its k-steps through a private ring of LDS stages with the LDS-DMA loads of the tiled kernel
// (whole 128-byte lines, 8 rows per instruction), depth - 1 k-steps ahead of the MFMAs.  The MFMA's A block is 32
// rows: rows 16-31 repeat rows 0-15 and their results are not stored (a row's result depends on its own A row only).
// Each wave streams its weight rows at a rate bounded by its own load latency, so more, smaller waves finish sooner:
// 16 rows per wave against 32 measured M = 2, N = 18 432, K = 3072: 11.0 -> 10.6 us; M = 5: 6.6 -> 5.8 us; M = 17:
// 4.8 -> 4.4 us; M = 32, K = 8192: 13.9 -> 12.0 us (8 rows per wave: between the two).  A stage holds the 16 weight
// rows and MB 8-row groups of token rows (MB = 1 for M <= 8, else 4; the lanes of token rows past 8 MB take zero
// operands); the ring is 4 stages deep for MB = 1 and 3 for MB = 4 (12 / 18 KiB).  No other wave reads the ring, so no
// barrier: the wave's own vmcnt wait publishes a stage and its own lgkmcnt wait releases it.
// Every output element goes through the same MFMA sequence as in gemm_kernel: v_mfma 32x32x64 with the weight row at
// A-row n % 32 and the token at B-column m % 32, the 64-deep k chunks in ascending order, two per 128-deep k-step (a
// chunk at or past K reads zeros, as the big tiles' last k-step does), and the same epilogue, so the output is bitwise
// the big kernel's.
constexpr int ROWS_MAX_M = 32;
constexpr int ROWS_RW = 16;                               // weight rows per wave

template <int MB>
struct RowsRing {
    static constexpr int STAGE = (ROWS_RW + 8 * MB) * ROWB;    // the weight rows, then 8 MB token rows
    static constexpr int DEPTH = MB == 1 ? 4 : 3;
    static constexpr int LOADS = ROWS_RW / 8 + MB;             // LDS-DMA instructions per k-step
    static_assert(DEPTH >= 2 && LOADS * (DEPTH - 1) <= 63, "vmcnt range");
};

// NT: the weight loads carry the non-temporal hint (chosen by the launcher, see launch_rows_t).
template <int OUT_DT, bool HAS_BIAS, bool AMAX, int MB, bool NT>
__global__ void __launch_bounds__(64) gemm_rows_kernel(GemmParams p) {
    constexpr int ROWS_DEPTH = RowsRing<MB>::DEPTH;
    constexpr int ROWS_STAGE = RowsRing<MB>::STAGE;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[ROWS_DEPTH * ROWS_STAGE];
    const int lane = threadIdx.x;
    const int r = lane & 31, h = lane >> 5;
    const int n0 = (int)blockIdx.x * ROWS_RW;
    const uint32_t lds0 = lds_addr(lds);
    const v4u dw = buffer_desc(p.w, p.w_bytes);
    const v4u da = buffer_desc(p.a, p.a_bytes);
    // LDS-DMA lane layout (as make_loader): lane l moves row 8 i + (l >> 3) of an 8-row group i, LDS chunk l & 7, which
    // holds logical chunk (l & 7) ^ swz(row); swz depends on the row's bit 3, so even and odd groups differ
    const int lrow = lane >> 3;
    const uint32_t lch[2] = {(uint32_t)((lane & 7) ^ swz(lrow)), (uint32_t)((lane & 7) ^ swz(lrow + 8))};
    uint32_t wrow[4], arow[4];                            // byte offsets of this lane's row in each 8-row group
                                                          // (weights: the first ROWS_RW / 8 groups)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int n = n0 + 8 * i + lrow, m = 8 * i + lrow;
        wrow[i] = n < p.N ? (uint32_t)((int64_t)n * p.ldw) : OOB;
        arow[i] = m < p.M ? (uint32_t)((int64_t)m * p.lda) : OOB;
    }
    const int nk = (p.K + BK - 1) / BK;
    // the RowsRing<MB>::LOADS = ROWS_RW / 8 + MB loads of k-step ks into ring slot `slot`: pieces at or past K read
    // zeros (K % 16 == 0)
    auto issue = [&](int slot, int ks) {
        const uint32_t st = lds0 + (uint32_t)slot * ROWS_STAGE;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t c = (uint32_t)ks * BK + 16u * lch[i & 1];
            const bool in = c < (uint32_t)p.K;
            if (i < ROWS_RW / 8) {
                const uint32_t off = in && wrow[i] != OOB ? wrow[i] + c : OOB;
                if (NT) dma16_nt(dw, st + (uint32_t)i * 8 * ROWB, off);
                else dma16(dw, st + (uint32_t)i * 8 * ROWB, off);
            }
            if (i < MB)
                dma16(da, st + ROWS_RW * ROWB + (uint32_t)i * 8 * ROWB, in && arow[i] != OOB ? arow[i] + c : OOB);
        }
    };
    auto kstep_mfma = [&](v16f& acc, int slot) {
        const uint8_t* st = lds + slot * ROWS_STAGE;
        const int alane = (r % ROWS_RW) | (lane & 32);    // A rows past ROWS_RW repeat rows r % ROWS_RW
        const v8i a0 = read_frag(st, alane, 0), a1 = read_frag(st, alane, 1);
        v8i b0 = {0, 0, 0, 0, 0, 0, 0, 0}, b1 = b0;
        if (MB == 4 || r < 8 * MB) {                    // token rows past 8 MB: zero operands, nothing staged
            b0 = read_frag(st + ROWS_RW * ROWB, lane, 0);
            b1 = read_frag(st + ROWS_RW * ROWB, lane, 1);
        }
        wait_lgkm0();                                   // the slot is read: the next issue may refill it
        acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a0, b0, acc, 0, 0, 0, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a1, b1, acc, 0, 0, 0, 0, 0, 0);
    };

    v16f acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.f;
#pragma unroll
    for (int s = 0; s < ROWS_DEPTH; ++s) issue(s, s);
    // every k-step issues ROWS_RW / 8 + MB loads (RowsRing::LOADS; past the last k-step out of range, touching no
    // memory), so when k-step ks is consumed exactly the loads of the ROWS_DEPTH - 1 younger k-steps may be in flight
    int ks = 0;
    for (; ks + ROWS_DEPTH <= nk; ks += ROWS_DEPTH) {
#pragma unroll
        for (int s = 0; s < ROWS_DEPTH; ++s) {
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(RowsRing<MB>::LOADS * (ROWS_DEPTH - 1)));
            asm volatile("" ::: "memory");
            kstep_mfma(acc, s);
            issue(s, ks + s + ROWS_DEPTH);
        }
    }
#pragma unroll
    for (int s = 0; s < ROWS_DEPTH - 1; ++s) {          // the last nk mod ROWS_DEPTH k-steps, already in flight
        if (ks + s < nk) {
            wait_vm0();
            asm volatile("" ::: "memory");
            kstep_mfma(acc, s);
        }
    }
    wait_vm0();                                         // the out-of-range tail loads have landed before the exit

    // epilogue: register 4q + rr holds weight row n0 + 8q + 4h + rr for token r (the MFMA result layout); rows at or
    // past ROWS_RW are the repeated ones
    const int m = r;
    const bool mok = m < p.M;
    const float sam = mok ? p.sa[(int64_t)m * p.sa_stride] : 0.f;
    uint32_t rmax = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int n = n0 + 8 * q + 4 * h;               // N % 16 == 0: a group of four is wholly in or out
        if (8 * q + 4 * h >= ROWS_RW || !mok || n >= p.N) continue;
        if (OUT_DT == H3FP8_DT_F32) {
            const v4f v = {acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
            *reinterpret_cast<v4f*>(reinterpret_cast<float*>(p.y) + (int64_t)m * p.ldy + n) = v;
            continue;
        }
        float v[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const float t = p.sb[(int64_t)(n + rr) * p.sb_stride] * acc[4 * q + rr];
            v[rr] = HAS_BIAS ? __builtin_fmaf(sam, t, load_bias(p.bias, n + rr, OUT_DT)) : sam * t;
        }
        uint32_t lo, hi2;
        if (OUT_DT) {
            lo = fp16_rne(v[0]) | (fp16_rne(v[1]) << 16);
            hi2 = fp16_rne(v[2]) | (fp16_rne(v[3]) << 16);
        } else {
            lo = cvt_bf16x2(v[0], v[1]);
            hi2 = cvt_bf16x2(v[2], v[3]);
        }
        if (AMAX)
            rmax = OUT_DT ? max_abs_f16x2(max_abs_f16x2(rmax, lo), hi2) : max_abs_bf16x2(max_abs_bf16x2(rmax, lo), hi2);
        *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(p.y) + (int64_t)m * p.ldy + n) = make_uint2(lo, hi2);
    }
    if (AMAX) {
        const uint32_t o = (uint32_t)__shfl_xor((int)rmax, 32, 64);
        rmax = rmax > o ? rmax : o;
        if (h == 0 && mok && rmax) atomicMax(reinterpret_cast<unsigned int*>(p.row_amax) + m, rmax);
    }
}

// With at least 4 waves per CU of the one-token-group form the weight stream is bandwidth-bound and its loads take the
// non-temporal hint; with fewer waves (each streaming more k-steps) or the four-group form the hint made it slower.
// Measured (one process, interleaved, median of 7, outputs identical), M x N x K: 2 x 18 432 x 3072 (1152 waves)
// 10.6 -> 9.2 us, 2 x 36 864 x 3072 19.1 -> 17.6, 5 x 18 432 x 3072 10.5 -> 9.3; but 2 x 9216 x 3072 (576 waves)
// 5.8 -> 6.2, 2 x 12 288 x 3072 6.7 -> 6.9, 32 x 18 432 x 3072 (four groups) 12.1 -> 14.2, 32 x 3072 x 8192
// 11.9 -> 15.3; 2 x 16 384 x 8192 (1024 waves of 64 k-steps) 23.0 either way.
template <int OUT_DT, bool HAS_BIAS, bool AMAX>
int launch_rows_t(const GemmParams& p, hipStream_t st) {
    const int waves = (p.N + ROWS_RW - 1) / ROWS_RW;
    const dim3 grid((unsigned)waves);
    if (p.M <= 8) {
        if (waves >= 4 * h3host::cu_count())
            hipLaunchKernelGGL((gemm_rows_kernel<OUT_DT, HAS_BIAS, AMAX, 1, true>), grid, dim3(64), 0, st, p);
        else
            hipLaunchKernelGGL((gemm_rows_kernel<OUT_DT, HAS_BIAS, AMAX, 1, false>), grid, dim3(64), 0, st, p);
    } else {
        hipLaunchKernelGGL((gemm_rows_kernel<OUT_DT, HAS_BIAS, AMAX, 4, false>), grid, dim3(64), 0, st, p);
    }
    H3_CHECK_HIP(hipGetLastError());
    return H3FP8_OK;
}

int launch_rows(const GemmParams& p, int epi, int out_dt, bool has_bias, hipStream_t st) {
    const bool amax = epi == EPI_AMAX;
    if (out_dt == H3FP8_DT_F32) return launch_rows_t<H3FP8_DT_F32, false, false>(p, st);
    if (out_dt == H3FP8_DT_BF16) {
        if (amax) return has_bias ? launch_rows_t<0, true, true>(p, st) : launch_rows_t<0, false, true>(p, st);
        return has_bias ? launch_rows_t<0, true, false>(p, st) : launch_rows_t<0, false, false>(p, st);
    }
    if (amax) return has_bias ? launch_rows_t<1, true, true>(p, st) : launch_rows_t<1, false, true>(p, st);
    return has_bias ? launch_rows_t<1, true, false>(p, st) : launch_rows_t<1, false, false>(p, st);
}

// ---- half tiles (256 tokens x 128 channels) with three stages ----
// The half-tile form runs a problem's last partial round and whole small problems (a 2048 x 3072 x 3072 linear is 96
// full tiles, i.e. 192 half tiles on 192 CUs).  A half tile's k-step has half the MFMAs of a full one, and with two
// stages its loads get about 1.25 k-steps to arrive: it waits on memory latency (about 1.1 us per k-step against
// 0.55 us of MFMAs).  Its stage is 48 KiB (128 weight rows, then 256 token rows), so three fit the LDS when the
// epilogue stores from registers instead of staging its tile: the loads of k-step g+3 go out during k-step g, one
// barrier per k-step both frees stage g and publishes stage g+1, and the loads get about 1.9 k-steps.
// Every output element goes through the same MFMA sequence and epilogue arithmetic as in the full tiles (weight row at
// A-row n % 32, token at B-column m % 32, k ascending), so the output is bitwise the full-tile kernel's.
// Each wave loads 32 weight rows and 64 token rows per k-step (12 LDS-DMA instructions) plus the two scale loads.
constexpr int H3S_STAGE = (128 + 256) * ROWB;       // 48 KiB
constexpr int H3S_A = 128 * ROWB;                   // token rows start after the 128 weight rows
constexpr int H3S_NSTAGE = 3;
constexpr int H3S_NSCALE = 4;                       // the cursor runs up to 3 tiles ahead (1 k-step per tile)
constexpr int H3S_SCALES_OFF = H3S_NSTAGE * H3S_STAGE;
constexpr int H3S_JUNK_OFF = H3S_SCALES_OFF + H3S_NSCALE * SCALE_SET;
constexpr int H3S_LDS = H3S_JUNK_OFF + 512;
static_assert(H3S_LDS <= 160 * 1024, "LDS of one CU");
constexpr int H3S_LOADS = 14;                       // per wave and k-step: 4 weight + 8 token + 2 scale loads

// Half-tile launch: workgroup id -> (tile position in the full-tile order, column half).  The full-tile launch before it
// took workgroups b < full of the XCD-contiguous map over all T full tiles, i.e. the first full / 8 positions of each of
// the 8 per-XCD ranges; the R = T - full positions left are the tails of those ranges.  They are listed range by range
// (so consecutive entries are consecutive positions), split in two halves each, and dealt to the half-tile workgroups
// by the same XCD-contiguous rule: the two halves of a tile and neighbouring tiles run on one XCD and share its L2.
__device__ __forceinline__ void half_tile_of(const GemmParams& p, int id, int n_half, int& tm, int& tn) {
    const int xcd = id & 7, local = id >> 3;
    const int per = n_half >> 3, rem = n_half & 7;
    const int lid = (xcd < rem) ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
    int k = lid >> 1;
    const int T = p.tiles_m * p.tiles_n, pT = T >> 3, rT = T & 7, done = p.half_first >> 3;
    int c = 0;
    for (; c < 7; ++c) {
        const int n_c = pT + (c < rT ? 1 : 0) - done;
        if (k < n_c) break;
        k -= n_c;
    }
    const int pos = ((c < rT) ? c * (pT + 1) : rT * (pT + 1) + (c - rT) * pT) + done + k;
    const int in_group = p.group_m * p.tiles_n;
    const int g = pos / in_group;
    const int first = g * p.group_m;
    const int gsz = min(p.tiles_m - first, p.group_m);
    const int r = pos - g * in_group;
    tm = first + r % gsz;
    tn = 2 * (r / gsz) + (lid & 1);
}

struct Half3Cursor {
    v4u rw, ra, rsa, rsb;
    uint32_t vw[2], va[2], vw_t[2], va_t[2];        // lane parts (even / odd 8-row groups); _t: the K-tail k-step
    uint32_t row8_w, row8_a;
    uint32_t sa_off, sb_off;
    uint32_t dsa, dsb;                              // this wave's share of the tile's scale set (junk when unused)
    int c, ks, nk;
    bool valid;
};

__device__ __forceinline__ void h3s_cursor_set(Half3Cursor& I, const GroupedParams& gp, int c, uint32_t lds0,
                                               int wave, int lane) {
    const int id = (int)blockIdx.x + c * (int)gridDim.x;
    I.c = c;
    I.ks = 0;
    I.valid = id < gp.total_tiles;
    const uint32_t set = lds0 + H3S_SCALES_OFF + (uint32_t)(c % H3S_NSCALE) * SCALE_SET;
    I.dsa = set + 256u * (uint32_t)wave;
    I.dsb = wave < 2 ? set + 1024u + 256u * (uint32_t)wave : lds0 + H3S_JUNK_OFF;
    if (!I.valid) {
#pragma unroll
        for (int e = 0; e < 2; ++e) I.vw[e] = I.va[e] = I.vw_t[e] = I.va_t[e] = OOB;
        I.sa_off = I.sb_off = OOB;
        I.nk = 1;
        return;
    }
    int tm, tn;
    const GemmParams& p = gp.g[0];
    half_tile_of(p, id, gp.total_tiles, tm, tn);
    I.nk = (p.K + BK - 1) / BK;
    const uint32_t lrow = (uint32_t)(lane >> 3);
    const uint32_t lch[2] = {(uint32_t)((lane & 7) ^ swz((int)lrow)), (uint32_t)((lane & 7) ^ swz((int)lrow + 8))};
    const int64_t wrow0 = (int64_t)tn * (BN / 2) + 32 * wave;    // this wave's 32 weight rows
    const int64_t arow0 = (int64_t)tm * BM + 64 * wave;          // ... and 64 token rows
    I.rw = buffer_desc(p.w, p.w_bytes);
    I.ra = buffer_desc(p.a, p.a_bytes);
    const uint32_t ktail = (uint32_t)(p.K % BK);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const uint32_t c16 = 16u * lch[e];
        I.vw[e] = (wrow0 >= p.N) ? OOB : (uint32_t)((wrow0 + lrow) * p.ldw) + c16;   // rows past N: past the range
        I.va[e] = (arow0 >= p.M) ? OOB : (uint32_t)((arow0 + lrow) * p.lda) + c16;   // rows past M: past the range
        const bool cut = ktail != 0 && c16 >= ktail;
        I.vw_t[e] = cut ? OOB : I.vw[e];
        I.va_t[e] = cut ? OOB : I.va[e];
    }
    I.row8_w = (uint32_t)(8 * p.ldw);
    I.row8_a = (uint32_t)(8 * p.lda);
    I.rsa = buffer_desc(p.sa, p.sa_stride ? (uint32_t)((p.M - 1) * p.sa_stride * 4 + 4) : 4u);
    I.rsb = buffer_desc(p.sb, p.sb_stride ? (uint32_t)((p.w_rows - 1) * p.sb_stride * 4 + 4) : 4u);
    const int64_t srow = arow0 + lane;                            // sa of token row 64 wave + lane
    I.sa_off = (srow < p.M) ? (uint32_t)(srow * p.sa_stride * 4) : OOB;
    const int64_t wr = (int64_t)tn * (BN / 2) + 64 * wave + lane;  // waves 0, 1: sb of the tile's 128 weight rows
    I.sb_off = (wave < 2 && wr < p.N) ? (uint32_t)(wr * p.sb_stride * 4) : OOB;
}

__device__ __forceinline__ void h3s_cursor_next(Half3Cursor& I, const GroupedParams& gp, uint32_t lds0, int wave,
                                                int lane) {
    if (++I.ks == I.nk) h3s_cursor_set(I, gp, I.c + 1, lds0, wave, lane);
}

// Load j (0..13) of the cursor's k-step into stage `st`: 0..3 the wave's weight rows (8 per instruction), 4..11 its
// token rows, 12 / 13 the scales (into the tile's scale set at its first k-step, else into the scratch slot).
__device__ __forceinline__ void h3s_issue_one(const Half3Cursor& I, uint32_t st, uint32_t lds0, int wave, int j) {
    const bool last = I.ks == I.nk - 1;
    const uint32_t k0 = (uint32_t)I.ks * BK;
    if (j < 4) {
        const uint32_t off = (last ? I.vw_t[j & 1] : I.vw[j & 1]);
        dma16(I.rw, st + (uint32_t)(32 * wave + 8 * j) * ROWB, off == OOB ? OOB : off + k0 + (uint32_t)j * I.row8_w);
    } else if (j < 12) {
        const int i = j - 4;
        const uint32_t off = (last ? I.va_t[i & 1] : I.va[i & 1]);
        dma16(I.ra, st + H3S_A + (uint32_t)(64 * wave + 8 * i) * ROWB,
              off == OOB ? OOB : off + k0 + (uint32_t)i * I.row8_a);
    } else {
        const bool real = I.valid && I.ks == 0;
        if (j == 12) dma4(I.rsa, real ? I.dsa : lds0 + H3S_JUNK_OFF, real ? I.sa_off : OOB);
        else dma4(I.rsb, real ? I.dsb : lds0 + H3S_JUNK_OFF, real ? I.sb_off : OOB);
    }
}

// Fragment f of a sub-step (0, 1: the wave's two 32-row weight tiles; 2..5: its four 32-row token tiles).
__device__ __forceinline__ void h3s_read(const uint8_t* stage, int wn, int wm, int lane, int sub, int f, v8i af[4],
                                         v8i bf[4]) {
    if (f < 2) af[f] = read_frag(stage + (wn * 64 + 32 * f) * ROWB, lane, sub);
    else bf[f - 2] = read_frag(stage + H3S_A + (wm * 128 + 32 * (f - 2)) * ROWB, lane, sub);
}

// One k-step over 16 MFMA slots (u < 8 sub-step 0, u >= 8 sub-step 1):
//   u < 6       the 6 sub-step-1 fragment reads of stage g;
//   u == 7      lgkmcnt(0) + vmcnt(14) + barrier: every wave's reads of stage g have returned (it is free) and k-step
//               g+1 has landed (only the loads of k-step g+2 may still be in flight);
//   8 <= u < 15 the 14 loads of k-step g+3 into stage g, two per MFMA;
//   8 <= u < 14 the 6 sub-step-0 fragment reads of k-step g+1.
template <bool READ_NEXT>
__device__ __forceinline__ void h3s_kstep(uint8_t* lds, uint32_t lds0, int s0, const Half3Cursor& I, int wave, int wn,
                                          int wm, int lane, v16f acc[4][4], v8i fa0[4], v8i fb0[4], v8i fa1[4],
                                          v8i fb1[4]) {
    const int s1 = s0 == H3S_NSTAGE - 1 ? 0 : s0 + 1;
    const uint8_t* cur = lds + s0 * H3S_STAGE;
    const uint8_t* nxt = lds + s1 * H3S_STAGE;
    const uint32_t st = lds0 + (uint32_t)s0 * H3S_STAGE;
    constexpr int NEXT_ORDER[6] = {0, 2, 3, 4, 5, 1};   // weight tile 0 and the token tiles first: MFMA t uses
                                                        // weight tile t / 4 and token tile t % 4
#pragma unroll
    for (int u = 0; u < 16; ++u) {
        if (u < 8) mfma_one(acc, fa0, fb0, u);
        else mfma_one(acc, fa1, fb1, u - 8);
        if (u < 6) h3s_read(cur, wn, wm, lane, 1, u, fa1, fb1);
        if (u == 7) {
            wait_lgkm0();
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(H3S_LOADS));
            barrier_nofence();
        }
        if (u >= 8 && u < 15) {
            h3s_issue_one(I, st, lds0, wave, 2 * (u - 8));
            h3s_issue_one(I, st, lds0, wave, 2 * (u - 8) + 1);
        }
        if (READ_NEXT && u >= 8 && u < 14) h3s_read(nxt, wn, wm, lane, 0, NEXT_ORDER[u - 8], fa0, fb0);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Epilogue of a wave's NI x NJ MFMA blocks from the accumulators: register 4q + r of block (i, j) is channel
// col0 + 32 i + 8 q + 4 (lane >> 5) + r of token mrow0 + 32 j + (lane & 31); sa_l[sa0 + t] and sb_l[sb0 + c] (LDS)
// hold the scales of token mrow0 + t and channel col0 + c.  Without staging each lane stores its 4 consecutive
// channels (8 bytes, 16 contiguous bytes with the partner lane l ^ 32), so a store instruction touches 32 rows.
// STAGED (bf16 / fp16 outputs): the 32 tokens of block row j go through the wave's LDS area `stg` (rows of NI x 64
// bytes at a stride padded by 16 bytes) and come back as 16-byte chunks, chunk c of row t at lane (32 t + c) % 64 of
// instruction (32 t + c) / 64 -- every store then writes whole row segments of NI x 64 bytes (the store path handles
// about one 128-byte line per cycle, so the lines an instruction touches are what it costs).  Rows past M fall
// outside the output descriptor's range, columns past N get an out-of-range offset.
template <int OUT_DT, bool HAS_BIAS, int EPI, int NI, int NJ, int AI, int AJ, bool STAGED = false>
__device__ __forceinline__ void reg_epilogue(const GemmParams& p, int col0, int mrow0, const float* sa_l, int sa0,
                                             const float* sb_l, int sb0, int lane, v16f (&acc)[AI][AJ],
                                             uint8_t* stg = nullptr) {
    constexpr int CH = NI * 4;                          // 16-byte chunks per staged token row
    constexpr int RS = CH * 16 + 16;                    // staged row stride (padded: rows fall on other banks)
    static_assert(!STAGED || (32 * CH) % 64 == 0, "whole store instructions per block row");
    static_assert(NI <= AI && NJ <= AJ, "blocks of the accumulator array");
    const int hi = lane >> 5, mj = lane & 31;
    if (OUT_DT == H3FP8_DT_F32) {
        float* yf = reinterpret_cast<float*>(p.y);
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const int n = col0 + 32 * i + 8 * q + 4 * hi;
                    const int m = mrow0 + 32 * j + mj;
                    if (n < p.N && m < p.M) {
                        const v4f v = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                                       acc[i][j][4 * q + 3]};
                        *reinterpret_cast<v4f*>(yf + (int64_t)m * p.ldy + n) = v;
                    }
                }
        return;
    }
    const __amdgpu_buffer_rsrc_t yr = make_rsrc(p.y, p.y_bytes);
    const uint32_t row2 = (uint32_t)p.ldy * 2u;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int m = mrow0 + 32 * j + mj;
        const float sam = sa_l[sa0 + 32 * j + mj];
        uint32_t rmax = 0;
        if (STAGED) wave_sync();                        // the previous block row's reads before these writes
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = col0 + 32 * i + 8 * q + 4 * hi;
                const v4f sbn = *reinterpret_cast<const v4f*>(sb_l + sb0 + 32 * i + 8 * q + 4 * hi);
                float bn[4] = {0, 0, 0, 0};
                if (HAS_BIAS) {
                    const int nc = n < p.N ? n : 0;
#pragma unroll
                    for (int r = 0; r < 4; ++r) bn[r] = load_bias(p.bias, nc + r, OUT_DT);
                }
                float v[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float t = sbn[r] * acc[i][j][4 * q + r];
                    v[r] = HAS_BIAS ? __builtin_fmaf(sam, t, bn[r]) : sam * t;
                }
                uint32_t lo, hi2;
                if (OUT_DT) {
                    lo = fp16_rne(v[0]) | (fp16_rne(v[1]) << 16);
                    hi2 = fp16_rne(v[2]) | (fp16_rne(v[3]) << 16);
                } else {
                    lo = cvt_bf16x2(v[0], v[1]);
                    hi2 = cvt_bf16x2(v[2], v[3]);
                }
                if (EPI == EPI_AMAX && n < p.N && m < p.M)
                    rmax = OUT_DT ? max_abs_f16x2(max_abs_f16x2(rmax, lo), hi2)
                                  : max_abs_bf16x2(max_abs_bf16x2(rmax, lo), hi2);
                const v2u32 val = {lo, hi2};
                if (STAGED) {
                    *reinterpret_cast<v2u32*>(stg + mj * RS + (4 * i + q) * 16 + 8 * hi) = val;
                } else {
                    const uint32_t off = (n < p.N) ? (uint32_t)m * row2 + (uint32_t)n * 2u : OOB;
                    __builtin_amdgcn_raw_buffer_store_b64(val, yr, off, 0, 0);
                }
            }
        if (STAGED) {
            wave_sync();                                // every lane's writes before any lane's reads
            constexpr int NS = 32 * CH / 64;
            v4u v[NS];
            uint32_t off[NS];
#pragma unroll
            for (int s2 = 0; s2 < NS; ++s2) {           // all reads before the first store
                const int idx = 64 * s2 + lane, t = idx / CH, c = idx - t * CH;
                v[s2] = *reinterpret_cast<const v4u*>(stg + t * RS + c * 16);
                const int n = col0 + 8 * c;
                off[s2] = (n < p.N) ? (uint32_t)(mrow0 + 32 * j + t) * row2 + (uint32_t)n * 2u : OOB;
            }
#pragma unroll
            for (int s2 = 0; s2 < NS; ++s2) __builtin_amdgcn_raw_buffer_store_b128(v[s2], yr, off[s2], 0, 0);
        }
        if (EPI == EPI_AMAX) {
            const uint32_t o = (uint32_t)__shfl_xor((int)rmax, 32, 64);
            rmax = rmax > o ? rmax : o;
            if (hi == 0 && m < p.M && rmax) atomicMax(reinterpret_cast<unsigned int*>(p.row_amax) + m, rmax);
        }
    }
}

// A half tile's wave owns 2 x 4 blocks: channels tn * 128 + 64 wn onwards, tokens tm * 256 + 128 wm onwards.
template <int OUT_DT, bool HAS_BIAS, int EPI>
__device__ __forceinline__ void h3s_epilogue(const GemmParams& p, int tm, int tn, const uint8_t* lds, int set, int wn,
                                             int wm, int lane, v16f (&acc)[4][4]) {
    const float* sa_l = reinterpret_cast<const float*>(lds + H3S_SCALES_OFF + set * SCALE_SET);
    const float* sb_l = sa_l + 256;
    reg_epilogue<OUT_DT, HAS_BIAS, EPI, 2, 4>(p, tn * (BN / 2) + wn * 64, tm * BM + wm * 128, sa_l, wm * 128, sb_l,
                                              wn * 64, lane, acc);
}

template <int OUT_DT, bool HAS_BIAS, int EPI>
__global__ void __launch_bounds__(256, 1) gemm_half3_kernel(GroupedParams gp) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[H3S_LDS];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int wn = wave & 1, wm = wave >> 1;
    const int G = (int)gridDim.x;
    const uint32_t lds0 = lds_addr(lds);
    Half3Cursor I;
    h3s_cursor_set(I, gp, 0, lds0, wave, lane);
    if (!I.valid) return;
    // prologue: k-steps 0, 1, 2 in flight (14 loads each), then stage 0 published
#pragma unroll
    for (int s = 0; s < H3S_NSTAGE; ++s) {
#pragma unroll
        for (int j = 0; j < H3S_LOADS; ++j) h3s_issue_one(I, lds0 + (uint32_t)s * H3S_STAGE, lds0, wave, j);
        if (I.valid) h3s_cursor_next(I, gp, lds0, wave, lane);
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * H3S_LOADS));
    barrier_nofence();
    v8i fa0[4], fb0[4], fa1[4], fb1[4];
#pragma unroll
    for (int f = 0; f < 6; ++f) h3s_read(lds, wn, wm, lane, 0, f, fa0, fb0);
    int s0 = 0;
    for (int c = 0;; ++c) {
        const int id = (int)blockIdx.x + c * G;
        int tm, tn;
        const GemmParams& p = gp.g[0];
        half_tile_of(p, id, gp.total_tiles, tm, tn);
        const int nk = (p.K + BK - 1) / BK;
        v16f acc[4][4];                                 // acc[0..1][*] used
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
        for (int ks = 0; ks < nk - 1; ++ks) {
            h3s_kstep<true>(lds, lds0, s0, I, wave, wn, wm, lane, acc, fa0, fb0, fa1, fb1);
            if (I.valid) h3s_cursor_next(I, gp, lds0, wave, lane);
            s0 = s0 == H3S_NSTAGE - 1 ? 0 : s0 + 1;
        }
        h3s_kstep<false>(lds, lds0, s0, I, wave, wn, wm, lane, acc, fa0, fb0, fa1, fb1);
        if (I.valid) h3s_cursor_next(I, gp, lds0, wave, lane);
        s0 = s0 == H3S_NSTAGE - 1 ? 0 : s0 + 1;
        h3s_epilogue<OUT_DT, HAS_BIAS, EPI>(p, tm, tn, lds, c % H3S_NSCALE, wn, wm, lane, acc);
        __builtin_amdgcn_sched_barrier(0);
        if (id + G >= gp.total_tiles) break;
#pragma unroll
        for (int f = 0; f < 6; ++f) h3s_read(lds + s0 * H3S_STAGE, wn, wm, lane, 0, f, fa0, fb0);
    }
    wait_vm0();                                         // the trailing zero-fill loads have landed before the exit
}

// ---- 128 x 192 tiles, one per workgroup (problems that fit one round) ----
// A problem whose 256 x 256 tiles number at most half the CUs runs as half tiles, which can still leave CUs idle: the
// single linear 2048 x 3072 x 3072 has 96 full tiles, 192 half tiles, on 256 CUs.  Tiles of 128 token rows x 192
// weight rows cover it with 16 x 16 = 256 workgroups, one per CU, each loading 40 KiB per k-step (half tiles: 48).
// The four waves own 96 weight rows x 64 token rows each (3 x 2 MFMA blocks).  Every output element gets the same
// MFMA sequence as in the other forms (k sub-steps of 64 in order from a zero accumulator), so the same bits.
constexpr int W192_WR = 192;                            // weight rows per tile
constexpr int W192_TR = 128;                            // token rows per tile
constexpr int W192_STAGE = (W192_WR + W192_TR) * ROWB;  // 40 KiB
constexpr int W192_A = W192_WR * ROWB;                  // token rows start after the weight rows
constexpr int W192_NSTAGE = 3;
constexpr int W192_SCALES_OFF = W192_NSTAGE * W192_STAGE;
constexpr int W192_JUNK_OFF = W192_SCALES_OFF + SCALE_SET;
constexpr int W192_STG_OFF = W192_JUNK_OFF + 512;      // the epilogue's staging: per wave 32 rows of 192 + 16 bytes
constexpr int W192_STG_PER_WAVE = 32 * (3 * 64 + 16);
constexpr int W192_LDS = W192_STG_OFF + 4 * W192_STG_PER_WAVE;
static_assert(W192_LDS <= 160 * 1024, "LDS of one CU");
constexpr int W192_LOADS = 12;                          // per wave and k-step: 6 weight + 4 token + 2 scale loads
constexpr int W192_GROUP_M = 8;                         // token-tile rows per group of the XCD-contiguous tile map
                                                        // (c1: an XCD's 32 tiles read 5.5 MB of operands, with 4 rows
                                                        // 6.3 MB; measured 1-3 % faster than 4)

struct W192Loader {
    v4u rw, ra, rsa, rsb;
    uint32_t vw[2], va[2], vw_t[2], va_t[2];            // lane parts (even / odd 8-row groups); _t: the K-tail k-step
    uint32_t row8_w, row8_a;
    uint32_t sa_off, sb_off;
    uint32_t dsa, dsb;                                  // this wave's share of the tile's scale set (junk when unused)
    int wgroups, agroups;                               // this wave's 8-row groups that start inside N / M
    int nk;
};

// Wave w loads weight rows 48 w .. 48 w + 47 and token rows 32 w .. 32 w + 31 of the tile (6 and 4 groups of 8 rows);
// waves 0, 1 the sa of the tile's 128 token rows, waves 0..2 the sb of its 192 weight rows.
__device__ __forceinline__ void w192_loader_set(W192Loader& L, const GemmParams& p, int tm, int tn, uint32_t lds0,
                                                int wave, int lane) {
    L.nk = (p.K + BK - 1) / BK;
    const uint32_t lrow = (uint32_t)(lane >> 3);
    const uint32_t lch[2] = {(uint32_t)((lane & 7) ^ swz((int)lrow)), (uint32_t)((lane & 7) ^ swz((int)lrow + 8))};
    const int64_t wrow0 = (int64_t)tn * W192_WR + 48 * wave;
    const int64_t arow0 = (int64_t)tm * W192_TR + 32 * wave;
    const int64_t wg = wrow0 < p.N ? (p.N - wrow0 + 7) / 8 : 0, ag = arow0 < p.M ? (p.M - arow0 + 7) / 8 : 0;
    L.wgroups = (int)(wg < 6 ? wg : 6);
    L.agroups = (int)(ag < 4 ? ag : 4);
    L.rw = buffer_desc(p.w, p.w_bytes);
    L.ra = buffer_desc(p.a, p.a_bytes);
    const uint32_t ktail = (uint32_t)(p.K % BK);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const uint32_t c16 = 16u * lch[e];
        L.vw[e] = L.wgroups ? (uint32_t)((wrow0 + lrow) * p.ldw) + c16 : OOB;
        L.va[e] = L.agroups ? (uint32_t)((arow0 + lrow) * p.lda) + c16 : OOB;
        const bool cut = ktail != 0 && c16 >= ktail;
        L.vw_t[e] = cut ? OOB : L.vw[e];
        L.va_t[e] = cut ? OOB : L.va[e];
    }
    L.row8_w = (uint32_t)(8 * p.ldw);
    L.row8_a = (uint32_t)(8 * p.lda);
    L.rsa = buffer_desc(p.sa, p.sa_stride ? (uint32_t)((p.M - 1) * p.sa_stride * 4 + 4) : 4u);
    L.rsb = buffer_desc(p.sb, p.sb_stride ? (uint32_t)((p.w_rows - 1) * p.sb_stride * 4 + 4) : 4u);
    const uint32_t set = lds0 + W192_SCALES_OFF;
    L.dsa = wave < 2 ? set + 256u * (uint32_t)wave : lds0 + W192_JUNK_OFF;
    L.dsb = wave < 3 ? set + 1024u + 256u * (uint32_t)wave : lds0 + W192_JUNK_OFF;
    const int64_t srow = (int64_t)tm * W192_TR + 64 * wave + lane;
    L.sa_off = (wave < 2 && srow < p.M) ? (uint32_t)(srow * p.sa_stride * 4) : OOB;
    const int64_t wr = (int64_t)tn * W192_WR + 64 * wave + lane;
    L.sb_off = (wave < 3 && wr < p.N) ? (uint32_t)(wr * p.sb_stride * 4) : OOB;
}

// Load j (0..11) of k-step kl into stage `st`: 0..5 the wave's weight rows (8 per instruction), 6..9 its token rows,
// 10 / 11 the scales (into the scale set at k-step 0, else into the scratch slot).  K-steps past the last one load
// zeros (every k-step issues the same 12 loads, which the vmcnt waits count on).
__device__ __forceinline__ void w192_issue_one(const W192Loader& L, int kl, uint32_t st, uint32_t lds0, int wave,
                                               int j) {
    const bool live = kl < L.nk;
    const bool last = kl == L.nk - 1;
    const uint32_t k0 = (uint32_t)kl * BK;
    if (j < 6) {
        const uint32_t off = last ? L.vw_t[j & 1] : L.vw[j & 1];
        const bool ok = live && j < L.wgroups && off != OOB;
        dma16(L.rw, st + (uint32_t)(48 * wave + 8 * j) * ROWB, ok ? off + k0 + (uint32_t)j * L.row8_w : OOB);
    } else if (j < 10) {
        const int i = j - 6;
        const uint32_t off = last ? L.va_t[i & 1] : L.va[i & 1];
        const bool ok = live && i < L.agroups && off != OOB;
        dma16(L.ra, st + W192_A + (uint32_t)(32 * wave + 8 * i) * ROWB, ok ? off + k0 + (uint32_t)i * L.row8_a : OOB);
    } else {
        const bool real = kl == 0;
        if (j == 10) dma4(L.rsa, real ? L.dsa : lds0 + W192_JUNK_OFF, real ? L.sa_off : OOB);
        else dma4(L.rsb, real ? L.dsb : lds0 + W192_JUNK_OFF, real ? L.sb_off : OOB);
    }
}

// Fragment f of a sub-step (0..2: the wave's three 32-row weight blocks; 3, 4: its two 32-row token blocks).
__device__ __forceinline__ void w192_read(const uint8_t* stage, int wn, int wm, int lane, int sub, int f, v8i af[3],
                                          v8i bf[2]) {
    if (f < 3) af[f] = read_frag(stage + (wn * 96 + 32 * f) * ROWB, lane, sub);
    else bf[f - 3] = read_frag(stage + W192_A + (wm * 64 + 32 * (f - 3)) * ROWB, lane, sub);
}

__device__ __forceinline__ void w192_mfma(v16f acc[3][2], const v8i af[3], const v8i bf[2], int t) {
    acc[t >> 1][t & 1] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(af[t >> 1], bf[t & 1], acc[t >> 1][t & 1], 0, 0,
                                                                         0, 0, 0, 0);
}

// K-step ks over 12 MFMA slots (u < 6 sub-step 0, u >= 6 sub-step 1):
//   u < 5        the 5 sub-step-1 fragment reads of stage ks;
//   u == 5       lgkmcnt(0) + vmcnt(12) + barrier: every wave's reads of stage ks have returned (it is free) and k-step
//                ks + 1 has landed (only the loads of k-step ks + 2 may still be in flight);
//   6 <= u < 12  the 12 loads of k-step ks + 3 into stage ks, two per MFMA;
//   6 <= u < 11  the 5 sub-step-0 fragment reads of k-step ks + 1.
template <bool READ_NEXT>
__device__ __forceinline__ void w192_kstep(uint8_t* lds, uint32_t lds0, int s0, int ks, const W192Loader& L, int wave,
                                           int wn, int wm, int lane, v16f acc[3][2], v8i fa0[3], v8i fb0[2],
                                           v8i fa1[3], v8i fb1[2]) {
    const int s1 = s0 == W192_NSTAGE - 1 ? 0 : s0 + 1;
    const uint8_t* cur = lds + s0 * W192_STAGE;
    const uint8_t* nxt = lds + s1 * W192_STAGE;
    const uint32_t st = lds0 + (uint32_t)s0 * W192_STAGE;
    constexpr int NEXT_ORDER[5] = {0, 3, 4, 1, 2};      // weight block 0 and the token blocks first: MFMA t uses
                                                        // weight block t / 2 and token block t % 2
#pragma unroll
    for (int u = 0; u < 12; ++u) {
        if (u < 6) w192_mfma(acc, fa0, fb0, u);
        else w192_mfma(acc, fa1, fb1, u - 6);
        if (u < 5) w192_read(cur, wn, wm, lane, 1, u, fa1, fb1);
        if (u == 5) {
            wait_lgkm0();
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(W192_LOADS));
            barrier_nofence();
        }
        if (u >= 6) {
            w192_issue_one(L, ks + 3, st, lds0, wave, 2 * (u - 6));
            w192_issue_one(L, ks + 3, st, lds0, wave, 2 * (u - 6) + 1);
        }
        if (READ_NEXT && u >= 6 && u < 11) w192_read(nxt, wn, wm, lane, 0, NEXT_ORDER[u - 6], fa0, fb0);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// One tile per workgroup: the launch has exactly as many workgroups as tiles, all resident at once (at most one per
// CU), so there is no persistent loop.
template <int OUT_DT, bool HAS_BIAS, int EPI>
__global__ void __launch_bounds__(256, 1) gemm_w192_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[W192_LDS];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int wn = wave & 1, wm = wave >> 1;
    const uint32_t lds0 = lds_addr(lds);
    const int tiles_m = (p.M + W192_TR - 1) / W192_TR, tiles_n = (p.N + W192_WR - 1) / W192_WR;
    int tm, tn;
    tile_of((int)blockIdx.x, tiles_m * tiles_n, tiles_m, tiles_n, W192_GROUP_M, tm, tn);
    W192Loader L;
    w192_loader_set(L, p, tm, tn, lds0, wave, lane);
    // prologue: k-steps 0, 1, 2 in flight (12 loads each), then stage 0 published
#pragma unroll
    for (int s = 0; s < W192_NSTAGE; ++s) {
#pragma unroll
        for (int j = 0; j < W192_LOADS; ++j) w192_issue_one(L, s, lds0 + (uint32_t)s * W192_STAGE, lds0, wave, j);
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * W192_LOADS));
    barrier_nofence();
    v8i fa0[3], fb0[2], fa1[3], fb1[2];
#pragma unroll
    for (int f = 0; f < 5; ++f) w192_read(lds, wn, wm, lane, 0, f, fa0, fb0);
    v16f acc[3][2];
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    int s0 = 0;
    for (int ks = 0; ks < L.nk - 1; ++ks) {
        w192_kstep<true>(lds, lds0, s0, ks, L, wave, wn, wm, lane, acc, fa0, fb0, fa1, fb1);
        s0 = s0 == W192_NSTAGE - 1 ? 0 : s0 + 1;
    }
    w192_kstep<false>(lds, lds0, s0, L.nk - 1, L, wave, wn, wm, lane, acc, fa0, fb0, fa1, fb1);
    const float* sa_l = reinterpret_cast<const float*>(lds + W192_SCALES_OFF);
    reg_epilogue<OUT_DT, HAS_BIAS, EPI, 3, 2, 3, 2, true>(p, tn * W192_WR + wn * 96, tm * W192_TR + wm * 64, sa_l,
                                                          wm * 64, sa_l + 256, wn * 96, lane, acc,
                                                          lds + W192_STG_OFF + wave * W192_STG_PER_WAVE);
    wait_vm0();                                         // the trailing zero-fill loads have landed before the exit
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

// Workgroups of a persistent launch over `tiles` tiles: one per CU, at most one per tile.
int grid_for(int tiles) { return std::max(1, std::min(tiles, h3host::cu_count())); }

template <int OUT_DT, bool HAS_BIAS, int EPI, bool GROUPED>
int launch_one(const GroupedParams& gp, hipStream_t st) {
    hipLaunchKernelGGL((gemm_kernel<OUT_DT, HAS_BIAS, EPI, GROUPED>), dim3(grid_for(gp.total_tiles)), dim3(256), 0, st,
                       gp);
    H3_CHECK_HIP(hipGetLastError());
    return H3FP8_OK;
}

template <int EPI>
int dispatch(const GroupedParams& gp, int out_dt, bool has_bias, hipStream_t st) {
    if (out_dt == H3FP8_DT_BF16) {
        return has_bias ? launch_one<0, true, EPI, false>(gp, st) : launch_one<0, false, EPI, false>(gp, st);
    }
    if (out_dt == H3FP8_DT_F32) return launch_one<H3FP8_DT_F32, false, EPI_PLAIN, false>(gp, st);
    return has_bias ? launch_one<1, true, EPI, false>(gp, st) : launch_one<1, false, EPI, false>(gp, st);
}

template <int OUT_DT, bool HAS_BIAS, int EPI>
int launch_half3(const GroupedParams& gp, hipStream_t st) {
    hipLaunchKernelGGL((gemm_half3_kernel<OUT_DT, HAS_BIAS, EPI>), dim3(grid_for(gp.total_tiles)), dim3(256), 0, st, gp);
    H3_CHECK_HIP(hipGetLastError());
    return H3FP8_OK;
}

int dispatch_half3(const GroupedParams& gp, int epi, int out_dt, bool has_bias, hipStream_t st) {
    if (out_dt == H3FP8_DT_F32) return launch_half3<H3FP8_DT_F32, false, EPI_PLAIN>(gp, st);
    if (epi == EPI_AMAX) {
        if (out_dt == H3FP8_DT_BF16)
            return has_bias ? launch_half3<0, true, EPI_AMAX>(gp, st) : launch_half3<0, false, EPI_AMAX>(gp, st);
        return has_bias ? launch_half3<1, true, EPI_AMAX>(gp, st) : launch_half3<1, false, EPI_AMAX>(gp, st);
    }
    if (out_dt == H3FP8_DT_BF16)
        return has_bias ? launch_half3<0, true, EPI_PLAIN>(gp, st) : launch_half3<0, false, EPI_PLAIN>(gp, st);
    return has_bias ? launch_half3<1, true, EPI_PLAIN>(gp, st) : launch_half3<1, false, EPI_PLAIN>(gp, st);
}

template <int OUT_DT, bool HAS_BIAS, int EPI>
int launch_w192(const GemmParams& p, int tiles, hipStream_t st) {
    hipLaunchKernelGGL((gemm_w192_kernel<OUT_DT, HAS_BIAS, EPI>), dim3(tiles), dim3(256), 0, st, p);
    H3_CHECK_HIP(hipGetLastError());
    return H3FP8_OK;
}

int dispatch_w192(const GemmParams& p, int tiles, int epi, int out_dt, bool has_bias, hipStream_t st) {
    if (out_dt == H3FP8_DT_F32) return launch_w192<H3FP8_DT_F32, false, EPI_PLAIN>(p, tiles, st);
    if (epi == EPI_AMAX) {
        if (out_dt == H3FP8_DT_BF16)
            return has_bias ? launch_w192<0, true, EPI_AMAX>(p, tiles, st) : launch_w192<0, false, EPI_AMAX>(p, tiles, st);
        return has_bias ? launch_w192<1, true, EPI_AMAX>(p, tiles, st) : launch_w192<1, false, EPI_AMAX>(p, tiles, st);
    }
    if (out_dt == H3FP8_DT_BF16)
        return has_bias ? launch_w192<0, true, EPI_PLAIN>(p, tiles, st) : launch_w192<0, false, EPI_PLAIN>(p, tiles, st);
    return has_bias ? launch_w192<1, true, EPI_PLAIN>(p, tiles, st) : launch_w192<1, false, EPI_PLAIN>(p, tiles, st);
}

// The last, partial round of a launch with full tiles leaves most CUs idle.  When its tiles fit one round as half
// tiles (256 tokens x 128 channels, the same MFMAs per output element, so the same bits), the full-tile launch stops
// at the last whole round and a half-tile launch covers the rest: a problem of T full tiles on G CUs runs
// floor(T / G) full rounds and, if T mod G <= G / 2, the remainder as 2 (T mod G) half tiles.  Kernel 3 (SwiGLU pairs
// gate and up rows inside a tile) always runs full tiles.  A problem that runs as half tiles alone takes 128 x 192
// tiles instead when they occupy more CUs and still fit one round (gemm_w192_kernel).
int launch_split(GroupedParams gp, int epi, int out_dt, bool has_bias, hipStream_t st) {
    const int T = gp.g[0].tiles_m * gp.g[0].tiles_n;
    const int G = h3host::cu_count();
    const int full = (epi == EPI_SWIGLU) ? T : (T / G) * G;
    const int rest = T - full;
    // half_tile_of takes the full-tile launch to have covered the first full / 8 positions of each per-XCD range,
    // which holds when full is a multiple of 8 (a CU count that is a multiple of 8, as on gfx950); otherwise the
    // launch keeps full tiles throughout
    const bool half = rest > 0 && 2 * rest <= G && full % 8 == 0;
    const int full_tiles = half ? full : T;
    if (full_tiles == 0) {
        const GemmParams& p = gp.g[0];
        const int64_t w192 = (int64_t)((p.M + W192_TR - 1) / W192_TR) * ((p.N + W192_WR - 1) / W192_WR);
        if (w192 <= G && w192 > 2 * (int64_t)rest) return dispatch_w192(p, (int)w192, epi, out_dt, has_bias, st);
    }
    int rc = H3FP8_OK;
    if (full_tiles > 0) {
        gp.total_tiles = full_tiles;
        if (epi == EPI_PLAIN) rc = dispatch<EPI_PLAIN>(gp, out_dt, has_bias, st);
        else if (epi == EPI_AMAX) rc = dispatch<EPI_AMAX>(gp, out_dt, has_bias, st);
        else rc = dispatch<EPI_SWIGLU>(gp, H3FP8_DT_BF16, has_bias, st);
        if (rc || !half) return rc;
    }
    gp.g[0].half_first = full_tiles;
    gp.total_tiles = 2 * rest;
    return dispatch_half3(gp, epi, out_dt, has_bias, st);
}

constexpr int64_t kMaxBufferBytes = 0x7fff0000LL;   // buffer offsets are 32-bit; keep clear of the OOB marker
constexpr int64_t kMallBytes = 256LL << 20;          // MI355X's last-level cache (MALL) in front of HBM

// Common argument checks.
int check_gemm(const void* a, int64_t lda, const void* w, int64_t ldw, const float* sa, int64_t sa_stride,
               const float* sb, int64_t sb_stride, const void* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
               int64_t w_rows, const char* who) {
    H3_REQUIRE(M >= 0 && N >= 0 && K >= 0, "%s: negative size", who);
    H3_REQUIRE(K % 16 == 0 && N % 16 == 0, "%s: K=%lld and N=%lld must be multiples of 16", who, (long long)K,
               (long long)N);
    H3_REQUIRE(M <= 0x7fffffff && N <= 0x7fffffff && K <= 0x7fffffff, "%s: size too large", who);
    if (M == 0 || N == 0) return H3FP8_OK;
    // an empty reduction is refused rather than run: the k-loops assume at least one k-step
    H3_REQUIRE(K > 0, "%s: K must be positive (got 0)", who);
    H3_REQUIRE(a && w && sa && sb && y, "%s: null pointer", who);
    H3_REQUIRE(lda >= K && lda % 16 == 0 && ldw >= K && ldw % 16 == 0, "%s: lda/ldw must be >= K and multiples of 16",
               who);
    H3_REQUIRE(ldy >= N && ldy % 8 == 0, "%s: ldy must be >= N and a multiple of 8", who);
    H3_REQUIRE(((uintptr_t)a & 15) == 0 && ((uintptr_t)w & 15) == 0 && ((uintptr_t)y & 15) == 0,
               "%s: a, w and y must be 16-byte aligned", who);
    H3_REQUIRE(((uintptr_t)sa & 3) == 0 && ((uintptr_t)sb & 3) == 0, "%s: scales must be 4-byte aligned", who);
    H3_REQUIRE(sa_stride >= 0 && sb_stride >= 0, "%s: negative scale stride", who);
    H3_REQUIRE((w_rows - 1) * ldw + K <= kMaxBufferBytes, "%s: weight too large for one buffer range", who);
    H3_REQUIRE((w_rows - 1) * sb_stride * 4 + 4 <= kMaxBufferBytes, "%s: sb too large", who);
    H3_REQUIRE(lda * 512 <= kMaxBufferBytes, "%s: lda too large", who);
    H3_REQUIRE(ldy * 4 * 512 <= kMaxBufferBytes, "%s: ldy too large", who);
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
    p.w_rows = (int)w_rows;
    p.a_bytes = (uint32_t)((M - 1) * lda + K);
    p.w_bytes = (uint32_t)((w_rows - 1) * ldw + K);
    p.y_bytes = (uint32_t)(((M - 1) * ldy + N) * 2);   // bf16 / fp16 (run_gemm resets it for fp32 outputs)
    const int64_t n_tile_cols = swiglu ? (BN / 2) : BN;
    p.tiles_m = (int)((M + BM - 1) / BM);
    p.tiles_n = (int)((N + n_tile_cols - 1) / n_tile_cols);
    p.group_m = 4;
    p.tile_offset = 0;
    return p;
}

// Launches one problem, splitting M so that every launch's activation and scale ranges fit 32-bit buffer offsets.
int run_gemm(int epi, const uint8_t* a, int64_t lda, const uint8_t* w, int64_t ldw, const float* sa,
             int64_t sa_stride, const float* sb, int64_t sb_stride, const void* bias, void* y, int64_t ldy,
             int out_dt, int64_t M, int64_t N, int64_t K, int64_t w_rows, float* row_amax, const uint16_t* silu,
             hipStream_t st) {
    if (epi != EPI_SWIGLU && M <= ROWS_MAX_M) {
        // weight-bound: one wave per 16 weight rows (gemm_rows_kernel), bitwise the tiled kernel's output
        const GemmParams p = make_params(a, lda, w, ldw, sa, sa_stride, sb, sb_stride, bias, y, ldy, M, N, K, w_rows,
                                         row_amax, silu, false);
        return launch_rows(p, epi, out_dt, bias != nullptr, st);
    }
    const int out_elem = (out_dt == H3FP8_DT_F32) ? 4 : 2;
    int64_t rows_per = std::max<int64_t>(BM, ((kMaxBufferBytes - K) / lda + 1) / BM * BM);
    if (sa_stride > 0) rows_per = std::min<int64_t>(rows_per, std::max<int64_t>(BM, kMaxBufferBytes / (4 * sa_stride) / BM * BM));
    // the output's byte offsets (stored through a range-checked descriptor) are 32-bit as well: rows of ldy elements of
    // out_elem bytes (a bf16 [91 728, 9216] output fits one launch)
    rows_per = std::min<int64_t>(rows_per, std::max<int64_t>(BM, kMaxBufferBytes / (out_elem * ldy) / BM * BM));
    for (int64_t r0 = 0; r0 < M; r0 += rows_per) {
        const int64_t Mi = std::min<int64_t>(rows_per, M - r0);
        GroupedParams gp{};
        gp.g[0] = make_params(a + r0 * lda, lda, w, ldw, sa + r0 * sa_stride, sa_stride, sb, sb_stride, bias,
                              reinterpret_cast<uint8_t*>(y) + r0 * ldy * out_elem, ldy, Mi, N, K, w_rows,
                              row_amax ? row_amax + r0 : nullptr, silu, epi == EPI_SWIGLU);
        gp.n = 1;
        if (epi == EPI_SWIGLU) gp.g[0].silu_rot = h3host::silu_rot_ptr();
        if (out_dt == H3FP8_DT_F32) {
            gp.g[0].y_bytes = (uint32_t)(((Mi - 1) * ldy + N) * 4);
            // a product larger than the MALL (256 MiB on MI355X) cannot stay cached for its consumer: the full tiles
            // store it non-temporally (measured, GEMM + scale pass: 16 740 x 9216 x 3072 570 -> 542 us, 31 248 x
            // 3072 x 3072 336 -> 328 us; a product that fits, 4100 x 5376 x 7168 (88 MB), 161.6 -> 167.1 us).  The
            // bf16 outputs gained nothing measurable from it (-0.8 to +0.4 % per GEMM of the 1344x768 15 s chain).
            gp.g[0].y_nt = M * N * 4 > kMallBytes;
        }
        const int rc = launch_split(gp, epi, out_dt, bias != nullptr, st);
        if (rc) return rc;
    }
    return H3FP8_OK;
}

}  // namespace

namespace h3host {
int quant_rows_amax_launch(const void* x, int64_t ldx, int64_t M, int64_t K, const float* row_amax, void* q,
                           int64_t ldq, float* scale, hipStream_t st);
int quant_args_ok(const void* x, int64_t ldx, int64_t M, int64_t K, const void* q, int64_t ldq, const float* scale);
}

// ---- the library-owned row-maxima buffer of h3fp8_gemm_quant_noalloc -------------------------------------------------
// One array per device (the loader gives every device its own copy at its own address), H3FP8_NOALLOC_MAX_ROWS fp32
// row maxima = 1 MiB, held until the process ends.  Its name is a host-side stand-in: host code uses only the device
// address that hipGetSymbolAddress returned for the device (g_scratch_ptr), never `scratch` itself.
static __device__ __align__(256) float scratch[H3FP8_NOALLOC_MAX_ROWS];

namespace {
constexpr int kScratchDevices = 64;
float* g_scratch_ptr[kScratchDevices] = {};
}  // namespace

namespace h3host {
// Called once per device by the library's set-up (ensure_device_init), with that device current.
int gemm_scratch_setup(int dev) {
    if (dev < 0 || dev >= kScratchDevices) {
        set_error("device index %d out of range", dev);
        return H3FP8_EINVAL;
    }
    float* p = nullptr;
    H3_CHECK_HIP(hipGetSymbolAddress((void**)&p, HIP_SYMBOL(scratch)));
    g_scratch_ptr[dev] = p;
    return H3FP8_OK;
}
}  // namespace h3host

extern "C" {

int h3fp8_gemm(const void* a, int64_t lda, const void* w, int64_t ldw, const float* sa, int64_t sa_stride,
               const float* sb, int64_t sb_stride, const void* bias, void* y, int64_t ldy, int out_dtype, int64_t M,
               int64_t N, int64_t K, float* row_amax, void* stream) {
    int rc = check_gemm(a, lda, w, ldw, sa, sa_stride, sb, sb_stride, y, ldy, M, N, K, N, "h3fp8_gemm");
    if (rc) return rc;
    H3_REQUIRE(out_dtype == H3FP8_DT_BF16 || out_dtype == H3FP8_DT_FP16 || out_dtype == H3FP8_DT_F32,
               "h3fp8_gemm: bad out_dtype %d", out_dtype);
    H3_REQUIRE(out_dtype != H3FP8_DT_F32 || (!bias && !row_amax && ldy % 4 == 0),
               "h3fp8_gemm: the raw fp32 accumulator output takes no bias or row_amax and needs ldy %% 4 == 0");
    if (M == 0 || N == 0) return H3FP8_OK;
    rc = h3host::ensure_device_init();
    if (rc) return rc;
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
    // the tail's arguments are checked before the GEMM is enqueued: a bad ldq leaves nothing launched
    int rc = h3host::quant_args_ok(y, ldy, M, N, q, ldq, scale);
    if (rc) return rc;
    rc = h3fp8_gemm(a, lda, w, ldw, sa, sa_stride, sb, sb_stride, bias, y, ldy, H3FP8_DT_BF16, M, N, K, amax_ws,
                        stream);
    if (rc) return rc;
    return h3host::quant_rows_amax_launch(y, ldy, M, N, amax_ws, q, ldq, scale, (hipStream_t)stream);
}

int h3fp8_gemm_quant_noalloc(const void* a, int64_t lda, const void* w, int64_t ldw, const float* sa,
                             int64_t sa_stride, const float* sb, int64_t sb_stride, const void* bias, void* y,
                             int64_t ldy, int64_t M, int64_t N, int64_t K, void* q, int64_t ldq, float* scale,
                             void* stream) {
    H3_REQUIRE(M >= 0 && M <= H3FP8_NOALLOC_MAX_ROWS,
               "h3fp8_gemm_quant_noalloc: M = %lld rows exceeds the library buffer's %d (use h3fp8_gemm_quant with a "
               "workspace)", (long long)M, H3FP8_NOALLOC_MAX_ROWS);
    H3_REQUIRE(M == 0 || (q && scale), "h3fp8_gemm_quant_noalloc: null output");
    int rc = check_gemm(a, lda, w, ldw, sa, sa_stride, sb, sb_stride, y, ldy, M, N, K, N, "h3fp8_gemm_quant_noalloc");
    if (rc) return rc;
    // the tail's arguments too, before the fill and the GEMM are enqueued (nothing is launched for a refused call)
    rc = h3host::quant_args_ok(y, ldy, M, N, q, ldq, scale);
    if (rc) return rc;
    if (M == 0 || N == 0) return H3FP8_OK;
    // no set-up here (it creates a stream and waits): the caller has run h3fp8_init on this device
    int dev = -1;
    H3_CHECK_HIP(hipGetDevice(&dev));
    H3_REQUIRE(h3host::device_ready(dev) && dev < kScratchDevices && g_scratch_ptr[dev],
               "h3fp8_gemm_quant_noalloc: call h3fp8_init on device %d first", dev);
    float* amax = g_scratch_ptr[dev];
    hipStream_t st = (hipStream_t)stream;
    rc = zero_rows(amax, M, st);                        // a fill kernel: also safe under stream capture
    if (rc) return rc;
    rc = run_gemm(EPI_AMAX, (const uint8_t*)a, lda, (const uint8_t*)w, ldw, sa, sa_stride, sb, sb_stride, bias, y, ldy,
                  H3FP8_DT_BF16, M, N, K, N, amax, nullptr, st);
    if (rc) return rc;
    return h3host::quant_rows_amax_launch(y, ldy, M, N, amax, q, ldq, scale, st);
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
    int rc = h3host::quant_args_ok(h_ws, F, M, F, q, ldq, scale);
    if (rc) return rc;
    rc = h3fp8_gemm_swiglu(a, lda, w_gate_up, ldw, sa, sa_stride, sb, sb_stride, bias, h_ws, F, amax_ws, M, F, K,
                               stream);
    if (rc) return rc;
    return h3host::quant_rows_amax_launch(h_ws, F, M, F, amax_ws, q, ldq, scale, (hipStream_t)stream);
}

int h3fp8_grouped_gemm(const h3fp8_group* groups, int n_groups, void* stream) {
    H3_REQUIRE(groups && n_groups >= 0 && n_groups <= H3FP8_MAX_GROUPS, "h3fp8_grouped_gemm: bad group list");
    for (int i = 0; i < n_groups; ++i) {
        const h3fp8_group& g = groups[i];
        int rc = check_gemm(g.a, g.lda, g.w, g.ldw, g.sa, g.sa_stride, g.sb, g.sb_stride, g.y, g.ldy, g.M, g.N, g.K,
                            g.N, "h3fp8_grouped_gemm");
        if (rc) return rc;
        H3_REQUIRE(g.M == 0 || (g.M - 1) * g.lda + g.K <= kMaxBufferBytes,
                   "h3fp8_grouped_gemm: group %d activation too large for one launch", i);
        H3_REQUIRE(g.M == 0 || ((g.M - 1) * g.ldy + g.N) * 2 <= kMaxBufferBytes,
                   "h3fp8_grouped_gemm: group %d output too large for one launch", i);
        H3_REQUIRE(g.M == 0 || (g.M - 1) * g.sa_stride * 4 + 4 <= kMaxBufferBytes,
                   "h3fp8_grouped_gemm: group %d scales too large for one launch", i);
    }
    // A tile costs ceil(K / 128) k-steps whatever its M and N, and workgroup b takes tiles b, b + G, ...: with the
    // groups' tile ranges in descending order of K, the last rounds are filled with the cheapest tiles (longest
    // processing time first), so the workgroups finish close together.
    int order[H3FP8_MAX_GROUPS];
    for (int i = 0; i < n_groups; ++i) order[i] = i;
    std::stable_sort(order, order + n_groups, [&](int x, int y) { return groups[x].K > groups[y].K; });
    GroupedParams gp{};
    int tiles = 0;
    for (int k = 0; k < n_groups; ++k) {
        const h3fp8_group& g = groups[order[k]];
        if (g.M == 0 || g.N == 0) continue;
        GemmParams p = make_params((const uint8_t*)g.a, g.lda, (const uint8_t*)g.w, g.ldw, g.sa, g.sa_stride, g.sb,
                                   g.sb_stride, nullptr, g.y, g.ldy, g.M, g.N, g.K, g.N, nullptr, nullptr, false);
        p.tile_offset = tiles;
        tiles += p.tiles_m * p.tiles_n;
        gp.g[gp.n++] = p;
    }
    if (tiles == 0) return H3FP8_OK;
    gp.total_tiles = tiles;
    int rc = h3host::ensure_device_init();
    if (rc) return rc;
    return launch_one<0, false, EPI_PLAIN, true>(gp, (hipStream_t)stream);
}

}  // extern "C"
