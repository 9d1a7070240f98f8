// W8A8 GEMM on the gfx950 matrix cores: C = epilogue(A[M, K] . B[N, K]^T), int8 x int8 -> int32.
//
// Tiling (one workgroup = 8 wavefronts = 512 threads, one workgroup per CU):
//   * workgroup tile 256 (M) x 256 (N); the 8 waves form a 4 (M) x 2 (N) grid, each owns 64 x 128 =
//     2 x 4 tiles of v_mfma_i32_32x32x32_i8 (128 int32 accumulators per lane).  The weight rows
//     are the MFMA's A operand and the activation rows its B operand, so a lane ends up with 4
//     consecutive output columns of one row.
//   * K is staged 64 bytes at a time through a ring of 4 LDS stages (4 x 32 KiB), filled by
//     buffer_load ... lds (global -> LDS without VGPRs), 3 slabs ahead of the MFMAs.  The buffer
//     resources carry the operand sizes, so rows past M / N and chunks past K read as zeros.
//   * software pipeline, one barrier per slab: every wave issues the operand reads of slab k + 1
//     and the DMA of slab k + 4 between the MFMAs of slab k; explicit vmcnt / lgkmcnt waits order
//     the DMA, because the compiler does not track LDS DMA across loop iterations.
//   * LDS rows are 64 bytes = 4 chunks of 16; chunk c of tile row r lives at chunk
//     c ^ ((r >> 2) & 3), which makes the MFMA operand reads (32 consecutive rows, one chunk,
//     16 bytes per lane) free of LDS bank conflicts; the DMA writes 1 KiB contiguous blocks.
//
// Schedule.  Tiles are numbered in an XCD-aware grouped order (tile_of).  The first dp_tiles run
// whole, one per workgroup per round.  When the tile count leaves a partial last round of few
// tiles with a long K, the remaining sk_tiles are split along K over the first sk_grid workgroups
// (stream-K): workgroup g < G = sk_grid takes the contiguous range [g W / G, (g + 1) W / G) of the
// W = sk_tiles * nk (tile, slab) iterations.  A workgroup that ends with part of a tile stores its int32 partial
// accumulators to the workspace, publishes them (device-scope release) and counts itself in the
// tile's arrival counter; the last of the tile's contributors to arrive adds the others' partials
// to its own (integer addition: exact in any order) and runs the epilogue, then re-zeroes the
// counter for the next launch.  Nobody waits for anybody, so the schedule cannot deadlock.
//
// Workgroup order: the hardware hands workgroup i to XCD i % 8, and each XCD has its own L2.
// Tiles are renumbered so each XCD gets one contiguous range of tiles, and inside a range tiles go
// in groups of kGroupM M-tiles, column by column, so the workgroups that run together on an XCD
// share A and B panels in that XCD's L2.
//
// Epilogue (per accumulator): y = (f32(acc) * sa[m]) * sb[n] (+ bias[n]) in this order
// (kernel_src/kernels.py:65-67, int8_runtime.py:186-190), converted with round-to-nearest-even
// (fp32 -> bf16 via v_cvt_pk_bf16_f32).  SILU_MUL pairs gate and up columns held by the same
// lane (see mica_amd.h).  The residual is added after that rounding.  16-bit outputs are staged
// through LDS so every lane stores 16 contiguous bytes of a row.

#include <mutex>

#include "common.h"
#include "gemm_i8_common.h"

namespace {

constexpr int BK = 64;      // bytes of K per LDS stage
constexpr int NST = 4;      // LDS stages
constexpr int KS = BK / 32; // MFMA k-steps per stage
constexpr int kTile = 256;  // edge of the schedule's (whole) tiles
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;

// A BM x BN workgroup tile computed by 8 waves in a 4 (M) x 2 (N) grid, each owning WM x WN.
template <int BM_, int BN_>
struct Cfg {
    static constexpr int BM = BM_, BN = BN_;
    static constexpr int WM = BM / 4;
    static constexpr int WN = BN / 2;
    static constexpr int MB = WM / 32;                      // 32x32 MFMA tiles along M
    static constexpr int NB = WN / 32;                      // ... along N
    static constexpr int kABytes = BM * BK;                 // A part of an LDS stage
    static constexpr int kStage = (BM + BN) * BK;
    static constexpr int kABlk = BM * BK / 1024 / kWaves;   // 1 KiB DMA blocks of A per wave per slab
    static constexpr int kBBlk = BN * BK / 1024 / kWaves;   // ... of B
    static constexpr int kDmaPerSlab = kABlk + kBBlk;       // buffer_load ... lds per wave per slab
    // staged epilogue: each wave's WM x WN 16-bit block, rows padded by 16 bytes
    static constexpr int kEpiPitch = WN * 2 + 16;
    static constexpr int kEpiWave = WM * kEpiPitch;
    static constexpr int kSmemMain = (NST * kStage > kWaves * kEpiWave) ? NST * kStage : kWaves * kEpiWave;
    // int32x4 vectors of one lane's accumulators (a split tile's partial sums)
    static constexpr int kPartialVecs = NB * MB * 4;
};
using CfgFull = Cfg<256, 256>; // waves of 64 x 128: 2 x 4 MFMA tiles, 4 DMA per slab
using CfgHalf = Cfg<256, 128>; // waves of 64 x 64: 2 x 2 MFMA tiles, 3 DMA per slab
using CfgQuarter = Cfg<128, 128>; // waves of 32 x 64: 1 x 2 MFMA tiles, 2 DMA per slab
using CfgHalfM = Cfg<128, 256>;   // waves of 32 x 128: 1 x 4 MFMA tiles, 3 DMA per slab (SiLU pairs intact)
static_assert(CfgFull::MB == 2 && CfgFull::NB == 4 && CfgFull::kABlk == 2 && CfgFull::kBBlk == 2, "schedule");
static_assert(CfgHalf::MB == 2 && CfgHalf::NB == 2 && CfgHalf::kABlk == 2 && CfgHalf::kBBlk == 1, "schedule");
static_assert(CfgQuarter::MB == 1 && CfgQuarter::NB == 2 && CfgQuarter::kABlk == 1 && CfgQuarter::kBBlk == 1,
              "schedule");
static_assert(CfgQuarter::kSmemMain <= CfgFull::kSmemMain, "LDS");
static_assert(CfgHalfM::MB == 1 && CfgHalfM::NB == 4 && CfgHalfM::kABlk == 1 && CfgHalfM::kBBlk == 2 &&
              CfgHalfM::WN == 128 && CfgHalfM::kSmemMain <= CfgFull::kSmemMain, "schedule");
// LDS: the larger configuration's stages / staging, then the tile's row scales, column scales and
// bias (fp32, 3 x 256), then the arrival count a split tile's contributors read back
constexpr int kSmemMain = CfgFull::kSmemMain > CfgHalf::kSmemMain ? CfgFull::kSmemMain : CfgHalf::kSmemMain;
constexpr int kScaleOff = kSmemMain;
constexpr int kFlagOff = kScaleOff + 3 * 256 * 4;
constexpr int kSmem = kFlagOff + 16;

// LDS placement of 16-byte chunk c of tile row r: chunk c ^ swz(r).  With 64-byte rows, the MFMA
// operand reads (32 consecutive rows, one chunk, 16 bytes per lane) then run at the LDS's full
// rate on gfx950; measured on the device against other XOR patterns (2-4x slower ones included).
MICA_DEVICE int swz(int row) { return (row >> 2) & 3; }

// Stream-K partition of W (tile, slab) iterations over G workgroups: workgroup g owns
// [sk_begin(g), sk_begin(g + 1)).  With W >= G every range is non-empty.
MICA_DEVICE long long sk_begin(int g, long long W, int G) { return (long long)g * W / G; }
// the workgroup whose range holds iteration i (the largest g with sk_begin(g) <= i)
MICA_DEVICE int sk_owner(long long i, long long W, int G) { return (int)(((i + 1) * G + W - 1) / W) - 1; }

// One workgroup tile of configuration C: its accumulators, the main loop that fills them from
// slabs [k0, k1) and the epilogue that writes them out.
template <class C, int EPI, int OUT, bool HAS_BIAS, bool HAS_RES>
struct TileEngine {
    static constexpr int WM = C::WM, WN = C::WN, MB = C::MB, NB = C::NB;
    static constexpr int kDmaPerSlab = C::kDmaPerSlab;
    static constexpr int kEpiPitch = C::kEpiPitch, kEpiWave = C::kEpiWave;

    v16i acc[NB][MB]; // [n tile][m tile]

    struct Ops {
        v4i x[KS][MB];
        v4i w[KS][NB];
    };

    // ---- slabs [k0, k1) of tile (m0, n0) into acc.  Every wave runs the same software pipeline,
    // one barrier per 64-byte slab k:
    //   wait: this wave's DMA of slab k + 1 landed, its reads of slab k (registers X) completed
    //   barrier: slab k + 1 is visible in LDS, and nobody reads slab k's stage any more
    //   then, interleaved instruction by instruction: the MFMAs of slab k (from X), the operand
    //   reads of slab k + 1 (into Y) and the DMA of slab k + 4 (into the stage slab k just left).
    // All 8 waves keep the LDS busy together (operand reads and DMA writes share it) while the
    // two waves of each SIMD keep its matrix core busy.  A DMA past slab k1 is still issued (it
    // fails the range check and writes zeros into a stage nobody reads), so every wave always has
    // exactly 3 younger slabs in flight when it waits for slab k + 1.
    // The tile's per-row / per-column epilogue factors are loaded before the prologue DMA and
    // written to LDS after it, so their latency hides under the DMA's.  Threads 0-255: sa and bias
    // of tile row / column tid, threads 256-511: sb of column tid - 256.
    MICA_DEVICE void run(const GemmParams &p, int8_t *smem, __amdgpu_buffer_rsrc_t rsrc_a,
                         __amdgpu_buffer_rsrc_t rsrc_b, int m0, int n0, int k0, int k1) {
        const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
        const int wm = wave / 2, wn = wave % 2;
        const int M = p.M, N = p.N, K = p.K;
        // DMA: lane i of 1 KiB block b of an operand writes LDS bytes [16 i, 16 i + 16): tile row
        // 16 b + i / 4, physical chunk i % 4, so it fetches logical chunk (i % 4) ^ swz(row)
        int a_off[C::kABlk], b_off[C::kBBlk];
#pragma unroll
        for (int j = 0; j < C::kABlk; ++j) {
            const int r = (wave * C::kABlk + j) * 16 + (lane >> 2);
            const int kc = ((lane & 3) ^ swz(r)) << 4;
            a_off[j] = m0 + r < M ? (m0 + r) * p.lda + kc : kOutOfRange;
        }
#pragma unroll
        for (int j = 0; j < C::kBBlk; ++j) {
            const int r = (wave * C::kBBlk + j) * 16 + (lane >> 2);
            const int kc = ((lane & 3) ^ swz(r)) << 4;
            b_off[j] = n0 + r < N ? (n0 + r) * p.ldb + kc : kOutOfRange;
        }
        const int kc_lane = ((lane & 3) ^ swz(lane >> 2)) << 4; // chunk column; swz(r) == swz(lane >> 2)
        auto dma1 = [&](int slab, int j, int op) {
            const int kb = slab * BK;
            int8_t *st = smem + (slab % NST) * C::kStage;
            const bool kin = slab < k1 && kb + kc_lane < K;
            const int row = op == 0 ? a_off[j] : b_off[j];
            const int off = (kin && row != kOutOfRange) ? row + kb : kOutOfRange;
            const int blk = wave * (op == 0 ? C::kABlk : C::kBBlk) + j;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(op == 0 ? rsrc_a : rsrc_b,
                                                     (lds_void *)(st + op * C::kABytes + blk * 1024), 16, off, 0, 0, 0);
        };
        auto dma = [&](int slab) {
#pragma unroll
            for (int j = 0; j < C::kABlk; ++j) dma1(slab, j, 0);
#pragma unroll
            for (int j = 0; j < C::kBBlk; ++j) dma1(slab, j, 1);
        };
        // MFMA operand offsets inside a stage: [tile][k-step]
        const int r32 = lane & 31, khalf = lane >> 5;
        int x_rd[MB][KS], w_rd[NB][KS];
#pragma unroll
        for (int i = 0; i < MB; ++i)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const int rx = wm * WM + i * 32 + r32;
                x_rd[i][ks] = rx * BK + (((ks * 2 + khalf) ^ swz(rx)) << 4);
            }
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const int rw = wn * WN + j * 32 + r32;
                w_rd[j][ks] = C::kABytes + rw * BK + (((ks * 2 + khalf) ^ swz(rw)) << 4);
            }
        auto lds_read = [&](Ops &o, int slab) {
            const int8_t *st = smem + (slab % NST) * C::kStage;
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
                for (int j = 0; j < NB; ++j) o.w[ks][j] = *(const v4i *)(st + w_rd[j][ks]);
#pragma unroll
                for (int i = 0; i < MB; ++i) o.x[ks][i] = *(const v4i *)(st + x_rd[i][ks]);
            }
        };
        auto mfma_half = [&](const Ops &o, int ks) {
#pragma unroll
            for (int j = 0; j < NB; ++j)
#pragma unroll
                for (int i = 0; i < MB; ++i)
                    acc[j][i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(o.w[ks][j], o.x[ks][i], acc[j][i], 0, 0, 0);
        };

#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int i = 0; i < MB; ++i) acc[j][i] = v16i{};
        float f1, f2 = 0.0f;
        {
            // branch-free: the index is clamped into range (values of rows / columns past the edge
            // are never used), so no load waits for another
            const int i = tid & 255;
            const bool row = tid < 256;
            const float *src = row ? p.sa : p.sb;
            const int base = row ? m0 : n0;
            const int lim = (row ? M : N) - base;
            f1 = src[base + (i < lim ? i : lim - 1)];
            if (HAS_BIAS) f2 = p.bias[n0 + (i < N - n0 ? i : N - n0 - 1)];
        }
        // the previous tile's epilogue (LDS staging, scale reads) is finished in every wave
        wait_lgkmcnt0();
        __builtin_amdgcn_s_barrier();
#pragma unroll
        for (int sl = 0; sl < NST; ++sl) dma(k0 + sl);
        {
            float *sc = (float *)(smem + kScaleOff);
            sc[tid] = f1;                       // [0, 256): sa, [256, 512): sb
            if (tid < 256) sc[512 + tid] = f2;  // [512, 768): bias
        }
        wait_vmcnt<(NST - 1) * kDmaPerSlab>(); // slab k0 landed in this wave's blocks ...
        __builtin_amdgcn_s_barrier();          // ... and in every wave's
        Ops X, Y;
        lds_read(X, k0);

        auto step = [&](Ops &cur, Ops &nxt, int k) {
            wait_vmcnt<(NST - 2) * kDmaPerSlab>(); // slab k + 1 landed (slabs k + 2, k + 3 may be in flight)
            wait_lgkmcnt0();                       // slab k's operands are in registers
            __builtin_amdgcn_s_barrier();
            const int8_t *st = smem + ((k + 1) % NST) * C::kStage;
            const int dslab = k + NST;
            if constexpr (NB == 4 && MB == 1) {
                // 10 reads, 3 DMA, 8 MFMA: 4 reads up front, then 3 x [M, R, M, R, D] + [M, M]
                nxt.w[0][0] = *(const v4i *)(st + w_rd[0][0]);
                nxt.w[0][1] = *(const v4i *)(st + w_rd[1][0]);
                nxt.x[0][0] = *(const v4i *)(st + x_rd[0][0]);
                nxt.w[0][2] = *(const v4i *)(st + w_rd[2][0]);
                nxt.w[0][3] = *(const v4i *)(st + w_rd[3][0]);
                nxt.w[1][0] = *(const v4i *)(st + w_rd[0][1]);
                nxt.w[1][1] = *(const v4i *)(st + w_rd[1][1]);
                nxt.x[1][0] = *(const v4i *)(st + x_rd[0][1]);
                nxt.w[1][2] = *(const v4i *)(st + w_rd[2][1]);
                nxt.w[1][3] = *(const v4i *)(st + w_rd[3][1]);
                dma1(dslab, 0, 0);
                dma1(dslab, 0, 1);
                dma1(dslab, 1, 1);
                mfma_half(cur, 0);
                mfma_half(cur, 1);
                __builtin_amdgcn_sched_group_barrier(0x100, 4, 0); // 4 DS reads
#pragma unroll
                for (int r = 0; r < 3; ++r) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); // DS read
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0); // VMEM read (the LDS DMA)
                }
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            } else if constexpr (NB == 4) {
                // 12 reads, 4 DMA, 16 MFMA: 4 reads up front, then 4 x [M, R, M, R, M, D, M]
                nxt.w[0][0] = *(const v4i *)(st + w_rd[0][0]);
                nxt.w[0][1] = *(const v4i *)(st + w_rd[1][0]);
                nxt.x[0][0] = *(const v4i *)(st + x_rd[0][0]);
                nxt.x[0][1] = *(const v4i *)(st + x_rd[1][0]);
                nxt.w[0][2] = *(const v4i *)(st + w_rd[2][0]);
                nxt.w[0][3] = *(const v4i *)(st + w_rd[3][0]);
                nxt.w[1][0] = *(const v4i *)(st + w_rd[0][1]);
                nxt.w[1][1] = *(const v4i *)(st + w_rd[1][1]);
                nxt.x[1][0] = *(const v4i *)(st + x_rd[0][1]);
                nxt.x[1][1] = *(const v4i *)(st + x_rd[1][1]);
                nxt.w[1][2] = *(const v4i *)(st + w_rd[2][1]);
                nxt.w[1][3] = *(const v4i *)(st + w_rd[3][1]);
                dma1(dslab, 0, 0);
                dma1(dslab, 0, 1);
                dma1(dslab, 1, 0);
                dma1(dslab, 1, 1);
                mfma_half(cur, 0);
                mfma_half(cur, 1);
                __builtin_amdgcn_sched_group_barrier(0x100, 4, 0); // 4 DS reads
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); // DS read
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0); // VMEM read (the LDS DMA)
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                }
            } else if constexpr (MB == 1) {
                // 6 reads, 2 DMA, 4 MFMA: 4 reads up front, then 2 x [M, R, M, D]
                nxt.w[0][0] = *(const v4i *)(st + w_rd[0][0]);
                nxt.w[0][1] = *(const v4i *)(st + w_rd[1][0]);
                nxt.x[0][0] = *(const v4i *)(st + x_rd[0][0]);
                nxt.w[1][0] = *(const v4i *)(st + w_rd[0][1]);
                nxt.w[1][1] = *(const v4i *)(st + w_rd[1][1]);
                nxt.x[1][0] = *(const v4i *)(st + x_rd[0][1]);
                dma1(dslab, 0, 0);
                dma1(dslab, 0, 1);
                mfma_half(cur, 0);
                mfma_half(cur, 1);
                __builtin_amdgcn_sched_group_barrier(0x100, 4, 0); // 4 DS reads
#pragma unroll
                for (int r = 0; r < 2; ++r) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); // DS read
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0); // VMEM read (the LDS DMA)
                }
            } else {
                // 8 reads, 3 DMA, 8 MFMA: 4 reads up front, then 3 x [M, R, M, D] + [M, R, M]
                nxt.w[0][0] = *(const v4i *)(st + w_rd[0][0]);
                nxt.w[0][1] = *(const v4i *)(st + w_rd[1][0]);
                nxt.x[0][0] = *(const v4i *)(st + x_rd[0][0]);
                nxt.x[0][1] = *(const v4i *)(st + x_rd[1][0]);
                nxt.w[1][0] = *(const v4i *)(st + w_rd[0][1]);
                nxt.w[1][1] = *(const v4i *)(st + w_rd[1][1]);
                nxt.x[1][0] = *(const v4i *)(st + x_rd[0][1]);
                nxt.x[1][1] = *(const v4i *)(st + x_rd[1][1]);
                dma1(dslab, 0, 0);
                dma1(dslab, 0, 1);
                dma1(dslab, 1, 0);
                mfma_half(cur, 0);
                mfma_half(cur, 1);
                __builtin_amdgcn_sched_group_barrier(0x100, 4, 0); // 4 DS reads
#pragma unroll
                for (int r = 0; r < 3; ++r) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); // DS read
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0); // VMEM read (the LDS DMA)
                }
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            }
        };
        int k = k0;
        for (; k + 1 < k1; k += 2) {
            step(X, Y, k);
            step(Y, X, k + 1);
        }
        if (k < k1) step(X, Y, k);
        wait_vmcnt<0>();
    }

    // ---- epilogue of tile (m0, n0) from acc.  acc[j][i][r]: n = 8 (r / 4) + 4 (lane / 32) + r % 4
    //      (4 consecutive per r / 4), m = lane % 32 within the 32 x 32 tile (j, i) ----
    MICA_DEVICE void epilogue(const GemmParams &p, int8_t *smem, int m0, int n0) {
        const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
        const int wm = wave / 2, wn = wave % 2;
        const int r32 = lane & 31, khalf = lane >> 5;
        const int M = p.M, N = p.N;
        const int mw = m0 + wm * WM;
        const int nw = n0 + wn * WN;
        const bool vec = p.vec_ok != 0;
        const float *sc = (const float *)(smem + kScaleOff); // [0, 256): sa, [256, 512): sb, [512, 768): bias
        float sav[MB];
#pragma unroll
        for (int i = 0; i < MB; ++i) sav[i] = sc[wm * WM + i * 32 + r32];
        if constexpr (OUT == MICA_BF16 || OUT == MICA_FP16) {
            // Staged through LDS: every wave writes its rounded 16-bit block (8 bytes per lane per
            // store) into its own padded region, then streams it out row-contiguously, 16 bytes per
            // lane, so each global store covers whole 128- or 256-byte row segments.
            wait_lgkmcnt0();
            __builtin_amdgcn_s_barrier(); // every wave is done reading the operand stages
            int8_t *ep = smem + wave * kEpiWave;
            constexpr int kCols = EPI == MICA_EPI_SCALE ? WN : WN / 2; // output columns of this wave
            const int col0 = EPI == MICA_EPI_SCALE ? nw : (nw >> 7) * 64;
            const int ncols_out = EPI == MICA_EPI_SCALE ? N : (N >> 1);
#pragma unroll
            for (int j = 0; j < (EPI == MICA_EPI_SCALE ? NB : 2); ++j) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int nl = j * 32 + 8 * q + 4 * khalf; // local output column of this lane's 4 values
                    float s1[4], s2[4], bv[4];
                    const int cb = wn * WN + nl; // tile-local column of this lane's 4 values
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        s1[t] = sc[256 + cb + t]; // SCALE: sb[n]; SILU_MUL: the gate rows' sb
                        s2[t] = EPI == MICA_EPI_SCALE ? 0.0f : sc[256 + cb + 64 + t]; // the matching up rows
                        bv[t] = HAS_BIAS ? sc[512 + cb + t] : 0.0f;
                    }
#pragma unroll
                    for (int i = 0; i < MB; ++i) {
                        float y[4];
#pragma unroll
                        for (int t = 0; t < 4; ++t) {
                            if (EPI == MICA_EPI_SCALE) {
                                y[t] = ((float)acc[j][i][4 * q + t] * sav[i]) * s1[t];
                                if (HAS_BIAS) y[t] = y[t] + bv[t];
                            } else {
                                const float gv = round_bf16(((float)acc[j][i][4 * q + t] * sav[i]) * s1[t]);
                                const float uv = round_bf16(((float)acc[j + 2][i][4 * q + t] * sav[i]) * s2[t]);
                                const float act = silu_bf16(gv);
                                y[t] = act * uv;
                            }
                        }
                        u32x2 w;
                        if (OUT == MICA_BF16) {
                            w[0] = pack_bf16x2(y[0], y[1]);
                            w[1] = pack_bf16x2(y[2], y[3]);
                        } else {
                            w[0] = (uint32_t)f32_to_f16(y[0]) | ((uint32_t)f32_to_f16(y[1]) << 16);
                            w[1] = (uint32_t)f32_to_f16(y[2]) | ((uint32_t)f32_to_f16(y[3]) << 16);
                        }
                        *(u32x2 *)(ep + (i * 32 + r32) * kEpiPitch + nl * 2) = w;
                    }
                }
            }
            wait_lgkmcnt0(); // a wave reads back only its own region: no barrier needed
            constexpr int kLanesPerRow = kCols / 8;          // lanes x 8 columns per row
            constexpr int kRowsPerPass = 64 / kLanesPerRow;
            const int cl = (lane % kLanesPerRow) * 8;        // local column of this lane's 8 values
            const int valid = ncols_out - (col0 + cl) < 8 ? (ncols_out - (col0 + cl) > 0 ? ncols_out - (col0 + cl) : 0) : 8;
            const bool vec8 = vec && (p.ldc % 8 == 0) && (!HAS_RES || p.ldr % 8 == 0);
#pragma unroll 4
            for (int r0 = 0; r0 < WM; r0 += kRowsPerPass) {
                const int rl = r0 + lane / kLanesPerRow;
                const int m = mw + rl;
                const u32x4 v = *(const u32x4 *)(ep + rl * kEpiPitch + cl * 2);
                if (m >= M || valid == 0) continue;
                u32x4 o = v;
                if (HAS_RES) {
                    const uint16_t *rp = (const uint16_t *)p.res + (long)m * p.ldr + col0 + cl;
                    u32x4 rv = {0u, 0u, 0u, 0u};
                    if (vec8 && valid == 8) rv = *(const u32x4 *)rp;
                    else for (int t = 0; t < valid; ++t) rv[t >> 1] |= (uint32_t)rp[t] << (16 * (t & 1));
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        float a0, a1, b0, b1;
                        if (OUT == MICA_BF16) {
                            a0 = bf16_lo(v[t]); a1 = bf16_hi(v[t]); b0 = bf16_lo(rv[t]); b1 = bf16_hi(rv[t]);
                            o[t] = pack_bf16x2(a0 + b0, a1 + b1);
                        } else {
                            a0 = f16_to_f32(v[t] & 0xffff); a1 = f16_to_f32(v[t] >> 16);
                            b0 = f16_to_f32(rv[t] & 0xffff); b1 = f16_to_f32(rv[t] >> 16);
                            o[t] = (uint32_t)f32_to_f16(a0 + b0) | ((uint32_t)f32_to_f16(a1 + b1) << 16);
                        }
                    }
                }
                uint16_t *cp = (uint16_t *)p.C + (long)m * p.ldc + col0 + cl;
                if (vec8 && valid == 8) {
                    *(u32x4 *)cp = o;
                } else {
                    for (int t = 0; t < valid; ++t) cp[t] = (uint16_t)(o[t >> 1] >> (16 * (t & 1)));
                }
            }
            return;
        }
        // 32-bit outputs (fp32 / raw int32): direct 16-byte stores from the accumulator layout
        if (EPI == MICA_EPI_SCALE) {
#pragma unroll
            for (int j = 0; j < NB; ++j) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int nb = nw + j * 32 + 8 * q + 4 * khalf;
                    const int valid = N - nb < 4 ? (N - nb > 0 ? N - nb : 0) : 4;
                    if (valid == 0) continue;
                    float sbv[4], bv[4];
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        sbv[t] = t < valid ? p.sb[nb + t] : 0.0f;
                        bv[t] = (HAS_BIAS && t < valid) ? p.bias[nb + t] : 0.0f;
                    }
#pragma unroll
                    for (int i = 0; i < MB; ++i) {
                        const int m = mw + i * 32 + r32;
                        if (m >= M) continue;
                        const long off = (long)m * p.ldc + nb;
                        if (OUT == MICA_INT32) {
                            int *c = (int *)p.C + off;
                            if (vec && valid == 4) {
                                *(v4i *)c = v4i{acc[j][i][4 * q], acc[j][i][4 * q + 1], acc[j][i][4 * q + 2],
                                                acc[j][i][4 * q + 3]};
                            } else {
                                for (int t = 0; t < valid; ++t) c[t] = acc[j][i][4 * q + t];
                            }
                            continue;
                        }
                        float y[4];
#pragma unroll
                        for (int t = 0; t < 4; ++t) {
                            y[t] = ((float)acc[j][i][4 * q + t] * sav[i]) * sbv[t];
                            if (HAS_BIAS) y[t] = y[t] + bv[t];
                        }
                        if (HAS_RES) {
                            float rv[4];
                            load4_res<OUT>(p.res, (long)m * p.ldr + nb, rv, valid, vec);
#pragma unroll
                            for (int t = 0; t < 4; ++t) y[t] = to_out_precision<OUT>(y[t]) + rv[t];
                        }
                        store4<OUT>(p.C, off, y, valid, vec);
                    }
                }
            }
        }
    }
};

template <int EPI, int OUT, bool HAS_BIAS, bool HAS_RES>
__global__ __launch_bounds__(kThreads, 1) void gemm_i8_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(1024))) int8_t smem[kSmem];
    static_assert(EPI == MICA_EPI_SCALE || CfgFull::WN == 128,
                  "the SiLU epilogue needs one 128-row gate/up group per wave");
    const int tid = threadIdx.x;
    const int K = p.K;
    const int nk = (K + BK - 1) / BK;
    const int G = gridDim.x;
    const __amdgpu_buffer_rsrc_t rsrc_a = __builtin_amdgcn_make_buffer_rsrc((void *)p.A, 0, p.M * p.lda, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rsrc_b = __builtin_amdgcn_make_buffer_rsrc((void *)p.B, 0, p.N * p.ldb, kBufferFlags);

    TileEngine<CfgFull, EPI, OUT, HAS_BIAS, HAS_RES> full;

    // ---- whole tiles: blockIdx.x, blockIdx.x + G, ... below dp_tiles ----
    for (int pid = blockIdx.x; pid < p.dp_tiles; pid += G) {
        int tm, tn;
        tile_of(pid, p.tiles_m, p.tiles_n, tm, tn);
        full.run(p, smem, rsrc_a, rsrc_b, tm * kTile, tn * kTile, 0, nk);
        full.epilogue(p, smem, tm * kTile, tn * kTile);
    }

    // ---- half tiles: the next half_tiles tiles, each as two 256 x 128 halves ----
    if constexpr (EPI == MICA_EPI_SCALE) {
        if (p.half_tiles > 0) {
            TileEngine<CfgHalf, EPI, OUT, HAS_BIAS, HAS_RES> half;
            for (int h = blockIdx.x; h < 2 * p.half_tiles; h += G) {
                int tm, tn;
                tile_of(p.dp_tiles + (h >> 1), p.tiles_m, p.tiles_n, tm, tn);
                const int n0 = tn * kTile + (h & 1) * CfgHalf::BN;
                half.run(p, smem, rsrc_a, rsrc_b, tm * kTile, n0, 0, nk);
                half.epilogue(p, smem, tm * kTile, n0);
            }
        }
        // ---- quarter tiles: the next quarter_tiles tiles, each as four 128 x 128 quarters (a
        // quarter wholly past M or N is skipped: the branch is uniform over the workgroup) ----
        if (p.quarter_tiles > 0) {
            TileEngine<CfgQuarter, EPI, OUT, HAS_BIAS, HAS_RES> quarter;
            for (int h = blockIdx.x; h < 4 * p.quarter_tiles; h += G) {
                int tm, tn;
                tile_of(p.dp_tiles + (h >> 2), p.tiles_m, p.tiles_n, tm, tn);
                const int m0 = tm * kTile + ((h >> 1) & 1) * CfgQuarter::BM;
                const int n0 = tn * kTile + (h & 1) * CfgQuarter::BN;
                if (m0 >= p.M || n0 >= p.N) continue;
                quarter.run(p, smem, rsrc_a, rsrc_b, m0, n0, 0, nk);
                quarter.epilogue(p, smem, m0, n0);
            }
        }
    }

    // ---- M-halves: the next mhalf_tiles tiles, each as two 128 x 256 halves along M (a half wholly
    // past M is skipped: uniform over the workgroup); the SiLU epilogue's gate/up column pairs stay
    // within one wave ----
    if constexpr (EPI == MICA_EPI_SILU_MUL) {
        if (p.mhalf_tiles > 0) {
            TileEngine<CfgHalfM, EPI, OUT, HAS_BIAS, HAS_RES> mhalf;
            for (int h = blockIdx.x; h < 2 * p.mhalf_tiles; h += G) {
                int tm, tn;
                tile_of(p.dp_tiles + (h >> 1), p.tiles_m, p.tiles_n, tm, tn);
                const int m0 = tm * kTile + (h & 1) * CfgHalfM::BM;
                if (m0 >= p.M) continue;
                mhalf.run(p, smem, rsrc_a, rsrc_b, m0, tn * kTile, 0, nk);
                mhalf.epilogue(p, smem, m0, tn * kTile);
            }
        }
    }

    if (p.sk_tiles == 0 || (int)blockIdx.x >= p.sk_grid) return;
    // ---- split tiles: this workgroup's stream-K range of (tile, slab) iterations.  A workgroup
    // ending with part of a tile publishes its partial sums; the tile's last contributor to
    // arrive adds the others' to its own and runs the epilogue ----
    int *flag = (int *)(smem + kFlagOff);
    const int S = p.sk_grid;
    const long long W = (long long)p.sk_tiles * nk;
    const long long my_begin = sk_begin(blockIdx.x, W, S);
    const long long my_end = sk_begin(blockIdx.x + 1, W, S);
    // Partial sums move with device-scope (sc1) buffer stores and loads: written through to the
    // device's coherence point and read from it, so no cache-wide write-back or invalidation (a
    // device-scope fence) is needed, only the ordering below.
    constexpr int kDeviceScope = 16; // cache policy bits: sc1
    constexpr int kSlotBytes = CfgFull::kPartialVecs * kThreads * 16;
    const __amdgpu_buffer_rsrc_t rsrc_p =
        __builtin_amdgcn_make_buffer_rsrc((void *)p.partials, 0, S * 2 * kSlotBytes, kBufferFlags);
    auto slot_off = [&](int g, int seg) { return (g * 2 + seg) * kSlotBytes + tid * 16; };
    auto fixup = [&](int rel) -> bool {
        const long long tb = (long long)rel * nk;      // the tile's first iteration
        const int seg = tb > my_begin ? 1 : 0;          // first (0) or last (1) range segment of this workgroup
        const int g0 = sk_owner(tb, W, S), g1 = sk_owner(tb + nk - 1, W, S);
        const int mine = slot_off(blockIdx.x, seg);
#pragma unroll
        for (int j = 0; j < CfgFull::NB; ++j)
#pragma unroll
            for (int i = 0; i < CfgFull::MB; ++i)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    __builtin_amdgcn_raw_buffer_store_b128(
                        v4i{full.acc[j][i][4 * q], full.acc[j][i][4 * q + 1], full.acc[j][i][4 * q + 2],
                            full.acc[j][i][4 * q + 3]},
                        rsrc_p, mine + ((j * CfgFull::MB + i) * 4 + q) * kThreads * 16, 0, kDeviceScope);
        wait_vmcnt<0>();  // this wave's partial sums reached the coherence point ...
        __syncthreads();  // ... and every wave's, before the arrival is counted
        if (tid == 0) *flag = __hip_atomic_fetch_add(p.arrivals + rel, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (*flag != g1 - g0) return false; // a later contributor finishes the tile
        for (int g = g0; g <= g1; ++g) {
            if (g == (int)blockIdx.x) continue;
            const int src = slot_off(g, tb > sk_begin(g, W, S) ? 1 : 0);
            // two halves of 64 registers each: the operand registers of the main loop are free
            // here, but not all 128 accumulators' worth on top of the accumulators themselves
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int j = h * CfgFull::NB / 2; j < (h + 1) * CfgFull::NB / 2; ++j)
#pragma unroll
                    for (int i = 0; i < CfgFull::MB; ++i)
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const v4i v = __builtin_amdgcn_raw_buffer_load_b128(
                                rsrc_p, src + ((j * CfgFull::MB + i) * 4 + q) * kThreads * 16, 0, kDeviceScope);
#pragma unroll
                            for (int t = 0; t < 4; ++t) full.acc[j][i][4 * q + t] += v[t];
                        }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if (tid == 0) __hip_atomic_store(p.arrivals + rel, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return true;
    };
    for (long long it = my_begin; it < my_end;) {
        const int rel = (int)(it / nk);
        const int k0 = (int)(it - (long long)rel * nk);
        const int k1 = (long long)(nk - k0) < my_end - it ? nk : k0 + (int)(my_end - it);
        int tm, tn;
        tile_of(p.dp_tiles + rel, p.tiles_m, p.tiles_n, tm, tn);
        it += k1 - k0;
        full.run(p, smem, rsrc_a, rsrc_b, tm * kTile, tn * kTile, k0, k1);
        if ((k0 != 0 || k1 != nk) && !fixup(rel)) continue;
        full.epilogue(p, smem, tm * kTile, tn * kTile);
    }
}

template <int EPI, int OUT>
int launch_out(const GemmParams &p, int grid_size, bool has_bias, bool has_res, hipStream_t st) {
    dim3 grid(grid_size), block(kThreads);
#define MICA_G(B_, R_) hipLaunchKernelGGL((gemm_i8_kernel<EPI, OUT, B_, R_>), grid, block, 0, st, p)
    if (EPI == MICA_EPI_SILU_MUL) MICA_G(false, false);
    else if (has_bias && has_res) MICA_G(true, true);
    else if (has_bias) MICA_G(true, false);
    else if (has_res) MICA_G(false, true);
    else MICA_G(false, false);
#undef MICA_G
    return mica_err(hipGetLastError());
}

// Workspace of the split-tile schedule on a device with `cus` compute units: the arrival counters
// (one per split tile, at most cus of them), padded to 4 KiB, then two partial-sum slots of
// kPartialVecs x kThreads int32x4 per workgroup.
constexpr long long kCounterBytes = 4096;
constexpr long long kSlotBytes = (long long)CfgFull::kPartialVecs * kThreads * 16;
long long workspace_bytes_for(int cus) { return kCounterBytes + (long long)cus * 2 * kSlotBytes; }

int cu_count(int device) {
    static int cached[64];
    if (device >= 0 && device < 64 && cached[device] > 0) return cached[device];
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || v <= 0) return 0;
    if (device >= 0 && device < 64) cached[device] = v;
    return v;
}

// Scratch of the no-allocation entry point (mica_mm_i8_noalloc): the split schedule's arrival
// counters, then two partial-sum slots for each of at most kScratchGroups split workgroups (16 split
// tiles of 4 workgroups).  Every device the library runs on holds its own copy until the process ends.
constexpr int kScratchGroups = 64;
constexpr long long kScratchBytes = kCounterBytes + (long long)kScratchGroups * 2 * kSlotBytes; // 32 MiB + 4 KiB

__global__ void clear_counters_kernel(int *counters, int n) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) counters[i] = 0;
}

// Validation, schedule and launch shared by mica_mm_i8 and mica_mm_i8_noalloc.  `noalloc`: the
// workspace is the static scratch (kScratchBytes), a split round needing more of it than that is
// rejected (MICA_MISS_RANGE) instead of being run as quarter / half tiles.
// Argument checks (no device call): 0 when the call is well-formed, else the miss code.
int mm_i8_check(const int8_t *A, int lda, const int8_t *B, int ldb, const float *sa, const float *sb,
                const float *bias, const void *residual, int ldr, void *C, int ldc, int out_dtype, int M, int N,
                int K, int epilogue, const void *workspace, long long workspace_bytes) {
    if (A == nullptr || B == nullptr || sa == nullptr || sb == nullptr || C == nullptr) return MICA_MISS_ARG;
    if (epilogue != MICA_EPI_SCALE && epilogue != MICA_EPI_SILU_MUL) return MICA_MISS_ARG;
    if (out_dtype != MICA_BF16 && out_dtype != MICA_FP16 && out_dtype != MICA_FP32 && out_dtype != MICA_INT32)
        return MICA_MISS_DTYPE;
    if (out_dtype == MICA_INT32 && epilogue != MICA_EPI_SCALE) return MICA_MISS_ARG;
    if (M < 0 || N <= 0 || K <= 0 || K % 16 != 0) return MICA_MISS_SHAPE;
    const int Nout = epilogue == MICA_EPI_SILU_MUL ? N / 2 : N;
    if (epilogue == MICA_EPI_SILU_MUL) {
        if (N % 128 != 0) return MICA_MISS_SHAPE;
        if (out_dtype != MICA_BF16 || bias != nullptr || residual != nullptr) return MICA_MISS_ARG;
    }
    if (lda < K || ldb < K || lda % 16 != 0 || ldb % 16 != 0 || ldc < Nout || (residual && ldr < Nout))
        return MICA_MISS_STRIDE;
    if ((long long)M * lda >= (1ll << 31) || (long long)N * ldb >= (1ll << 31) ||
        (long long)M * ldc >= (1ll << 31) || (residual && (long long)M * ldr >= (1ll << 31)))
        return MICA_MISS_RANGE;
    if (!mica_aligned16(A) || !mica_aligned16(B) || !mica_aligned16(sa) || !mica_aligned16(sb) ||
        !mica_aligned16(C) || (bias && !mica_aligned16(bias)) || (residual && !mica_aligned16(residual)) ||
        (workspace && !mica_aligned16(workspace)))
        return MICA_MISS_ALIGN;
    if (workspace_bytes < 0) return MICA_MISS_ARG;
    return 0;
}

int mm_i8_run(const int8_t *A, int lda, const int8_t *B, int ldb, const float *sa, const float *sb,
              const float *bias, const void *residual, int ldr, void *C, int ldc, int out_dtype, int M, int N, int K,
              int epilogue, void *workspace, long long workspace_bytes, bool noalloc, hipStream_t st) {
    const int bad = mm_i8_check(A, lda, B, ldb, sa, sb, bias, residual, ldr, C, ldc, out_dtype, M, N, K, epilogue,
                                workspace, workspace_bytes);
    if (bad != 0) return bad;
    if (M == 0) return 0;
    const int Nout = epilogue == MICA_EPI_SILU_MUL ? N / 2 : N;
    GemmParams p{};
    p.A = A; p.B = B; p.sa = sa; p.sb = sb; p.bias = bias; p.res = residual; p.C = C;
    p.lda = lda; p.ldb = ldb; p.ldr = ldr; p.ldc = ldc; p.M = M; p.N = N; p.K = K;
    p.tiles_m = (M + kTile - 1) / kTile;
    p.tiles_n = (N + kTile - 1) / kTile;
    p.vec_ok = (ldc % 4 == 0) && (Nout % 4 == 0) && (!residual || ldr % 4 == 0);
    const long long tiles = (long long)p.tiles_m * p.tiles_n;
    if (tiles >= (1ll << 31)) return MICA_MISS_RANGE;
    // Schedule over a grid of at most one workgroup per CU.  Whole tiles, one per workgroup per
    // round; when the last round would be at most a quarter full, its tiles run as four 128 x 128
    // quarters each, and when at most half full, as two 256 x 128 halves (SCALE epilogue; the pieces
    // fill up to one round).  For the SiLU epilogue, whose waves need 128 columns (gate / up pairs), a
    // last round at most half full runs as two 128 x 256 halves along M (measured: 36.2 -> 27.2 us at
    // 128 x 19456 x 2560, 86.8 -> 73.8 us at M = 1024).  With a workspace and int32 / fp32 outputs (the
    // 16-bit ones have the 128-row split above), a partial last round of at most cus / kSplit tiles
    // whose K has at least kSplit * kMinSplitSlabs slabs is instead split along K, kSplit workgroups
    // per tile, for M <= 256, where a tile's lower quarters are mostly or wholly empty.  A split tile costs its last
    // contributor a serial sum of the others' 256 KiB partials plus the partial-sum round trip
    // (measured about 15 us + 3 us per partial), so the split pays only when a quarter of the tile's
    // K still takes longer than that; with more contributors per tile the sum grows faster than
    // the K share shrinks.  Measured against quarters at K >= 8192: split 41.7 vs 44.4 us at
    // M = 128, 43.1 vs 44.9 at M = 256; quarters 42.3 vs 43.3 at M = 512, 44.7 vs 52.2 at M = 1024.
#ifndef MICA_GEMM_QUARTERS
#define MICA_GEMM_QUARTERS 1
#endif
    constexpr bool kQuarters = MICA_GEMM_QUARTERS != 0;
#ifndef MICA_GEMM_MHALVES
#define MICA_GEMM_MHALVES 1
#endif
    constexpr bool kMHalves = MICA_GEMM_MHALVES != 0;
#ifndef MICA_GEMM_AGPR
#define MICA_GEMM_AGPR 1
#endif
    constexpr bool kAgpr = MICA_GEMM_AGPR != 0;
#ifndef MICA_GEMM_SMALL
#define MICA_GEMM_SMALL 1
#endif
    constexpr bool kSmall = MICA_GEMM_SMALL != 0;
    constexpr long long kSplit = 4;
    constexpr long long kMinSplitSlabs = 32;
    p.dp_tiles = (int)tiles;
    p.half_tiles = 0;
    p.quarter_tiles = 0;
    p.mhalf_tiles = 0;
    p.sk_tiles = 0;
    p.sk_grid = 0;
    int grid = (int)tiles;
    int dev = 0;
    const int cus = hipGetDevice(&dev) == hipSuccess ? cu_count(dev) : 0;
    // Few tiles and a long K (a short request's down projection, e.g. 128 x 2560 x 9728: 16 tiles of
    // 128 x 160 on 256 CUs): with a workspace, one round of 128-row tiles split along K into `parts`
    // pieces whose int32 partial sums each tile's last part adds (agpr_split_launch; same bits as every
    // other schedule).  The hand-off costs ~5 us (the partial sums' write-through, the arrival count,
    // the read-back, each a round trip to the device's coherence point) plus ~2 us per further part
    // read back, so it pays only for a long K: measured on MI355X (us, unsplit / 2 / 3 / 4 parts):
    // 128 x 2560 x 9728: 29.4 / 22.9 / 20.5 / 19.5; 512 x 2560 x 9728: 31.4 / 26.6 / 26.0 / 28.3;
    // 1024 x 2560 x 9728: 33.6 / 35.3; 128 x 2560 x 4096: 13.4 / 15.1 / 14.8 / 15.8; 128 x 6144 x 2560:
    // 10.5 / 12.4 / 14.2 / 15.8; SiLU 128 x 19456 x 2560: 21.5 / 26.9 / 36.0.  Hence K >= 8192 and
    // about one part per 20 slabs of 128 bytes, at least 3 (capped by the CUs and the workspace).
#ifndef MICA_GEMM_SPLIT_SMALL
#define MICA_GEMM_SPLIT_SMALL 1
#endif
    if (MICA_GEMM_SPLIT_SMALL && workspace != nullptr && cus > 0 && K % 256 == 0 && K >= 8192 &&
        (epilogue == MICA_EPI_SILU_MUL || out_dtype == MICA_BF16 || out_dtype == MICA_FP16) && ldc % 8 == 0 &&
        Nout % 8 == 0 && (!residual || ldr % 8 == 0) && (long long)(M + kTile) * lda < (1ll << 31) &&
        (long long)(N + kTile) * ldb < (1ll << 31) && (long long)kTile * ldc * 4 < (1ll << 31) &&
        (!residual || (long long)kTile * ldr * 4 < (1ll << 31))) {
        const int bn = agpr_split_tile_n(epilogue);
        const long long tiles_s = (long long)((M + 127) / 128) * ((N + bn - 1) / bn);
        const long long slabs = K / 128;
        long long parts = slabs / 20;
#ifdef MICA_GEMM_SPLIT_PARTS
        parts = MICA_GEMM_SPLIT_PARTS;
#endif
        if (parts > cus / tiles_s) parts = cus / tiles_s;
        if (parts > slabs / 4) parts = slabs / 4;
        const long long slot = agpr_split_slot_bytes(epilogue);
        while (parts >= 3 && kCounterBytes + tiles_s * parts * slot > workspace_bytes) --parts;
        if (parts >= 3 && tiles_s <= kCounterBytes / 4) {
            p.tiles_m = (M + 127) / 128;
            p.tiles_n = (N + bn - 1) / bn;
            p.dp_tiles = 0;
            p.sk_tiles = (int)tiles_s;
            p.sk_grid = (int)(tiles_s * parts);
            p.arrivals = (int *)workspace;
            p.partials = (v4i *)((char *)workspace + kCounterBytes);
            return agpr_split_launch(p, epilogue, out_dtype, bias != nullptr, residual != nullptr, st);
        }
    }
    const long long nk = (K + BK - 1) / BK;
    const long long rem = cus > 0 ? tiles % cus : 0;
    if (rem != 0 && cus <= 1024) {
        const bool quarters = kQuarters && epilogue == MICA_EPI_SCALE && 4 * rem <= cus;
        // (16-bit outputs no longer take it: the AGPR kernel's quarter / half tiles and the 128-row split
        // above serve them faster, e.g. 128 x 2560 x 9728 in 29.4 / 19.5 us against 48.9 us here)
        const bool want_split = workspace != nullptr && rem * kSplit <= cus && nk >= kSplit * kMinSplitSlabs &&
                                !(quarters && M > 256) && (out_dtype == MICA_INT32 || out_dtype == MICA_FP32);
        // the existing entry point splits with a workspace of mica_mm_i8_workspace_bytes(device); the
        // no-allocation one with the scratch, which holds kScratchGroups split workgroups
        const bool fits = noalloc ? rem * kSplit <= kScratchGroups : workspace_bytes >= workspace_bytes_for(cus);
        if (want_split && noalloc && !fits) return MICA_MISS_RANGE;
        if (want_split && fits) {
            p.dp_tiles = (int)(tiles - rem);
            p.sk_tiles = (int)rem;
            p.sk_grid = (int)(rem * kSplit);
            p.arrivals = (int *)workspace;
            p.partials = (v4i *)((char *)workspace + kCounterBytes);
            grid = tiles > rem ? cus : p.sk_grid;
        } else if (quarters) {
            p.dp_tiles = (int)(tiles - rem);
            p.quarter_tiles = (int)rem;
            grid = cus < tiles ? cus : (int)tiles;
            if (grid < 4 * rem) grid = (int)(4 * rem);
        } else if (kMHalves && epilogue == MICA_EPI_SILU_MUL && 2 * rem <= cus) {
            p.dp_tiles = (int)(tiles - rem);
            p.mhalf_tiles = (int)rem;
            grid = cus < tiles ? cus : (int)tiles;
            if (grid < 2 * rem) grid = (int)(2 * rem);
        } else if (epilogue == MICA_EPI_SCALE && 2 * rem <= cus) {
            p.dp_tiles = (int)(tiles - rem);
            p.half_tiles = (int)rem;
            grid = cus < tiles ? cus : (int)tiles;
            if (grid < 2 * rem) grid = (int)(2 * rem);
        }
    }
    const bool hb = bias != nullptr, hr = residual != nullptr;
    // K a multiple of 256 (an even number of 128-byte slabs) and no split: the wide kernel
    // (gemm_i8_wide.hip) runs the same schedule of whole tiles and tail pieces, with the same bits;
    // its grid stays persistent (one workgroup per CU) also when the tiles fill whole rounds
    // (the operands addressable with 32-bit offsets one tile past their last row, and a 256-row span
    // of C or of the residual)
    const bool wide_ok = K % 256 == 0 && p.sk_tiles == 0 && (long long)(M + kTile) * lda < (1ll << 31) &&
                         (long long)(N + kTile) * ldb < (1ll << 31) && (long long)kTile * ldc * 4 < (1ll << 31) &&
                         (!residual || (long long)kTile * ldr * 4 < (1ll << 31));
    if (wide_ok) {
        if (rem == 0 && cus > 0 && tiles > cus) grid = cus;
        // Fewer whole tiles than CUs, too many for four quarters each to fit one round (the halves
        // schedule above): one round of 128 x 160 tiles when they fit it (the AGPR kernel's small tiles,
        // same bits).  Each CU then streams (128 + 160) rows of operands instead of a half tile's 384.
        // The SiLU epilogue with fewer whole tiles than CUs: one round of 128 x 128 tiles, one gate / up
        // group each, when they fit one (same bits).  Each streams 256 rows of operands against the
        // M-halves' 384, on up to twice as many CUs (M <= 128: the lower halves had no rows).  Measured
        // on one box (us, M-halves or whole tiles / these): 128 x 19456 x 2560 21.5 / 14.2, 300 x 3072 x
        // 2560 17.8 / 11.2, 700 x 3072 x 2560 19.1 / 12.7; over more than one round they lose
        // (256 x 19456 x 2560: 23.2 / 25.4) or tie (512 x 19456 x 2560: 37.7 / 36.6).
        const long long tiles_silu = (long long)((M + 127) / 128) * ((N + 127) / 128);
        if (kAgpr && kSmall && epilogue == MICA_EPI_SILU_MUL && cus > 0 && tiles < cus && tiles_silu <= cus &&
            K >= 512 && ldc % 8 == 0 && Nout % 8 == 0) {
            p.tiles_m = (M + 127) / 128;
            p.tiles_n = (N + 127) / 128;
            p.dp_tiles = (int)tiles_silu;
            p.mhalf_tiles = 0;
            return agpr_silu_small_launch(p, (int)tiles_silu, st);
        }
        const long long tiles_small = (long long)((M + 127) / 128) * ((N + 159) / 160);
        const bool small = kAgpr && kSmall && epilogue == MICA_EPI_SCALE && p.half_tiles == tiles && cus > 0 &&
                           4 * tiles > cus && tiles_small <= cus && K >= 512 &&
                           (out_dtype == MICA_BF16 || out_dtype == MICA_FP16) && ldc % 8 == 0 && Nout % 8 == 0 &&
                           (!residual || ldr % 8 == 0);
        if (small) {
            p.tiles_m = (M + 127) / 128;
            p.tiles_n = (N + 159) / 160;
            p.dp_tiles = (int)tiles_small;
            p.half_tiles = 0;
            return agpr_small_launch(p, out_dtype, (int)tiles_small, hb, hr, st);
        }
        // One partial round of whole tiles with no tail pieces (more than half the CUs busy, e.g.
        // 4096 x 2560: 160 tiles on 256 CUs) runs as 256 x 160 tiles instead when those still fit one
        // round (256 of them there): each costs about 0.65 of a whole tile and more CUs work.
        const long long tiles160 = (long long)p.tiles_m * ((N + 159) / 160);
        const bool narrow = epilogue == MICA_EPI_SCALE && (out_dtype == MICA_BF16 || out_dtype == MICA_FP16) &&
                            cus > 0 && p.dp_tiles == tiles && tiles < cus && tiles160 > tiles && tiles160 <= cus &&
                            (long long)(N + 160) * ldb < (1ll << 31);
        if (narrow) {
            p.tiles_n = (N + 159) / 160;
            p.dp_tiles = (int)tiles160;
            grid = (int)tiles160;
            // the AGPR kernel's 4 x 1 wave grid on the same tiles and bits (16-byte output row units),
            // when the tiles fill more than 3/4 of the CUs.  Measured (same box, bit-identical):
            // 4096 x 2560 x 4096: 37.5 vs 40.4 us, 4096 x 2560 x 9728: 77.7 vs 81.4; with half the CUs
            // or fewer busy the 8-wave kernel is ahead (2048 x 2560 x 4096: 26.4 vs 25.2 us).
            if (kAgpr && K >= 512 && 4 * tiles160 > 3 * (long long)cus && ldc % 8 == 0 && Nout % 8 == 0 &&
                (!residual || ldr % 8 == 0))
                return agpr_narrow_launch(p, out_dtype, grid, hb, hr, st);
            return wide_launch(p, epilogue, out_dtype, grid, hb, hr, true, st);
        }
        // 16-bit outputs in whole 16-byte row units and at least 4 slabs of K: the AGPR kernel
        // (gemm_i8_agpr.hip), same schedule and bits, one wave per SIMD
        // Measured (same box, bit-identical): faster from one whole round of tiles on; below that,
        // wherever tail pieces run with a long K or at M >= 512 or for the SiLU epilogue (1024 x 2560 x
        // 9728: 33.1 vs 48.7 us; 512 x 9728 x 2560: 19.8 vs 21.5; 128 x 19456 x 2560 SiLU: 22.4 vs
        // 24.9), but not for quarters at M <= 256 with K = 2560 (11.0 vs 10.6 us at 256 x 6144) nor
        // for fewer whole tiles than CUs with no pieces (33.8 vs 33.2 at 2048 x 6144).
        const bool pieces = p.dp_tiles < tiles;
        const bool agpr_wins = tiles >= cus || (pieces && (K >= 4096 || M >= 512 || epilogue == MICA_EPI_SILU_MUL));
        const bool agpr_ok = kAgpr && K >= 512 && cus > 0 && agpr_wins &&
                             (out_dtype == MICA_BF16 || out_dtype == MICA_FP16) && ldc % 8 == 0 &&
                             Nout % 8 == 0 && (!residual || ldr % 8 == 0);
        if (agpr_ok) return agpr_launch(p, epilogue, out_dtype, grid, hb, hr, st);
        return wide_launch(p, epilogue, out_dtype, grid, hb, hr, false, st);
    }
    if (epilogue == MICA_EPI_SILU_MUL) return launch_out<MICA_EPI_SILU_MUL, MICA_BF16>(p, grid, false, false, st);
    if (out_dtype == MICA_BF16) return launch_out<MICA_EPI_SCALE, MICA_BF16>(p, grid, hb, hr, st);
    if (out_dtype == MICA_FP16) return launch_out<MICA_EPI_SCALE, MICA_FP16>(p, grid, hb, hr, st);
    if (out_dtype == MICA_INT32) return launch_out<MICA_EPI_SCALE, MICA_INT32>(p, grid, false, false, st);
    return launch_out<MICA_EPI_SCALE, MICA_FP32>(p, grid, hb, hr, st);
}

}  // namespace

// The scratch array.  In host code `scratch` names a host-side stand-in, not device memory: only the
// per-device address hipGetSymbolAddress returns (scratch_on) is ever passed to a kernel.
static __device__ __align__(256) int8_t scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];

// The scratch's device address on the current device, looked up once per device.  The first lookup
// also clears the arrival counters on `st` (static storage starts zeroed; every split launch leaves
// them zero again), so calls ordered after the first one see zero counters.
int scratch_on(hipStream_t st, void **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return -(int)e;
    if (dev < 0 || dev >= kMaxDevices) return MICA_MISS_DEVICE;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return -(int)e;
        if (ptr == nullptr) return -(int)hipErrorInvalidSymbol;
        hipLaunchKernelGGL(clear_counters_kernel, dim3(1), dim3(256), 0, st, (int *)ptr, (int)(kCounterBytes / 4));
        e = hipGetLastError();
        if (e != hipSuccess) return -(int)e;
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return 0;
}

}  // namespace

extern "C" long long mica_mm_i8_workspace_bytes(int device) {
    const int cus = cu_count(device);
    if (cus <= 0 || cus > 1024) return -(long long)hipErrorInvalidDevice;
    return workspace_bytes_for(cus);
}

extern "C" int mica_mm_i8(const int8_t *A, int lda, const int8_t *B, int ldb, const float *sa, const float *sb,
                          const float *bias, const void *residual, int ldr, void *C, int ldc, int out_dtype, int M,
                          int N, int K, int epilogue, void *workspace, long long workspace_bytes,
                          mica_stream_t stream) {
    return mm_i8_run(A, lda, B, ldb, sa, sb, bias, residual, ldr, C, ldc, out_dtype, M, N, K, epilogue, workspace,
                     workspace_bytes, false, (hipStream_t)stream);
}

extern "C" long long mica_mm_i8_noalloc_scratch_bytes(void) { return kScratchBytes; }

extern "C" int mica_mm_i8_noalloc(const int8_t *A, int lda, const int8_t *B, int ldb, const float *sa,
                                  const float *sb, const float *bias, const void *residual, int ldr, void *C, int ldc,
                                  int out_dtype, int M, int N, int K, int epilogue, mica_stream_t stream) {
    // arguments first (a rejected call touches no device), then the scratch of the current device
    const int bad = mm_i8_check(A, lda, B, ldb, sa, sb, bias, residual, ldr, C, ldc, out_dtype, M, N, K, epilogue,
                                nullptr, 0);
    if (bad != 0 || M == 0) return bad;
    void *ws = nullptr;
    const int rc = scratch_on((hipStream_t)stream, &ws);
    if (rc != 0) return rc;
    return mm_i8_run(A, lda, B, ldb, sa, sb, bias, residual, ldr, C, ldc, out_dtype, M, N, K, epilogue, ws,
                     kScratchBytes, true, (hipStream_t)stream);
}
