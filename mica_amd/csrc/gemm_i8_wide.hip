// W8A8 GEMM for large aligned shapes (K a multiple of 256, whole 256 x 256 tiles plus a tail of
// halves): C = epilogue(A[M, K] . B[N, K]^T) on v_mfma_i32_16x16x64_i8.
//
// Why this shape of kernel (measured on MI355X, random int8 operands):
//   * v_mfma_i32_16x16x64_i8 with two waves per SIMD keeps the shader clock near 2.1 GHz at full issue,
//     where back-to-back v_mfma_i32_32x32x32_i8 drops it to 1.5-1.7 GHz: 4.2 vs 2.9-3.5 POP/s of pure
//     MFMA work.  A single wave per SIMD cannot issue the 16x16x64 form back to back, so the
//     workgroup is 8 waves (2 per SIMD), each with a 64 x 128 block of the 256 x 256 tile.
//   * LDS DMA (buffer_load ... lds) moves ~1.5x more bytes per clock when every 16 lanes of an
//     instruction fetch two whole 128-byte lines instead of four half lines, so K is staged 128 bytes
//     at a time: a slab is 256 rows x 128 bytes of A and of B (64 KiB), and an instruction loads 8 rows.
// Tiling: 8 waves in a 4 (M) x 2 (N) grid.  A wave's block is MB x NB tiles of 16 x 16; the weight rows
// are the MFMA's A operand and the activation rows its B operand, so lane (r16 = lane % 16, kq =
// lane / 16) of tile (j, i) holds row i * 16 + r16, columns j * 16 + 4 kq .. + 3: four consecutive
// output columns of one row.  For the SiLU epilogue a wave's 128 weight rows are one group of 64 gate
// rows and the matching 64 up rows (the packing of int8_runtime.pack_gate_up).
// Pipeline: two LDS stages of one slab each.  K-step 0 of a slab runs while k-step 1's fragments are
// read; then one barrier (slab k + 1 has landed in every wave's share, every wave has read slab k),
// the DMA of slab k + 2 into slab k's stage, and k-step 1 while slab k + 1's k-step 0 is read.
// LDS rows are 128 bytes; 16-byte chunk g of row r sits at position g ^ (r % 8).  Measured with the
// LDS bank-conflict counters on gfx950 (256 bytes per clock, a ds_read_b128 in 4 clocks when free of
// conflicts): this keeps the 16-row x 4-chunk operand reads of both k-steps conflict-free, where
// g ^ ((r % 8) ^ (r / 8 % 2)) or an unswizzled layout cost 2x and 4x.
// Tiles overlap: the DMA that would fetch slab nk of a tile fetches slab 0 of the workgroup's next
// tile instead, its scales are loaded as the epilogue starts, and its slab 1 goes out right after the
// output stores, once the epilogue has finished with the LDS it shares with stage 1 (the 16-bit output
// staging).  The stores are buffer stores, a fixed number per wave (lanes past the edge get an offset
// that fails the range check), so the next tile waits for its slab 0 and scales with an exact vmcnt.
// Schedule: a persistent grid of at most one workgroup per CU walks the whole tiles in the XCD-aware
// order of gemm_i8_common.h, then the tail tiles as two halves each (256 x 128 for the SCALE epilogue,
// 128 x 256 along M for SiLU, whose waves need their 128 gate / up rows) or four quarters.
// Epilogue order: y = (f32(acc) * sa[m]) * sb[n] (+ bias[n]), rounded to the output type; the
// residual is added after that rounding (kernel_src/kernels.py:63-68, int8_runtime.py:186-192).

#include <type_traits>

#include "common.h"
#include "gemm_i8_common.h"

namespace {

constexpr int WBK = 128;                 // bytes of K per slab
constexpr int kWideWaves = 8, kWideThreads = 64 * kWideWaves;

typedef float v4f __attribute__((ext_vector_type(4)));

// A BM x BN tile on 8 waves in a 4 (M) x 2 (N) grid.
template <int BM_, int BN_>
struct WCfg {
    static constexpr int BM = BM_, BN = BN_;
    static constexpr int WM = BM / 4, WN = BN / 2;
    static constexpr int MB = WM / 16, NB = WN / 16;
    static constexpr int kAHalf = BM * WBK;                  // one stage of A
    static constexpr int kBHalf = BN * WBK;                  // one stage of B
    static constexpr int kBBase = 2 * kAHalf;                // B stages follow both A stages
    static constexpr int kADma = BM / 8 / kWideWaves;        // 1 KiB DMA instructions per wave per slab
    // B's 8-row blocks: the first kBWide waves take kBDma of them, the others kBDma - 1 (BN = 160: 3, 2)
    static constexpr int kBBlocks = BN / 8;
    static constexpr int kBDma = (kBBlocks + kWideWaves - 1) / kWideWaves;
    static constexpr int kBWide = kBBlocks - (kBDma - 1) * kWideWaves;
    static constexpr int kDma = kADma + kBDma;               // the most any wave issues per slab
    static_assert(BM % (8 * kWideWaves) == 0 && BN % 8 == 0, "DMA blocks");
    MICA_DEVICE static int bdma_count(int wave) {
        if constexpr (kBWide == kWideWaves) return kBDma;
        else return wave < kBWide ? kBDma : kBDma - 1;
    }
    MICA_DEVICE static int bdma_first(int wave) {
        if constexpr (kBWide == kWideWaves) return wave * kBDma;
        else return wave < kBWide ? wave * kBDma : kBWide * kBDma + (wave - kBWide) * (kBDma - 1);
    }
};
using WFull = WCfg<256, 256>;   // waves of 64 x 128
using WHalfN = WCfg<256, 128>;  // waves of 64 x 64 (SCALE tail)
using WHalfM = WCfg<128, 256>;  // waves of 32 x 128 (SiLU tail)
using WQuart = WCfg<128, 128>;  // waves of 32 x 64 (SCALE tail at most a quarter of a round)
using W160 = WCfg<256, 160>;    // waves of 64 x 80: whole tiles for N = 2560 at M = 4096 (256 tiles)

// LDS: A stages 0 and 1, then B stages 0 and 1 (every operand read of either stage then reaches
// its data with the 16-bit offset of ds_read_b128 from one base register per operand and k-step).
// The 16-bit epilogue stages its output outside stage 0, which by then holds the next tile's slab 0:
// the first kLowWaves waves in A stage 1, the others from the end of B stage 1 on.  Then two
// buffers of tile scales (sa, sb, bias: 3 x 256 fp32), for this tile and the next.
constexpr int kWScale = 96 * 1024 + 5 * 64 * 144;  // past the largest staging (WFull, SiLU)
constexpr int kWScaleBuf = 3 * 256 * 4;
constexpr int kWSmem = kWScale + 2 * kWScaleBuf;
static_assert(kWSmem <= 160 * 1024, "LDS");

MICA_DEVICE int wswz(int r) { return r & 7; }

// This lane's index in its wave, computed afresh (mbcnt over a full mask) wherever it is used: the
// per-lane offsets derived from it are recomputed for every tile (a few VALU operations) instead of
// being held across the persistent loop, where at 256 VGPRs they (or threadIdx.x itself) would be
// spilled, and a reload waits for every DMA in flight.  The wave index lives in an SGPR.
MICA_DEVICE int fresh_lane() {
    int l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
}

// A buffer offset the compiler cannot see through.  A per-lane choice between an offset and
// kOutOfRange must reach its load / store as one value: split into two exec-masked copies of the
// instruction, an empty side would be skipped and the number of operations issued (which the vmcnt
// waits count on) would vary with the data.
MICA_DEVICE int opaque(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

template <class C, int EPI, int OUT, bool HAS_BIAS, bool HAS_RES>
struct WideTile {
    static constexpr int WM = C::WM, WN = C::WN, MB = C::MB, NB = C::NB;
    static constexpr bool k16 = OUT == MICA_BF16 || OUT == MICA_FP16;
    // 16-bit epilogue: output columns per wave, staging pitch, rows staged per pass (two passes when
    // a whole 64 x 128 block does not fit the staging space), and the stores each wave issues
    static constexpr int kCols = EPI == MICA_EPI_SCALE ? WN : WN / 2;
    static constexpr int kPitch = kCols * 2 + 16;
    static constexpr int kPassRows = (WM * kPitch <= 64 * 144) ? WM : WM / 2;
    static constexpr int kPasses = WM / kPassRows;
    // lanes per staged row (8 columns each; a power of 2, lanes past kCols / 8 idle: kCols = 80 -> 16)
    static constexpr int kLanesPerRow = kCols / 8 <= 8 ? 8 : (kCols / 8 <= 16 ? 16 : 32);
    static constexpr int kRowsPerStore = 64 / kLanesPerRow;
    static constexpr int kReadsPerPass = kPassRows / kRowsPerStore;
    static constexpr int kStores = k16 ? WM / kRowsPerStore : 0;
    // staging: per-wave regions of kRegion bytes, kLowWaves of them in A stage 1
    static constexpr int kRegion = kPassRows * kPitch;
    static constexpr int kLowWaves = C::kAHalf / kRegion < kWideWaves ? C::kAHalf / kRegion : kWideWaves;
    static_assert(C::kBBase + C::kBHalf + (kWideWaves - kLowWaves) * kRegion <= kWScale, "staging");
    static_assert(kPassRows % 16 == 0 && kPassRows % kRowsPerStore == 0, "passes");
    static_assert(C::kDma + kStores < 64, "vmcnt");
    static_assert(kCols % 8 == 0 && kCols / 8 <= kLanesPerRow && kLanesPerRow <= 64, "staged rows");

    // s_waitcnt until this wave has at most N + (its DMA instructions per slab) vector memory operations
    // outstanding (the count differs between waves when B's blocks do not divide evenly)
    template <int N>
    MICA_DEVICE static void wait_dma_plus(int wave) {
        if constexpr (C::kBWide == kWideWaves) {
            wait_vmcnt<C::kDma + N>();
        } else {
            if (wave < C::kBWide) wait_vmcnt<C::kDma + N>();
            else wait_vmcnt<C::kDma - 1 + N>();
        }
    }

    v4i acc[NB][MB];

    struct Ops {
        v4i x[MB];
        v4i w[NB];
    };

    // DMA of tile rows: lane l of 1 KiB instruction j (A: j < kADma) covers row (wave * kADma + j) * 8 +
    // l / 8, LDS position l % 8, i.e. global chunk (l % 8) ^ (l / 8) (the row's r % 8 is l / 8).  The
    // VGPR offset of instruction j is the lane's base offset (dma_base) plus j rows of 8; rows past M /
    // N lie past the end of their buffer and read zeros (the launcher keeps (M + 256) * lda and
    // (N + 256) * ldb below 2^31).  The slab's K offset is the SGPR offset.
    MICA_DEVICE static int dma_base(int row0, int ld, int lane) {
        return (row0 + (lane >> 3)) * ld + (((lane & 7) ^ ((lane >> 3) & 7)) << 4);
    }
    // DMA of slab `slab` of tile (m0, n0) into LDS stage `stage`
    MICA_DEVICE static void tile_dma(const GemmParams &p, int8_t *smem, __amdgpu_buffer_rsrc_t rsrc_a,
                                     __amdgpu_buffer_rsrc_t rsrc_b, int wave, int m0, int n0, int slab, int stage) {
        const int lane = fresh_lane();
        const int kb = slab * WBK;
        const int bfirst = C::bdma_first(wave), bcount = C::bdma_count(wave);
        const int a0 = dma_base(m0 + wave * C::kADma * 8, p.lda, lane);
        const int b0 = dma_base(n0 + bfirst * 8, p.ldb, lane);
        int8_t *sa_ = smem + stage * C::kAHalf + wave * C::kADma * 1024;
        int8_t *sb_ = smem + C::kBBase + stage * C::kBHalf + bfirst * 1024;
#pragma unroll
        for (int j = 0; j < C::kADma; ++j)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_a, (lds_void *)(sa_ + j * 1024), 16, a0 + j * 8 * p.lda, kb, 0, 0);
#pragma unroll
        for (int j = 0; j < C::kBDma; ++j)
            if (j < bcount)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_b, (lds_void *)(sb_ + j * 1024), 16, b0 + j * 8 * p.ldb, kb, 0, 0);
    }

    // tile (m0, n0)'s scales into scale buffer buf by LDS DMA (no VGPRs held while they travel):
    // waves 0-3 fetch sa of tile rows [64 w, 64 w + 64) into [0, 256) and the bias of the same
    // columns into [512, 768), waves 4-7 sb into [256, 512); entries past the edge read 0 (unused)
    MICA_DEVICE static void scales_dma(const GemmParams &p, int8_t *smem, int wave, int buf, int m0, int n0) {
        const int i = (wave & 3) * 64 + fresh_lane();
        int8_t *sc = smem + kWScale + buf * kWScaleBuf;
        if (wave < 4) {
            const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void *)p.sa, 0, p.M * 4, kBufferFlags);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void *)(sc + wave * 256), 4, (m0 + i) * 4, 0, 0, 0);
            if (HAS_BIAS) {
                const __amdgpu_buffer_rsrc_t rb =
                    __builtin_amdgcn_make_buffer_rsrc((void *)p.bias, 0, p.N * 4, kBufferFlags);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void *)(sc + 2048 + wave * 256), 4, (n0 + i) * 4, 0,
                                                         0, 0);
            }
        } else {
            const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void *)p.sb, 0, p.N * 4, kBufferFlags);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void *)(sc + wave * 256), 4, (n0 + i) * 4, 0, 0, 0);
        }
    }

    // ---- slabs of tile (m0, n0) into acc.  On entry slab 0 is visible in stage 0 and slab 1 is in
    // flight into stage 1.  has_next: slab 0 of tile (m0n, n0n) is fetched into stage 0 once this
    // tile's last use of it is over.
    MICA_DEVICE void run(const GemmParams &p, int8_t *smem, __amdgpu_buffer_rsrc_t rsrc_a,
                         __amdgpu_buffer_rsrc_t rsrc_b, int wave, int m0, int n0, bool has_next, int m0n, int n0n) {
        const int lane = fresh_lane();
        const int wm = wave >> 1, wn = wave & 1;
        const int r16 = lane & 15, kq = lane >> 4;
        const int nk = p.K / WBK;  // even
        const int bfirst = C::bdma_first(wave), bcount = C::bdma_count(wave);
        const int a0 = opaque(dma_base(m0 + wave * C::kADma * 8, p.lda, lane));
        const int b0 = opaque(dma_base(n0 + bfirst * 8, p.ldb, lane));
        // the per-instruction offsets are formed at each DMA (one add each): held across the loop
        // they would cost 6 more VGPRs
        auto dma = [&](int slab) {
            const int kb = slab * WBK;
            const int a = opaque(a0), b = opaque(b0);
            int8_t *sa_ = smem + (slab & 1) * C::kAHalf + wave * C::kADma * 1024;
            int8_t *sb_ = smem + C::kBBase + (slab & 1) * C::kBHalf + bfirst * 1024;
#pragma unroll
            for (int j = 0; j < C::kADma; ++j)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_a, (lds_void *)(sa_ + j * 1024), 16, a + j * 8 * p.lda, kb, 0, 0);
#pragma unroll
            for (int j = 0; j < C::kBDma; ++j)
                if (j < bcount)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_b, (lds_void *)(sb_ + j * 1024), 16, b + j * 8 * p.ldb, kb, 0, 0);
        };
        // operand reads: k-step s of row r is chunk 4 s + kq.  The stage and the 16-row block are
        // compile-time offsets (they fit the 16-bit offset of ds_read_b128), so two base registers per
        // operand suffice
        int x_rd[2], w_rd[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int pos = ((4 * s + kq) ^ wswz(r16)) << 4;
            x_rd[s] = (wm * WM + r16) * WBK + pos;
            w_rd[s] = C::kBBase + (wn * WN + r16) * WBK + pos;
        }
        auto reads = [&](Ops &o, auto st_c, int s) {
            constexpr int ST = decltype(st_c)::value;
#pragma unroll
            for (int j = 0; j < NB; ++j) o.w[j] = *(const v4i *)(smem + w_rd[s] + ST * C::kBHalf + j * 16 * WBK);
#pragma unroll
            for (int i = 0; i < MB; ++i) o.x[i] = *(const v4i *)(smem + x_rd[s] + ST * C::kAHalf + i * 16 * WBK);
        };
        auto mfmas = [&](const Ops &o) {
#pragma unroll
            for (int j = 0; j < NB; ++j)
#pragma unroll
                for (int i = 0; i < MB; ++i)
                    acc[j][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(o.w[j], o.x[i], acc[j][i], 0, 0, 0);
        };
        constexpr int kReads = MB + NB, kMfma = MB * NB;
        static_assert(kMfma >= kReads, "schedule");
        // The next k-step's reads (and, after a barrier, the DMA) go out first, one per MFMA, so they
        // have landed long before the k-step that uses them; the rest of the MFMAs follow
        auto interleave = [&](auto dma_c) {
            constexpr bool DMA = decltype(dma_c)::value;
#pragma unroll
            for (int g = 0; g < kReads; ++g) {
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                if (DMA && g < C::kDma) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0); // LDS DMA
            }
            __builtin_amdgcn_sched_group_barrier(0x008, kMfma - kReads, 0);
        };
        using T = std::integral_constant<bool, true>;
        using F = std::integral_constant<bool, false>;
        // what goes out after a slab's barrier: nothing, this tile's slab k + 2, or the next tile's slab 0
        using DNone = std::integral_constant<int, 0>;
        using DOwn = std::integral_constant<int, 1>;
        using DNext = std::integral_constant<int, 2>;
        Ops R0, R1;
        // one slab from stage ST (R0 holds its k-step 0).  NEXT: another slab follows (barrier before
        // k-step 1, then its k-step 0 is read into R0)
        auto slab = [&](auto st_c, auto next_c, auto dk_c, int k) {
            constexpr int ST = decltype(st_c)::value;
            constexpr int DK = decltype(dk_c)::value;
            reads(R1, st_c, 1);
            mfmas(R0);
            interleave(F{});
            __builtin_amdgcn_sched_barrier(0);  // k-step 0 stays before the wait and the barrier
            if constexpr (decltype(next_c)::value) {
                wait_vmcnt<0>();   // slab k + 1 landed (this wave's share)
                wait_lgkmcnt0();   // k-step 1's fragments are in registers
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (DK == 1) dma(k + 2);
                if constexpr (DK == 2) {
                    if (has_next) tile_dma(p, smem, rsrc_a, rsrc_b, wave, m0n, n0n, 0, 0);
                }
                reads(R0, std::integral_constant<int, ST ^ 1>{}, 0);
                mfmas(R1);
                interleave(std::integral_constant<bool, DK == 1>{});
            } else {
                mfmas(R1);
            }
            // keep the next slab's k-step 0 MFMAs (whose fragments were just read) out of this one
            __builtin_amdgcn_sched_barrier(0);
        };

#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int i = 0; i < MB; ++i) acc[j][i] = v4i{};
        using S0 = std::integral_constant<int, 0>;
        using S1 = std::integral_constant<int, 1>;
        reads(R0, S0{}, 0);
        int k = 0;
        for (; k + 2 < nk; k += 2) {
            slab(S0{}, T{}, DOwn{}, k);
            slab(S1{}, T{}, DOwn{}, k + 1);
        }
        slab(S0{}, T{}, DNext{}, k);
        slab(S1{}, F{}, DNone{}, k + 1);
    }

    // ---- epilogue of tile (m0, n0) from acc, with its scales in buffer buf.  With has_next, the next
    // tile's scales go to buffer buf ^ 1 and, last, its slab 1 into stage 1; between the scales and
    // that DMA this wave issues exactly kStores vector memory operations that may still be in flight
    // (the stores; anything else is waited for).
    MICA_DEVICE void epilogue(const GemmParams &p, int8_t *smem, __amdgpu_buffer_rsrc_t rsrc_a,
                              __amdgpu_buffer_rsrc_t rsrc_b, int wave, int m0, int n0, int buf, bool has_next,
                              int m0n, int n0n) {
        const int lane = fresh_lane();
        const int wm = wave >> 1, wn = wave & 1;
        const int r16 = lane & 15, kq = lane >> 4;
        const int M = p.M, N = p.N;
        const int mw = m0 + wm * WM;
        const bool vec = p.vec_ok != 0;
        const float *sc = (const float *)(smem + kWScale + buf * kWScaleBuf); // sa, sb, bias
        if (has_next) scales_dma(p, smem, wave, buf ^ 1, m0n, n0n);
        float sav[MB];
#pragma unroll
        for (int i = 0; i < MB; ++i) sav[i] = sc[wm * WM + i * 16 + r16];
        // every wave is done reading stage 1 (the staging below overlaps it)
        wait_lgkmcnt0();
        __builtin_amdgcn_s_barrier();
        if constexpr (k16) {
            // Staged through LDS: every wave writes its rounded 16-bit block (8 bytes per lane per store)
            // into its own padded region, reads it back row-contiguously (16 bytes per lane), and stores
            // it once stage 1 is handed to the next tile.
            int8_t *ep = smem + (wave < kLowWaves ? C::kAHalf + wave * kRegion
                                                  : C::kBBase + C::kBHalf + (wave - kLowWaves) * kRegion);
            const int col0 = EPI == MICA_EPI_SCALE ? n0 + wn * WN : (n0 >> 1) + wn * (WN / 2);
            const int ncols_out = EPI == MICA_EPI_SCALE ? N : (N >> 1);
            // local column of this lane's 8 values (lanes past the wave's columns read a valid place and
            // store nothing)
            const bool lane_on = kCols / 8 == kLanesPerRow || (lane % kLanesPerRow) * 8 < kCols;
            const int cl = lane_on ? (lane % kLanesPerRow) * 8 : kCols - 8;
            u32x4 outv[kStores];
#pragma unroll
            for (int pass = 0; pass < kPasses; ++pass) {
                if (pass > 0) wait_lgkmcnt0();  // the previous pass's read-back has landed
#pragma unroll
                for (int j = 0; j < (EPI == MICA_EPI_SCALE ? NB : NB / 2); ++j) {
                    const int nl = j * 16 + 4 * kq;  // local output column of this lane's 4 values
                    const int cb = wn * WN + nl;     // tile-local column (SiLU: of the gate row)
                    const v4f s1 = *(const v4f *)(sc + 256 + cb);  // SCALE: sb[n]; SILU_MUL: the gate rows' sb
                    v4f s2 = {}, bv = {};
                    if (EPI != MICA_EPI_SCALE) s2 = *(const v4f *)(sc + 256 + cb + WN / 2);  // the up rows
                    if (HAS_BIAS) bv = *(const v4f *)(sc + 512 + cb);
#pragma unroll
                    for (int ii = 0; ii < kPassRows / 16; ++ii) {
                        const int i = pass * (kPassRows / 16) + ii;
                        float y[4];
#pragma unroll
                        for (int t = 0; t < 4; ++t) {
                            if (EPI == MICA_EPI_SCALE) {
                                y[t] = ((float)acc[j][i][t] * sav[i]) * s1[t];
                                if (HAS_BIAS) y[t] = y[t] + bv[t];
                            } else {
                                const float gv = round_bf16(((float)acc[j][i][t] * sav[i]) * s1[t]);
                                const float uv = round_bf16(((float)acc[j + NB / 2][i][t] * sav[i]) * s2[t]);
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
                        *(u32x2 *)(ep + (ii * 16 + r16) * kPitch + nl * 2) = w;
                    }
                }
                wait_lgkmcnt0(); // a wave reads back only its own region: no barrier needed
#pragma unroll
                for (int r = 0; r < kReadsPerPass; ++r)
                    outv[pass * kReadsPerPass + r] =
                        *(const u32x4 *)(ep + (r * kRowsPerStore + lane / kLanesPerRow) * kPitch + cl * 2);
            }
            // output row of store s: mw + s * kRowsPerStore + lane / kLanesPerRow
            const bool fast = vec && (p.ldc % 8 == 0) && (!HAS_RES || p.ldr % 8 == 0) && (ncols_out % 8 == 0);
            const int rows_in = M - m0 < C::BM ? M - m0 : C::BM;  // valid rows of this tile
            const bool col_ok = lane_on && col0 + cl < ncols_out;  // with fast: all 8 columns, or none
            u32x4 rv[HAS_RES ? kStores : 1];
            if (fast && HAS_RES) {
                const __amdgpu_buffer_rsrc_t rsrc_r = __builtin_amdgcn_make_buffer_rsrc(
                    (void *)((const uint16_t *)p.res + (long)m0 * p.ldr), 0, rows_in * p.ldr * 2, kBufferFlags);
#pragma unroll
                for (int s = 0; s < kStores; ++s) {
                    const int rl = wm * WM + s * kRowsPerStore + lane / kLanesPerRow;  // tile-local row
                    const int off = opaque(col_ok ? (rl * p.ldr + col0 + cl) * 2 : kOutOfRange);
                    rv[s] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc_r, off, 0, 0));
                }
            }
            if (fast) {
                if (HAS_RES) {
                    wait_vmcnt<0>();  // the residual rows
#pragma unroll
                    for (int s = 0; s < kStores; ++s) {
#pragma unroll
                        for (int t = 0; t < 4; ++t) {
                            const uint32_t v = outv[s][t], r = rv[s][t];
                            if (OUT == MICA_BF16) {
                                outv[s][t] = pack_bf16x2(bf16_lo(v) + bf16_lo(r), bf16_hi(v) + bf16_hi(r));
                            } else {
                                const float a0 = f16_to_f32(v & 0xffff), a1 = f16_to_f32(v >> 16);
                                const float b0 = f16_to_f32(r & 0xffff), b1 = f16_to_f32(r >> 16);
                                outv[s][t] = (uint32_t)f32_to_f16(a0 + b0) | ((uint32_t)f32_to_f16(a1 + b1) << 16);
                            }
                        }
                    }
                }
                const __amdgpu_buffer_rsrc_t rsrc_c = __builtin_amdgcn_make_buffer_rsrc(
                    (void *)((uint16_t *)p.C + (long)m0 * p.ldc), 0, rows_in * p.ldc * 2, kBufferFlags);
#pragma unroll
                for (int s = 0; s < kStores; ++s) {
                    const int rl = wm * WM + s * kRowsPerStore + lane / kLanesPerRow;
                    const int off = opaque(col_ok ? (rl * p.ldc + col0 + cl) * 2 : kOutOfRange);
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i, outv[s]), rsrc_c, off, 0, 0);
                }
            } else {
                // unaligned output: element stores, then nothing left in flight
                const int valid = !lane_on ? 0 : ncols_out - (col0 + cl) < 8 ? (ncols_out - (col0 + cl) > 0 ? ncols_out - (col0 + cl) : 0) : 8;
#pragma unroll
                for (int s = 0; s < kStores; ++s) {
                    const int m = mw + s * kRowsPerStore + lane / kLanesPerRow;
                    if (m >= M || valid == 0) continue;
                    const u32x4 v = outv[s];
                    u32x4 o = v;
                    if (HAS_RES) {
                        const uint16_t *rp = (const uint16_t *)p.res + (long)m * p.ldr + col0 + cl;
                        u32x4 r = {0u, 0u, 0u, 0u};
                        for (int t = 0; t < valid; ++t) r[t >> 1] |= (uint32_t)rp[t] << (16 * (t & 1));
#pragma unroll
                        for (int t = 0; t < 4; ++t) {
                            if (OUT == MICA_BF16) {
                                o[t] = pack_bf16x2(bf16_lo(v[t]) + bf16_lo(r[t]), bf16_hi(v[t]) + bf16_hi(r[t]));
                            } else {
                                const float a0 = f16_to_f32(v[t] & 0xffff), a1 = f16_to_f32(v[t] >> 16);
                                const float b0 = f16_to_f32(r[t] & 0xffff), b1 = f16_to_f32(r[t] >> 16);
                                o[t] = (uint32_t)f32_to_f16(a0 + b0) | ((uint32_t)f32_to_f16(a1 + b1) << 16);
                            }
                        }
                    }
                    uint16_t *cp = (uint16_t *)p.C + (long)m * p.ldc + col0 + cl;
                    for (int t = 0; t < valid; ++t) cp[t] = (uint16_t)(o[t >> 1] >> (16 * (t & 1)));
                }
                if (has_next) wait_vmcnt<0>();
            }
            // every wave's read-back is done: stage 1 belongs to the next tile
            wait_lgkmcnt0();
            __builtin_amdgcn_s_barrier();
            if (has_next) tile_dma(p, smem, rsrc_a, rsrc_b, wave, m0n, n0n, 1, 1);
            return;
        }
        // 32-bit outputs (fp32 / raw int32): 16-byte stores straight from the accumulator layout, then
        // nothing left in flight
        if constexpr (EPI == MICA_EPI_SCALE) {
            const int nw = n0 + wn * WN;
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const int nb = nw + j * 16 + 4 * kq;
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
                    const int m = mw + i * 16 + r16;
                    if (m >= M) continue;
                    const long off = (long)m * p.ldc + nb;
                    if (OUT == MICA_INT32) {
                        int *c = (int *)p.C + off;
                        if (vec && valid == 4) *(v4i *)c = acc[j][i];
                        else for (int t = 0; t < valid; ++t) c[t] = acc[j][i][t];
                        continue;
                    }
                    float y[4];
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        y[t] = ((float)acc[j][i][t] * sav[i]) * sbv[t];
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
        if (has_next) {
            wait_vmcnt<0>();
            tile_dma(p, smem, rsrc_a, rsrc_b, wave, m0n, n0n, 1, 1);
        }
    }
};

// The pieces h = h0, h0 + G, ... < hend of one schedule phase (all of one tile shape C), on this
// workgroup; piece(h, m0, n0) gives a piece's origin, false for a piece wholly past the edge.
template <class C, int EPI, int OUT, bool HAS_BIAS, bool HAS_RES, class Piece>
MICA_DEVICE void run_phase(const GemmParams &p, int8_t *smem, __amdgpu_buffer_rsrc_t rsrc_a,
                           __amdgpu_buffer_rsrc_t rsrc_b, int wave, int h0, int hend, int G, Piece piece) {
    using Tile = WideTile<C, EPI, OUT, HAS_BIAS, HAS_RES>;
    int h = h0, m0 = 0, n0 = 0;
    while (h < hend && !piece(h, m0, n0)) h += G;
    if (h >= hend) return;
    Tile t;
    // the previous phase's epilogue is finished with the stages, the staging and the scales
    wait_lgkmcnt0();
    __builtin_amdgcn_s_barrier();
    Tile::scales_dma(p, smem, wave, 0, m0, n0);
    Tile::tile_dma(p, smem, rsrc_a, rsrc_b, wave, m0, n0, 0, 0);
    Tile::tile_dma(p, smem, rsrc_a, rsrc_b, wave, m0, n0, 1, 1);
    Tile::template wait_dma_plus<0>(wave);  // scales and slab 0 landed (slab 1 may be in flight)
    __builtin_amdgcn_s_barrier();
    int buf = 0;
    for (;;) {
        int hn = h + G, m0n = 0, n0n = 0;
        while (hn < hend && !piece(hn, m0n, n0n)) hn += G;
        const bool has_next = hn < hend;
        t.run(p, smem, rsrc_a, rsrc_b, wave, m0, n0, has_next, m0n, n0n);
        t.epilogue(p, smem, rsrc_a, rsrc_b, wave, m0, n0, buf, has_next, m0n, n0n);
        if (!has_next) break;
        // the next tile's slab 0 and scales landed: all but this epilogue's stores and its slab 1
        Tile::template wait_dma_plus<Tile::kStores>(wave);
        __builtin_amdgcn_s_barrier();
        buf ^= 1;
        h = hn;
        m0 = m0n;
        n0 = n0n;
    }
}

template <int EPI, int OUT, bool HAS_BIAS, bool HAS_RES, bool NARROW>
__global__ __launch_bounds__(kWideThreads, 1) void gemm_i8_wide_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(1024))) int8_t smem[kWSmem];
    static_assert(EPI == MICA_EPI_SCALE || WFull::WN == 128, "the SiLU epilogue needs one 128-row gate/up group per wave");
    const int G = gridDim.x;
    const __amdgpu_buffer_rsrc_t rsrc_a = __builtin_amdgcn_make_buffer_rsrc((void *)p.A, 0, p.M * p.lda, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rsrc_b = __builtin_amdgcn_make_buffer_rsrc((void *)p.B, 0, p.N * p.ldb, kBufferFlags);
    const int tm_n = p.tiles_m, tn_n = p.tiles_n, dp = p.dp_tiles, M = p.M, N = p.N;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    if constexpr (NARROW) {
        // 256 x 160 tiles only (tiles_n counts 160-column tiles)
        run_phase<W160, EPI, OUT, HAS_BIAS, HAS_RES>(p, smem, rsrc_a, rsrc_b, wave, blockIdx.x, dp, G,
                                                     [&](int h, int &m0, int &n0) {
                                                         int tm, tn;
                                                         tile_of(h, tm_n, tn_n, tm, tn);
                                                         m0 = tm * 256;
                                                         n0 = tn * 160;
                                                         return true;
                                                     });
        return;
    }
    run_phase<WFull, EPI, OUT, HAS_BIAS, HAS_RES>(p, smem, rsrc_a, rsrc_b, wave, blockIdx.x, dp, G,
                                                  [&](int h, int &m0, int &n0) {
                                                      int tm, tn;
                                                      tile_of(h, tm_n, tn_n, tm, tn);
                                                      m0 = tm * 256;
                                                      n0 = tn * 256;
                                                      return true;
                                                  });
    if constexpr (EPI == MICA_EPI_SCALE) {
        // the next half_tiles tiles as two 256 x 128 halves each
        if (p.half_tiles > 0)
            run_phase<WHalfN, EPI, OUT, HAS_BIAS, HAS_RES>(p, smem, rsrc_a, rsrc_b, wave, blockIdx.x, 2 * p.half_tiles, G,
                                                           [&](int h, int &m0, int &n0) {
                                                               int tm, tn, t, part;
                                                               tail_piece(h, 2, dp, p.half_tiles, t, part);
                                                               tile_of(t, tm_n, tn_n, tm, tn);
                                                               m0 = tm * 256;
                                                               n0 = tn * 256 + part * 128;
                                                               return n0 < N;
                                                           });
        // or the next quarter_tiles tiles as four 128 x 128 quarters each
        if (p.quarter_tiles > 0)
            run_phase<WQuart, EPI, OUT, HAS_BIAS, HAS_RES>(p, smem, rsrc_a, rsrc_b, wave, blockIdx.x, 4 * p.quarter_tiles, G,
                                                           [&](int h, int &m0, int &n0) {
                                                               int tm, tn, t, part;
                                                               tail_piece(h, 4, dp, p.quarter_tiles, t, part);
                                                               tile_of(t, tm_n, tn_n, tm, tn);
                                                               m0 = tm * 256 + ((part >> 1) & 1) * 128;
                                                               n0 = tn * 256 + (part & 1) * 128;
                                                               return m0 < M && n0 < N;
                                                           });
    } else {
        // the next mhalf_tiles tiles as two 128 x 256 halves each along M (gate / up pairs intact)
        if (p.mhalf_tiles > 0)
            run_phase<WHalfM, EPI, OUT, HAS_BIAS, HAS_RES>(p, smem, rsrc_a, rsrc_b, wave, blockIdx.x, 2 * p.mhalf_tiles, G,
                                                           [&](int h, int &m0, int &n0) {
                                                               int tm, tn, t, part;
                                                               tail_piece(h, 2, dp, p.mhalf_tiles, t, part);
                                                               tile_of(t, tm_n, tn_n, tm, tn);
                                                               m0 = tm * 256 + part * 128;
                                                               n0 = tn * 256;
                                                               return m0 < M;
                                                           });
    }
}

template <int EPI, int OUT, bool NARROW = false>
int wide_launch_out(const GemmParams &p, int grid, bool has_bias, bool has_res, hipStream_t st) {
    dim3 g(grid), b(kWideThreads);
#define MICA_W(B_, R_) hipLaunchKernelGGL((gemm_i8_wide_kernel<EPI, OUT, B_, R_, NARROW>), g, b, 0, st, p)
    if constexpr (EPI == MICA_EPI_SILU_MUL || OUT == MICA_INT32) {
        static_assert(!NARROW, "narrow tiles: SCALE epilogue with 16-bit outputs only");
        MICA_W(false, false);
    } else {
        if (has_bias && has_res) MICA_W(true, true);
        else if (has_bias) MICA_W(true, false);
        else if (has_res) MICA_W(false, true);
        else MICA_W(false, false);
    }
#undef MICA_W
    return mica_err(hipGetLastError());
}

}  // namespace

// Launch of the wide kernel for the schedule in p (dp_tiles whole tiles, then half_tiles, quarter_tiles
// or mhalf_tiles as pieces; no split).  Called by mica_mm_i8 after its checks, only for K % 256 == 0
// and row pitches whose 256-row tile spans stay below 2^31 bytes (the buffer offsets of the stores).
// narrow: dp_tiles 256 x 160 tiles and nothing else (SCALE epilogue, bf16 / fp16 outputs).
int mica_gemm::wide_launch(const GemmParams &p, int epilogue, int out_dtype, int grid, bool has_bias, bool has_res,
                           bool narrow, hipStream_t st) {
    if (narrow) {
        if (epilogue != MICA_EPI_SCALE || p.half_tiles || p.quarter_tiles || p.mhalf_tiles || p.sk_tiles)
            return MICA_MISS_ARG;
        if (out_dtype == MICA_BF16) return wide_launch_out<MICA_EPI_SCALE, MICA_BF16, true>(p, grid, has_bias, has_res, st);
        if (out_dtype == MICA_FP16) return wide_launch_out<MICA_EPI_SCALE, MICA_FP16, true>(p, grid, has_bias, has_res, st);
        return MICA_MISS_ARG;
    }
    if (epilogue == MICA_EPI_SILU_MUL) return wide_launch_out<MICA_EPI_SILU_MUL, MICA_BF16>(p, grid, false, false, st);
    if (out_dtype == MICA_BF16) return wide_launch_out<MICA_EPI_SCALE, MICA_BF16>(p, grid, has_bias, has_res, st);
    if (out_dtype == MICA_FP16) return wide_launch_out<MICA_EPI_SCALE, MICA_FP16>(p, grid, has_bias, has_res, st);
    if (out_dtype == MICA_INT32) return wide_launch_out<MICA_EPI_SCALE, MICA_INT32>(p, grid, false, false, st);
    return wide_launch_out<MICA_EPI_SCALE, MICA_FP32>(p, grid, has_bias, has_res, st);
}
