// W8A8 GEMM with the accumulators in AGPRs: C = epilogue(A[M, K] . B[N, K]^T) on
// v_mfma_i32_16x16x64_i8, 4 waves per workgroup (one per SIMD), 16-bit outputs.
//
// Why this shape of kernel (measured on MI355X, random int8 operands):
//   * One wave per SIMD issues independent v_mfma_i32_16x16x64_i8 back to back at ~94 % of the rate
//     of two waves per SIMD when its 64 accumulators stay in AGPRs (3.82 vs 4.06 POP/s of pure MFMA
//     work over the chip).  With two waves per SIMD sharing the MFMA pipe, the pipe's arbitration lets
//     one wave of the pair run ahead; at every workgroup barrier the other then issues alone, and
//     that skew, not the MFMA work, set the pace of the 8-wave kernel (gemm_i8_wide.hip).  Here the
//     four waves run the same instruction stream on four pipes and reach each barrier together.
//   * A 256 x 256 tile over 4 waves is 128 x 128 per wave: 8 x 8 MFMA tiles of 16 x 16, i.e. 256
//     accumulator registers, which only AGPRs can hold next to the operand double buffer (2 x 16
//     fragments of 16 bytes per lane = 128 VGPRs).  Per k-step a wave reads 16 fragments for 64 MFMAs
//     (the 8-wave kernel: 12 for 32).
//   * The first k-step of a tile accumulates onto the inline constant 0, so no register is cleared.
// Operand feed (as in the 8-wave kernel): K moves in 128-byte slabs by LDS DMA, 2 stages of one slab
// (A 32 KiB + B 32 KiB each); 16-byte chunk g of LDS row r sits at position g ^ (r % 8), which keeps
// the 16-row x 4-chunk fragment reads conflict-free.  One barrier per slab, after k-step 0: slab k + 1
// has landed in every wave's share and every wave has read slab k, whose stage then receives slab k + 2.
// Epilogue without LDS staging: a lane of MFMA tile (j, i) holds 4 consecutive output columns of one
// row; v_permlane16_swap between the lanes of rows kq and kq ^ 1 of two neighbouring tiles j, j + 1
// leaves every lane with 8 consecutive columns (16 bytes) of one output row, stored straight from
// registers.  Stage 1 is therefore free as soon as the last slab has been read: the next tile's slab 1
// goes out at the start of the epilogue, its slab 0 during the last slab.
// Schedule: a persistent grid of at most one workgroup per CU walks the whole tiles in the XCD-aware
// order of gemm_i8_common.h, then the tail tiles as two halves (256 x 128 for the SCALE epilogue,
// 128 x 256 along M for SiLU, whose waves need their 128 gate / up rows) or four 128 x 128 quarters.
// Launches of few tiles with a long K run as 128-row tiles split along K over several workgroups
// (gemm_i8_agpr_split_kernel), whose int32 partial sums the last part of each tile adds.
// Epilogue order: y = (f32(acc) * sa[m]) * sb[n] (+ bias[n]), rounded to the output type; the residual
// is added after that rounding (kernel_src/kernels.py:63-68, int8_runtime.py:186-192); SiLU:
// bf16(bf16(silu(bf16 g)) * bf16 u) (fast_runtime.py:126-132 with the gate / up pairing of
// int8_runtime.pack_gate_up).

#include <type_traits>

#include "common.h"
#include "gemm_i8_common.h"

namespace {

constexpr int QBK = 128;                // bytes of K per slab
constexpr int kQWaves = 4, kQThreads = 64 * kQWaves;

typedef float v4f __attribute__((ext_vector_type(4)));

// A BM x BN tile on 4 waves in a WGM (M) x WGN (N) grid, NS LDS stages of one slab each; CPOL: the
// cache policy bits of its output stores (0, or 2: nt).
template <int BM_, int BN_, int NS_ = 2, int WGM_ = 2, int WGN_ = 2, int CPOL_ = 0>
struct QCfg {
    static constexpr int BM = BM_, BN = BN_, NS = NS_, WGM = WGM_, WGN = WGN_, CPOL = CPOL_;
    static_assert(WGM * WGN == kQWaves, "wave grid");
    static constexpr int WM = BM / WGM, WN = BN / WGN;
    static constexpr int MB = WM / 16, NB = WN / 16;
    static constexpr int kAHalf = BM * QBK;                 // one stage of A
    static constexpr int kBHalf = BN * QBK;                 // one stage of B
    static constexpr int kBBase = NS * kAHalf;              // B stages follow the A stages
    static constexpr int kADma = BM / 8 / kQWaves;          // 1 KiB DMA instructions per wave per slab
    static constexpr int kBDma = BN / 8 / kQWaves;
    static constexpr int kDma = kADma + kBDma;
    static_assert(BM % (8 * kQWaves) == 0 && BN % (8 * kQWaves) == 0, "DMA blocks");
    static_assert(NB % 2 == 0, "tile pairs for the 16-byte stores");
};
// Tail pieces (one per workgroup: the launcher gives a tail at most one piece per CU) store their outputs
// non-temporally (the last writes of a launch; same bits, measured 0.3-0.9 % faster over the headline,
// QKV, gate+up and 1024 x 2560 x 9728, interleaved on one box) and keep three slabs
// in LDS, two in flight while one is read: they need 48 B of DMA per MFMA clock against 32 for whole
// tiles, and with one slab of lookahead their loop ran 35 K cycles (256 x 128 x 2560) against 28 K
// with every operand resident in L2.
using QFull = QCfg<256, 256>;      // waves of 128 x 128
using QHalfN = QCfg<256, 128, 3, 2, 2, 2>;  // waves of 128 x 64 (SCALE tail)
using QHalfM = QCfg<128, 256, 3, 2, 2, 2>;  // waves of 64 x 128 (SiLU tail)
using QQuart = QCfg<128, 128, 3, 2, 2, 2>;  // waves of 64 x 64 (SCALE tail at most a quarter of a round)
// One partial round of 256 x 256 tiles run as 256 x 160 tiles (e.g. N = 2560 at M = 4096: 160 tiles
// become 256): waves of 64 x 160 stacked along M, 10 x 4 MFMA tiles = 160 accumulators per lane.
using QNarrow = QCfg<256, 160, 2, 4, 1>;
// One round of 128 x 160 tiles for launches whose 256 x 256 tiles fill less than a round and are too
// many for 128 x 128 quarters to fit one (e.g. 512 x 2560 x 9728: 76 tiles, 244 of these): waves of
// 32 x 160 stacked along M, 2 x 10 MFMA tiles = 80 accumulators per lane, four LDS stages (one tile
// per workgroup, nothing to prefetch for a successor: three slabs stay in flight, against two with three
// stages, whose DMA waited on memory latency).  Such a tile is bound by its DMA feed, (128 + 160) rows x
// K against 384 rows for the 256 x 128 half tile it replaces.
// Its outputs are stored non-temporally: 512 x 9728 x 2560 16.4 -> 15.5 us (same bits), where whole
// 256 x 256 tiles lost by it (4096 x 9728 x 2560 86.5 -> 91.7 us, 4096 x 6144 x 2560 57.3 -> 58.6, the
// 256 x 160 tiles of 4096 x 2560 x 9728 79.0 -> 80.0; interleaved on one box).
using QSmall = QCfg<128, 160, 4, 4, 1, 2>;
// The SiLU epilogue's counterpart for launches of at most 128 rows (a short request's gate+up): one round
// of 128 x 128 tiles, each one 64-row group of gate weights and its 64 up rows, on waves of 32 x 128
// stacked along M (2 x 8 MFMA tiles, 64 accumulators per lane), so every wave pairs gate and up columns
// in its own lanes.  128 x 19456 x 2560: 152 tiles on 152 CUs, where the 128 x 256 M-halves keep 76
// busy (and 76 with no rows).
using QSiluSmall = QCfg<128, 128, 4, 4, 1>;

// LDS: the A stages, the B stages, then (at a fixed place past the largest stage set) two buffers of
// tile scales (sa, sb, bias: 3 x 256 fp32), for this tile and the next.
constexpr int kQScale = 144 * 1024;
constexpr int kQScaleBuf = 3 * 256 * 4;
constexpr int kQSmem = kQScale + 2 * kQScaleBuf;
static_assert(kQSmem <= 160 * 1024, "LDS");
template <class C>
constexpr bool stages_fit = C::NS * (C::kAHalf + C::kBHalf) <= kQScale;
static_assert(stages_fit<QFull> && stages_fit<QHalfN> && stages_fit<QHalfM> && stages_fit<QQuart> &&
                  stages_fit<QNarrow> && stages_fit<QSmall> && stages_fit<QSiluSmall>, "stages");

// This lane's index, computed afresh where it is used (a few VALU operations per tile instead of a
// register held across the persistent loop).  The wave index lives in an SGPR.
MICA_DEVICE int lane_id() {
    int l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
}

// A buffer offset the compiler cannot see through: a per-lane choice between an offset and
// kOutOfRange reaches its load / store as one instruction, so the number of vector memory operations
// (which the vmcnt waits count) does not depend on the data.
MICA_DEVICE int opaque_off(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

// LDS address (byte offset in the workgroup's LDS) of a shared-memory pointer
MICA_DEVICE uint32_t lds_addr(const int8_t *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) int8_t *)p;
}

// N operand fragments (16 bytes per lane) at a + OFF + 2048 i, i < N, by ds_read_b128 written as inline
// assembly: the destinations are plain VGPRs (the compiler's own LDS loads may target AGPRs, which
// pushes accumulators out of the AGPRs into copies every k-step).  The compiler does not see these
// loads: every use waits with an explicit s_waitcnt lgkmcnt and a scheduling barrier.  (An LDS load
// may overwrite a register an MFMA issued just before reads as srcA / srcB: the compiler itself emits
// that order with no wait states for gfx950.)
template <int OFF, int N, int I = 0>
MICA_DEVICE void frag_reads(v4i (&r)[N], uint32_t a) {
    if constexpr (I < N) {
        asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r[I]) : "v"(a), "i"(OFF + I * 16 * QBK));
        frag_reads<OFF, N, I + 1>(r, a);
    }
}

template <class C, int EPI, int OUT, bool HAS_BIAS, bool HAS_RES>
struct QTile {
    static constexpr int WM = C::WM, WN = C::WN, MB = C::MB, NB = C::NB;
    static_assert(OUT == MICA_BF16 || OUT == MICA_FP16, "16-bit outputs");
    static_assert(EPI == MICA_EPI_SCALE || (OUT == MICA_BF16 && !HAS_BIAS && !HAS_RES), "SiLU: bf16 only");
    // output tiles of 16 columns per wave row block (SiLU: gate tiles j < NB / 2 pair with up tiles
    // j + NB / 2), and 16-byte stores per row block (one per pair of output tiles)
    static constexpr int kOutTiles = EPI == MICA_EPI_SCALE ? NB : NB / 2;
    static constexpr int kS = kOutTiles / 2;
    static constexpr int kStores = MB * kS;
    static_assert(kOutTiles % 2 == 0, "pairs");
    static_assert(C::kDma + kStores <= 63 && C::kDma + 2 * kS <= 63, "vmcnt");

    v4i acc[NB][MB];

    struct Ops {
        v4i x[MB];
        v4i w[NB];
    };

    // DMA of tile rows: lane l of 1 KiB instruction j covers row (wave * kDma_ + j) * 8 + l / 8 at LDS
    // position l % 8, i.e. global chunk (l % 8) ^ (l / 8).  Rows past M / N read zeros (the launcher
    // keeps (M + 256) * lda and (N + 256) * ldb below 2^31); the slab's K offset is the SGPR offset.
    MICA_DEVICE static int dma_base(int row0, int ld, int lane) {
        return (row0 + (lane >> 3)) * ld + (((lane & 7) ^ ((lane >> 3) & 7)) << 4);
    }
    MICA_DEVICE static void tile_dma(const GemmParams &p, int8_t *smem, __amdgpu_buffer_rsrc_t rsrc_a,
                                     __amdgpu_buffer_rsrc_t rsrc_b, int wave, int m0, int n0, int slab, int stage) {
        const int lane = lane_id();
        const int kb = slab * QBK;
        const int a0 = dma_base(m0 + wave * C::kADma * 8, p.lda, lane);
        const int b0 = dma_base(n0 + wave * C::kBDma * 8, p.ldb, lane);
        int8_t *sa_ = smem + stage * C::kAHalf + wave * C::kADma * 1024;
        int8_t *sb_ = smem + C::kBBase + stage * C::kBHalf + wave * C::kBDma * 1024;
#pragma unroll
        for (int j = 0; j < C::kADma; ++j)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_a, (lds_void *)(sa_ + j * 1024), 16, a0 + j * 8 * p.lda, kb, 0, 0);
#pragma unroll
        for (int j = 0; j < C::kBDma; ++j)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_b, (lds_void *)(sb_ + j * 1024), 16, b0 + j * 8 * p.ldb, kb, 0, 0);
    }

    // tile (m0, n0)'s scales into scale buffer buf by LDS DMA: wave w fetches sa of tile rows
    // [64 w, 64 w + 64), sb (and the bias) of tile columns [64 w, 64 w + 64); entries past the edge
    // read 0 (unused).  2 or 3 vector memory operations per wave.
    static constexpr int kScaleOps = HAS_BIAS ? 3 : 2;
    MICA_DEVICE static void scales_dma(const GemmParams &p, int8_t *smem, int wave, int buf, int m0, int n0) {
        const int i = wave * 64 + lane_id();
        int8_t *sc = smem + kQScale + buf * kQScaleBuf;
        const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void *)p.sa, 0, p.M * 4, kBufferFlags);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void *)(sc + wave * 256), 4, (m0 + i) * 4, 0, 0, 0);
        const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc((void *)p.sb, 0, p.N * 4, kBufferFlags);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void *)(sc + 1024 + wave * 256), 4, (n0 + i) * 4, 0, 0, 0);
        if (HAS_BIAS) {
            const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc((void *)p.bias, 0, p.N * 4, kBufferFlags);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rc, (lds_void *)(sc + 2048 + wave * 256), 4, (n0 + i) * 4, 0, 0, 0);
        }
    }

    // ---- one k-step: MFMA m = MB j + i accumulates w[j] x x[i] of cur (FIRST: onto 0).  With READ, the
    // next k-step's fragments go out first, one ahead of each of the first kReads MFMAs, in that
    // order (a scheduling barrier after each pair), at LDS offsets OFFW / OFFX from wa / xa.
    static constexpr int kReads = MB + NB, kMfma = MB * NB;
    static_assert(kMfma >= kReads, "schedule");
    template <int M, bool FIRST>
    MICA_DEVICE void mfma_one(const Ops &cur) {
        constexpr int j = M / MB, i = M % MB;
        if constexpr (FIRST) {
            // the tile's first k-step accumulates onto 0 and defines the accumulator in AGPRs (as
            // inline assembly: left to the compiler, these fresh values start in VGPRs and are
            // shuffled into AGPRs later); the next MFMA on it is a k-step (kMfma MFMAs) later
            asm("v_mfma_i32_16x16x64_i8 %0, %1, %2, 0" : "=a"(acc[j][i]) : "v"(cur.w[j]), "v"(cur.x[i]));
        } else {
            acc[j][i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(cur.w[j], cur.x[i], acc[j][i], 0, 0, 0);
        }
    }
    // The DMA of one slab into one stage, issued one instruction at a time: A rows first (kADma
    // instructions), then B rows.  A plan with zero-sized buffers (no next tile) loads zeros into a
    // stage nothing reads any more, so every wave issues the same instructions either way.
    struct DmaPlan {
        __amdgpu_buffer_rsrc_t ra, rb;
        int a0, b0, kb, lda, ldb;
        int8_t *sa, *sb;
        MICA_DEVICE void issue(int d) const {
            if (d < C::kADma)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void *)(sa + d * 1024), 16, a0 + d * 8 * lda, kb, 0, 0);
            else
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void *)(sb + (d - C::kADma) * 1024), 16,
                                                         b0 + (d - C::kADma) * 8 * ldb, kb, 0, 0);
        }
    };
    // the plan for slab `slab` of tile (m0, n0) into stage `stage`; valid = false: zero-sized buffers
    MICA_DEVICE static DmaPlan tile_plan(const GemmParams &p, int8_t *smem, int wave, int lane, int m0, int n0,
                                         int slab, int stage, bool valid) {
        DmaPlan d;
        d.ra = __builtin_amdgcn_make_buffer_rsrc((void *)p.A, 0, valid ? p.M * p.lda : 0, kBufferFlags);
        d.rb = __builtin_amdgcn_make_buffer_rsrc((void *)p.B, 0, valid ? p.N * p.ldb : 0, kBufferFlags);
        d.a0 = dma_base(m0 + wave * C::kADma * 8, p.lda, lane);
        d.b0 = dma_base(n0 + wave * C::kBDma * 8, p.ldb, lane);
        d.kb = slab * QBK;
        d.lda = p.lda;
        d.ldb = p.ldb;
        d.sa = smem + stage * C::kAHalf + wave * C::kADma * 1024;
        d.sb = smem + C::kBBase + stage * C::kBHalf + wave * C::kBDma * 1024;
        return d;
    }
    // DMA instructions go out one per kDStride MFMAs: issued together after the barrier they back up
    // the address unit, and the stalled issue starves this wave's MFMA pipe (measured: 66 K -> 45 K
    // cycles per 256 x 256 x 2560 tile without any DMA in the loop)
    // (whole tiles issue all kDma in their k-step; smaller tiles, whose k-steps are shorter, issue
    // the rest early in the next one)
    static constexpr int kDStride = 4;
    static constexpr int kDFirst = (kMfma + kDStride - 1) / kDStride < C::kDma ? (kMfma + kDStride - 1) / kDStride : C::kDma;
    static_assert(C::kDma - kDFirst <= kDFirst, "DMA spread over at most two k-steps");
    template <int M, bool READ, int OFFW, int OFFX, bool FIRST, int D0>
    MICA_DEVICE void ks_body(Ops &nx, const Ops &cur, uint32_t wa, uint32_t xa, const DmaPlan &dp) {
        if constexpr (M < kMfma) {
            if constexpr (READ && M < kReads) {
                if constexpr (M < NB)
                    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(nx.w[M]) : "v"(wa), "i"(OFFW + M * 16 * QBK));
                else
                    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(nx.x[M - NB]) : "v"(xa), "i"(OFFX + (M - NB) * 16 * QBK));
            }
            // D0 < 0: no DMA in this k-step; else instructions D0, D0 + 1, ... (below the slab's kDma
            // and, in the first k-step, below kDFirst)
            if constexpr (D0 >= 0 && M % kDStride == 0 && D0 + M / kDStride < (D0 == 0 ? kDFirst : C::kDma))
                dp.issue(D0 + M / kDStride);
            mfma_one<M, FIRST>(cur);
            __builtin_amdgcn_sched_barrier(0);
            ks_body<M + 1, READ, OFFW, OFFX, FIRST, D0>(nx, cur, wa, xa, dp);
        }
    }
    // READ: the next k-step's fragments (stage ST) into nx, one ahead of each of the first kReads
    // MFMAs; D0 >= 0: the plan's instructions from D0 on, one per kDStride MFMAs
    template <bool READ, int ST, bool FIRST, int D0>
    MICA_DEVICE void kstep(Ops &nx, const Ops &cur, uint32_t wa, uint32_t xa, const DmaPlan &dp) {
        ks_body<0, READ, ST * C::kBHalf, ST * C::kAHalf, FIRST, D0>(nx, cur, wa, xa, dp);
        __builtin_amdgcn_sched_barrier(0);
    }

    // ---- slabs of tile (m0, n0) into acc.  On entry slab 0 is visible in stage 0 and slab 1 is in
    // flight into stage 1.  has_next: slab 0 of tile (m0n, n0n) goes into stage 0 once this tile's
    // last use of it is over.  The fragment loads are inline assembly (frag reads above): each k-step
    // starts with an explicit wait for the fragments it consumes.
    MICA_DEVICE void run(const GemmParams &p, int8_t *smem, __amdgpu_buffer_rsrc_t rsrc_a,
                         __amdgpu_buffer_rsrc_t rsrc_b, int wave, int m0, int n0, bool has_next, int m0n, int n0n) {
        const int lane = lane_id();
        const int wm = wave / C::WGN, wn = wave % C::WGN;
        const int r16 = lane & 15, kq = lane >> 4;
        const int nk = p.K / QBK;  // even, at least 4
        const int a0 = opaque_off(dma_base(m0 + wave * C::kADma * 8, p.lda, lane));
        const int b0 = opaque_off(dma_base(n0 + wave * C::kBDma * 8, p.ldb, lane));
        DmaPlan own{rsrc_a, rsrc_b, a0, b0, 0, p.lda, p.ldb, nullptr, nullptr};
        // fragment addresses: k-step s of row r is chunk 4 s + kq (stage and 16-row block are
        // compile-time offsets within the 16-bit offset of ds_read_b128)
        const uint32_t lds0 = lds_addr(smem);
        uint32_t xa[2], wa[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int pos = ((4 * s + kq) ^ (r16 & 7)) << 4;
            xa[s] = lds0 + (wm * WM + r16) * QBK + pos;
            wa[s] = lds0 + C::kBBase + (wn * WN + r16) * QBK + pos;
        }
        Ops R0, R1;
        // The k-steps run as A / B halves: A(k) = k-step 0 of slab k (its k-step 1 fragments read into
        // R1 alongside); B(k) = slab k + 1 landed (this wave's share) and every wave past its reads of
        // slab k: a barrier, the DMA into slab k's stage (DK: 1 = this tile's slab k + 2, 2 = the next
        // tile's slab 0), then k-step 1 of slab k with k-step 0 of slab k + 1 read into R0.
        // the DMA that half_b started, continued in the next half_a when it has more instructions
        constexpr int kDMore = C::kDma > kDFirst ? kDFirst : -1;
        DmaPlan cont = own;
        auto half_a = [&](auto st_c, auto first_c) {
            wait_lgkmcnt0();   // k-step 0's fragments (read one k-step ago) are in registers
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (decltype(first_c)::value)
                kstep<true, decltype(st_c)::value, true, -1>(R1, R0, wa[1], xa[1], own);
            else
                kstep<true, decltype(st_c)::value, false, kDMore>(R1, R0, wa[1], xa[1], cont);
        };
        auto half_b = [&](auto st_c, const DmaPlan &dp) {
            constexpr int ST = decltype(st_c)::value;
            wait_vmcnt<0>();   // slab k + 1 landed (this wave's share)
            wait_lgkmcnt0();   // k-step 1's fragments are in registers
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            cont = dp;
            kstep<true, ST ^ 1, false, 0>(R0, R1, wa[0], xa[0], dp);
        };
        // the DMA of this tile's slab `slab` into its stage
        auto own_plan = [&](int slab) {
            DmaPlan d = own;
            d.kb = slab * QBK;
            d.sa = smem + (slab & 1) * C::kAHalf + wave * C::kADma * 1024;
            d.sb = smem + C::kBBase + (slab & 1) * C::kBHalf + wave * C::kBDma * 1024;
            return d;
        };
        using T = std::integral_constant<bool, true>;
        using F = std::integral_constant<bool, false>;
        using S0 = std::integral_constant<int, 0>;
        using S1 = std::integral_constant<int, 1>;
        frag_reads<0, NB>(R0.w, wa[0]);
        frag_reads<0, MB>(R0.x, xa[0]);
        half_a(S0{}, T{});
        int k = 0;
        for (; k + 4 <= nk; k += 2) {
            half_b(S0{}, own_plan(k + 2));
            half_a(S1{}, F{});
            half_b(S1{}, own_plan(k + 3));
            half_a(S0{}, F{});
        }
        // k = nk - 2: slab nk - 2's stage takes the next tile's slab 0 (zeros without a next tile)
        half_b(S0{}, tile_plan(p, smem, wave, lane, m0n, n0n, 0, 0, has_next));
        half_a(S1{}, F{});
        wait_lgkmcnt0();
        __builtin_amdgcn_sched_barrier(0);
        kstep<false, 0, false, -1>(R0, R1, wa[0], xa[0], own);
    }

    // ---- slabs ks0 .. ks0 + nk - 1 of a piece with no successor to prefetch for (C::NS >= 3 stages; nk
    // at least NS): on entry the range's slab 0 is visible in stage 0 and its slabs 1 .. NS - 1 are in
    // flight into stages 1 .. NS - 1.  Slab s of the range lives in stage s % NS; after the barrier of
    // B(k) (slab k + 1 landed, slab k read by every wave) slab k + NS goes into slab k's stage, so NS - 1
    // slabs are in flight while one is read.  Stage offsets beyond the 16-bit offset of ds_read_b128
    // ride on the base registers.
    MICA_DEVICE void run_deep(const GemmParams &p, int8_t *smem, int wave, int m0, int n0, int ks0, int nk) {
        constexpr int NS = C::NS;
        static_assert(NS == 3 || NS == 4, "stages");
        static_assert((NS - 2) * C::kDma < 64, "vmcnt");
        const int lane = lane_id();
        const int wm = wave / C::WGN, wn = wave % C::WGN;
        const int r16 = lane & 15, kq = lane >> 4;
        const uint32_t lds0 = lds_addr(smem);
        uint32_t xa[2], wa[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const int pos = ((4 * s + kq) ^ (r16 & 7)) << 4;
            xa[s] = lds0 + (wm * WM + r16) * QBK + pos;
            wa[s] = lds0 + C::kBBase + (wn * WN + r16) * QBK + pos;
        }
        constexpr int kDMore = C::kDma > kDFirst ? kDFirst : -1;
        Ops R0, R1;
        DmaPlan cont = tile_plan(p, smem, wave, lane, m0, n0, 0, 0, false);
        // the plan for slab `slab` (stage ST = slab % NS): zero-sized past the last slab, so every wave
        // issues the same instructions and the waits below count them
        auto plan = [&](int slab, auto st_c) {
            return tile_plan(p, smem, wave, lane, m0, n0, ks0 + slab, decltype(st_c)::value, slab < nk);
        };
        // A: k-step 0 of the slab in stage ST (in R0), its k-step 1 read into R1
        auto half_a = [&](auto st_c, auto first_c) {
            constexpr int ST = decltype(st_c)::value;
            wait_lgkmcnt0();
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (decltype(first_c)::value)
                kstep<true, 0, true, -1>(R1, R0, wa[1] + ST * C::kBHalf, xa[1] + ST * C::kAHalf, cont);
            else
                kstep<true, 0, false, kDMore>(R1, R0, wa[1] + ST * C::kBHalf, xa[1] + ST * C::kAHalf, cont);
        };
        // B: slab k + 1 (stage ST + 1) landed -- only the NS - 2 slabs after it may be in flight
        auto half_b = [&](auto st_c, const DmaPlan &dp) {
            constexpr int ST = decltype(st_c)::value;
            constexpr int SN = (ST + 1) % NS;
            wait_vmcnt<(NS - 2) * C::kDma>();
            wait_lgkmcnt0();
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            cont = dp;
            kstep<true, 0, false, 0>(R0, R1, wa[0] + SN * C::kBHalf, xa[0] + SN * C::kAHalf, dp);
        };
        using T = std::integral_constant<bool, true>;
        using F = std::integral_constant<bool, false>;
        using S0 = std::integral_constant<int, 0>;
        using S1 = std::integral_constant<int, 1>;
        using S2 = std::integral_constant<int, 2>;
        using S3 = std::integral_constant<int, NS - 1>;   // stage 3 (NS == 4)
        frag_reads<0, NB>(R0.w, wa[0]);
        frag_reads<0, MB>(R0.x, xa[0]);
        half_a(S0{}, T{});
        int k = 0;
        for (; k + NS <= nk - 1; k += NS) {
            half_b(S0{}, plan(k + NS, S0{}));
            half_a(S1{}, F{});
            half_b(S1{}, plan(k + NS + 1, S1{}));
            half_a(S2{}, F{});
            if constexpr (NS == 3) {
                half_b(S2{}, plan(k + 5, S2{}));
                half_a(S0{}, F{});
            } else {
                half_b(S2{}, plan(k + 6, S2{}));
                half_a(S3{}, F{});
                half_b(S3{}, plan(k + 7, S3{}));
                half_a(S0{}, F{});
            }
        }
        // the last nk - 1 - k (0 to NS - 1) pairs, from stage 0
        if (k + 1 <= nk - 1) {
            half_b(S0{}, plan(k + NS, S0{}));
            half_a(S1{}, F{});
        }
        if (k + 2 <= nk - 1) {
            half_b(S1{}, plan(k + NS + 1, S1{}));
            half_a(S2{}, F{});
        }
        if constexpr (NS == 4) {
            if (k + 3 <= nk - 1) {
                half_b(S2{}, plan(k + 6, S2{}));
                half_a(S3{}, F{});
            }
        }
        wait_lgkmcnt0();
        __builtin_amdgcn_sched_barrier(0);
        kstep<false, 0, false, -1>(R0, R1, wa[0], xa[0], cont);
    }

    // 16 bytes of one output row from MFMA tiles ja and ja + 1 of row block i: lanes of rows kq, kq ^ 1
    // exchange their halves (v_permlane16_swap swaps the odd 16-lane rows of the first operand with the
    // even rows of the second), so lane (r16, kq) ends with columns 16 (ja + kq % 2) + 8 (kq / 2) + 0..7
    // of row 16 i + r16.
    MICA_DEVICE static u32x4 pair16(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1) {
        const auto s0 = __builtin_amdgcn_permlane16_swap(a0, b0, false, false);
        const auto s1 = __builtin_amdgcn_permlane16_swap(a1, b1, false, false);
        return u32x4{s0[0], s1[0], s0[1], s1[1]};
    }
    MICA_DEVICE static uint32_t pack2(float lo, float hi) {
        if (OUT == MICA_BF16) return pack_bf16x2(lo, hi);
        return (uint32_t)f32_to_f16(lo) | ((uint32_t)f32_to_f16(hi) << 16);
    }
    MICA_DEVICE static uint32_t add2(uint32_t v, uint32_t r) {
        if (OUT == MICA_BF16) return pack_bf16x2(bf16_lo(v) + bf16_lo(r), bf16_hi(v) + bf16_hi(r));
        const float a0 = f16_to_f32(v & 0xffff), a1 = f16_to_f32(v >> 16);
        const float b0 = f16_to_f32(r & 0xffff), b1 = f16_to_f32(r >> 16);
        return (uint32_t)f32_to_f16(a0 + b0) | ((uint32_t)f32_to_f16(a1 + b1) << 16);
    }

    // ---- a tile split along K over `parts` workgroups (gemm_i8_agpr_split_kernel), this one being part
    // `part`: its int32 accumulators go to its slot t * parts + part of p.partials (slot = int32x4 vector
    // v of thread x at (v * kQThreads + x) * 16), then it counts itself in p.arrivals[t].  The part that
    // arrives last adds the other parts' slots to its accumulators, re-zeroes the count for the next
    // launch and returns true (it runs the epilogue); the others return false.  Integer sums are exact
    // in any order.  Slots move with device-scope (sc1) buffer stores and loads, written through to the
    // device's coherence point and read from it; the count is a device-scope atomic taken after every
    // wave's stores were acknowledged (vmcnt 0, then a workgroup barrier).  Nobody waits for another
    // workgroup, so no co-residency is assumed.
    static constexpr int kSlotVecs = NB * MB;
    MICA_DEVICE bool split_fixup(const GemmParams &p, int8_t *smem, int t, int part, int parts) {
        constexpr int kDeviceScope = 16;  // cache policy bits: sc1
        const int tid = threadIdx.x;
        const __amdgpu_buffer_rsrc_t rsrc_p = __builtin_amdgcn_make_buffer_rsrc(
            (void *)p.partials, 0, p.sk_grid * kSlotVecs * kQThreads * 16, kBufferFlags);
        auto off = [&](int slot, int v) { return ((slot * kSlotVecs + v) * kQThreads + tid) * 16; };
        const int mine = t * parts + part;
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int i = 0; i < MB; ++i)
                __builtin_amdgcn_raw_buffer_store_b128(acc[j][i], rsrc_p, off(mine, j * MB + i), 0, kDeviceScope);
        wait_vmcnt<0>();   // this wave's partial sums reached the coherence point ...
        __syncthreads();   // ... and every wave's, before the arrival is counted
        int *flag = (int *)(smem + kQScale + kQScaleBuf);  // the second scale buffer (unused by a split tile)
        if (tid == 0) *flag = __hip_atomic_fetch_add(p.arrivals + t, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (*flag != parts - 1) return false;  // a later part finishes the tile
        // each read-back is a round trip to the coherence point: a whole chunk of a slot's vectors goes
        // out before any is added (left to the compiler, the loads of a slot went out a few at a time)
        constexpr int kChunk = kSlotVecs <= 20 ? kSlotVecs : kSlotVecs / 2;
        static_assert(kSlotVecs % kChunk == 0, "chunks");
        for (int o = 0; o < parts; ++o) {
            if (o == part) continue;
            const int slot = t * parts + o;
#pragma unroll
            for (int c = 0; c < kSlotVecs; c += kChunk) {
                v4i buf[kChunk];
#pragma unroll
                for (int v = 0; v < kChunk; ++v)
                    buf[v] = __builtin_amdgcn_raw_buffer_load_b128(rsrc_p, off(slot, c + v), 0, kDeviceScope);
#pragma unroll
                for (int v = 0; v < kChunk; ++v) acc[(c + v) / MB][(c + v) % MB] += buf[v];
            }
        }
        if (tid == 0) __hip_atomic_store(p.arrivals + t, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return true;
    }

    // ---- epilogue of tile (m0, n0) from acc, with its scales in buffer buf.  With has_next, the next
    // tile's scales go to buffer buf ^ 1 and its slab 1 into stage 1.  Vector memory operations in
    // issue order: next scales, [res(0), res(1)], next slab 1, then per row block i the stores st(i)
    // and [res(i + 2)]; every residual wait counts exactly what was issued after it.
    MICA_DEVICE void epilogue(const GemmParams &p, int8_t *smem, __amdgpu_buffer_rsrc_t rsrc_a,
                              __amdgpu_buffer_rsrc_t rsrc_b, int wave, int m0, int n0, int buf, bool has_next,
                              int m0n, int n0n) {
        const int lane = lane_id();
        const int wm = wave / C::WGN, wn = wave % C::WGN;
        const int r16 = lane & 15, kq = lane >> 4;
        const float *sc = (const float *)(smem + kQScale + buf * kQScaleBuf);  // sa, sb, bias
        // nothing of the epilogue moves up into the last k-steps (its registers would not fit there)
        asm volatile("" ::: "memory");
        // every wave has read the last slab from stage 1: the next tile's slab 1 may overwrite it
        wait_lgkmcnt0();
        __builtin_amdgcn_s_barrier();
        if (has_next) scales_dma(p, smem, wave, buf ^ 1, m0n, n0n);
        const int ncols_out = EPI == MICA_EPI_SCALE ? p.N : (p.N >> 1);
        const int col0 = EPI == MICA_EPI_SCALE ? n0 + wn * WN : (n0 >> 1) + wn * (WN / 2);
        const int rows_in = p.M - m0 < C::BM ? p.M - m0 : C::BM;  // valid rows of this tile
        // this lane's output column (tile-local to the wave) in store jp, and whether it is in range
        auto col_of = [&](int jp) { return (2 * jp + (kq & 1)) * 16 + (kq >> 1) * 8; };
        auto row_of = [&](int i) { return wm * WM + i * 16 + r16; };  // tile-local row
        // (built for every variant; without a residual it is never used)
        const __amdgpu_buffer_rsrc_t rsrc_r = __builtin_amdgcn_make_buffer_rsrc(
            (void *)((const uint16_t *)p.res + (long)m0 * p.ldr), 0, rows_in * p.ldr * 2, kBufferFlags);
        u32x4 rv[MB][kS];
        auto res_load = [&](int i) {
#pragma unroll
            for (int jp = 0; jp < kS; ++jp) {
                const int col = col0 + col_of(jp);
                const int off = opaque_off(col < ncols_out ? (row_of(i) * p.ldr + col) * 2 : kOutOfRange);
                rv[i][jp] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc_r, off, 0, 0));
            }
        };
        if constexpr (HAS_RES) {
            res_load(0);
            res_load(1);
        }
        // the next tile's slab 1: with a residual at once (its waits count it), else spread over the
        // row blocks so the VALU stream never waits for the address unit
        if constexpr (HAS_RES) {
            if (has_next) tile_dma(p, smem, rsrc_a, rsrc_b, wave, m0n, n0n, 1, 1);
        }
        const DmaPlan slab1 = tile_plan(p, smem, wave, lane, m0n, n0n, 1, 1, has_next);
        const __amdgpu_buffer_rsrc_t rsrc_c = __builtin_amdgcn_make_buffer_rsrc(
            (void *)((uint16_t *)p.C + (long)m0 * p.ldc), 0, rows_in * p.ldc * 2, kBufferFlags);
        // this lane's scales: sa of its rows, sb (SiLU: of the gate and the up rows) and the bias of
        // its 4 columns in each output tile, read once per tile
        float sav[MB];
#pragma unroll
        for (int i = 0; i < MB; ++i) sav[i] = sc[row_of(i)];
        v4f s1v[kOutTiles], s2v[EPI == MICA_EPI_SCALE ? 1 : kOutTiles], bvv[HAS_BIAS ? kOutTiles : 1];
#pragma unroll
        for (int j = 0; j < kOutTiles; ++j) {
            const int cb = wn * WN + j * 16 + 4 * kq;  // tile-local weight row of this lane's values
            s1v[j] = *(const v4f *)(sc + 256 + cb);
            if constexpr (EPI != MICA_EPI_SCALE) s2v[j] = *(const v4f *)(sc + 256 + cb + WN / 2);
            if constexpr (HAS_BIAS) bvv[j] = *(const v4f *)(sc + 512 + cb);
        }
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            if constexpr (!HAS_RES) {
#pragma unroll
                for (int d = i * C::kDma / MB; d < (i + 1) * C::kDma / MB; ++d)
                    if (has_next) slab1.issue(d);
            }
            u32x4 outv[kS];
#pragma unroll
            for (int jp = 0; jp < kS; ++jp) {
                uint32_t pk[2][2];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int j = 2 * jp + h;            // output tile (SiLU: the gate tile)
                    const v4f s1 = s1v[j];
                    v4f s2 = {}, bv = {};
                    if constexpr (EPI != MICA_EPI_SCALE) s2 = s2v[j];
                    if constexpr (HAS_BIAS) bv = bvv[j];
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
                    pk[h][0] = pack2(y[0], y[1]);
                    pk[h][1] = pack2(y[2], y[3]);
                }
                outv[jp] = pair16(pk[0][0], pk[0][1], pk[1][0], pk[1][1]);
            }
            if constexpr (HAS_RES) {
                // res(i) landed: count what was issued after it
                if (i == 0) {
                    if (has_next) wait_vmcnt<kS + C::kDma>();
                    else wait_vmcnt<kS>();
                } else if (i == 1) {
                    constexpr int after = kS + (MB > 2 ? kS : 0);  // st(0) [+ res(2)]
                    if (has_next) wait_vmcnt<C::kDma + after>();   // [slab 1] issued before st(0)
                    else wait_vmcnt<after>();
                } else {
                    if (i + 1 < MB) wait_vmcnt<2 * kS>();  // st(i - 1), res(i + 1)
                    else wait_vmcnt<kS>();                 // st(i - 1)
                }
#pragma unroll
                for (int jp = 0; jp < kS; ++jp)
#pragma unroll
                    for (int t = 0; t < 4; ++t) outv[jp][t] = add2(outv[jp][t], rv[i][jp][t]);
            }
#pragma unroll
            for (int jp = 0; jp < kS; ++jp) {
                const int col = col0 + col_of(jp);
                const int off = opaque_off(col < ncols_out ? (row_of(i) * p.ldc + col) * 2 : kOutOfRange);
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4i, outv[jp]), rsrc_c, off, 0, C::CPOL);
            }
            if constexpr (HAS_RES) {
                if (i + 2 < MB) res_load(i + 2);
            }
        }
    }
};

// The pieces h = h0, h0 + G, ... < hend of one schedule phase (all of one tile shape C), on this
// workgroup; piece(h, m0, n0) gives a piece's origin, false for a piece wholly past the edge.
template <class C, int EPI, int OUT, bool HAS_BIAS, bool HAS_RES, class Piece>
MICA_DEVICE void run_qphase(const GemmParams &p, int8_t *smem, __amdgpu_buffer_rsrc_t rsrc_a,
                            __amdgpu_buffer_rsrc_t rsrc_b, int wave, int h0, int hend, int G, Piece piece) {
    using Tile = QTile<C, EPI, OUT, HAS_BIAS, HAS_RES>;
    int h = h0, m0 = 0, n0 = 0;
    while (h < hend && !piece(h, m0, n0)) h += G;
    if (h >= hend) return;
    Tile t;
    if constexpr (C::NS >= 3) {
        // pieces with no successor, each on its own: slabs 0 .. NS - 1 out, slab 0 and the scales
        // waited for
        for (; h < hend; h += G) {
            if (!piece(h, m0, n0)) continue;
            wait_vmcnt<0>();
            wait_lgkmcnt0();
            __builtin_amdgcn_s_barrier();
            Tile::scales_dma(p, smem, wave, 0, m0, n0);
            Tile::tile_dma(p, smem, rsrc_a, rsrc_b, wave, m0, n0, 0, 0);
            Tile::tile_dma(p, smem, rsrc_a, rsrc_b, wave, m0, n0, 1, 1);
            Tile::tile_dma(p, smem, rsrc_a, rsrc_b, wave, m0, n0, 2, 2);
            if constexpr (C::NS > 3) Tile::tile_dma(p, smem, rsrc_a, rsrc_b, wave, m0, n0, 3, 3);
            wait_vmcnt<(C::NS - 1) * C::kDma>();  // scales and slab 0 landed (slabs 1 .. NS - 1 may be in flight)
            __builtin_amdgcn_s_barrier();
            t.run_deep(p, smem, wave, m0, n0, 0, p.K / QBK);
            t.epilogue(p, smem, rsrc_a, rsrc_b, wave, m0, n0, 0, false, 0, 0);
        }
        return;
    }
    // the previous phase's last epilogue is finished with the stages and the scales
    wait_vmcnt<0>();
    wait_lgkmcnt0();
    __builtin_amdgcn_s_barrier();
    Tile::scales_dma(p, smem, wave, 0, m0, n0);
    Tile::tile_dma(p, smem, rsrc_a, rsrc_b, wave, m0, n0, 0, 0);
    Tile::tile_dma(p, smem, rsrc_a, rsrc_b, wave, m0, n0, 1, 1);
    wait_vmcnt<C::kDma>();  // scales and slab 0 landed (slab 1 may be in flight)
    __builtin_amdgcn_s_barrier();
    int buf = 0;
    for (;;) {
        int hn = h + G, m0n = 0, n0n = 0;
        while (hn < hend && !piece(hn, m0n, n0n)) hn += G;
        const bool has_next = hn < hend;
        t.run(p, smem, rsrc_a, rsrc_b, wave, m0, n0, has_next, m0n, n0n);
        t.epilogue(p, smem, rsrc_a, rsrc_b, wave, m0, n0, buf, has_next, m0n, n0n);
        if (!has_next) break;
        // the next tile's slab 0 and scales landed: at most its slab 1 and this epilogue's stores
        // (and residual loads, all waited for) were issued after them
        wait_vmcnt<C::kDma + Tile::kStores>();
        __builtin_amdgcn_s_barrier();
        buf ^= 1;
        h = hn;
        m0 = m0n;
        n0 = n0n;
    }
}

template <int EPI, int OUT, bool HAS_BIAS, bool HAS_RES>
__global__ __launch_bounds__(kQThreads, 1) void gemm_i8_agpr_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(1024))) int8_t smem[kQSmem];
    const int G = gridDim.x;
    const __amdgpu_buffer_rsrc_t rsrc_a = __builtin_amdgcn_make_buffer_rsrc((void *)p.A, 0, p.M * p.lda, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rsrc_b = __builtin_amdgcn_make_buffer_rsrc((void *)p.B, 0, p.N * p.ldb, kBufferFlags);
    const int tm_n = p.tiles_m, tn_n = p.tiles_n, dp = p.dp_tiles, M = p.M, N = p.N;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    run_qphase<QFull, EPI, OUT, HAS_BIAS, HAS_RES>(p, smem, rsrc_a, rsrc_b, wave, blockIdx.x, dp, G,
                                                   [&](int h, int &m0, int &n0) {
                                                       int tm, tn;
                                                       tile_of(h, tm_n, tn_n, tm, tn);
                                                       m0 = tm * 256;
                                                       n0 = tn * 256;
                                                       return true;
                                                   });
    if constexpr (EPI == MICA_EPI_SCALE) {
        if (p.half_tiles > 0)
            run_qphase<QHalfN, EPI, OUT, HAS_BIAS, HAS_RES>(p, smem, rsrc_a, rsrc_b, wave, blockIdx.x, 2 * p.half_tiles, G,
                                                            [&](int h, int &m0, int &n0) {
                                                                int tm, tn, t, part;
                                                                tail_piece(h, 2, dp, p.half_tiles, t, part);
                                                                tile_of(t, tm_n, tn_n, tm, tn);
                                                                m0 = tm * 256;
                                                                n0 = tn * 256 + part * 128;
                                                                return n0 < N;
                                                            });
        if (p.quarter_tiles > 0)
            run_qphase<QQuart, EPI, OUT, HAS_BIAS, HAS_RES>(p, smem, rsrc_a, rsrc_b, wave, blockIdx.x, 4 * p.quarter_tiles, G,
                                                            [&](int h, int &m0, int &n0) {
                                                                int tm, tn, t, part;
                                                                tail_piece(h, 4, dp, p.quarter_tiles, t, part);
                                                                tile_of(t, tm_n, tn_n, tm, tn);
                                                                m0 = tm * 256 + ((part >> 1) & 1) * 128;
                                                                n0 = tn * 256 + (part & 1) * 128;
                                                                return m0 < M && n0 < N;
                                                            });
    } else {
        if (p.mhalf_tiles > 0)
            run_qphase<QHalfM, EPI, OUT, HAS_BIAS, HAS_RES>(p, smem, rsrc_a, rsrc_b, wave, blockIdx.x, 2 * p.mhalf_tiles, G,
                                                            [&](int h, int &m0, int &n0) {
                                                                int tm, tn, t, part;
                                                                tail_piece(h, 2, dp, p.mhalf_tiles, t, part);
                                                                tile_of(t, tm_n, tn_n, tm, tn);
                                                                m0 = tm * 256 + part * 128;
                                                                n0 = tn * 256;
                                                                return m0 < M;
                                                            });
    }
    // every store of this workgroup has left before the waves end
    wait_vmcnt<0>();
}

// One round of 256 x 160 tiles (dp_tiles of them over tiles_m x tiles_n, one per workgroup), SCALE
// epilogue.
template <int OUT, bool HAS_BIAS, bool HAS_RES>
__global__ __launch_bounds__(kQThreads, 1) void gemm_i8_agpr_narrow_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(1024))) int8_t smem[kQSmem];
    const __amdgpu_buffer_rsrc_t rsrc_a = __builtin_amdgcn_make_buffer_rsrc((void *)p.A, 0, p.M * p.lda, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rsrc_b = __builtin_amdgcn_make_buffer_rsrc((void *)p.B, 0, p.N * p.ldb, kBufferFlags);
    const int tm_n = p.tiles_m, tn_n = p.tiles_n;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    run_qphase<QNarrow, MICA_EPI_SCALE, OUT, HAS_BIAS, HAS_RES>(p, smem, rsrc_a, rsrc_b, wave, blockIdx.x, p.dp_tiles,
                                                               gridDim.x, [&](int h, int &m0, int &n0) {
                                                                   int tm, tn;
                                                                   tile_of(h, tm_n, tn_n, tm, tn);
                                                                   m0 = tm * 256;
                                                                   n0 = tn * 160;
                                                                   return true;
                                                               });
    // every store of this workgroup has left before the waves end
    wait_vmcnt<0>();
}

// One round of 128 x 160 tiles (dp_tiles of them over tiles_m x tiles_n, one per workgroup), SCALE
// epilogue.
template <int OUT, bool HAS_BIAS, bool HAS_RES>
__global__ __launch_bounds__(kQThreads, 1) void gemm_i8_agpr_small_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(1024))) int8_t smem[kQSmem];
    const __amdgpu_buffer_rsrc_t rsrc_a = __builtin_amdgcn_make_buffer_rsrc((void *)p.A, 0, p.M * p.lda, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rsrc_b = __builtin_amdgcn_make_buffer_rsrc((void *)p.B, 0, p.N * p.ldb, kBufferFlags);
    const int tm_n = p.tiles_m, tn_n = p.tiles_n;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    run_qphase<QSmall, MICA_EPI_SCALE, OUT, HAS_BIAS, HAS_RES>(p, smem, rsrc_a, rsrc_b, wave, blockIdx.x, p.dp_tiles,
                                                              gridDim.x, [&](int h, int &m0, int &n0) {
                                                                  int tm, tn;
                                                                  tile_of(h, tm_n, tn_n, tm, tn);
                                                                  m0 = tm * QSmall::BM;
                                                                  n0 = tn * QSmall::BN;
                                                                  return true;
                                                              });
    // every store of this workgroup has left before the waves end
    wait_vmcnt<0>();
}

// One round of 128 x 128 tiles (dp_tiles of them over tiles_m x tiles_n, one per workgroup), SiLU
// epilogue (bf16 out).
__global__ __launch_bounds__(kQThreads, 1) void gemm_i8_agpr_silu_small_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(1024))) int8_t smem[kQSmem];
    const __amdgpu_buffer_rsrc_t rsrc_a = __builtin_amdgcn_make_buffer_rsrc((void *)p.A, 0, p.M * p.lda, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rsrc_b = __builtin_amdgcn_make_buffer_rsrc((void *)p.B, 0, p.N * p.ldb, kBufferFlags);
    const int tm_n = p.tiles_m, tn_n = p.tiles_n;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    run_qphase<QSiluSmall, MICA_EPI_SILU_MUL, MICA_BF16, false, false>(
        p, smem, rsrc_a, rsrc_b, wave, blockIdx.x, p.dp_tiles, gridDim.x, [&](int h, int &m0, int &n0) {
            int tm, tn;
            tile_of(h, tm_n, tn_n, tm, tn);
            m0 = tm * QSiluSmall::BM;
            n0 = tn * QSiluSmall::BN;
            return true;
        });
    // every store of this workgroup has left before the waves end
    wait_vmcnt<0>();
}

// One round of tiles split along K (few tiles and a long K, e.g. a short request's projections):
// p.sk_tiles tiles of 128 x 160 (SiLU: 128 x 256) over tiles_m x tiles_n (M-major), each in
// parts = sk_grid / sk_tiles pieces of K.  Workgroup g is part g % parts of tile g / parts and runs
// slabs [part nk / parts, (part + 1) nk / parts) of the nk 128-byte slabs (at least 4 of them; the
// launcher checks), then split_fixup; the last part of each tile runs the epilogue.
template <int EPI, int OUT, bool HAS_BIAS, bool HAS_RES>
__global__ __launch_bounds__(kQThreads, 1) void gemm_i8_agpr_split_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(1024))) int8_t smem[kQSmem];
    using C = std::conditional_t<EPI == MICA_EPI_SILU_MUL, QHalfM, QSmall>;
    using Tile = QTile<C, EPI, OUT, HAS_BIAS, HAS_RES>;
    const __amdgpu_buffer_rsrc_t rsrc_a = __builtin_amdgcn_make_buffer_rsrc((void *)p.A, 0, p.M * p.lda, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rsrc_b = __builtin_amdgcn_make_buffer_rsrc((void *)p.B, 0, p.N * p.ldb, kBufferFlags);
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int parts = p.sk_grid / p.sk_tiles;
    const int t = (int)blockIdx.x / parts, part = (int)blockIdx.x - t * parts;
    const int m0 = (t % p.tiles_m) * C::BM, n0 = (t / p.tiles_m) * C::BN;
    const int nk = p.K / QBK;
    const int k0 = part * nk / parts, k1 = (part + 1) * nk / parts;
    Tile tile;
    Tile::scales_dma(p, smem, wave, 0, m0, n0);
#pragma unroll
    for (int s = 0; s < C::NS; ++s) Tile::tile_dma(p, smem, rsrc_a, rsrc_b, wave, m0, n0, k0 + s, s);
    wait_vmcnt<(C::NS - 1) * C::kDma>();  // scales and slab k0 landed (the next NS - 1 may be in flight)
    __builtin_amdgcn_s_barrier();
    tile.run_deep(p, smem, wave, m0, n0, k0, k1 - k0);
    if (tile.split_fixup(p, smem, t, part, parts))
        tile.epilogue(p, smem, rsrc_a, rsrc_b, wave, m0, n0, 0, false, 0, 0);
    // every store of this workgroup has left before the waves end
    wait_vmcnt<0>();
}

// Explicit instantiations: hipcc's host pass left the launch stubs of the variants without a residual
// undefined when they were only instantiated implicitly by the launches below.
template __global__ void gemm_i8_agpr_split_kernel<MICA_EPI_SILU_MUL, MICA_BF16, false, false>(GemmParams);
template __global__ void gemm_i8_agpr_split_kernel<MICA_EPI_SCALE, MICA_BF16, false, false>(GemmParams);
template __global__ void gemm_i8_agpr_split_kernel<MICA_EPI_SCALE, MICA_BF16, true, false>(GemmParams);
template __global__ void gemm_i8_agpr_split_kernel<MICA_EPI_SCALE, MICA_BF16, false, true>(GemmParams);
template __global__ void gemm_i8_agpr_split_kernel<MICA_EPI_SCALE, MICA_BF16, true, true>(GemmParams);
template __global__ void gemm_i8_agpr_split_kernel<MICA_EPI_SCALE, MICA_FP16, false, false>(GemmParams);
template __global__ void gemm_i8_agpr_split_kernel<MICA_EPI_SCALE, MICA_FP16, true, false>(GemmParams);
template __global__ void gemm_i8_agpr_split_kernel<MICA_EPI_SCALE, MICA_FP16, false, true>(GemmParams);
template __global__ void gemm_i8_agpr_split_kernel<MICA_EPI_SCALE, MICA_FP16, true, true>(GemmParams);

template <int EPI, int OUT>
int agpr_split_out(const GemmParams &p, bool has_bias, bool has_res, hipStream_t st) {
    dim3 g(p.sk_grid), b(kQThreads);
#define MICA_QX(B_, R_) hipLaunchKernelGGL((gemm_i8_agpr_split_kernel<EPI, OUT, B_, R_>), g, b, 0, st, p)
    if constexpr (EPI == MICA_EPI_SILU_MUL) {
        MICA_QX(false, false);
    } else {
        if (has_bias && has_res) MICA_QX(true, true);
        else if (has_bias) MICA_QX(true, false);
        else if (has_res) MICA_QX(false, true);
        else MICA_QX(false, false);
    }
#undef MICA_QX
    return mica_err(hipGetLastError());
}

template <int OUT>
int agpr_small_out(const GemmParams &p, int grid, bool has_bias, bool has_res, hipStream_t st) {
    dim3 g(grid), b(kQThreads);
#define MICA_QS(B_, R_) hipLaunchKernelGGL((gemm_i8_agpr_small_kernel<OUT, B_, R_>), g, b, 0, st, p)
    if (has_bias && has_res) MICA_QS(true, true);
    else if (has_bias) MICA_QS(true, false);
    else if (has_res) MICA_QS(false, true);
    else MICA_QS(false, false);
#undef MICA_QS
    return mica_err(hipGetLastError());
}

template <int OUT>
int agpr_narrow_out(const GemmParams &p, int grid, bool has_bias, bool has_res, hipStream_t st) {
    dim3 g(grid), b(kQThreads);
#define MICA_QN(B_, R_) hipLaunchKernelGGL((gemm_i8_agpr_narrow_kernel<OUT, B_, R_>), g, b, 0, st, p)
    if (has_bias && has_res) MICA_QN(true, true);
    else if (has_bias) MICA_QN(true, false);
    else if (has_res) MICA_QN(false, true);
    else MICA_QN(false, false);
#undef MICA_QN
    return mica_err(hipGetLastError());
}

template <int EPI, int OUT>
int agpr_launch_out(const GemmParams &p, int grid, bool has_bias, bool has_res, hipStream_t st) {
    dim3 g(grid), b(kQThreads);
#define MICA_Q(B_, R_) hipLaunchKernelGGL((gemm_i8_agpr_kernel<EPI, OUT, B_, R_>), g, b, 0, st, p)
    if constexpr (EPI == MICA_EPI_SILU_MUL) {
        MICA_Q(false, false);
    } else {
        if (has_bias && has_res) MICA_Q(true, true);
        else if (has_bias) MICA_Q(true, false);
        else if (has_res) MICA_Q(false, true);
        else MICA_Q(false, false);
    }
#undef MICA_Q
    return mica_err(hipGetLastError());
}

}  // namespace

// Launch of the AGPR kernel for the schedule in p (dp_tiles whole tiles, then half_tiles, quarter_tiles
// or mhalf_tiles as pieces; no split).  Called by mica_mm_i8 after its checks, only for K % 256 == 0,
// 16-bit outputs whose rows (and the residual's) are whole 16-byte units (ldc, ldr and the output width
// multiples of 8), and row pitches whose 256-row tile spans stay below 2^31 bytes.
int mica_gemm::agpr_launch(const GemmParams &p, int epilogue, int out_dtype, int grid, bool has_bias, bool has_res,
                           hipStream_t st) {
    if (epilogue == MICA_EPI_SILU_MUL) {
        if (out_dtype != MICA_BF16 || has_bias || has_res) return MICA_MISS_ARG;
        return agpr_launch_out<MICA_EPI_SILU_MUL, MICA_BF16>(p, grid, false, false, st);
    }
    if (out_dtype == MICA_BF16) return agpr_launch_out<MICA_EPI_SCALE, MICA_BF16>(p, grid, has_bias, has_res, st);
    if (out_dtype == MICA_FP16) return agpr_launch_out<MICA_EPI_SCALE, MICA_FP16>(p, grid, has_bias, has_res, st);
    return MICA_MISS_ARG;
}

// Launch of the 256 x 160 AGPR kernel for one round of tiles (p.tiles_n counts 160-column tiles; SCALE
// epilogue, 16-bit outputs; the same conditions as agpr_launch, and (N + 160) * ldb below 2^31).
int mica_gemm::agpr_narrow_launch(const GemmParams &p, int out_dtype, int grid, bool has_bias, bool has_res,
                                  hipStream_t st) {
    if (out_dtype == MICA_BF16) return agpr_narrow_out<MICA_BF16>(p, grid, has_bias, has_res, st);
    if (out_dtype == MICA_FP16) return agpr_narrow_out<MICA_FP16>(p, grid, has_bias, has_res, st);
    return MICA_MISS_ARG;
}

// Launch of the 128 x 160 AGPR kernel for one round of tiles (p.tiles_m / p.tiles_n count 128-row /
// 160-column tiles; SCALE epilogue, 16-bit outputs; the same conditions as agpr_launch).
int mica_gemm::agpr_small_launch(const GemmParams &p, int out_dtype, int grid, bool has_bias, bool has_res,
                                 hipStream_t st) {
    if (out_dtype == MICA_BF16) return agpr_small_out<MICA_BF16>(p, grid, has_bias, has_res, st);
    if (out_dtype == MICA_FP16) return agpr_small_out<MICA_FP16>(p, grid, has_bias, has_res, st);
    return MICA_MISS_ARG;
}

// Launch of the 128 x 128 SiLU kernel for one round of tiles (p.tiles_m / p.tiles_n count 128-row /
// 128-column tiles of the gate / up weight rows; bf16 output; the same conditions as agpr_launch).
int mica_gemm::agpr_silu_small_launch(const GemmParams &p, int grid, hipStream_t st) {
    hipLaunchKernelGGL(gemm_i8_agpr_silu_small_kernel, dim3(grid), dim3(kQThreads), 0, st, p);
    return mica_err(hipGetLastError());
}

// Tile shape of the split schedule: 128 x 160 for the SCALE epilogue, 128 x 256 for SiLU (whose waves
// need 128 columns of gate / up pairs).
int mica_gemm::agpr_split_tile_n(int epilogue) { return epilogue == MICA_EPI_SILU_MUL ? QHalfM::BN : QSmall::BN; }
// Bytes of one part's slot of partial sums.
long long mica_gemm::agpr_split_slot_bytes(int epilogue) {
    return epilogue == MICA_EPI_SILU_MUL ? (long long)QHalfM::MB * QHalfM::NB * kQThreads * 16
                                         : (long long)QSmall::MB * QSmall::NB * kQThreads * 16;
}
static_assert(QSmall::BM == 128 && QHalfM::BM == 128, "split tiles are 128 rows");

// Launch of the split schedule in p (tiles_m x tiles_n tiles of 128 x agpr_split_tile_n columns,
// sk_tiles of them, sk_grid workgroups = sk_tiles x parts, arrivals zero, partials with sk_grid slots).
// The same conditions as agpr_launch, and K / 128 at least 4 x parts.
int mica_gemm::agpr_split_launch(const GemmParams &p, int epilogue, int out_dtype, bool has_bias, bool has_res,
                                 hipStream_t st) {
    if (p.sk_tiles <= 0 || p.sk_grid % p.sk_tiles != 0 || p.K / QBK < 4 * (p.sk_grid / p.sk_tiles))
        return MICA_MISS_ARG;
    if (epilogue == MICA_EPI_SILU_MUL) {
        if (out_dtype != MICA_BF16 || has_bias || has_res) return MICA_MISS_ARG;
        return agpr_split_out<MICA_EPI_SILU_MUL, MICA_BF16>(p, false, false, st);
    }
    if (out_dtype == MICA_BF16) return agpr_split_out<MICA_EPI_SCALE, MICA_BF16>(p, has_bias, has_res, st);
    if (out_dtype == MICA_FP16) return agpr_split_out<MICA_EPI_SCALE, MICA_FP16>(p, has_bias, has_res, st);
    return MICA_MISS_ARG;
}
