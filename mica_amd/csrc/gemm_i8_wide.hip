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
// LDS rows are 128 bytes; 16-byte chunk g of row r sits at position g ^ swz(r), which keeps the
// 16-row x 4-chunk operand reads free of bank conflicts.
// Schedule: a persistent grid of at most one workgroup per CU walks the whole tiles in the XCD-aware
// order of gemm_i8_common.h, then the tail tiles as two halves each (256 x 128 for the SCALE epilogue,
// 128 x 256 along M for SiLU, whose waves need their 128 gate / up rows).
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
    static constexpr int kBDma = BN / 8 / kWideWaves;
    static constexpr int kDma = kADma + kBDma;
};
using WFull = WCfg<256, 256>;   // waves of 64 x 128
using WHalfN = WCfg<256, 128>;  // waves of 64 x 64 (SCALE tail)
using WHalfM = WCfg<128, 256>;  // waves of 32 x 128 (SiLU tail)
using WQuart = WCfg<128, 128>;  // waves of 32 x 64 (SCALE tail at most a quarter of a round)

// LDS: the larger of the stages (128 KiB) and the 16-bit epilogue staging (8 waves x 64 rows x
// (128 columns x 2 + 16) bytes), then the tile's scales (sa, sb, bias: 3 x 256 fp32)
constexpr int kWStaging = kWideWaves * 64 * (128 * 2 + 16);
constexpr int kWMain = (4 * 256 * WBK > kWStaging) ? 4 * 256 * WBK : kWStaging;
constexpr int kWScale = kWMain;
constexpr int kWSmem = kWScale + 3 * 256 * 4;
static_assert(kWSmem <= 160 * 1024, "LDS");

MICA_DEVICE int wswz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// threadIdx.x through an opaque move: the per-lane offsets derived from it are recomputed for every
// tile (a few VALU operations) instead of being held across the persistent loop, where at 256 VGPRs
// they would be spilled and their reloads would wait for every DMA in flight
MICA_DEVICE int fresh_tid() {
    int t;
    asm volatile("v_mov_b32 %0, %1" : "=v"(t) : "v"((int)threadIdx.x));
    return t;
}

template <class C, int EPI, int OUT, bool HAS_BIAS, bool HAS_RES>
struct WideTile {
    static constexpr int WM = C::WM, WN = C::WN, MB = C::MB, NB = C::NB;
    v4i acc[NB][MB];

    struct Ops {
        v4i x[MB];
        v4i w[NB];
    };

    // ---- slabs of tile (m0, n0) into acc
    MICA_DEVICE void run(const GemmParams &p, int8_t *smem, __amdgpu_buffer_rsrc_t rsrc_a,
                         __amdgpu_buffer_rsrc_t rsrc_b, int m0, int n0) {
        const int tid = fresh_tid(), lane = tid & 63;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int wm = wave >> 1, wn = wave & 1;
        const int r16 = lane & 15, kq = lane >> 4;
        const int M = p.M, N = p.N;
        const int nk = p.K / WBK;  // even
        // DMA: lane l of 1 KiB instruction j (A: j < kADma) covers row (wave * kADma + j) * 8 + l / 8,
        // position l % 8, i.e. global chunk (l % 8) ^ wswz(row); rows past M / N read zeros
        int a_off[C::kADma], b_off[C::kBDma];
#pragma unroll
        for (int j = 0; j < C::kADma; ++j) {
            const int r = (wave * C::kADma + j) * 8 + (lane >> 3);
            a_off[j] = m0 + r < M ? (m0 + r) * p.lda + (((lane & 7) ^ wswz(r)) << 4) : kOutOfRange;
        }
#pragma unroll
        for (int j = 0; j < C::kBDma; ++j) {
            const int r = (wave * C::kBDma + j) * 8 + (lane >> 3);
            b_off[j] = n0 + r < N ? (n0 + r) * p.ldb + (((lane & 7) ^ wswz(r)) << 4) : kOutOfRange;
        }
        // kOutOfRange + kb stays at or above 2^31, past every buffer: no select per slab
        auto dma = [&](int slab) {
            const int kb = slab * WBK;
            int8_t *sa_ = smem + (slab & 1) * C::kAHalf + wave * C::kADma * 1024;
            int8_t *sb_ = smem + C::kBBase + (slab & 1) * C::kBHalf + wave * C::kBDma * 1024;
#pragma unroll
            for (int j = 0; j < C::kADma; ++j)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_a, (lds_void *)(sa_ + j * 1024), 16, a_off[j] + kb, 0, 0, 0);
#pragma unroll
            for (int j = 0; j < C::kBDma; ++j)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc_b, (lds_void *)(sb_ + j * 1024), 16, b_off[j] + kb, 0, 0, 0);
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
        // MFMAs interleaved with the next k-step's reads (and, after a barrier, the DMA)
        auto interleave = [&](auto dma_c) {
            constexpr bool DMA = decltype(dma_c)::value;
            constexpr int per = kMfma / kReads > 0 ? kMfma / kReads : 1;
#pragma unroll
            for (int g = 0; g < kReads; ++g) {
                __builtin_amdgcn_sched_group_barrier(0x008, per, 0); // MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
                if (DMA && g < C::kDma) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0); // LDS DMA
            }
            if (kMfma > per * kReads) __builtin_amdgcn_sched_group_barrier(0x008, kMfma - per * kReads, 0);
        };
        using T = std::integral_constant<bool, true>;
        using F = std::integral_constant<bool, false>;
        Ops R0, R1;
        // one slab from stage ST (R0 holds its k-step 0).  NEXT: another slab follows (barrier before
        // k-step 1, then its k-step 0 is read into R0); DMA: the DMA of slab k + 2 goes after the barrier
        auto slab = [&](auto st_c, auto next_c, auto dma_c, int k) {
            constexpr int ST = decltype(st_c)::value;
            reads(R1, st_c, 1);
            mfmas(R0);
            interleave(F{});
            if constexpr (decltype(next_c)::value) {
                wait_vmcnt<0>();   // slab k + 1 landed (this wave's share)
                wait_lgkmcnt0();   // k-step 1's fragments are in registers
                __builtin_amdgcn_s_barrier();
                if constexpr (decltype(dma_c)::value) dma(k + 2);
                reads(R0, std::integral_constant<int, ST ^ 1>{}, 0);
                mfmas(R1);
                interleave(dma_c);
            } else {
                mfmas(R1);
            }
        };

#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int i = 0; i < MB; ++i) acc[j][i] = v4i{};
        // this tile's scales, loaded branch-free before the DMA (the index is clamped into range;
        // values of rows / columns past the edge are never used): threads 0-255 sa and bias of tile row /
        // column tid, threads 256-511 sb of column tid - 256
        float f1, f2 = 0.0f;
        {
            const int i = tid & 255;
            const bool row = wave < 4;  // wave-uniform: the selects below stay scalar
            const float *src = row ? p.sa : p.sb;
            const int base = row ? m0 : n0;
            const int lim = (row ? M : N) - base;
            f1 = src[base + (i < lim ? i : lim - 1)];
            if (HAS_BIAS) f2 = p.bias[n0 + (i < N - n0 ? i : N - n0 - 1)];
        }
        // the previous tile's epilogue (LDS staging, scale reads) is finished in every wave
        wait_lgkmcnt0();
        __builtin_amdgcn_s_barrier();
        dma(0);
        dma(1);
        {
            float *sc = (float *)(smem + kWScale);
            sc[tid] = f1;                                   // [0, 256): sa, [256, 512): sb
            if (HAS_BIAS && tid < 256) sc[512 + tid] = f2;  // [512, 768): bias
        }
        wait_vmcnt<C::kDma>();  // slab 0 landed (slab 1 may be in flight)
        __builtin_amdgcn_s_barrier();
        using S0 = std::integral_constant<int, 0>;
        using S1 = std::integral_constant<int, 1>;
        reads(R0, S0{}, 0);
        int k = 0;
        for (; k + 2 < nk; k += 2) {
            slab(S0{}, T{}, T{}, k);
            slab(S1{}, T{}, T{}, k + 1);
        }
        slab(S0{}, T{}, F{}, k);
        slab(S1{}, F{}, F{}, k + 1);
    }

    // ---- epilogue of tile (m0, n0) from acc
    MICA_DEVICE void epilogue(const GemmParams &p, int8_t *smem, int m0, int n0) {
        const int tid = fresh_tid(), lane = tid & 63;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const int wm = wave >> 1, wn = wave & 1;
        const int r16 = lane & 15, kq = lane >> 4;
        const int M = p.M, N = p.N;
        const int mw = m0 + wm * WM;
        const bool vec = p.vec_ok != 0;
        const float *sc = (const float *)(smem + kWScale); // [0, 256): sa, [256, 512): sb, [512, 768): bias
        float sav[MB];
#pragma unroll
        for (int i = 0; i < MB; ++i) sav[i] = sc[wm * WM + i * 16 + r16];
        if constexpr (OUT == MICA_BF16 || OUT == MICA_FP16) {
            // Staged through LDS: every wave writes its rounded 16-bit block (8 bytes per lane per store)
            // into its own padded region, then streams it out row-contiguously, 16 bytes per lane.
            wait_lgkmcnt0();
            __builtin_amdgcn_s_barrier(); // every wave is done reading the operand stages
            constexpr int kCols = EPI == MICA_EPI_SCALE ? WN : WN / 2;   // output columns of this wave
            constexpr int kPitch = kCols * 2 + 16;
            int8_t *ep = smem + wave * (WM * kPitch);
            const int col0 = EPI == MICA_EPI_SCALE ? n0 + wn * WN : (n0 >> 1) + wn * (WN / 2);
            const int ncols_out = EPI == MICA_EPI_SCALE ? N : (N >> 1);
#pragma unroll
            for (int j = 0; j < (EPI == MICA_EPI_SCALE ? NB : NB / 2); ++j) {
                const int nl = j * 16 + 4 * kq;  // local output column of this lane's 4 values
                const int cb = wn * WN + nl;     // tile-local column (SiLU: of the gate row)
                float s1[4], s2[4], bv[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    s1[t] = sc[256 + cb + t];  // SCALE: sb[n]; SILU_MUL: the gate rows' sb
                    s2[t] = EPI == MICA_EPI_SCALE ? 0.0f : sc[256 + cb + WN / 2 + t]; // the matching up rows
                    bv[t] = HAS_BIAS ? sc[512 + cb + t] : 0.0f;
                }
#pragma unroll
                for (int i = 0; i < MB; ++i) {
                    float y[4];
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        if (EPI == MICA_EPI_SCALE) {
                            y[t] = ((float)acc[j][i][t] * sav[i]) * s1[t];
                            if (HAS_BIAS) y[t] = y[t] + bv[t];
                        } else {
                            const float gv = round_bf16(((float)acc[j][i][t] * sav[i]) * s1[t]);
                            const float uv = round_bf16(((float)acc[j + NB / 2][i][t] * sav[i]) * s2[t]);
                            const float act = round_bf16(gv / (1.0f + expf(-gv)));
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
                    *(u32x2 *)(ep + (i * 16 + r16) * kPitch + nl * 2) = w;
                }
            }
            wait_lgkmcnt0(); // a wave reads back only its own region: no barrier needed
            constexpr int kLanesPerRow = kCols / 8;   // lanes x 8 columns per row
            constexpr int kRowsPerPass = 64 / kLanesPerRow;
            const int cl = (lane % kLanesPerRow) * 8; // local column of this lane's 8 values
            const int valid = ncols_out - (col0 + cl) < 8 ? (ncols_out - (col0 + cl) > 0 ? ncols_out - (col0 + cl) : 0) : 8;
            const bool vec8 = vec && (p.ldc % 8 == 0) && (!HAS_RES || p.ldr % 8 == 0);
#pragma unroll 4
            for (int r0 = 0; r0 < WM; r0 += kRowsPerPass) {
                const int rl = r0 + lane / kLanesPerRow;
                const int m = mw + rl;
                const u32x4 v = *(const u32x4 *)(ep + rl * kPitch + cl * 2);
                if (m >= M || valid == 0) continue;
                u32x4 o = v;
                if (HAS_RES) {
                    const uint16_t *rp = (const uint16_t *)p.res + (long)m * p.ldr + col0 + cl;
                    u32x4 rv = {0u, 0u, 0u, 0u};
                    if (vec8 && valid == 8) rv = *(const u32x4 *)rp;
                    else for (int t = 0; t < valid; ++t) rv[t >> 1] |= (uint32_t)rp[t] << (16 * (t & 1));
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        if (OUT == MICA_BF16) {
                            o[t] = pack_bf16x2(bf16_lo(v[t]) + bf16_lo(rv[t]), bf16_hi(v[t]) + bf16_hi(rv[t]));
                        } else {
                            const float a0 = f16_to_f32(v[t] & 0xffff), a1 = f16_to_f32(v[t] >> 16);
                            const float b0 = f16_to_f32(rv[t] & 0xffff), b1 = f16_to_f32(rv[t] >> 16);
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
        // 32-bit outputs (fp32 / raw int32): 16-byte stores straight from the accumulator layout
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
    }
};

template <int EPI, int OUT, bool HAS_BIAS, bool HAS_RES>
__global__ __launch_bounds__(kWideThreads, 1) void gemm_i8_wide_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(1024))) int8_t smem[kWSmem];
    static_assert(EPI == MICA_EPI_SCALE || WFull::WN == 128, "the SiLU epilogue needs one 128-row gate/up group per wave");
    const int G = gridDim.x;
    const __amdgpu_buffer_rsrc_t rsrc_a = __builtin_amdgcn_make_buffer_rsrc((void *)p.A, 0, p.M * p.lda, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rsrc_b = __builtin_amdgcn_make_buffer_rsrc((void *)p.B, 0, p.N * p.ldb, kBufferFlags);
    {
        WideTile<WFull, EPI, OUT, HAS_BIAS, HAS_RES> full;
        for (int pid = blockIdx.x; pid < p.dp_tiles; pid += G) {
            int tm, tn;
            tile_of(pid, p.tiles_m, p.tiles_n, tm, tn);
            full.run(p, smem, rsrc_a, rsrc_b, tm * 256, tn * 256);
            full.epilogue(p, smem, tm * 256, tn * 256);
        }
    }
    if constexpr (EPI == MICA_EPI_SCALE) {
        // the next half_tiles tiles as two 256 x 128 halves each
        if (p.half_tiles > 0) {
            WideTile<WHalfN, EPI, OUT, HAS_BIAS, HAS_RES> half;
            for (int h = blockIdx.x; h < 2 * p.half_tiles; h += G) {
                int tm, tn;
                tile_of(p.dp_tiles + (h >> 1), p.tiles_m, p.tiles_n, tm, tn);
                const int n0 = tn * 256 + (h & 1) * 128;
                if (n0 >= p.N) continue;  // uniform over the workgroup
                half.run(p, smem, rsrc_a, rsrc_b, tm * 256, n0);
                half.epilogue(p, smem, tm * 256, n0);
            }
        }
        // or the next quarter_tiles tiles as four 128 x 128 quarters each
        if (p.quarter_tiles > 0) {
            WideTile<WQuart, EPI, OUT, HAS_BIAS, HAS_RES> quarter;
            for (int h = blockIdx.x; h < 4 * p.quarter_tiles; h += G) {
                int tm, tn;
                tile_of(p.dp_tiles + (h >> 2), p.tiles_m, p.tiles_n, tm, tn);
                const int m0 = tm * 256 + ((h >> 1) & 1) * 128;
                const int n0 = tn * 256 + (h & 1) * 128;
                if (m0 >= p.M || n0 >= p.N) continue;  // uniform over the workgroup
                quarter.run(p, smem, rsrc_a, rsrc_b, m0, n0);
                quarter.epilogue(p, smem, m0, n0);
            }
        }
    } else {
        // the next mhalf_tiles tiles as two 128 x 256 halves each along M (gate / up pairs intact)
        if (p.mhalf_tiles > 0) {
            WideTile<WHalfM, EPI, OUT, HAS_BIAS, HAS_RES> mhalf;
            for (int h = blockIdx.x; h < 2 * p.mhalf_tiles; h += G) {
                int tm, tn;
                tile_of(p.dp_tiles + (h >> 1), p.tiles_m, p.tiles_n, tm, tn);
                const int m0 = tm * 256 + (h & 1) * 128;
                if (m0 >= p.M) continue;  // uniform over the workgroup
                mhalf.run(p, smem, rsrc_a, rsrc_b, m0, tn * 256);
                mhalf.epilogue(p, smem, m0, tn * 256);
            }
        }
    }
}

template <int EPI, int OUT>
int wide_launch_out(const GemmParams &p, int grid, bool has_bias, bool has_res, hipStream_t st) {
    dim3 g(grid), b(kWideThreads);
#define MICA_W(B_, R_) hipLaunchKernelGGL((gemm_i8_wide_kernel<EPI, OUT, B_, R_>), g, b, 0, st, p)
    if constexpr (EPI == MICA_EPI_SILU_MUL || OUT == MICA_INT32) {
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
// or mhalf_tiles as pieces; no split).  Called by mica_mm_i8 after its checks, only for K % 256 == 0.
int mica_gemm::wide_launch(const GemmParams &p, int epilogue, int out_dtype, int grid, bool has_bias, bool has_res,
                           hipStream_t st) {
    if (epilogue == MICA_EPI_SILU_MUL) return wide_launch_out<MICA_EPI_SILU_MUL, MICA_BF16>(p, grid, false, false, st);
    if (out_dtype == MICA_BF16) return wide_launch_out<MICA_EPI_SCALE, MICA_BF16>(p, grid, has_bias, has_res, st);
    if (out_dtype == MICA_FP16) return wide_launch_out<MICA_EPI_SCALE, MICA_FP16>(p, grid, has_bias, has_res, st);
    if (out_dtype == MICA_INT32) return wide_launch_out<MICA_EPI_SCALE, MICA_INT32>(p, grid, false, false, st);
    return wide_launch_out<MICA_EPI_SCALE, MICA_FP32>(p, grid, has_bias, has_res, st);
}
