// Row kernels of the W8A8 hot path on gfx950:
//   * fused RMSNorm (+ residual add) + per-token INT8 quantizer  (mica_rmsnorm_quant)
//   * standalone per-token INT8 quantizer                        (mica_act_quant)
//   * elementwise SwiGLU                                          (mica_swiglu)
//
// Layout: one 64-lane wavefront owns one row at a time and keeps the whole row in registers,
// so x is read from HBM once and q (int8) + s (fp32) are written once.  Lane l holds the
// 8-element chunks [c * 512 + 8 l, c * 512 + 8 l + 8) for c < NCH = ceil(K / 512): every
// load is a 16-byte vector and a wave's 64 lanes cover 1 KiB of contiguous bf16 per chunk.
// The sum of squares and the absmax are wavefront reductions (no LDS, no barrier).
// Waves walk rows with a grid stride over a grid sized to the CU count; rows of up to 2560
// elements keep the next row's load in flight while the current one is processed.
// The int8 rows are written with non-temporal stores (streamed out once, read by the next
// kernel), measured faster than cached stores on MI355X; cached loads measured faster than
// non-temporal ones.

#include <atomic>

#include "common.h"

namespace {

constexpr int kChunk = 8;          // elements per lane per chunk
constexpr int kRowStep = 64 * kChunk; // elements per chunk across the wave


constexpr int kMaxOut = 4; // quantized copies one row launch can write (mica_rmsnorm_quant_multi)

struct RowParams {
    const void *x;
    const void *res;
    const void *w;
    // the quantized outputs: n_out of them, each with its own smoothing factors (or NULL), int8
    // rows (row stride ldq) and per-row scales
    const float *inv[kMaxOut];
    int8_t *q[kMaxOut];
    float *s[kMaxOut];
    int ldq[kMaxOut];
    int n_out;
    void *y;
    void *sum;
    int ldx, ldr, ldy, lds;
    int M, K;
    int w_dtype;
    int rounding;
    float offset, eps;
};

// 16-bit element j of a packed chunk as fp32
template <int XT>
MICA_DEVICE float elem16(const u32x4 &c, int j) {
    uint32_t word = c[j >> 1];
    uint16_t h = (j & 1) ? (uint16_t)(word >> 16) : (uint16_t)(word & 0xffffu);
    if (XT == MICA_BF16) return bf16_to_f32(h);
    return f16_to_f32(h);
}

template <int XT>
MICA_DEVICE uint16_t to16(float f) {
    if (XT == MICA_BF16) return f32_to_bf16(f);
    return f32_to_f16(f);
}

template <int XT>
MICA_DEVICE void unpack8(const u32x4 &c, float (&v)[kChunk]) {
#pragma unroll
    for (int j = 0; j < kChunk; ++j) v[j] = elem16<XT>(c, j);
}

template <int XT>
MICA_DEVICE u32x4 pack8(const float (&v)[kChunk]) {
    u32x4 c;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if (XT == MICA_BF16) c[j] = pack_bf16x2(v[2 * j], v[2 * j + 1]);
        else c[j] = (uint32_t)to16<XT>(v[2 * j]) | ((uint32_t)to16<XT>(v[2 * j + 1]) << 16);
    }
    return c;
}

MICA_DEVICE void load_w8(const void *w, int w_dtype, int idx, float (&v)[kChunk]) {
    if (w_dtype == MICA_FP32) {
        const float4 *p = (const float4 *)((const float *)w + idx);
        float4 a = p[0], b = p[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
        u32x4 c = *(const u32x4 *)((const uint16_t *)w + idx);
        if (w_dtype == MICA_BF16) unpack8<MICA_BF16>(c, v);
        else unpack8<MICA_FP16>(c, v);
    }
}

MICA_DEVICE void load_inv8(const float *inv, int idx, float (&v)[kChunk]) {
    const float4 *p = (const float4 *)(inv + idx);
    float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// Quantize one chunk of 8 fp32 values with the row's scale s (r = 1 / s) and store 8 bytes; the
// reference's q = clamp(round(x / s), -127, 127) with x / s the IEEE fp32 quotient
// (int8_quant.py:70; kernel_src/kernels.py:34-36 for half away).  RND: the rounding mode
// (MICA_ROUND_EVEN / MICA_ROUND_AWAY, or 2: the one given at run time).
//
// The quotient is y = x * r corrected once: y + fma(-y, s, x) * r.  For bf16 x with a bf16 absmax
// (kFast: unsmoothed bf16 rows; the row kernels take this path for half-away rounding, and the
// one-FMA quantizer of common.h for half even) its rounded integer equals the IEEE quotient's for every input
// (tests/native/quotient_check.c, exhaustive).  For other values (SmoothQuant-scaled rows, fp16 and
// fp32 activations) the plain product y = x * r is used.  With |x / s| <= 127.5, the exact product x r
// is within 127.5 * 2^-24 < 2^-17 of x / s (r = RN(1 / s)), y's rounding adds at most 2^-18, and the
// IEEE quotient RN(x / s) is within 2^-18 of x / s: so y and RN(x / s) lie within 2^-16 of each other,
// and their integers can only differ when y is within 2^-16 of a boundary k + 0.5.  Lanes whose y lies
// within kTieWindow = 2^-15 of one (|fract(y) - 0.5| <= 2^-15, v_fract_f32) recompute the chunk with
// the IEEE division.  A wave takes that path when any of its 512 values is that close: ~3 % of the
// chunks of a smoothed row, against ~12 % for a 2^-13 window.
//
// Half even without kFast is one step shorter: the exact product x r (one FMA with 1.5 * 2^23) is
// rounded to an integer directly, and the guard looks at u = RN(x r + 0.5 + 2^-15): x r within 2^-16
// of k + 0.5 puts u within 2^-15 +- (2^-16 + 2^-18) of the integer k + 1 (|u| < 128, so its rounding
// is at most 2^-18), i.e. fract(u) in (0, 2^-14), and those lanes take the IEEE division.
// tests/native/guarded_quotient_check.c checks both forms on 2^28 random pairs and on every x within
// the window around every boundary k + 0.5 for 2^15 values of s (the computation is invariant under
// scaling x and s by the same power of two, so s in [1, 2) covers every normal scale).
//
// Half even rounds with the 1.5 * 2^23 trick: for |t| < 2^22, t + 12582912 is an integer-valued
// float (its rounding is the IEEE round-half-even of t), whose low mantissa byte is that integer in
// two's complement; v_perm_b32 gathers the four low bytes into one dword.  No clamp is needed:
// |x| <= amax and s = RN(max(amax, 1e-8) / 127) give |x / s| <= 127 / (1 - 2^-24) < 127.5, so
// round(x / s) is already within +-127 (the reference's clamp is the identity on finite rows; a row
// holding Inf or NaN yields 0 for those elements).
constexpr float kTieWindow = 0x1p-15f;

template <bool kFast, int RND>
MICA_DEVICE void quant_store8r(const float (&v)[kChunk], float s, float r, int rounding, int8_t *dst) {
    const int mode = RND == 2 ? rounding : RND;
    if (!kFast && mode == MICA_ROUND_EVEN) {
        uint32_t b[kChunk];
        float low = 1.0f;
#pragma unroll
        for (int j = 0; j < kChunk; ++j) {
            b[j] = __float_as_uint(__builtin_fmaf(v[j], r, kMagicRne));
            low = __builtin_fminf(low, __builtin_amdgcn_fractf(__builtin_fmaf(v[j], r, 0.5f + kTieWindow)));
        }
        if (low < 2.0f * kTieWindow) {
#pragma unroll
            for (int j = 0; j < kChunk; ++j) b[j] = __float_as_uint(v[j] / s + kMagicRne);
        }
        u32x2 packed;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t lo = __builtin_amdgcn_perm(b[4 * h + 1], b[4 * h], 0x0c0c0400u);
            const uint32_t hi = __builtin_amdgcn_perm(b[4 * h + 3], b[4 * h + 2], 0x0c0c0400u);
            packed[h] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
        }
        __builtin_nontemporal_store(packed, (u32x2 *)dst);
        return;
    }
    float t[kChunk];
#pragma unroll
    for (int j = 0; j < kChunk; ++j) {
        const float y = v[j] * r;
        t[j] = kFast ? __builtin_fmaf(__builtin_fmaf(-y, s, v[j]), r, y) : y;
    }
    if (!kFast) {
        // fract(y) - 0.5 is exact; v_fract_f32 returns at most 1 - 2^-24 (for tiny negative y), far
        // from the window
        float gap = 1.0f;
#pragma unroll
        for (int j = 0; j < kChunk; ++j) gap = __builtin_fminf(gap, __builtin_fabsf(__builtin_amdgcn_fractf(t[j]) - 0.5f));
        const bool near = gap <= kTieWindow;
        if (near) {
#pragma unroll
            for (int j = 0; j < kChunk; ++j) t[j] = v[j] / s;
        }
    }
    u32x2 packed;
    if (mode == MICA_ROUND_EVEN) {
        uint32_t b[kChunk];
#pragma unroll
        for (int j = 0; j < kChunk; ++j) b[j] = __float_as_uint(t[j] + 12582912.0f);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t lo = __builtin_amdgcn_perm(b[4 * h + 1], b[4 * h], 0x0c0c0400u);
            const uint32_t hi = __builtin_amdgcn_perm(b[4 * h + 3], b[4 * h + 2], 0x0c0c0400u);
            packed[h] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
        }
    } else {
        int qv[kChunk];
#pragma unroll
        for (int j = 0; j < kChunk; ++j) {
            const float a = __builtin_truncf(t[j] >= 0.0f ? t[j] + 0.5f : t[j] - 0.5f);
            qv[j] = (int)__builtin_fminf(__builtin_fmaxf(a, -127.0f), 127.0f);
        }
        packed[0] = pack_i8x4(qv[0], qv[1], qv[2], qv[3]);
        packed[1] = pack_i8x4(qv[4], qv[5], qv[6], qv[7]);
    }
    __builtin_nontemporal_store(packed, (u32x2 *)dst); // written once, read by the next kernel
}

// XT: dtype of x / residual / y / sum (bf16 or fp16).  NORM: apply the RMSNorm first.
// HAS_INV: some output multiplies by its inv_smooth before the absmax (that output then uses the
// IEEE-division quotient).
// FULL: K == NCH * 512, so no chunk needs a bounds mask.  RND: rounding mode (2: at run time).
// Each wave prefetches its next row while it works on the current one; the row is unpacked to
// fp32 once, and after the norm it stays in fp32 registers (already rounded to XT), so the
// absmax and the quantizer work on registers.
// ONE: every wave owns exactly one row (the launch covers M with one wave per row, all resident at
// once): no next row to prefetch, and the bf16 weights are loaded with the row and widened where
// they are used instead of being held as fp32, which keeps the kernel within 4+ waves per SIMD
// (measured at T = 4096, K = 2560 against weights formed once per workgroup in LDS: 6.0 vs 6.3 us).
template <int NCH, int XT, bool NORM, bool HAS_INV, bool FULL, int RND, bool ONE = false>
MICA_DEVICE void row16_body(const RowParams &p) {
    constexpr bool kFast = XT == MICA_BF16; // the fast quotient is exact for unsmoothed bf16 rows
    const int lane = threadIdx.x & 63;
    const int nwaves = gridDim.x * (blockDim.x >> 6);
    const int K = p.K;
    auto live = [&](int c) { return FULL || c * kRowStep + lane * kChunk < K; };

    auto load_row = [&](u32x4 (&raw)[NCH], int row) {
        const uint16_t *xr = (const uint16_t *)p.x + (long)row * p.ldx;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int idx = c * kRowStep + lane * kChunk;
            raw[c] = live(c) ? *(const u32x4 *)(xr + idx) : u32x4{0u, 0u, 0u, 0u};
        }
    };
    // the wave's first row is requested before the weights, so the two latencies overlap
    int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    u32x4 bufA[NCH], bufB[NCH <= 5 && !ONE ? NCH : 1];
    if (row < p.M) load_row(bufA, row);
    // ONE: the raw bf16 weights of this lane's chunks, widened at their use
    u32x4 wraw[ONE && NORM ? NCH : 1];
    if (ONE && NORM) {
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int idx = c * kRowStep + lane * kChunk;
            wraw[c] = live(c) ? *(const u32x4 *)((const uint16_t *)p.w + idx) : u32x4{0u, 0u, 0u, 0u};
        }
    }

    // rows of up to 2560 elements with smoothing factors: the workgroup copies every output's factors
    // into LDS once (n_out x K fp32, dynamic shared memory), so the two passes of every row read them
    // there instead of through the vector memory path.  Chunk ch = c * 64 + lane of output o sits at
    // float4 X = (o * NCH + c) * 64 + lane (its first 4 factors) and kHalf + X (its last 4): a wave's
    // 16-byte reads then cover consecutive addresses, free of bank conflicts.
    constexpr bool kInvLds = HAS_INV && NCH <= 5;
    extern __shared__ float4 inv_sh[];
    const int kHalf = p.n_out * NCH * 64;
    if (kInvLds) {
        for (int o = 0; o < p.n_out; ++o) {
            if (p.inv[o] == nullptr) continue;
            for (int ch = threadIdx.x; ch < NCH * 64; ch += blockDim.x) {
                float4 a = {0.0f, 0.0f, 0.0f, 0.0f}, b = a;
                if (FULL || ch * kChunk < K) {
                    a = ((const float4 *)(p.inv[o] + ch * kChunk))[0];
                    b = ((const float4 *)(p.inv[o] + ch * kChunk))[1];
                }
                inv_sh[o * NCH * 64 + ch] = a;
                inv_sh[kHalf + o * NCH * 64 + ch] = b;
            }
        }
        __syncthreads();
    }

    // per-lane weight multipliers (offset + w), fp32, cached across the rows this wave visits
    float w1[NORM && !ONE ? NCH : 1][kChunk];
    if (NORM && !ONE) {
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int idx = c * kRowStep + lane * kChunk;
            if (live(c)) {
                load_w8(p.w, p.w_dtype, idx, w1[c]);
#pragma unroll
                for (int j = 0; j < kChunk; ++j) w1[c][j] = p.offset + w1[c][j];
            } else {
#pragma unroll
                for (int j = 0; j < kChunk; ++j) w1[c][j] = 0.0f;
            }
        }
    }

    // one row, held in cur (raw bits).  Short rows (kF32) are unpacked to fp32 once and stay in
    // fp32 registers through the norm, the absmax and the quantizer; long rows stay packed and are
    // unpacked again in each pass, which keeps enough waves resident.
    constexpr bool kF32 = NCH <= 8;
    // long rows already keep enough bytes in flight per wave; smoothed rows spend the registers on
    // their factors' products instead
    constexpr bool kPrefetch = NCH <= 5 && !HAS_INV && !ONE;
    auto process = [&](u32x4 (&cur)[NCH], int row) {
        if (NORM && p.res != nullptr) {
            // v = (x + r) rounded to the activation dtype (fused_kernels.py:27-30, :52)
            const uint16_t *rr = (const uint16_t *)p.res + (long)row * p.ldr;
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                const int idx = c * kRowStep + lane * kChunk;
                if (live(c)) {
                    u32x4 rc = *(const u32x4 *)(rr + idx);
                    float a[kChunk], b[kChunk];
                    unpack8<XT>(cur[c], a);
                    unpack8<XT>(rc, b);
#pragma unroll
                    for (int j = 0; j < kChunk; ++j) a[j] = a[j] + b[j];
                    cur[c] = pack8<XT>(a);
                    if (p.sum != nullptr) *(u32x4 *)((uint16_t *)p.sum + (long)row * p.lds + idx) = cur[c];
                }
            }
        }
        float v[kF32 ? NCH : 1][kChunk];
        if (kF32) {
#pragma unroll
            for (int c = 0; c < NCH; ++c) unpack8<XT>(cur[c], v[kF32 ? c : 0]);
        }
        if (NORM) {
            float ss = 0.0f;
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                float t[kChunk];
                if (!kF32) unpack8<XT>(cur[c], t);
                const float(&a)[kChunk] = kF32 ? v[kF32 ? c : 0] : t;
#pragma unroll
                for (int j = 0; j < kChunk; ++j) ss = __builtin_fmaf(a[j], a[j], ss);
            }
            ss = wave_sum(ss);
            const float mean = ss / (float)K;
            const float rstd = 1.0f / __builtin_sqrtf(mean + p.eps);
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                const int idx = c * kRowStep + lane * kChunk;
                float t[kChunk];
                if (!kF32) unpack8<XT>(cur[c], t);
                float(&a)[kChunk] = kF32 ? v[kF32 ? c : 0] : t;
                if (ONE) {
                    float wv[kChunk];
                    unpack8<MICA_BF16>(wraw[ONE && NORM ? c : 0], wv);
#pragma unroll
                    for (int j = 0; j < kChunk; ++j) a[j] = (a[j] * rstd) * (p.offset + wv[j]);
                } else {
#pragma unroll
                    for (int j = 0; j < kChunk; ++j) a[j] = (a[j] * rstd) * w1[ONE ? 0 : c][j];
                }
                const u32x4 packed = pack8<XT>(a);
                if (kF32) unpack8<XT>(packed, a);
                else cur[c] = packed;
                if (p.y != nullptr && live(c)) *(u32x4 *)((uint16_t *)p.y + (long)row * p.ldy + idx) = packed;
            }
        }
        // the quantized outputs: per output, the absmax of the (smoothed) row, its scale, then the
        // int8 row.  The smoothing product x * inv is formed on the fly in both passes, so the row
        // itself stays unsmoothed for the next output.  Masked chunks hold zeros.
#pragma unroll 1
        for (int o = 0; o < p.n_out; ++o) {
            const float *inv = HAS_INV ? p.inv[o] : nullptr;
            auto chunk = [&](int c, float (&t)[kChunk]) {
                if (kF32) {
#pragma unroll
                    for (int j = 0; j < kChunk; ++j) t[j] = v[kF32 ? c : 0][j];
                } else {
                    unpack8<XT>(cur[c], t);
                }
                if (HAS_INV && inv != nullptr) {
                    float iv[kChunk];
                    if (kInvLds) {
                        const float4 a = inv_sh[(o * NCH + c) * 64 + lane];
                        const float4 b = inv_sh[kHalf + (o * NCH + c) * 64 + lane];
                        iv[0] = a.x; iv[1] = a.y; iv[2] = a.z; iv[3] = a.w;
                        iv[4] = b.x; iv[5] = b.y; iv[6] = b.z; iv[7] = b.w;
                    } else if (live(c)) {
                        load_inv8(inv, c * kRowStep + lane * kChunk, iv);
                    } else {
                        for (int j = 0; j < kChunk; ++j) iv[j] = 0.0f;
                    }
#pragma unroll
                    for (int j = 0; j < kChunk; ++j) t[j] = t[j] * iv[j];
                }
            };
            float amax = 0.0f;
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                float t[kChunk];
                chunk(c, t);
#pragma unroll
                for (int j = 0; j < kChunk; ++j) amax = __builtin_fmaxf(amax, __builtin_fabsf(t[j]));
            }
            amax = wave_max(amax);
            if (!kF32) {
                // the quantizer unpacks the row again: keep the compiler from holding the first
                // pass's fp32 values live instead (that would cost the registers kF32 = false saves)
#pragma unroll
                for (int c = 0; c < NCH; ++c) __asm__ volatile("" : "+v"(cur[c]));
            }
            const float sc = row_scale(amax);
            const float r = 1.0f / sc;
            if (lane == 0) p.s[o][row] = sc;
            int8_t *qr = p.q[o] + (long)row * p.ldq[o];
            const bool smoothed = HAS_INV && inv != nullptr;
            // unsmoothed bf16 rows rounded half even: one FMA per element (fma_quant_recip)
            const bool one_fma = kFast && !smoothed && (RND == 2 ? p.rounding : RND) == MICA_ROUND_EVEN;
            const float rf = one_fma ? fma_quant_recip(amax, sc, r) : r;
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                float t[kChunk];
                chunk(c, t);
                if (!live(c)) continue;
                int8_t *dst = qr + c * kRowStep + lane * kChunk;
                if (one_fma) __builtin_nontemporal_store(fma_quant8(t, rf), (u32x2 *)dst);
                // smoothed values are fp32 products (not bf16): IEEE quotient
                else if (smoothed) quant_store8r<false, RND>(t, sc, r, p.rounding, dst);
                else quant_store8r<kFast, RND>(t, sc, r, p.rounding, dst);
            }
        }
    };

    if constexpr (ONE) {
        if (row < p.M) process(bufA, row);
    } else if constexpr (kPrefetch) {
        // two row buffers used in turn (no registers are copied between rows); each wave's next
        // row is requested before the current one is worked on
        for (;;) {
            if (row >= p.M) break;
            if (row + nwaves < p.M) load_row(bufB, row + nwaves);
            process(bufA, row);
            row += nwaves;
            if (row >= p.M) break;
            if (row + nwaves < p.M) load_row(bufA, row + nwaves);
            process(bufB, row);
            row += nwaves;
        }
    } else {
        for (; row < p.M; row += nwaves) {
            if (row != blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) load_row(bufA, row);
            process(bufA, row);
        }
    }
}

template <int NCH, int XT, bool NORM, bool HAS_INV, bool FULL, int RND>
__global__ __launch_bounds__(256) void row16_kernel(RowParams p) {
    row16_body<NCH, XT, NORM, HAS_INV, FULL, RND>(p);
}

// One row per wave (see row16_body): for a launch whose rows all fit the resident waves at once.
#ifndef MICA_ONE_THREADS
#define MICA_ONE_THREADS 256
#endif
constexpr int kOneThreads = MICA_ONE_THREADS;
template <int NCH, int XT, bool NORM, bool FULL, int RND>
__global__ __launch_bounds__(kOneThreads) void row16_one_kernel(RowParams p) {
    row16_body<NCH, XT, NORM, false, FULL, RND, true>(p);
}

// Smoothed rows of up to 2560 elements, held to 168 registers (a few spill) so that 3 waves per SIMD
// stay resident, against 2 at the compiler's own choice (213 registers).
template <int NCH, int XT, bool NORM, bool FULL, int RND>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void row16_smooth_kernel(RowParams p) {
    row16_body<NCH, XT, NORM, true, FULL, RND>(p);
}

// Smoothed bf16 rows of exactly NCH * 512 elements where each of the NOUT outputs has its own
// factors, one row per wave with every row of the launch resident at once.  Against the grid-stride
// kernel above: no next row held, the norm's multipliers offset + w formed once per workgroup in LDS
// next to the factors, no run-time test of which outputs are smoothed, and each output's smoothed
// row held in registers from its absmax to its quantizer.  Same arithmetic, same bits: the row
// (+ residual, rounded to bf16), the norm (x * rstd) * (offset + w) rounded to bf16, t = x * inv in
// fp32, s = max(absmax(t), 1e-8) / 127, q from the guarded quotient t / s.
#ifndef MICA_SMOOTH_THREADS
#define MICA_SMOOTH_THREADS 1024
#endif
constexpr int kSmoothThreads = MICA_SMOOTH_THREADS;  // a whole CU's 16 rows share one copy of the factors
// SMOOTH = false: the same kernel for unsmoothed outputs, whose int8 rows are then all equal: the
// row is quantized once (the one-FMA half-even quantizer of common.h, exact for bf16 rows) and
// stored to each output.
template <int NCH, bool NORM, int NOUT, int RND, bool SMOOTH = true>
__global__ __launch_bounds__(kSmoothThreads) __attribute__((amdgpu_waves_per_eu(4))) void smooth_one_kernel(RowParams p) {
    constexpr int XT = MICA_BF16;
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (kSmoothThreads / 64) + (threadIdx.x >> 6);
    const bool on = row < p.M;
    const bool has_res = NORM && p.res != nullptr;
    // every output's factors go to LDS: chunk ch = c * 64 + lane of output o at float4
    // X = (o * NCH + c) * 64 + lane (its first 4 factors) and kHalf + X (its last 4), so a wave's 16-byte
    // reads cover consecutive addresses, free of bank conflicts; with the norm, the multipliers
    // offset + w (fp32) after them as output NOUT.  This thread's share is loaded first, the row second: the memory counter retires
    // loads in issue order, so the LDS fill waits for the factors alone, and the barrier after it waits
    // for LDS only -- each wave then starts on its row as soon as that row has arrived, instead of the
    // whole workgroup waiting for its slowest row (which a full __syncthreads() fence would do).
    extern __shared__ float4 inv_sh[];
    constexpr int kSets = SMOOTH ? NOUT : 0;  // factor sets before the norm's multipliers
    constexpr int kFill = (NCH * 64 + kSmoothThreads - 1) / kSmoothThreads;  // chunks per thread and set
    constexpr int kHalf = (kSets + (NORM ? 1 : 0)) * NCH * 64;
    float4 fin[kSets > 0 ? kSets : 1][kFill][2];
    u32x4 win[NORM ? kFill : 1];
    // (both loads are issued on every path, idle lanes re-reading the last valid chunk or row, so that
    // the compiler's wait before the LDS fill counts only the loads issued after the factors')
#pragma unroll
    for (int i = 0; i < kFill; ++i) {
        const int ch = (int)threadIdx.x + i * kSmoothThreads;
        const int chc = ch < NCH * 64 ? ch : NCH * 64 - 1;
#pragma unroll
        for (int o = 0; o < kSets; ++o) {
            fin[o][i][0] = ((const float4 *)(p.inv[o] + chc * kChunk))[0];
            fin[o][i][1] = ((const float4 *)(p.inv[o] + chc * kChunk))[1];
        }
        if (NORM) win[i] = *(const u32x4 *)((const uint16_t *)p.w + chc * kChunk);
    }
    // the scheduler keeps the multiplier loads ahead of the row loads; with smoothing factors held too,
    // pinning that order makes the compiler spill them, so it keeps its own order there
    if constexpr (!SMOOTH) __builtin_amdgcn_sched_barrier(0);
    u32x4 cur[NCH], rc[NORM ? NCH : 1];
    const int rowc = on ? row : p.M - 1;  // a launched block holds at least one row (M >= 1)
    {
        const uint16_t *xr = (const uint16_t *)p.x + (long)rowc * p.ldx;
#pragma unroll
        for (int c = 0; c < NCH; ++c) cur[c] = *(const u32x4 *)(xr + c * kRowStep + lane * kChunk);
        if (has_res) {
            const uint16_t *rr = (const uint16_t *)p.res + (long)rowc * p.ldr;
#pragma unroll
            for (int c = 0; c < NCH; ++c) rc[NORM ? c : 0] = *(const u32x4 *)(rr + c * kRowStep + lane * kChunk);
        }
    }
#pragma unroll
    for (int i = 0; i < kFill; ++i) {
        const int ch = (int)threadIdx.x + i * kSmoothThreads;
        if (ch < NCH * 64) {
#pragma unroll
            for (int o = 0; o < kSets; ++o) {
                inv_sh[o * NCH * 64 + ch] = fin[o][i][0];
                inv_sh[kHalf + o * NCH * 64 + ch] = fin[o][i][1];
            }
            if (NORM) {
                float wv[kChunk];
                unpack8<MICA_BF16>(win[i], wv);
                inv_sh[kSets * NCH * 64 + ch] = float4{p.offset + wv[0], p.offset + wv[1], p.offset + wv[2], p.offset + wv[3]};
                inv_sh[kHalf + kSets * NCH * 64 + ch] = float4{p.offset + wv[4], p.offset + wv[5], p.offset + wv[6], p.offset + wv[7]};
            }
        }
    }
    // LDS-only barrier: release and acquire fences of workgroup scope restricted to the LDS address
    // space around the barrier.  They order the LDS stores above before, and the LDS loads below after,
    // the barrier in the compiler's memory model, and lower to a wait on the LDS counter alone
    // (lgkmcnt 0), leaving the row's global loads in flight
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    if (!on) return;

    float v[NCH][kChunk];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        const int idx = c * kRowStep + lane * kChunk;
        if (has_res) {
            // v = (x + r) rounded to the activation dtype (fused_kernels.py:27-30, :52)
            float b[kChunk];
            unpack8<XT>(cur[c], v[c]);
            unpack8<XT>(rc[NORM ? c : 0], b);
#pragma unroll
            for (int j = 0; j < kChunk; ++j) v[c][j] = v[c][j] + b[j];
            cur[c] = pack8<XT>(v[c]);
            if (p.sum != nullptr) *(u32x4 *)((uint16_t *)p.sum + (long)row * p.lds + idx) = cur[c];
        }
        unpack8<XT>(cur[c], v[c]);
    }
    auto factors = [&](int o, int c, float (&iv)[kChunk]) {
        const float4 a = inv_sh[(o * NCH + c) * 64 + lane];
        const float4 b = inv_sh[kHalf + (o * NCH + c) * 64 + lane];
        iv[0] = a.x; iv[1] = a.y; iv[2] = a.z; iv[3] = a.w;
        iv[4] = b.x; iv[5] = b.y; iv[6] = b.z; iv[7] = b.w;
    };
    if (NORM) {
        float ss = 0.0f;
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
            for (int j = 0; j < kChunk; ++j) ss = __builtin_fmaf(v[c][j], v[c][j], ss);
        ss = wave_sum(ss);
        const float mean = ss / (float)p.K;
        const float rstd = 1.0f / __builtin_sqrtf(mean + p.eps);
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            float w1[kChunk];
            factors(kSets, c, w1);
#pragma unroll
            for (int j = 0; j < kChunk; ++j) v[c][j] = (v[c][j] * rstd) * w1[j];
            const u32x4 packed = pack8<XT>(v[c]);
            unpack8<XT>(packed, v[c]);
            if (p.y != nullptr) *(u32x4 *)((uint16_t *)p.y + (long)row * p.ldy + c * kRowStep + lane * kChunk) = packed;
        }
    }
    if constexpr (!SMOOTH) {
        float am = 0.0f;
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
            for (int j = 0; j < kChunk; ++j) am = __builtin_fmaxf(am, __builtin_fabsf(v[c][j]));
        am = wave_max(am);
        const float sc = row_scale(am);
        const float rr = 1.0f / sc;
        const float rf = RND == MICA_ROUND_EVEN ? fma_quant_recip(am, sc, rr) : rr;
        if (lane == 0) {
#pragma unroll
            for (int o = 0; o < NOUT; ++o) p.s[o][row] = sc;
        }
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            if (RND == MICA_ROUND_EVEN) {
                const u32x2 packed = fma_quant8(v[c], rf);
#pragma unroll
                for (int o = 0; o < NOUT; ++o)
                    __builtin_nontemporal_store(packed, (u32x2 *)(p.q[o] + (long)row * p.ldq[o] + c * kRowStep + lane * kChunk));
            } else {
#pragma unroll
                for (int o = 0; o < NOUT; ++o)
                    quant_store8r<true, RND>(v[c], sc, rr, p.rounding, p.q[o] + (long)row * p.ldq[o] + c * kRowStep + lane * kChunk);
            }
        }
        return;
    }
    // one output at a time: its smoothed row t stays in registers from the absmax to the quantizer
    // (the factors are read from LDS once per output)
#pragma unroll
    for (int o = 0; o < NOUT; ++o) {
        float t[NCH][kChunk];
        float am = 0.0f;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            float iv[kChunk];
            factors(o, c, iv);
#pragma unroll
            for (int j = 0; j < kChunk; ++j) {
                t[c][j] = v[c][j] * iv[j];
                am = __builtin_fmaxf(am, __builtin_fabsf(t[c][j]));
            }
        }
        const float sc = row_scale(wave_max(am));
        const float rr = 1.0f / sc;
        if (lane == 0) p.s[o][row] = sc;
        int8_t *qrow = p.q[o] + (long)row * p.ldq[o] + lane * kChunk;
#pragma unroll
        for (int c = 0; c < NCH; ++c) quant_store8r<false, RND>(t[c], sc, rr, p.rounding, qrow + c * kRowStep);
    }
}

template <int NCH, int XT, bool NORM, bool HAS_INV, bool FULL, int RND>
constexpr void (*row16_for())(RowParams) {
    if constexpr (HAS_INV && NCH <= 5) return row16_smooth_kernel<NCH, XT, NORM, FULL, RND>;
    else return row16_kernel<NCH, XT, NORM, HAS_INV, FULL, RND>;
}

// fp32 activations (act_quant only): same structure, two 16-byte loads per chunk.
template <int NCH, bool HAS_INV>
__global__ __launch_bounds__(256) void row32_kernel(RowParams p) {
    const int lane = threadIdx.x & 63;
    const int nwaves = gridDim.x * (blockDim.x >> 6);
    const int K = p.K;
    for (int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); row < p.M; row += nwaves) {
        float v[NCH][kChunk];
        const float *xr = (const float *)p.x + (long)row * p.ldx;
        float amax = 0.0f;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int idx = c * kRowStep + lane * kChunk;
            if (idx < K) {
                float4 a = *(const float4 *)(xr + idx), b = *(const float4 *)(xr + idx + 4);
                v[c][0] = a.x; v[c][1] = a.y; v[c][2] = a.z; v[c][3] = a.w;
                v[c][4] = b.x; v[c][5] = b.y; v[c][6] = b.z; v[c][7] = b.w;
                if (HAS_INV) {
                    float iv[kChunk];
                    load_inv8(p.inv[0], idx, iv);
#pragma unroll
                    for (int j = 0; j < kChunk; ++j) v[c][j] = v[c][j] * iv[j];
                }
            } else {
#pragma unroll
                for (int j = 0; j < kChunk; ++j) v[c][j] = 0.0f;
            }
#pragma unroll
            for (int j = 0; j < kChunk; ++j) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[c][j]));
        }
        amax = wave_max(amax);
        const float s = row_scale(amax);
        const float r = 1.0f / s;
        if (lane == 0) p.s[0][row] = s;
        int8_t *qr = p.q[0] + (long)row * p.ldq[0];
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int idx = c * kRowStep + lane * kChunk;
            if (idx < K) quant_store8r<false, 2>(v[c], s, r, p.rounding, qr + idx);
        }
    }
}

// Elementwise SwiGLU on bf16: y = bf16(bf16(silu(g)) * u), 8 elements per thread.
__global__ __launch_bounds__(256) void swiglu_kernel(const uint16_t *g, const uint16_t *u, uint16_t *y, long long n) {
    const long long i0 = ((long long)blockIdx.x * blockDim.x + threadIdx.x) * kChunk;
    if (i0 >= n) return;
    if (i0 + kChunk <= n) {
        u32x4 gc = *(const u32x4 *)(g + i0), uc = *(const u32x4 *)(u + i0);
        float gv[kChunk], uv[kChunk], out[kChunk];
        unpack8<MICA_BF16>(gc, gv);
        unpack8<MICA_BF16>(uc, uv);
#pragma unroll
        for (int j = 0; j < kChunk; ++j) {
            const float act = silu_bf16(gv[j]);
            out[j] = act * uv[j];
        }
        *(u32x4 *)(y + i0) = pack8<MICA_BF16>(out);
    } else {
        for (long long i = i0; i < n; ++i) {
            const float gv = bf16_to_f32(g[i]);
            const float act = silu_bf16(gv);
            y[i] = f32_to_bf16(act * bf16_to_f32(u[i]));
        }
    }
}

// Workgroups (4 waves each) per CU that a row launch asks for: 3 per CU keep every wave of the
// hot kernels (3 to 4 waves per SIMD) resident from the start, each walking its rows with a grid
// stride (its weights are loaded once, its next row is always in flight); measured against 4, 6
// and 12 per CU on MI355X.
#ifndef MICA_ROW_BLOCKS_PER_CU
#define MICA_ROW_BLOCKS_PER_CU 3
#endif

int cu_count_of_current_device() {
    static int cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] > 0) return cached[dev];
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) return 256;
    cached[dev] = v;
    return v;
}

int row_grid(int M) {
    const int blocks = (M + 3) / 4;
    const int cap = cu_count_of_current_device() * MICA_ROW_BLOCKS_PER_CU;
    return blocks < cap ? blocks : cap;
}

// dynamic LDS of a row16_kernel launch: the smoothing factors of rows of up to 2560 elements
template <int NCH>
unsigned inv_lds_bytes(const RowParams &p, bool has_inv) {
    return (has_inv && NCH <= 5) ? (unsigned)(p.n_out * NCH * 64 * 2 * sizeof(float4)) : 0u;
}

// Launch a row kernel on a grid of at most MICA_ROW_BLOCKS_PER_CU workgroups per CU, fewer when its
// registers or LDS let fewer be resident at once (a workgroup beyond that would only start when a
// resident one ends, and its rows would then finish last).
// The residency is queried once per kernel and output count (the LDS size depends on nothing else)
// and kept; concurrent first calls store the same value.
template <void (*Kernel)(RowParams)>
int launch_rows(const RowParams &p, unsigned lds, hipStream_t st) {
    static std::atomic<int> cached[kMaxOut + 1];
    std::atomic<int> &slot = cached[lds ? p.n_out : 0];
    int per_cu = slot.load(std::memory_order_relaxed);
    if (per_cu <= 0) {
        int occ = 0;
        per_cu = MICA_ROW_BLOCKS_PER_CU;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, Kernel, 256, lds) == hipSuccess && occ > 0 &&
            occ < per_cu)
            per_cu = occ;
        slot.store(per_cu, std::memory_order_relaxed);
    }
    const int blocks = (p.M + 3) / 4, cap = cu_count_of_current_device() * per_cu;
    hipLaunchKernelGGL(Kernel, dim3(blocks < cap ? blocks : cap), dim3(256), lds, st, p);
    return mica_err(hipGetLastError());
}

// Launch a one-row-per-wave kernel when every row fits the waves that can be resident at once
// (measured at T = 4096, K = 2560: the grid-stride kernel at 3 workgroups per CU leaves a third of
// its waves a second row); returns -1 when the rows do not fit, for the caller's grid-stride path.
template <void (*Kernel)(RowParams)>
int launch_one(const RowParams &p, hipStream_t st) {
    static std::atomic<int> cached{0};
    int per_cu = cached.load(std::memory_order_relaxed);
    if (per_cu <= 0) {
        int occ = 0;
        per_cu = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, Kernel, kOneThreads, 0) == hipSuccess && occ > 0 ? occ : 1;
        cached.store(per_cu, std::memory_order_relaxed);
    }
    const long long blocks = ((long long)p.M + kOneThreads / 64 - 1) / (kOneThreads / 64);
    if (blocks > (long long)cu_count_of_current_device() * per_cu) return -1;
    hipLaunchKernelGGL(Kernel, dim3((unsigned)blocks), dim3(kOneThreads), 0, st, p);
    return mica_err(hipGetLastError());
}

template <int NCH>
int launch16(const RowParams &p, int xt, bool norm, bool has_inv, hipStream_t st) {
#define MICA_ROW16(XT_, NORM_, INV_) \
    return launch_rows<row16_for<NCH, XT_, NORM_, INV_, false, 2>()>(p, inv_lds_bytes<NCH>(p, INV_), st)
    if (xt == MICA_BF16) {
        if (norm) { if (has_inv) MICA_ROW16(MICA_BF16, true, true); else MICA_ROW16(MICA_BF16, true, false); }
        else { if (has_inv) MICA_ROW16(MICA_BF16, false, true); else MICA_ROW16(MICA_BF16, false, false); }
    } else {
        if (norm) { if (has_inv) MICA_ROW16(MICA_FP16, true, true); else MICA_ROW16(MICA_FP16, true, false); }
        else { if (has_inv) MICA_ROW16(MICA_FP16, false, true); else MICA_ROW16(MICA_FP16, false, false); }
    }
#undef MICA_ROW16
}

// smooth_one_kernel when every row of the launch fits the resident waves; -1 otherwise (the caller
// then takes the grid-stride path)
template <int NCH, bool NORM, int NOUT, int RND, bool SMOOTH = true>
int launch_smooth_one(const RowParams &p, hipStream_t st) {
    constexpr auto kern = smooth_one_kernel<NCH, NORM, NOUT, RND, SMOOTH>;
    const unsigned lds = (unsigned)(((SMOOTH ? NOUT : 0) + (NORM ? 1 : 0)) * NCH * 64 * 2 * sizeof(float4));
    // the kernel writes exactly NOUT quantized rows and scales per row: never launch it for another
    // output count (a norm-only call has n_out = 0 and no q / s at all)
    if (lds == 0 || p.n_out != NOUT) return -1;
    for (int o = 0; o < NOUT; ++o)
        if (p.q[o] == nullptr || p.s[o] == nullptr || (SMOOTH && p.inv[o] == nullptr)) return -1;
    static std::atomic<int> cached{0};
    int per_cu = cached.load(std::memory_order_relaxed);
    if (per_cu <= 0) {
        int occ = 0;
        per_cu = hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kern, kSmoothThreads, lds) == hipSuccess && occ > 0 ? occ : 1;
        cached.store(per_cu, std::memory_order_relaxed);
    }
    constexpr int kRows = kSmoothThreads / 64;
    const long long blocks = ((long long)p.M + kRows - 1) / kRows;
    if (blocks > (long long)cu_count_of_current_device() * per_cu) return -1;
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(kSmoothThreads), lds, st, p);
    return mica_err(hipGetLastError());
}

template <int NCH, bool NORM, int NOUT, bool SMOOTH = true>
int launch_smooth_one_rnd(const RowParams &p, hipStream_t st) {
    if (p.rounding == MICA_ROUND_EVEN) return launch_smooth_one<NCH, NORM, NOUT, MICA_ROUND_EVEN, SMOOTH>(p, st);
    return launch_smooth_one<NCH, NORM, NOUT, MICA_ROUND_AWAY, SMOOTH>(p, st);
}

// bf16 rows of exactly NCH * 512 elements (the hot widths): no masks, rounding fixed at compile time
template <int NCH>
int launch16_full(const RowParams &p, bool norm, bool has_inv, hipStream_t st) {
    // rows of up to 2560 elements without smoothing: one wave per row when they all fit
    if constexpr (NCH <= 5) {
#ifndef MICA_NORM_ONE_LDS
#define MICA_NORM_ONE_LDS 1
#endif
        // one normed, quantized output: the kernel with the multipliers offset + w in LDS (measured at
        // T = 4096, K = 2560: 5.65 against 6.0 us for the kernel below, which stays faster for several
        // outputs: 8.0 against 8.3 us for three)
        if (MICA_NORM_ONE_LDS && !has_inv && norm && p.w_dtype == MICA_BF16 && p.n_out == 1) {
            const int rc = launch_smooth_one_rnd<NCH, true, 1, false>(p, st);
            if (rc >= 0) return rc;
        }
        if (!has_inv && (!norm || p.w_dtype == MICA_BF16)) {
            int rc = -1;
            if (norm && p.rounding == MICA_ROUND_EVEN) rc = launch_one<row16_one_kernel<NCH, MICA_BF16, true, true, MICA_ROUND_EVEN>>(p, st);
            else if (norm) rc = launch_one<row16_one_kernel<NCH, MICA_BF16, true, true, MICA_ROUND_AWAY>>(p, st);
            else if (p.rounding == MICA_ROUND_EVEN) rc = launch_one<row16_one_kernel<NCH, MICA_BF16, false, true, MICA_ROUND_EVEN>>(p, st);
            else rc = launch_one<row16_one_kernel<NCH, MICA_BF16, false, true, MICA_ROUND_AWAY>>(p, st);
            if (rc >= 0) return rc;
        }
        // every output smoothed (1 to 3 of them): one wave per row when they all fit
        bool all_inv = has_inv && p.n_out >= 1 && p.n_out <= 3 && (!norm || p.w_dtype == MICA_BF16);
        for (int o = 0; o < p.n_out; ++o) all_inv = all_inv && p.inv[o] != nullptr;
        if (all_inv) {
            int rc = -1;
            if (norm) {
                if (p.n_out == 1) rc = launch_smooth_one_rnd<NCH, true, 1>(p, st);
                else if (p.n_out == 2) rc = launch_smooth_one_rnd<NCH, true, 2>(p, st);
                else rc = launch_smooth_one_rnd<NCH, true, 3>(p, st);
            } else {
                if (p.n_out == 1) rc = launch_smooth_one_rnd<NCH, false, 1>(p, st);
                else if (p.n_out == 2) rc = launch_smooth_one_rnd<NCH, false, 2>(p, st);
                else rc = launch_smooth_one_rnd<NCH, false, 3>(p, st);
            }
            if (rc >= 0) return rc;
        }
    }
#define MICA_ROWF(NORM_, INV_, RND_) \
    return launch_rows<row16_for<NCH, MICA_BF16, NORM_, INV_, true, RND_>()>(p, inv_lds_bytes<NCH>(p, INV_), st)
#define MICA_ROWF2(NORM_, INV_) \
    if (p.rounding == MICA_ROUND_EVEN) MICA_ROWF(NORM_, INV_, MICA_ROUND_EVEN); else MICA_ROWF(NORM_, INV_, MICA_ROUND_AWAY);
    if (norm) { if (has_inv) { MICA_ROWF2(true, true) } else { MICA_ROWF2(true, false) } }
    else { if (has_inv) { MICA_ROWF2(false, true) } else { MICA_ROWF2(false, false) } }
#undef MICA_ROWF2
#undef MICA_ROWF
}

template <int NCH>
int launch32(const RowParams &p, bool has_inv, hipStream_t st) {
    dim3 grid(row_grid(p.M)), block(256);
    if (has_inv) hipLaunchKernelGGL((row32_kernel<NCH, true>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((row32_kernel<NCH, false>), grid, block, 0, st, p);
    return mica_err(hipGetLastError());
}

// NCH = ceil(K / 512) in 1..32 (K <= 16384).  bf16 rows of the hot widths (K = 2560: 5,
// 4096: 8, 9216: 18, 9728: 19) run unmasked with the rounding mode compiled in; any other width
// runs on the next larger instantiation, whose surplus chunks are masked off.
int dispatch_rows(const RowParams &p, int xt, bool norm, bool has_inv, hipStream_t st) {
    const int nch = (p.K + kRowStep - 1) / kRowStep;
    if (xt == MICA_BF16 && p.K == nch * kRowStep) {
        if (nch == 5) return launch16_full<5>(p, norm, has_inv, st);
        if (nch == 8) return launch16_full<8>(p, norm, has_inv, st);
        if (nch == 18) return launch16_full<18>(p, norm, has_inv, st);
        if (nch == 19) return launch16_full<19>(p, norm, has_inv, st);
    }
#define MICA_CASE(N_) \
    if (nch <= N_) return xt == MICA_FP32 ? launch32<N_>(p, has_inv, st) : launch16<N_>(p, xt, norm, has_inv, st);
    MICA_CASE(1) MICA_CASE(2) MICA_CASE(4) MICA_CASE(5) MICA_CASE(8) MICA_CASE(12) MICA_CASE(16) MICA_CASE(18)
    MICA_CASE(19) MICA_CASE(24) MICA_CASE(32)
#undef MICA_CASE
    return MICA_MISS_SHAPE;
}

bool ld_ok(int ld, int K) { return ld >= K && ld % 8 == 0; }

}  // namespace

extern "C" int mica_act_quant(const void *x, int x_dtype, int ldx, const float *inv_smooth, int8_t *q, int ldq,
                              float *s, int M, int K, int rounding, mica_stream_t stream) {
    if (x == nullptr || q == nullptr || s == nullptr) return MICA_MISS_ARG;
    if (x_dtype != MICA_BF16 && x_dtype != MICA_FP16 && x_dtype != MICA_FP32) return MICA_MISS_DTYPE;
    if (rounding != MICA_ROUND_EVEN && rounding != MICA_ROUND_AWAY) return MICA_MISS_ARG;
    if (M < 0 || K < 8 || K > 16384 || K % 8 != 0) return MICA_MISS_SHAPE;
    if (!ld_ok(ldx, K) || !ld_ok(ldq, K)) return MICA_MISS_STRIDE;
    if ((long long)M * ldx >= (1ll << 31) || (long long)M * ldq >= (1ll << 31)) return MICA_MISS_RANGE;
    if (!mica_aligned16(x) || !mica_aligned16(q) || !mica_aligned16(s) ||
        (inv_smooth != nullptr && !mica_aligned16(inv_smooth)))
        return MICA_MISS_ALIGN;
    if (M == 0) return 0;
    RowParams p{};
    p.x = x;
    p.inv[0] = inv_smooth; p.q[0] = q; p.s[0] = s; p.ldq[0] = ldq; p.n_out = 1;
    p.ldx = ldx; p.M = M; p.K = K; p.rounding = rounding;
    return dispatch_rows(p, x_dtype, false, inv_smooth != nullptr, (hipStream_t)stream);
}

namespace {

// Checks and launch shared by the one- and several-output RMSNorm + quantizer entry points.
int rmsnorm_quant_n(const void *x, int x_dtype, int ldx, const void *residual, int ldr, const void *w, int w_dtype,
                    float offset, float eps, int n_out, const float *const *inv_smooth, int8_t *const *q,
                    const int *ldq, float *const *s, void *y, int ldy, void *sum, int lds, int M, int K, int rounding,
                    mica_stream_t stream) {
    if (x == nullptr || w == nullptr || (n_out == 0 && y == nullptr)) return MICA_MISS_ARG;
    if (n_out < 0 || n_out > kMaxOut) return MICA_MISS_ARG;
    if (sum != nullptr && residual == nullptr) return MICA_MISS_ARG;
    if (x_dtype != MICA_BF16 && x_dtype != MICA_FP16) return MICA_MISS_DTYPE;
    if (w_dtype != MICA_BF16 && w_dtype != MICA_FP16 && w_dtype != MICA_FP32) return MICA_MISS_DTYPE;
    if (rounding != MICA_ROUND_EVEN && rounding != MICA_ROUND_AWAY) return MICA_MISS_ARG;
    if (M < 0 || K < 8 || K > 16384 || K % 8 != 0) return MICA_MISS_SHAPE;
    if (!ld_ok(ldx, K) || (residual && !ld_ok(ldr, K)) || (y && !ld_ok(ldy, K)) || (sum && !ld_ok(lds, K)))
        return MICA_MISS_STRIDE;
    long long maxld = ldx;
    if (residual && ldr > maxld) maxld = ldr;
    if (y && ldy > maxld) maxld = ldy;
    if (sum && lds > maxld) maxld = lds;
    bool has_inv = false;
    for (int o = 0; o < n_out; ++o) {
        if (q[o] == nullptr || s[o] == nullptr) return MICA_MISS_ARG;
        if (!ld_ok(ldq[o], K)) return MICA_MISS_STRIDE;
        if (ldq[o] > maxld) maxld = ldq[o];
        if (!mica_aligned16(q[o]) || !mica_aligned16(s[o]) || (inv_smooth[o] && !mica_aligned16(inv_smooth[o])))
            return MICA_MISS_ALIGN;
        has_inv = has_inv || inv_smooth[o] != nullptr;
    }
    if ((long long)M * maxld >= (1ll << 31)) return MICA_MISS_RANGE;
    if (!mica_aligned16(x) || !mica_aligned16(w) || (residual && !mica_aligned16(residual)) ||
        (y && !mica_aligned16(y)) || (sum && !mica_aligned16(sum)))
        return MICA_MISS_ALIGN;
    if (M == 0) return 0;
    RowParams p{};
    p.x = x; p.res = residual; p.w = w; p.y = y; p.sum = sum;
    for (int o = 0; o < n_out; ++o) {
        p.inv[o] = inv_smooth[o]; p.q[o] = q[o]; p.s[o] = s[o]; p.ldq[o] = ldq[o];
    }
    p.n_out = n_out;
    p.ldx = ldx; p.ldr = ldr; p.ldy = ldy; p.lds = lds;
    p.M = M; p.K = K; p.w_dtype = w_dtype; p.rounding = rounding; p.offset = offset; p.eps = eps;
    return dispatch_rows(p, x_dtype, true, has_inv, (hipStream_t)stream);
}

}  // namespace

extern "C" int mica_rmsnorm_quant(const void *x, int x_dtype, int ldx, const void *residual, int ldr, const void *w,
                                  int w_dtype, float offset, float eps, const float *inv_smooth, int8_t *q, int ldq,
                                  float *s, void *y, int ldy, void *sum, int lds, int M, int K, int rounding,
                                  mica_stream_t stream) {
    if (q != nullptr && s == nullptr) return MICA_MISS_ARG;
    const int n_out = q != nullptr ? 1 : 0;
    return rmsnorm_quant_n(x, x_dtype, ldx, residual, ldr, w, w_dtype, offset, eps, n_out, &inv_smooth, &q, &ldq, &s, y,
                           ldy, sum, lds, M, K, rounding, stream);
}

extern "C" int mica_rmsnorm_quant_multi(const void *x, int x_dtype, int ldx, const void *residual, int ldr,
                                        const void *w, int w_dtype, float offset, float eps, int n_out,
                                        const float *const *inv_smooth, int8_t *const *q, const int *ldq,
                                        float *const *s, void *y, int ldy, void *sum, int lds, int M, int K,
                                        int rounding, mica_stream_t stream) {
    if (n_out < 1 || n_out > kMaxOut || inv_smooth == nullptr || q == nullptr || ldq == nullptr || s == nullptr)
        return MICA_MISS_ARG;
    return rmsnorm_quant_n(x, x_dtype, ldx, residual, ldr, w, w_dtype, offset, eps, n_out, inv_smooth, q, ldq, s, y,
                           ldy, sum, lds, M, K, rounding, stream);
}

extern "C" int mica_swiglu(const void *g, const void *u, void *y, long long n, int dtype, mica_stream_t stream) {
    if (g == nullptr || u == nullptr || y == nullptr) return MICA_MISS_ARG;
    if (dtype != MICA_BF16) return MICA_MISS_DTYPE;
    if (n < 0) return MICA_MISS_SHAPE;
    if (!mica_aligned16(g) || !mica_aligned16(u) || !mica_aligned16(y)) return MICA_MISS_ALIGN;
    if (n == 0) return 0;
    const long long threads = (n + kChunk - 1) / kChunk;
    const long long blocks = (threads + 255) / 256;
    if (blocks >= (1ll << 31)) return MICA_MISS_RANGE;
    hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t *)g, (const uint16_t *)u, (uint16_t *)y, n);
    return mica_err(hipGetLastError());
}
