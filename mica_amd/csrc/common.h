// Device helpers shared by the gfx950 kernels of the W8A8 hot path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mica_amd.h"

#define MICA_DEVICE __device__ __forceinline__

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---- bf16 / fp16 <-> fp32 ------------------------------------------------------------------
MICA_DEVICE float bf16_lo(uint32_t packed) { return __uint_as_float(packed << 16); }
MICA_DEVICE float bf16_hi(uint32_t packed) { return __uint_as_float(packed & 0xffff0000u); }
MICA_DEVICE float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// fp32 -> bf16 bits, round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
MICA_DEVICE uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
// Two values packed low | high << 16, each rounded to nearest even: one v_cvt_pk_bf16_f32.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
MICA_DEVICE uint32_t pack_bf16x2(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}
// Round an fp32 value to the nearest bf16 and return it as fp32.
MICA_DEVICE float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// bf16(silu(g)) for a bf16 value g, silu(g) = g / (1 + exp(-g)) as F.silu evaluates it on bf16 (fp32 exp,
// fp32 quotient, rounded to bf16; fused_kernels.py:86-87): exp(-g) as v_exp_f32 of g * -log2(e), and
// 1 / (1 + e) as v_rcp_f32 refined by one Newton step (0 once 1 + e overflows), times g.  v_rcp_f32
// flushes results below 2^-126, so a denominator of 2^64 or more is scaled by 2^-64 first (exactly) and
// the product scaled back.  For every finite bf16 g this rounds to the same bf16 as a float64 exp and an
// IEEE fp32 quotient do, also with v_exp_f32 and v_rcp_f32 each one ulp off (exhaustive on the CPU with a
// flushing reciprocal; the GPU suite runs all 65536 codes).  ~15 VALU operations against ~23 for expf
// and an IEEE division.
MICA_DEVICE float silu_bf16(float g) {
    const float e = __builtin_amdgcn_exp2f(g * -1.44269504088896341f);
    const float d = 1.0f + e;
    const float s = d >= 0x1p64f ? 0x1p-64f : 1.0f;
    const float ds = d * s;
    const float r0 = __builtin_amdgcn_rcpf(ds);
    const float r = ds < __builtin_inff() ? __builtin_fmaf(r0, __builtin_fmaf(-ds, r0, 1.0f), r0) : 0.0f;
    return round_bf16((g * r) * s);
}

// Rotary embedding of 8 pairs (x[i], x[i + h]) of one head, in bf16 arithmetic as transformers'
// apply_rotary_pos_emb computes it (q * cos + rotate_half(q) * sin, each product rounded to bf16, then
// their sum):  ya[i] = bf16(bf16(a[i] c[i]) + bf16(b[i] (-s[i]))),  yb[i] = bf16(bf16(b[i] c[i]) + bf16(a[i] s[i])).
// a / b: the 8 first-half / second-half elements, c / s: the 8 cos / sin table entries, all packed bf16.
MICA_DEVICE void rope_pairs8(const u32x4 &a, const u32x4 &b, const u32x4 &c, const u32x4 &s, u32x4 &ya, u32x4 &yb) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float x0l = bf16_lo(a[e]), x0h = bf16_hi(a[e]), x1l = bf16_lo(b[e]), x1h = bf16_hi(b[e]);
        const float cl = bf16_lo(c[e]), ch = bf16_hi(c[e]), sl = bf16_lo(s[e]), sh = bf16_hi(s[e]);
        // the four products of both pairs of this word, each pair rounded to bf16 by one conversion
        const uint32_t pc0 = pack_bf16x2(x0l * cl, x0h * ch), ps1 = pack_bf16x2(x1l * -sl, x1h * -sh);
        const uint32_t pc1 = pack_bf16x2(x1l * cl, x1h * ch), ps0 = pack_bf16x2(x0l * sl, x0h * sh);
        ya[e] = pack_bf16x2(bf16_lo(pc0) + bf16_lo(ps1), bf16_hi(pc0) + bf16_hi(ps1));
        yb[e] = pack_bf16x2(bf16_lo(pc1) + bf16_lo(ps0), bf16_hi(pc1) + bf16_hi(ps0));
    }
}

MICA_DEVICE float f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
// fp32 -> fp16, round to nearest even, of the fp32 value as rounded.  The empty asm keeps the
// compiler from folding a preceding multiply into the conversion (v_fma_mix*_f16 would round the
// product once, straight to fp16, instead of to fp32 first).
MICA_DEVICE uint16_t f32_to_f16(float f) {
    __asm__ volatile("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// Load element i of a row of dtype (bf16 / fp16 / fp32) as fp32.
MICA_DEVICE float load_as_f32(const void *p, int dtype, long i) {
    if (dtype == MICA_BF16) return bf16_to_f32(((const uint16_t *)p)[i]);
    if (dtype == MICA_FP16) return f16_to_f32(((const uint16_t *)p)[i]);
    return ((const float *)p)[i];
}

// Round/convert an fp32 value to dtype and return it widened back to fp32.
MICA_DEVICE float round_to(float f, int dtype) {
    if (dtype == MICA_BF16) return round_bf16(f);
    if (dtype == MICA_FP16) return f16_to_f32(f32_to_f16(f));
    return f;
}

// ---- wavefront (64 lanes) reductions -------------------------------------------------------
// 64-lane reductions (every lane must be active; every lane gets the same bits): DPP steps within
// each 16-lane row (quad swaps, half-row mirror, row mirror: each lane of a pair adds the same two
// values, so a row ends uniform), then the four row results are read into scalars and combined in
// the same order in every lane.  No LDS traffic, a few cycles per step.
template <bool MAX>
MICA_DEVICE float row16_reduce(float v) {
    auto op = [](float a, float b) { return MAX ? __builtin_fmaxf(a, b) : a + b; };
#define MICA_DPP(x, ctrl) __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), ctrl, 0xF, 0xF, true))
    v = op(v, MICA_DPP(v, 0xB1));  // quad_perm [1, 0, 3, 2]
    v = op(v, MICA_DPP(v, 0x4E));  // quad_perm [2, 3, 0, 1]
    v = op(v, MICA_DPP(v, 0x141)); // row_half_mirror
    v = op(v, MICA_DPP(v, 0x140)); // row_mirror
#undef MICA_DPP
    return v;
}
// sum over each 16-lane row (lanes 16 r .. 16 r + 15, all active); every lane of a row gets the same bits
MICA_DEVICE float row16_sum(float v) { return row16_reduce<false>(v); }

template <bool MAX>
MICA_DEVICE float wave_reduce(float v) {
    auto op = [](float a, float b) { return MAX ? __builtin_fmaxf(a, b) : a + b; };
    v = row16_reduce<MAX>(v);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return op(op(r0, r1), op(r2, r3));
}
MICA_DEVICE float wave_sum(float v) { return wave_reduce<false>(v); }
MICA_DEVICE float wave_max(float v) { return wave_reduce<true>(v); }

// Pack four int8 values (given as int) into one dword, element 0 in the low byte.
MICA_DEVICE uint32_t pack_i8x4(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
           ((uint32_t)(d & 0xff) << 24);
}

// scale of a row from its absmax: max(amax, 1e-8) / 127 (int8_quant.py:68, EPS :13, QMAX :11)
MICA_DEVICE float row_scale(float amax) { return __builtin_fmaxf(amax, 1e-8f) / 127.0f; }

// The multiplier of the one-FMA half-even quantizer for a row of bf16 values x with a bf16 absmax
// a (|x| <= a), s = row_scale(a), inv = 1 / s:  q = low byte of fmaf(x, r, 1.5 * 2^23), which
// rounds the exact product x r to an integer in one step.  r is inv, moved one ulp toward the
// reference's answer for x = a / 2 when rint(x r) and rint(x / s) (IEEE quotient) disagree there;
// with that, q == clamp(rint(x / s), -127, 127) for every bf16 pair (x, a) (checked exhaustively
// on the CPU, tests/native/fma_quotient_check.c).  Costs two divisions per row, saves three
// instructions per element against the corrected quotient.
constexpr float kMagicRne = 12582912.0f; // 1.5 * 2^23
MICA_DEVICE float fma_quant_recip(float a, float s, float inv) {
    const float h = a * 0.5f;
    const float qh = __builtin_rintf(h / s);
    const float qf = __builtin_fmaf(h, inv, kMagicRne) - kMagicRne;
    const int dir = qh > qf ? 1 : (qh < qf ? -1 : 0);
    return __uint_as_float(__float_as_uint(inv) + (uint32_t)dir);
}
// 8 values -> 8 int8 (element 0 in the low byte) with the multiplier above
MICA_DEVICE u32x2 fma_quant8(const float (&x)[8], float r) {
    uint32_t b[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) b[j] = __float_as_uint(__builtin_fmaf(x[j], r, kMagicRne));
    u32x2 q;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t lo = __builtin_amdgcn_perm(b[4 * h + 1], b[4 * h], 0x0c0c0400u);
        const uint32_t hi = __builtin_amdgcn_perm(b[4 * h + 3], b[4 * h + 2], 0x0c0c0400u);
        q[h] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
    }
    return q;
}

// ---- host-side helpers ---------------------------------------------------------------------
static inline bool mica_aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }
static inline int mica_err(hipError_t e) { return e == hipSuccess ? 0 : -(int)e; }
