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
MICA_DEVICE float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
MICA_DEVICE float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Pack four int8 values (given as int) into one dword, element 0 in the low byte.
MICA_DEVICE uint32_t pack_i8x4(int a, int b, int c, int d) {
    return (uint32_t)(a & 0xff) | ((uint32_t)(b & 0xff) << 8) | ((uint32_t)(c & 0xff) << 16) |
           ((uint32_t)(d & 0xff) << 24);
}

// scale of a row from its absmax: max(amax, 1e-8) / 127 (int8_quant.py:68, EPS :13, QMAX :11)
MICA_DEVICE float row_scale(float amax) { return __builtin_fmaxf(amax, 1e-8f) / 127.0f; }

// ---- host-side helpers ---------------------------------------------------------------------
static inline bool mica_aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }
static inline int mica_err(hipError_t e) { return e == hipSuccess ? 0 : -(int)e; }
