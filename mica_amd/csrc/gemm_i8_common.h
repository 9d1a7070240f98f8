// Pieces shared by the two W8A8 GEMM kernels (gemm_i8.hip, gemm_i8_wide.hip): the launch parameters,
// the XCD-aware tile order, wait helpers and the epilogue's 4-value loads and stores.
#pragma once

#include "common.h"

// A named namespace: both kernels' translation units, and the launcher one calls in the other, see the
// same GemmParams type.
namespace mica_gemm {

constexpr int kGroupM = 4; // M-tiles per group of the tile order
constexpr int kXcds = 8;   // workgroup i runs on XCD i % 8, each with its own L2

// word 3 of a gfx9 buffer resource (raw buffer, 32-bit data format), as used by CK for gfx9xx
constexpr int kBufferFlags = 0x00020000;
// a buffer offset that fails the range check (every buffer here is < 2^31 bytes)
constexpr int kOutOfRange = (int)0x80000000u;

typedef __attribute__((address_space(3))) void lds_void;

struct GemmParams {
    const int8_t *A;
    const int8_t *B;
    const float *sa;
    const float *sb;
    const float *bias;
    const void *res;
    void *C;
    int lda, ldb, ldr, ldc;
    int M, N, K;
    int tiles_m, tiles_n; // 256 x 256 tiles (the wide kernel's narrow schedule: 256 x 160)
    int vec_ok;           // ldc, ldr, N all multiples of 4: 4-column vector stores
    // schedule over the tiles in grouped order (tile_of): [0, dp_tiles) run whole, one per workgroup
    // per round; the next half_tiles run as two 256 x 128 halves each, or the next quarter_tiles as
    // four 128 x 128 quarters each; the next sk_tiles are split along K over workgroups [0, sk_grid)
    // (at most one of half_tiles, quarter_tiles, sk_tiles is nonzero)
    // the next mhalf_tiles (SiLU epilogue) run as two 128 x 256 halves each along M
    int dp_tiles, half_tiles, quarter_tiles, mhalf_tiles, sk_tiles, sk_grid;
    v4i *partials; // [gridDim.x][2][kPartialVecs][kThreads]: a workgroup's partial accumulators
    int *arrivals; // [sk_tiles]: contributors arrived so far; zero between launches
};

// s_waitcnt with only one counter constrained (gfx9 encoding: vmcnt [3:0] + [15:14], expcnt [6:4],
// lgkmcnt [11:8]; the other fields at their maxima)
template <int N>
MICA_DEVICE void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
MICA_DEVICE void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4)); }

// Map the hardware workgroup id to a tile (tm, tn).
MICA_DEVICE void tile_of(int pid, int tiles_m, int tiles_n, int &tm, int &tn) {
    const int nt = tiles_m * tiles_n;
    // XCD-contiguous renumbering: XCD x = pid % 8 receives tiles [x * per + min(x, rem), ...)
    const int per = nt / kXcds, rem = nt % kXcds;
    const int x = pid % kXcds, local = pid / kXcds;
    const int t = x * per + (x < rem ? x : rem) + local;
    // grouped order: kGroupM M-tiles per group, walking N within the group
    const int width = kGroupM * tiles_n;
    const int first = (t / width) * kGroupM;
    const int gsize = (tiles_m - first) < kGroupM ? (tiles_m - first) : kGroupM;
    const int in = t % width;
    tm = first + in % gsize;
    tn = in / gsize;
}

// Piece h of the tail, whose rem tiles (tile ids dp .. dp + rem - 1 of tile_of) run as S pieces each
// (S = 2 halves or 4 quarters) on workgroups h, h + G, ...: the tile id and the piece's index in it.
// Workgroup h runs on XCD h % 8 and tile_of places tile id t on XCD t % 8; when every XCD holds the
// same number of tail tiles (rem % 8 == 0), the S pieces of a tile go to workgroups h on that XCD, so
// they share the tile's rows in one L2 (measured: a 256 x 128 half tile of 4096 x 9728 x 2560 had
// its pieces on different XCDs and ran 35 K cycles against 28 K with its operands resident in L2).
MICA_DEVICE void tail_piece(int h, int S, int dp, int rem, int &tile, int &part) {
    if (rem % kXcds == 0) {
        tile = dp + kXcds * (h / (kXcds * S)) + h % kXcds;
        part = (h / kXcds) % S;
    } else {
        tile = dp + h / S;
        part = h % S;
    }
}

template <int OUT>
MICA_DEVICE float to_out_precision(float v) {
    if (OUT == MICA_BF16) return round_bf16(v);
    if (OUT == MICA_FP16) return f16_to_f32(f32_to_f16(v));
    return v;
}

// store 4 consecutive outputs of one row (vector store when allowed, else element by element)
template <int OUT>
MICA_DEVICE void store4(void *C, long off, const float (&v)[4], int valid, bool vec) {
    if (OUT == MICA_BF16 || OUT == MICA_FP16) {
        uint16_t h[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) h[t] = OUT == MICA_BF16 ? f32_to_bf16(v[t]) : f32_to_f16(v[t]);
        uint16_t *p = (uint16_t *)C + off;
        if (vec && valid == 4) {
            u32x2 w;
            w[0] = (uint32_t)h[0] | ((uint32_t)h[1] << 16);
            w[1] = (uint32_t)h[2] | ((uint32_t)h[3] << 16);
            *(u32x2 *)p = w;
        } else {
            for (int t = 0; t < valid; ++t) p[t] = h[t];
        }
    } else {
        float *p = (float *)C + off;
        if (vec && valid == 4) *(float4 *)p = make_float4(v[0], v[1], v[2], v[3]);
        else for (int t = 0; t < valid; ++t) p[t] = v[t];
    }
}

template <int OUT>
MICA_DEVICE void load4_res(const void *R, long off, float (&v)[4], int valid, bool vec) {
    if (OUT == MICA_FP32) {
        const float *p = (const float *)R + off;
        if (vec && valid == 4) {
            const float4 t = *(const float4 *)p;
            v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
        } else {
            for (int t = 0; t < 4; ++t) v[t] = t < valid ? p[t] : 0.0f;
        }
        return;
    }
    const uint16_t *p = (const uint16_t *)R + off;
    uint16_t h[4] = {0, 0, 0, 0};
    if (vec && valid == 4) {
        const u32x2 w = *(const u32x2 *)p;
        h[0] = w[0] & 0xffff; h[1] = w[0] >> 16; h[2] = w[1] & 0xffff; h[3] = w[1] >> 16;
    } else {
        for (int t = 0; t < valid; ++t) h[t] = p[t];
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) v[t] = OUT == MICA_BF16 ? bf16_to_f32(h[t]) : f16_to_f32(h[t]);
}

// the wide kernel's launcher (gemm_i8_wide.hip)
int wide_launch(const GemmParams &p, int epilogue, int out_dtype, int grid, bool has_bias, bool has_res,
                bool narrow, hipStream_t st);
// the AGPR kernel's launcher (gemm_i8_agpr.hip): SCALE (bf16 / fp16) and SiLU (bf16) epilogues
int agpr_launch(const GemmParams &p, int epilogue, int out_dtype, int grid, bool has_bias, bool has_res,
                hipStream_t st);
int agpr_narrow_launch(const GemmParams &p, int out_dtype, int grid, bool has_bias, bool has_res, hipStream_t st);
int agpr_small_launch(const GemmParams &p, int out_dtype, int grid, bool has_bias, bool has_res, hipStream_t st);
int agpr_silu_small_launch(const GemmParams &p, int grid, hipStream_t st);
// the AGPR kernel's split-along-K schedule for few 128-row tiles (gemm_i8_agpr.hip)
int agpr_split_tile_n(int epilogue);
long long agpr_split_slot_bytes(int epilogue);
int agpr_split_launch(const GemmParams &p, int epilogue, int out_dtype, bool has_bias, bool has_res, hipStream_t st);

}  // namespace mica_gemm

using namespace mica_gemm;
