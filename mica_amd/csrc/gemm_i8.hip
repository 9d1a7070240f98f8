// W8A8 GEMM on the gfx950 matrix cores: C = epilogue(A[M, K] . B[N, K]^T), int8 x int8 -> int32.
//
// Tiling (one workgroup = 4 wavefronts = 256 threads, one workgroup per CU):
//   * workgroup tile 256 (M) x 256 (N), K staged 128 bytes at a time;
//   * the 4 waves form a 2 x 2 grid, each owns a 128 x 128 block = 4 x 4 tiles of
//     v_mfma_i32_32x32x32_i8 (256 int32 accumulators per lane, held in AGPRs);
//   * A and B K-slabs ([256][128] bytes each) are double-buffered in LDS (128 KiB total):
//     while the waves run the MFMAs of slab k, the 16-byte global loads of slab k + 1 are in
//     flight, and are written to the other buffer afterwards; one barrier per slab;
//   * LDS rows are 128 bytes = 8 chunks of 16 bytes; chunk c of row r is stored at chunk
//     c ^ ((r ^ (r >> 3)) & 7).  The 16-byte reads of an MFMA operand (32 consecutive rows,
//     one chunk) and the 16-byte writes of a slab (8 lanes per row) then touch every bank once
//     per 8 (32 banks) or 16 (64 banks) lanes: no bank conflicts in either direction.
//
// Workgroup order: the hardware hands workgroup i to XCD i % 8, and each XCD has its own L2.
// Workgroups are renumbered so each XCD gets one contiguous range of tiles, and inside a range
// tiles go in groups of kGroupM M-tiles, column by column, so the workgroups that run together
// on an XCD share A and B panels in that XCD's L2.
//
// Epilogue (per accumulator): y = (f32(acc) * sa[m]) * sb[n] (+ bias[n]) in this order
// (kernel_src/kernels.py:65-67, int8_runtime.py:186-190), converted with round-to-nearest-even
// (fp32 -> bf16 via v_cvt_pk_bf16_f32).  SILU_MUL pairs gate and up columns held by the same
// lane (see mica_amd.h).  The residual is added after that rounding.

#include "common.h"

namespace {

constexpr int BM = 256;
constexpr int BN = 256;
constexpr int BK = 128;     // bytes of K per LDS slab
constexpr int WM = 128;     // wave tile
constexpr int WN = 128;
constexpr int MB = WM / 32; // 32x32 MFMA tiles per wave along M
constexpr int NB = WN / 32;
constexpr int KS = BK / 32; // MFMA k-steps per slab
constexpr int kThreads = 256;
constexpr int kLoadIters = BM * BK / 16 / kThreads; // 16-byte chunks per thread per operand = 8
constexpr int kSlab = (BM + BN) * BK;               // bytes of one LDS stage
constexpr int kGroupM = 8;
constexpr int kXcds = 8;
// word 3 of a gfx9 buffer resource (raw buffer, 32-bit data format), as used by CK for gfx9xx
constexpr int kBufferFlags = 0x00020000;
// a buffer offset that fails the range check (every buffer here is < 2^31 bytes)
constexpr int kOutOfRange = (int)0x80000000u;

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
    int tiles_m, tiles_n;
};

MICA_DEVICE int swz(int row) { return (row ^ (row >> 3)) & 7; }

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

template <int OUT>
MICA_DEVICE void store_out(void *C, long off, float v) {
    if (OUT == MICA_BF16) ((uint16_t *)C)[off] = f32_to_bf16(v);
    else if (OUT == MICA_INT32) return; // raw accumulators are stored by the caller
    else if (OUT == MICA_FP16) ((uint16_t *)C)[off] = f32_to_f16(v);
    else ((float *)C)[off] = v;
}

template <int OUT>
MICA_DEVICE float load_res(const void *R, long off) {
    if (OUT == MICA_BF16) return bf16_to_f32(((const uint16_t *)R)[off]);
    if (OUT == MICA_FP16) return f16_to_f32(((const uint16_t *)R)[off]);
    return ((const float *)R)[off];
}

template <int EPI, int OUT, bool HAS_BIAS, bool HAS_RES>
__global__ __launch_bounds__(kThreads, 1) void gemm_i8_kernel(GemmParams p) {
    __shared__ __attribute__((aligned(16))) int8_t smem[2 * kSlab];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    int tm, tn;
    tile_of(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int M = p.M, N = p.N, K = p.K;

    // ---- global -> register -> LDS staging: thread owns chunk (tid & 7) of rows j*32 + tid/8 ----
    // Raw buffer loads: offsets are 32-bit and a load whose offset lies past the buffer's
    // range returns zeros, so rows past M / N and chunks past K read as 0 without branches.
    const __amdgpu_buffer_rsrc_t rsrc_a =
        __builtin_amdgcn_make_buffer_rsrc((void *)p.A, 0, p.M * p.lda, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rsrc_b =
        __builtin_amdgcn_make_buffer_rsrc((void *)p.B, 0, p.N * p.ldb, kBufferFlags);
    const int lrow = tid >> 3, lkc = tid & 7;
    int a_off[kLoadIters], b_off[kLoadIters], l_off[kLoadIters];
#pragma unroll
    for (int j = 0; j < kLoadIters; ++j) {
        const int row = j * 32 + lrow;
        a_off[j] = m0 + row < M ? (m0 + row) * p.lda + lkc * 16 : kOutOfRange;
        b_off[j] = n0 + row < N ? (n0 + row) * p.ldb + lkc * 16 : kOutOfRange;
        l_off[j] = row * BK + ((lkc ^ swz(row)) << 4);
    }
    v4i ra[kLoadIters], rb[kLoadIters];
    auto gload = [&](int k0) {
        const bool kout = k0 + lkc * 16 >= K; // K % 16 == 0: a chunk is all in or all out
#pragma unroll
        for (int j = 0; j < kLoadIters; ++j) {
            const int oa = kout ? kOutOfRange : a_off[j] + k0;
            const int ob = kout ? kOutOfRange : b_off[j] + k0;
            ra[j] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rsrc_a, oa, 0, 0));
            rb[j] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rsrc_b, ob, 0, 0));
        }
    };
    auto lstore = [&](int buf) {
        int8_t *As = smem + buf * kSlab;
        int8_t *Bs = As + BM * BK;
#pragma unroll
        for (int j = 0; j < kLoadIters; ++j) {
            *(v4i *)(As + l_off[j]) = ra[j];
            *(v4i *)(Bs + l_off[j]) = rb[j];
        }
    };

    v16i acc[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = v16i{};

    const int khalf = lane >> 5;
    const int r32 = lane & 31;

    gload(0);
    lstore(0);
    __syncthreads();

    const int nk = (K + BK - 1) / BK;
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * BK);
        const int8_t *As = smem + buf * kSlab;
        const int8_t *Bs = As + BM * BK;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int kc = ks * 2 + khalf;
            v4i a[MB], b[NB];
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                const int row = wm * WM + i * 32 + r32;
                a[i] = *(const v4i *)(As + row * BK + ((kc ^ swz(row)) << 4));
            }
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const int row = wn * WN + j * 32 + r32;
                b[j] = *(const v4i *)(Bs + row * BK + ((kc ^ swz(row)) << 4));
            }
#pragma unroll
            for (int i = 0; i < MB; ++i)
#pragma unroll
                for (int j = 0; j < NB; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) lstore(buf ^ 1);
        __syncthreads();
    }

    // ---- epilogue.  acc[i][j][r]: row = 8 (r / 4) + 4 (lane / 32) + r % 4, col = lane % 32 ----
    const int mw = m0 + wm * WM;
    const int nw = n0 + wn * WN;
    if (EPI == MICA_EPI_SCALE) {
        float sbv[NB], bv[NB];
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int n = nw + j * 32 + r32;
            sbv[j] = n < N ? p.sb[n] : 0.0f;
            bv[j] = (HAS_BIAS && n < N) ? p.bias[n] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < MB; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = mw + i * 32 + 8 * (r >> 2) + 4 * khalf + (r & 3);
                if (m >= M) continue;
                const float sav = p.sa[m];
#pragma unroll
                for (int j = 0; j < NB; ++j) {
                    const int n = nw + j * 32 + r32;
                    if (n >= N) continue;
                    if (OUT == MICA_INT32) {
                        ((int *)p.C)[(long)m * p.ldc + n] = acc[i][j][r];
                        continue;
                    }
                    float y = ((float)acc[i][j][r] * sav) * sbv[j];
                    if (HAS_BIAS) y = y + bv[j];
                    if (HAS_RES) {
                        y = round_to(y, OUT) + load_res<OUT>(p.res, (long)m * p.ldr + n);
                    }
                    store_out<OUT>(p.C, (long)m * p.ldc + n, y);
                }
            }
        }
    } else {
        // SILU_MUL: this wave's 128 B-rows are one interleave group g = nw / 128:
        // rows [0, 64) are gate columns 64 g + [0, 64), rows [64, 128) the matching up columns.
        const int g = nw >> 7;
        float sgv[2], suv[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int ng = nw + j * 32 + r32;
            sgv[j] = ng < N ? p.sb[ng] : 0.0f;
            suv[j] = ng + 64 < N ? p.sb[ng + 64] : 0.0f;
        }
        const int Nout = N >> 1;
#pragma unroll
        for (int i = 0; i < MB; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = mw + i * 32 + 8 * (r >> 2) + 4 * khalf + (r & 3);
                if (m >= M) continue;
                const float sav = p.sa[m];
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int col = g * 64 + j * 32 + r32;
                    if (col >= Nout) continue;
                    const float gv = round_bf16(((float)acc[i][j][r] * sav) * sgv[j]);
                    const float uv = round_bf16(((float)acc[i][j + 2][r] * sav) * suv[j]);
                    const float act = round_bf16(gv / (1.0f + expf(-gv)));
                    ((uint16_t *)p.C)[(long)m * p.ldc + col] = f32_to_bf16(act * uv);
                }
            }
        }
    }
}

template <int EPI, int OUT>
int launch_out(const GemmParams &p, bool has_bias, bool has_res, hipStream_t st) {
    dim3 grid(p.tiles_m * p.tiles_n), block(kThreads);
#define MICA_G(B_, R_) hipLaunchKernelGGL((gemm_i8_kernel<EPI, OUT, B_, R_>), grid, block, 0, st, p)
    if (EPI == MICA_EPI_SILU_MUL) MICA_G(false, false);
    else if (has_bias && has_res) MICA_G(true, true);
    else if (has_bias) MICA_G(true, false);
    else if (has_res) MICA_G(false, true);
    else MICA_G(false, false);
#undef MICA_G
    return mica_err(hipGetLastError());
}

}  // namespace

extern "C" int mica_mm_i8(const int8_t *A, int lda, const int8_t *B, int ldb, const float *sa, const float *sb,
                          const float *bias, const void *residual, int ldr, void *C, int ldc, int out_dtype, int M,
                          int N, int K, int epilogue, mica_stream_t stream) {
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
        !mica_aligned16(C) || (bias && !mica_aligned16(bias)) || (residual && !mica_aligned16(residual)))
        return MICA_MISS_ALIGN;
    if (M == 0) return 0;
    GemmParams p{};
    p.A = A; p.B = B; p.sa = sa; p.sb = sb; p.bias = bias; p.res = residual; p.C = C;
    p.lda = lda; p.ldb = ldb; p.ldr = ldr; p.ldc = ldc; p.M = M; p.N = N; p.K = K;
    p.tiles_m = (M + BM - 1) / BM;
    p.tiles_n = (N + BN - 1) / BN;
    if ((long long)p.tiles_m * p.tiles_n >= (1ll << 31)) return MICA_MISS_RANGE;
    hipStream_t st = (hipStream_t)stream;
    const bool hb = bias != nullptr, hr = residual != nullptr;
    if (epilogue == MICA_EPI_SILU_MUL) return launch_out<MICA_EPI_SILU_MUL, MICA_BF16>(p, false, false, st);
    if (out_dtype == MICA_BF16) return launch_out<MICA_EPI_SCALE, MICA_BF16>(p, hb, hr, st);
    if (out_dtype == MICA_FP16) return launch_out<MICA_EPI_SCALE, MICA_FP16>(p, hb, hr, st);
    if (out_dtype == MICA_INT32) return launch_out<MICA_EPI_SCALE, MICA_INT32>(p, false, false, st);
    return launch_out<MICA_EPI_SCALE, MICA_FP32>(p, hb, hr, st);
}
