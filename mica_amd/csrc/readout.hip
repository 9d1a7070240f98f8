// Last-position readout: gather each request's last hidden row, apply the final RMSNorm,
// dot it (fp32) with the allowed answer rows only, and softmax each request's slice.
//
// Two launches: logits over a (request, 16 label rows) grid, so the label rows' loads of all
// requests are in flight at once (one workgroup per request took ~300 us, each lane waiting for
// one 16-byte load at a time), then one small softmax workgroup per request.  The normed row lives
// in LDS as fp32; a wavefront reduction finishes each dot.  Work is B x L x K multiply-adds
// (8 x 257 x 2560 = 5.3 M) and the label rows (2.6 MB fp32) read once per request.

#include "common.h"

namespace {

constexpr int kMaxK = 8192;
constexpr int kMaxL = 8192;
constexpr int kThreads = 256;

struct ReadoutParams {
    const uint16_t *h;
    const int *rows;
    const void *norm_w;
    const void *W;
    const int *ids;
    const int *lo;
    const int *cnt;
    float *logits;
    float *probs;
    int ldh, ldw, ldp;
    int n_rows, w_rows;
    int B, L, K;
    int norm_dtype, w_dtype;
    float offset, eps;
};

__device__ float block_sum(float v, float *scratch) {
    v = wave_sum(v);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < kThreads / 64; ++i) t += scratch[i];
    return t;
}

__device__ float block_max(float v, float *scratch) {
    v = wave_max(v);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    float t = -INFINITY;
    for (int i = 0; i < kThreads / 64; ++i) t = fmaxf(t, scratch[i]);
    return t;
}

constexpr int kRowsPerBlock = 16; // label rows per workgroup of the logits kernel (4 per wave)
constexpr int kBatch = 8;          // 16-byte weight loads a lane issues before using any of them

// Logits: grid (B, ceil(L / 16)).  Every workgroup gathers and norms its request's row into LDS (a
// few KB, recomputed per workgroup), then each wave dots 4 label rows with it; a lane walks K with
// stride 64 x 4 (fp32) or 64 x 8 (bf16) elements and issues kBatch loads before the multiply-adds.
__global__ __launch_bounds__(kThreads) void readout_logits_kernel(ReadoutParams p) {
    __shared__ float xs[kMaxK];
    __shared__ float red[kThreads / 64];
    const int b = blockIdx.x, j0 = blockIdx.y * kRowsPerBlock;
    const int K = p.K, L = p.L;
    const int row = p.rows[b];
    if (row < 0 || row >= p.n_rows) { // an index the host could not check: NaN results, no access
        for (int j = j0 + (int)threadIdx.x; j < L && j < j0 + kRowsPerBlock; j += kThreads)
            p.logits[(long)b * L + j] = __builtin_nanf("");
        return;
    }
    const uint16_t *hr = p.h + (long)row * p.ldh;

    // gather the row (bf16 -> fp32) and its sum of squares
    float ss = 0.0f;
    for (int k = threadIdx.x; k < K; k += kThreads) {
        const float v = bf16_to_f32(hr[k]);
        xs[k] = v;
        ss = __builtin_fmaf(v, v, ss);
    }
    if (p.norm_w != nullptr) {
        ss = block_sum(ss, red);
        const float rstd = 1.0f / __builtin_sqrtf(ss / (float)K + p.eps);
        for (int k = threadIdx.x; k < K; k += kThreads) {
            const float w1 = p.offset + load_as_f32(p.norm_w, p.norm_dtype, k);
            xs[k] = round_bf16((xs[k] * rstd) * w1); // body.norm returns bf16 (fused_kernels.py:55)
        }
    }
    __syncthreads();

    // logits[b, j] = sum_k x[k] * W[row_j, k]
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int j = j0 + wave; j < L && j < j0 + kRowsPerBlock; j += kThreads / 64) {
        const int wi = p.ids != nullptr ? p.ids[j] : j;
        if (wi < 0 || wi >= p.w_rows) {
            if (lane == 0) p.logits[(long)b * L + j] = __builtin_nanf("");
            continue;
        }
        const long wr = (long)wi * p.ldw;
        float acc = 0.0f;
        if (p.w_dtype == MICA_FP32) {
            const float *wrow = (const float *)p.W + wr;
            for (int k0 = lane * 4; k0 < K; k0 += 256 * kBatch) {
                float4 w4[kBatch];
#pragma unroll
                for (int u = 0; u < kBatch; ++u)
                    if (k0 + 256 * u < K) w4[u] = *(const float4 *)(wrow + k0 + 256 * u);
#pragma unroll
                for (int u = 0; u < kBatch; ++u) {
                    const int k = k0 + 256 * u;
                    if (k >= K) break;
                    acc = __builtin_fmaf(xs[k], w4[u].x, acc);
                    acc = __builtin_fmaf(xs[k + 1], w4[u].y, acc);
                    acc = __builtin_fmaf(xs[k + 2], w4[u].z, acc);
                    acc = __builtin_fmaf(xs[k + 3], w4[u].w, acc);
                }
            }
        } else {
            const uint16_t *wrow = (const uint16_t *)p.W + wr;
            for (int k0 = lane * 8; k0 < K; k0 += 512 * kBatch) {
                u32x4 c[kBatch];
#pragma unroll
                for (int u = 0; u < kBatch; ++u)
                    if (k0 + 512 * u < K) c[u] = *(const u32x4 *)(wrow + k0 + 512 * u);
#pragma unroll
                for (int u = 0; u < kBatch; ++u) {
                    const int k = k0 + 512 * u;
                    if (k >= K) break;
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        acc = __builtin_fmaf(xs[k + 2 * t], bf16_lo(c[u][t]), acc);
                        acc = __builtin_fmaf(xs[k + 2 * t + 1], bf16_hi(c[u][t]), acc);
                    }
                }
            }
        }
        acc = wave_sum(acc);
        if (lane == 0) p.logits[(long)b * L + j] = acc;
    }
}

// Softmax over logits[b, lo, lo + n) (release_runtime.py:509-517), one workgroup per request; the
// slice [lo, lo + n) is clipped to the logits and to the probs row.
__global__ __launch_bounds__(kThreads) void readout_softmax_kernel(ReadoutParams p) {
    __shared__ float red[kThreads / 64];
    const int b = blockIdx.x, L = p.L;
    float *pr = p.probs + (long)b * p.ldp;
    const int row = p.rows[b];
    if (row < 0 || row >= p.n_rows) {
        for (int i = threadIdx.x; i < p.ldp; i += kThreads) pr[i] = __builtin_nanf("");
        return;
    }
    const float *zs = p.logits + (long)b * L;
    int lo = p.lo != nullptr ? p.lo[b] : 0;
    int n = p.cnt != nullptr ? p.cnt[b] : L;
    lo = lo < 0 ? 0 : (lo > L ? L : lo);
    n = n < 0 ? 0 : n;
    n = n > L - lo ? L - lo : n;
    n = n > p.ldp ? p.ldp : n;
    float mx = -INFINITY;
    for (int i = threadIdx.x; i < n; i += kThreads) mx = fmaxf(mx, zs[lo + i]);
    mx = block_max(mx, red);
    float se = 0.0f;
    for (int i = threadIdx.x; i < n; i += kThreads) se += expf(zs[lo + i] - mx);
    se = block_sum(se, red);
    for (int i = threadIdx.x; i < n; i += kThreads) pr[i] = expf(zs[lo + i] - mx) / se;
}

}  // namespace

extern "C" int mica_gather_logits(const void *h, int ldh, int n_rows, const int *rows, int B, const void *norm_w,
                                  int norm_dtype, float offset, float eps, const void *W, int w_dtype, int ldw,
                                  int w_rows, const int *ids, int L, int K, float *logits, const int *lo,
                                  const int *cnt, float *probs, int ldp, mica_stream_t stream) {
    if (h == nullptr || rows == nullptr || W == nullptr || logits == nullptr) return MICA_MISS_ARG;
    if ((lo == nullptr) != (cnt == nullptr)) return MICA_MISS_ARG;
    if (w_dtype != MICA_FP32 && w_dtype != MICA_BF16) return MICA_MISS_DTYPE;
    if (norm_w != nullptr && norm_dtype != MICA_BF16 && norm_dtype != MICA_FP16 && norm_dtype != MICA_FP32)
        return MICA_MISS_DTYPE;
    if (B < 0 || L <= 0 || L > kMaxL || K <= 0 || K > kMaxK) return MICA_MISS_SHAPE;
    if (K % (w_dtype == MICA_FP32 ? 4 : 8) != 0) return MICA_MISS_SHAPE;
    if (n_rows <= 0 || w_rows <= 0 || (ids == nullptr && w_rows < L)) return MICA_MISS_SHAPE;
    if (ldh < K || ldw < K || ldw % 8 != 0 || (probs != nullptr && ldp <= 0)) return MICA_MISS_STRIDE;
    if (!mica_aligned16(W)) return MICA_MISS_ALIGN;
    if (B == 0) return 0;
    ReadoutParams p{};
    p.h = (const uint16_t *)h; p.rows = rows; p.norm_w = norm_w; p.W = W; p.ids = ids; p.lo = lo; p.cnt = cnt;
    p.logits = logits; p.probs = probs; p.ldh = ldh; p.ldw = ldw; p.ldp = ldp; p.B = B; p.L = L; p.K = K;
    p.n_rows = n_rows; p.w_rows = w_rows;
    p.norm_dtype = norm_dtype; p.w_dtype = w_dtype; p.offset = offset; p.eps = eps;
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(readout_logits_kernel, dim3(B, (L + kRowsPerBlock - 1) / kRowsPerBlock), dim3(kThreads), 0, st, p);
    if (p.probs != nullptr) hipLaunchKernelGGL(readout_softmax_kernel, dim3(B), dim3(kThreads), 0, st, p);
    return mica_err(hipGetLastError());
}
