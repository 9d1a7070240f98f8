// Last-position readout: gather each request's last hidden row, apply the final RMSNorm,
// dot it (fp32) with the allowed answer rows only, and softmax each request's slice.
//
// One workgroup (256 threads) per request.  The normed row lives in LDS as fp32; each of the
// 4 wavefronts takes every 4th label row, its lanes stride over K with 16-byte loads, and a
// wavefront reduction finishes the dot.  Logits stay in LDS for the softmax.  Work is
// B x L x K multiply-adds (8 x 257 x 2560 = 5.3 M): latency bound, one launch.

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

__global__ __launch_bounds__(kThreads) void readout_kernel(ReadoutParams p) {
    __shared__ float xs[kMaxK];
    __shared__ float zs[kMaxL];
    __shared__ float red[kThreads / 64];
    const int b = blockIdx.x;
    const int K = p.K, L = p.L;
    const int row = p.rows[b];
    if (row < 0 || row >= p.n_rows) { // an index the host could not check: NaN results, no access
        for (int j = threadIdx.x; j < L; j += kThreads) p.logits[(long)b * L + j] = __builtin_nanf("");
        if (p.probs != nullptr)
            for (int i = threadIdx.x; i < p.ldp; i += kThreads) p.probs[(long)b * p.ldp + i] = __builtin_nanf("");
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
    for (int j = wave; j < L; j += kThreads / 64) {
        const int wi = p.ids != nullptr ? p.ids[j] : j;
        if (wi < 0 || wi >= p.w_rows) {
            if (lane == 0) {
                zs[j] = __builtin_nanf("");
                p.logits[(long)b * L + j] = __builtin_nanf("");
            }
            continue;
        }
        const long wr = (long)wi * p.ldw;
        float acc = 0.0f;
        if (p.w_dtype == MICA_FP32) {
            const float *wrow = (const float *)p.W + wr;
            for (int k = lane * 4; k < K; k += 256) {
                const float4 w4 = *(const float4 *)(wrow + k);
                acc = __builtin_fmaf(xs[k], w4.x, acc);
                acc = __builtin_fmaf(xs[k + 1], w4.y, acc);
                acc = __builtin_fmaf(xs[k + 2], w4.z, acc);
                acc = __builtin_fmaf(xs[k + 3], w4.w, acc);
            }
        } else {
            const uint16_t *wrow = (const uint16_t *)p.W + wr;
            for (int k = lane * 8; k < K; k += 512) {
                const u32x4 c = *(const u32x4 *)(wrow + k);
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    acc = __builtin_fmaf(xs[k + 2 * t], bf16_lo(c[t]), acc);
                    acc = __builtin_fmaf(xs[k + 2 * t + 1], bf16_hi(c[t]), acc);
                }
            }
        }
        acc = wave_sum(acc);
        if (lane == 0) {
            zs[j] = acc;
            p.logits[(long)b * L + j] = acc;
        }
    }
    __syncthreads();
    if (p.probs == nullptr) return;

    // softmax over logits[lo, lo + n) (release_runtime.py:509-517)
    // the slice [lo, lo + n) is clipped to the logits and to the probs row
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
    float *pr = p.probs + (long)b * p.ldp;
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
    hipLaunchKernelGGL(readout_kernel, dim3(B), dim3(kThreads), 0, (hipStream_t)stream, p);
    return mica_err(hipGetLastError());
}
