// The full-attention layers' extra steps around the attention kernel (the reference model's attention,
// fast_runtime.py:229-241, prefill_engine.py:123-130 and :317-331):
//
//   * head_norm_rope_kernel: per-head RMSNorm of the q and k heads (q_norm / k_norm, the zero-centred
//     Qwen3.5 RMSNorm that fork.install_norms routes to fused_kernels.rms_norm, fork.py:179-204:
//     y = bf16((x * rsqrt(mean(x^2) + eps)) * (offset + w))), then RoPE on the first rot_dim dims of each
//     head (partial rotary: rope_one, prefill_engine.py:83-89, x[..., :d] * cos + rotate_half(x[..., :d]) * sin
//     in bf16 ops, the other dims passed through), in place on the rows of the fused QKV projection.
//   * gate_quant_kernel: the output gate o * sigmoid(gate) (fast_runtime.py:240) in bf16 ops, then the
//     o_proj's per-token int8 quantization of the gated row (int8_quant.quant_act, half even), so the
//     gated bf16 row never goes to memory.
//
// Layouts: bf16 rows, head j of a segment at offset seg_off + j * head_dim of its row.

#include "common.h"

namespace {

// ---- per-head RMSNorm + partial RoPE ------------------------------------------------------------
// Thread = 8 consecutive dims (16 bytes) of one head; a head is head_dim / 8 consecutive lanes (a power
// of two dividing 64), so its reductions and the RoPE partner exchange stay inside the wave.
struct NormRopeParams {
    uint16_t *x; long long ldx;
    int T, q_off, n_q, k_off, n_k, head_dim;
    const uint16_t *wq, *wk;     // bf16 [head_dim] norm weights, or null: that segment is not normed
    float offset, eps;
    int rot_dim;                 // dims rotated at the head's start (0: none); cos / sin bf16 [n_pos][rot_dim / 2]
    const uint16_t *cs, *sn;
    const int *pos;              // int32 [T] positions, or null: t % period
    int period, n_pos;
    int tpl_log2;                // log2(head_dim / 8): lanes per head
};

constexpr int kNrThreads = 256;
constexpr int kNrRows = 4;   // tokens per thread and step

// sum over the `width` lanes of this lane's group (width a power of two <= 64, groups aligned): every
// lane of the group gets the same bits (a butterfly: lane l adds l ^ m's value, in the same order)
MICA_DEVICE float group_sum(float v, int width) {
    for (int m = 1; m < width; m <<= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// Grid (ceil((n_q + n_k) * lanes per head / 256), min(ceil(T / kNrRows), 65535)): blockIdx.x walks the
// heads of a token, blockIdx.y its tokens (grid-stride, kNrRows at a time), so a thread's head and dims
// come from shifts and no 64-bit division runs per thread.
__global__ __launch_bounds__(kNrThreads) void head_norm_rope_kernel(NormRopeParams p) {
    const int lg = p.tpl_log2;                             // lanes per head = 1 << lg
    const int per_tok = p.n_q + p.n_k;
    const int item = blockIdx.x * kNrThreads + threadIdx.x;
    // lanes past the token's last head keep the group's shuffles company on a valid head, and store nothing
    const bool live = item < (per_tok << lg);
    const int h = live ? item >> lg : per_tok - 1;
    const int part = item & ((1 << lg) - 1);               // this lane's 8 dims: 8 part .. 8 part + 7
    const bool is_q = h < p.n_q;
    const int col = is_q ? p.q_off + h * p.head_dim : p.k_off + (h - p.n_q) * p.head_dim;
    const uint16_t *w = is_q ? p.wq : p.wk;
    // kRows tokens per step, their loads issued before any of them is worked on (one 16-byte load per
    // token is too little in flight per wave to keep the memory busy)
    const int G = gridDim.y;
    for (int t0 = blockIdx.y; t0 < p.T; t0 += kNrRows * G) {
        u32x4 raws[kNrRows];
#pragma unroll
        for (int u = 0; u < kNrRows; ++u) {
            const int t = t0 + u * G;
            raws[u] = t < p.T ? *(const u32x4 *)(p.x + (long long)t * p.ldx + col + 8 * part) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < kNrRows; ++u) {
        const int t = t0 + u * G;
        if (t >= p.T) break;
        uint16_t *xh = p.x + (long long)t * p.ldx + col;
        float v[8];
        {
            const u32x4 raw = raws[u];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[2 * e] = bf16_lo(raw[e]);
                v[2 * e + 1] = bf16_hi(raw[e]);
            }
        }
        // the norm: every lane of a head takes the same branch (w is per segment)
        if (w != nullptr) {
            float ss = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(v[e], v[e], ss);
            ss = group_sum(ss, 1 << lg);
            const float rstd = 1.0f / __builtin_sqrtf(ss / (float)p.head_dim + p.eps);
            const u32x4 wr = *(const u32x4 *)(w + 8 * part);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[2 * e] = round_bf16((v[2 * e] * rstd) * (p.offset + bf16_lo(wr[e])));
                v[2 * e + 1] = round_bf16((v[2 * e + 1] * rstd) * (p.offset + bf16_hi(wr[e])));
            }
        }
        // RoPE on dims < rot_dim: dim i < rot_dim / 2 pairs with i + rot_dim / 2, held by lane part ^ (rot_dim / 16)
        u32x4 out;
        if (p.rot_dim > 0) {
            const int hl = p.rot_dim >> 4;                     // lanes per rotated half
            float o[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = __shfl_xor(v[e], hl, 64);
            const int pv = p.pos ? p.pos[t] : t % p.period;
            const bool rot = part < 2 * hl && pv >= 0 && pv < p.n_pos;   // out-of-table positions left unrotated
            if (rot) {
                const bool upper = part >= hl;
                const int i0 = (part & (hl - 1)) * 8;          // index into cos / sin (0 .. rot_dim / 2 - 1)
                const u32x4 c = *(const u32x4 *)(p.cs + (long long)pv * (p.rot_dim >> 1) + i0);
                const u32x4 s = *(const u32x4 *)(p.sn + (long long)pv * (p.rot_dim >> 1) + i0);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float cv = (e & 1) ? bf16_hi(c[e >> 1]) : bf16_lo(c[e >> 1]);
                    const float sv = (e & 1) ? bf16_hi(s[e >> 1]) : bf16_lo(s[e >> 1]);
                    // lower half: x_i cos_i - x_{i+h} sin_i; upper half: x_{i+h} cos_i + x_i sin_i
                    v[e] = upper ? round_bf16(v[e] * cv) + round_bf16(o[e] * sv)
                                 : round_bf16(v[e] * cv) + round_bf16(o[e] * -sv);
                }
            }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) out[e] = pack_bf16x2(v[2 * e], v[2 * e + 1]);
        if (live) *(u32x4 *)(xh + 8 * part) = out;
        }
    }
}

// ---- output gate + per-token int8 quantization ---------------------------------------------------
// One wave per row: lane l holds the 8 elements at c * 512 + 8 l of chunk c; y = bf16(a * bf16(sigmoid(g)))
// stays in registers from the absmax to the quantizer (the one-FMA half-even quantizer: exact for bf16
// rows).
struct GateQuantParams {
    const uint16_t *a; long long lda;
    const uint16_t *g; long long ldg;
    int8_t *q; long long ldq;
    float *s;
    uint16_t *y; long long ldy;   // optional bf16 gated rows
    int M;
};

// bf16(sigmoid(g)) for a bf16 value g: 1 / (1 + exp(-g)) with torch's fp32 steps (fp32 exp, fp32
// quotient, rounded to bf16): exp(-g) as v_exp_f32 of g * -log2(e), the reciprocal as v_rcp_f32 refined
// by one Newton step (0 once 1 + e overflows; a denominator of 2^64 or more scaled by 2^-64 first, since
// v_rcp_f32 flushes results below 2^-126).  The silu_bf16 construction of common.h, without the factor g.
MICA_DEVICE float sigmoid_bf16(float g) {
    const float e = __builtin_amdgcn_exp2f(g * -1.44269504088896341f);
    const float d = 1.0f + e;
    const float sc = d >= 0x1p64f ? 0x1p-64f : 1.0f;
    const float ds = d * sc;
    const float r0 = __builtin_amdgcn_rcpf(ds);
    const float r = ds < __builtin_inff() ? __builtin_fmaf(r0, __builtin_fmaf(-ds, r0, 1.0f), r0) : 0.0f;
    return round_bf16(r * sc);
}

template <int NCH>
__global__ __launch_bounds__(256) void gate_quant_kernel(GateQuantParams p) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= p.M) return;   // a whole wave leaves together
    const uint16_t *ar = p.a + (long long)row * p.lda + lane * 8;
    const uint16_t *gr = p.g + (long long)row * p.ldg + lane * 8;
    u32x4 araw[NCH], graw[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        araw[c] = *(const u32x4 *)(ar + c * 512);
        graw[c] = *(const u32x4 *)(gr + c * 512);
    }
    float y[NCH][8];
    float am = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            y[c][2 * e] = round_bf16(bf16_lo(araw[c][e]) * sigmoid_bf16(bf16_lo(graw[c][e])));
            y[c][2 * e + 1] = round_bf16(bf16_hi(araw[c][e]) * sigmoid_bf16(bf16_hi(graw[c][e])));
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) am = __builtin_fmaxf(am, __builtin_fabsf(y[c][j]));
    }
    am = wave_max(am);
    const float sc = row_scale(am);
    const float rf = fma_quant_recip(am, sc, 1.0f / sc);
    if (lane == 0) p.s[row] = sc;
    int8_t *qr = p.q + (long long)row * p.ldq + lane * 8;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        __builtin_nontemporal_store(fma_quant8(y[c], rf), (u32x2 *)(qr + c * 512));
        if (p.y != nullptr) {
            u32x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = pack_bf16x2(y[c][2 * e], y[c][2 * e + 1]);
            *(u32x4 *)(p.y + (long long)row * p.ldy + lane * 8 + c * 512) = o;
        }
    }
}

bool pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

}  // namespace

extern "C" int mica_head_norm_rope(void *x, long long ldx, int T, int q_off, int n_q, int k_off, int n_k,
                                   int head_dim, const void *q_norm_w, const void *k_norm_w, float offset, float eps,
                                   int rot_dim, const void *cos_tab, const void *sin_tab, int n_pos, const int *pos,
                                   int period, mica_stream_t stream) {
    if (x == nullptr) return MICA_MISS_ARG;
    if (T < 0 || n_q < 0 || n_k < 0 || q_off < 0 || k_off < 0 || head_dim < 16 || head_dim > 512 ||
        !pow2(head_dim))
        return MICA_MISS_SHAPE;
    if (rot_dim != 0 && (rot_dim < 16 || rot_dim > head_dim || !pow2(rot_dim))) return MICA_MISS_SHAPE;
    if (rot_dim != 0 && (cos_tab == nullptr || sin_tab == nullptr || n_pos <= 0 || (pos == nullptr && period <= 0)))
        return MICA_MISS_ARG;
    if (q_off % 8 || k_off % 8 || ldx % 8 || ldx < (long long)q_off + (long long)n_q * head_dim ||
        ldx < (long long)k_off + (long long)n_k * head_dim)
        return MICA_MISS_STRIDE;
    if (!mica_aligned16(x) || (q_norm_w && !mica_aligned16(q_norm_w)) || (k_norm_w && !mica_aligned16(k_norm_w)) ||
        (rot_dim && (!mica_aligned16(cos_tab) || !mica_aligned16(sin_tab))))
        return MICA_MISS_ALIGN;
    const long long heads = (long long)T * (n_q + n_k);
    if (heads == 0) return 0;
    const long long per_tok = (long long)(n_q + n_k) * (head_dim / 8);   // (head, 8 dims) items of a token
    const long long bx = (per_tok + kNrThreads - 1) / kNrThreads;
    if (bx >= (1LL << 31) || (long long)T * ldx >= (1LL << 62)) return MICA_MISS_RANGE;
    NormRopeParams p{};
    p.x = (uint16_t *)x; p.ldx = ldx; p.T = T; p.q_off = q_off; p.n_q = n_q; p.k_off = k_off; p.n_k = n_k;
    p.head_dim = head_dim; p.wq = (const uint16_t *)q_norm_w; p.wk = (const uint16_t *)k_norm_w;
    p.offset = offset; p.eps = eps; p.rot_dim = rot_dim; p.cs = (const uint16_t *)cos_tab;
    p.sn = (const uint16_t *)sin_tab; p.pos = pos; p.period = period; p.n_pos = n_pos;
    p.tpl_log2 = __builtin_ctz((unsigned)(head_dim / 8));
    const int gy = (T + kNrRows - 1) / kNrRows;
    hipLaunchKernelGGL(head_norm_rope_kernel, dim3((unsigned)bx, (unsigned)(gy < 65535 ? gy : 65535)), dim3(kNrThreads), 0,
                       (hipStream_t)stream, p);
    return mica_err(hipGetLastError());
}

extern "C" int mica_gate_quant(const void *a, long long lda, const void *gate, long long ldg, int8_t *q, long long ldq,
                               float *s, void *y, long long ldy, int M, int K, int rounding, mica_stream_t stream) {
    if (a == nullptr || gate == nullptr || q == nullptr || s == nullptr) return MICA_MISS_ARG;
    if (rounding != MICA_ROUND_EVEN) return MICA_MISS_ARG;
    if (M < 0 || K < 512 || K % 512 != 0 || K > 8192) return MICA_MISS_SHAPE;
    if (lda < K || ldg < K || ldq < K || (y && ldy < K) || lda % 8 || ldg % 8 || ldq % 16 || (y && ldy % 8))
        return MICA_MISS_STRIDE;
    if (!mica_aligned16(a) || !mica_aligned16(gate) || !mica_aligned16(q) || !mica_aligned16(s) ||
        (y && !mica_aligned16(y)))
        return MICA_MISS_ALIGN;
    if (M == 0) return 0;
    GateQuantParams p{};
    p.a = (const uint16_t *)a; p.lda = lda; p.g = (const uint16_t *)gate; p.ldg = ldg; p.q = q; p.ldq = ldq;
    p.s = s; p.y = (uint16_t *)y; p.ldy = ldy; p.M = M;
    const unsigned blocks = (unsigned)((M + 3) / 4);
    hipStream_t st = (hipStream_t)stream;
    switch (K / 512) {
#define MICA_GQ(n) case n: hipLaunchKernelGGL(gate_quant_kernel<n>, dim3(blocks), dim3(256), 0, st, p); break;
        MICA_GQ(1) MICA_GQ(2) MICA_GQ(3) MICA_GQ(4) MICA_GQ(5) MICA_GQ(6) MICA_GQ(7) MICA_GQ(8)
        MICA_GQ(9) MICA_GQ(10) MICA_GQ(11) MICA_GQ(12) MICA_GQ(13) MICA_GQ(14) MICA_GQ(15) MICA_GQ(16)
#undef MICA_GQ
        default: return MICA_MISS_SHAPE;
    }
    return mica_err(hipGetLastError());
}
