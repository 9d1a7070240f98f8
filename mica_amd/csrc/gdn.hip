// Gated delta net (GDN) token mixer on gfx950: the causal depthwise convolution in front of it and
// the chunked gated-delta-rule scan (the reference's causal_conv1d_fn + chunk_gated_delta_rule,
// v0.5/serving/lib/fork.py:71-147; the scan's arithmetic is that of flash-linear-attention 0.5.2's
// chunk_gated_delta_rule, which the reference calls).
//
// Recurrence, per sequence b and value head h, state S [128 (dk), 128 (dv)]:
//     S <- exp(g_t) S;   S <- S + k_t (beta_t (v_t - S^T k_t))^T;   o_t = scale S^T q_t
// computed 64 tokens (one chunk) at a time in the WY form:
//     G = in-chunk cumulative sum of g;  L[i][j] = beta_i (k_i . k_j) exp(G_i - G_j), j < i
//     T = (I + L)^-1;  W = T (beta exp(G) K);  U = T (beta V)                       (prep kernel)
//     v_new = U - W S;  o = scale (exp(G) (Q S) + [(Q K^T) exp(G_i - G_j)]_{j<=i} v_new)
//     S <- exp(G_63) S + K^T (exp(G_63 - G) v_new)                                   (scan kernel)
// Matrix products run on v_mfma_f32_32x32x16_bf16 with bf16 operands and fp32 accumulation;
// T, W, U, S, v_new and the masked Q K^T are rounded to bf16 where they enter a product, as in the
// reference's kernels.  The state stays in fp32 accumulators between chunks.
//
// Work split.  prep: one workgroup per (sequence, value head, chunk) -- fully parallel -- writes
// W and U in the register layouts the scan consumes, plus G.  scan: one workgroup per (sequence,
// value head), 8 waves; chunks in order; every product of a chunk is one MFMA pass over
// LDS-resident tiles, two barriers per chunk.  No per-chunk state is stored to memory.

#include "common.h"

namespace {

constexpr int kDk = 128, kDv = 128; // head dims (Qwen3.5 GDN: linear_key_head_dim = linear_value_head_dim = 128)
constexpr int kC = 64;              // chunk length
constexpr int kGdnThreads = 256;    // 4 waves

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

MICA_DEVICE f32x16 mfma(const bf16x8 &a, const bf16x8 &b, const f32x16 &c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
MICA_DEVICE bf16x8 as_bf16x8(const u32x4 &v) { return __builtin_bit_cast(bf16x8, v); }
MICA_DEVICE bf16x8 ld_frag(const void *p) { return __builtin_bit_cast(bf16x8, *(const u32x4 *)p); }

// Accumulator element r of a 32 x 32 tile in lane l: row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32.
MICA_DEVICE int acc_row(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

// exp(x) as v_exp_f32 (2^x) of x log2(e): a few ulps, enough for the decay factors (all <= 1 here)
MICA_DEVICE float fexp(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }
// silu(x) = x / (1 + exp(-x)) with the hardware exp2 and reciprocal (a few ulps in fp32; the
// outputs are rounded to bf16 after it)
MICA_DEVICE float fsilu(float x) { return x * __builtin_amdgcn_rcpf(1.0f + fexp(-x)); }

// Sum of a value over the 4 lanes of each quad (DPP quad permutations [1,0,3,2] and [2,3,0,1]);
// each move can fold into the add that follows it (v_add_f32 with a DPP source).
MICA_DEVICE float quad_sum(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));
    return v;
}

// ================================================================================================
// Causal depthwise convolution (width W <= 4) + optional SiLU, then optional l2 normalisation of
// each of the first n_norm 128-channel heads (the q / k heads).  One thread: kConvT consecutive
// tokens x 8 channels; its kConvT + 3 input rows are loaded together before any math, and the
// weights once.  out[t][c] = act(bias[c] + sum_j w[c][j] x[t - W + 1 + j][c]) in fp32 (the order
// of causal_conv1d_fn), rounded to bf16; the l2 norm rescales the rounded values by
// 1 / sqrt(sum x^2 + eps) and rounds again.
constexpr int kConvThreads = 256; // 2048 channels per workgroup
constexpr int kConvT = 8;         // tokens per thread

struct ConvParams {
    const uint16_t *x; long long sbx; int ldx;   // bf16 [B][T][C], strides in elements
    const void *w; const void *bias; int w_dtype; int width; // [C][width]
    int w_vec;                                   // width 4, bf16, 16-byte aligned: vector weight loads
    const uint16_t *init;                        // bf16 [B][C][width - 1] or null
    uint16_t *final_state;                       // bf16 [B][C][width - 1] or null
    uint16_t *y; long long sby; int ldy;         // bf16 out
    int B, T, C, silu, n_norm; float eps;
};

template <int W>
__global__ __launch_bounds__(kConvThreads) void conv_kernel(ConvParams p) {
    const int b = blockIdx.z, t0 = blockIdx.y * kConvT;
    const int c0 = (blockIdx.x * kConvThreads + threadIdx.x) * 8;
    const bool active = c0 < p.C;
    // slot j holds input row t0 - 3 + j (j = 0 .. kConvT + 2); output t0 + i uses slots i + 4 - W .. i + 3
    u32x4 rows[kConvT + 3];
#pragma unroll
    for (int j = 0; j < kConvT + 3; ++j) {
        const int s = t0 - 3 + j;
        rows[j] = u32x4{0u, 0u, 0u, 0u};
        if (!active || s >= p.T || s < -(W - 1)) continue;
        if (s >= 0) {
            rows[j] = *(const u32x4 *)(p.x + b * p.sbx + (long)s * p.ldx + c0);
        } else if (p.init) {
            const uint16_t *h = p.init + ((long)b * p.C + c0) * (W - 1) + (W - 1 + s);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                rows[j][e] = (uint32_t)h[(2 * e) * (W - 1)] | ((uint32_t)h[(2 * e + 1) * (W - 1)] << 16);
        }
    }
    float w[8][4], bs[8];
    if (active && p.w_vec) {
        const u32x4 *wp = (const u32x4 *)((const uint16_t *)p.w + (long)c0 * 4); // 8 channels x 4 taps
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
            const u32x4 v = wp[e2]; // channels 2 e2, 2 e2 + 1
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                w[2 * e2 + u][0] = bf16_lo(v[2 * u]);
                w[2 * e2 + u][1] = bf16_hi(v[2 * u]);
                w[2 * e2 + u][2] = bf16_lo(v[2 * u + 1]);
                w[2 * e2 + u][3] = bf16_hi(v[2 * u + 1]);
            }
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                w[e][j] = (active && j < W) ? load_as_f32(p.w, p.w_dtype, (long)(c0 + e) * W + j) : 0.0f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) bs[e] = (active && p.bias) ? load_as_f32(p.bias, p.w_dtype, c0 + e) : 0.0f;
    const bool norm = active && (c0 >> 7) < p.n_norm;

#pragma unroll
    for (int i = 0; i < kConvT; ++i) {
        const int t = t0 + i;
        if (t >= p.T) break; // uniform: every thread of the workgroup has the same t0
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float a = bs[e];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (j >= W) continue;
                const uint32_t r = rows[i + 4 - W + j][e >> 1];
                a += w[e][j] * ((e & 1) ? bf16_hi(r) : bf16_lo(r));
            }
            if (p.silu) a = fsilu(a);
            o[e] = round_bf16(a);
        }
        float ss = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += o[e] * o[e];
        // the 16 threads of a 128-channel head are the 16 lanes of one DPP row
        ss = row16_sum(ss);
        if (norm) {
            const float r = __builtin_amdgcn_rsqf(ss + p.eps);
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] *= r;
        }
        if (active) {
            u32x4 out;
#pragma unroll
            for (int e = 0; e < 4; ++e) out[e] = pack_bf16x2(o[2 * e], o[2 * e + 1]);
            __builtin_nontemporal_store(out, (u32x4 *)(p.y + b * p.sby + (long)t * p.ldy + c0));
        }
    }
    // the last W - 1 input rows (history included when T < W - 1) become the next call's initial
    // state: inputs T - W + 1 .. T - 1 are slots T - W + 4 - t0 .. T + 2 - t0
    if (p.final_state && active && t0 + kConvT >= p.T) {
        for (int j = 0; j < W - 1; ++j) {
            const int slot = p.T - W + 4 + j - t0;
            u32x4 r = {0u, 0u, 0u, 0u};
#pragma unroll
            for (int k = 0; k < kConvT + 3; ++k)
                if (k == slot) r = rows[k];
#pragma unroll
            for (int e = 0; e < 8; ++e)
                p.final_state[((long)b * p.C + c0 + e) * (W - 1) + j] = (uint16_t)(r[e >> 1] >> (16 * (e & 1)));
        }
    }
}

// ================================================================================================
// Shared by prep and scan.
struct GdnParams {
    const uint16_t *q; long long sbq; int ldq;  // bf16 [B][T][HK][128] (token stride ldq, batch stride sbq)
    const uint16_t *k; long long sbk; int ldk;
    const uint16_t *v; long long sbv; int ldv;  // bf16 [B][T][HV][128]
    const float *g;                             // fp32 [B][T][HV]
    const void *beta; int beta_dtype;           // [B][T][HV], bf16 or fp32
    const float *h0;                            // fp32 [B][HV][128][128] or null
    float *hT;                                  // fp32 [B][HV][128][128] or null
    uint16_t *o;                                // bf16 [B][T][HV][128]
    uint16_t *wf, *uf;                          // workspace: per (b, h, chunk) 8192 + 8192 bf16
    float *gc;                                  // workspace: per (b, h) NT * 64 fp32 (G)
    float scale;
    int B, T, HK, HV, NT;
};

// per (b, h, chunk) workspace blocks
MICA_DEVICE long chunk_id(const GdnParams &p, int b, int h, int c) { return ((long)b * p.HV + h) * p.NT + c; }

// ---- prep: one workgroup per (chunk, value head, sequence) ------------------------------------
// LDS (bytes): K rows, V rows (64 x 128 bf16, rows padded to 272 B), L (64 x 64 fp32, rows padded to
// 272 B), G, exp(G), beta.  The blocked solve keeps its fp32 blocks of T in L's space (the diagonal
// blocks in place of L's, the off-diagonal ones in the unused upper triangle); the bf16 T (64 x 64,
// rows padded to 144 B) then reuses that space once every wave holds its blocks in registers, and the
// W staging (64 x 128 bf16) reuses K's once W and U are done: 52 KB, three workgroups per CU.
constexpr int kRowP = 136;          // bf16 elements per padded 128-wide row
constexpr int kRowC = 72;           // bf16 elements per padded 64-wide row
constexpr int kLs = 68;             // fp32 elements per padded row of L (A-operand reads free of conflicts)
constexpr int kPrepK = 0;
constexpr int kPrepV = kPrepK + kC * kRowP * 2;
constexpr int kPrepL = kPrepV + kC * kRowP * 2;
constexpr int kPrepT = kPrepL;                     // after the solve
constexpr int kPrepW = kPrepK;                     // after W and U
constexpr int kPrepG = kPrepL + kC * kLs * 4;
constexpr int kPrepSmem = kPrepG + 3 * kC * 4;
static_assert(kC * kRowC * 2 <= kC * kLs * 4, "T fits in L's space");
static_assert(3 * kPrepSmem <= 160 * 1024, "three prep workgroups per CU");

// ---- 16 x 16 fp32 blocks on v_mfma_f32_16x16x4f32 (the blocked solve of T) ----
// Operand layouts of one k-step (4 of the 16 inner indices): lane i + 16 k holds A[i][k] and
// B[k][i]; the 16 x 16 result ("C layout"): lane j + 16 g holds rows 4 g .. 4 g + 3 of column j.
typedef float f32x4 __attribute__((ext_vector_type(4)));
MICA_DEVICE f32x4 mfma16(float a, float b, const f32x4 &c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }
// c + A B with both blocks in LDS (row stride kLs)
MICA_DEVICE f32x4 blk_mm(const float *A, const float *B, f32x4 c, int lane) {
    const int r = lane & 15, k = lane >> 4;
#pragma unroll
    for (int s = 0; s < 4; ++s) c = mfma16(A[r * kLs + 4 * s + k], B[(4 * s + k) * kLs + r], c);
    return c;
}
// c + A X with A in LDS and X in this wave's registers in the C layout: k-step s takes the inner
// indices m = 4 k + s (k = 0..3), whose X rows lane j + 16 k holds in its register s
MICA_DEVICE f32x4 blk_mm_reg(const float *A, const f32x4 &x, f32x4 c, int lane) {
    const int r = lane & 15, k = lane >> 4;
#pragma unroll
    for (int s = 0; s < 4; ++s) c = mfma16(A[r * kLs + 4 * k + s], x[s], c);
    return c;
}
// store a C-layout block at (row 16 bi, column 16 bj) of an fp32 matrix with row stride kLs
MICA_DEVICE void blk_store(float *M, int bi, int bj, const f32x4 &x, int lane) {
    const int j = lane & 15, g = lane >> 4;
#pragma unroll
    for (int v = 0; v < 4; ++v) M[(16 * bi + 4 * g + v) * kLs + 16 * bj + j] = x[v];
}
// the same block as bf16 into T (row stride kRowC)
MICA_DEVICE void blk_store_bf16(uint16_t *T, int bi, int bj, const f32x4 &x, int lane) {
    const int j = lane & 15, g = lane >> 4;
#pragma unroll
    for (int v = 0; v < 4; ++v) T[(16 * bi + 4 * g + v) * kRowC + 16 * bj + j] = f32_to_bf16(x[v]);
}

__global__ __launch_bounds__(kGdnThreads) void gdn_prep_kernel(GdnParams p) {
    __shared__ __attribute__((aligned(16))) int8_t smem[kPrepSmem];
    uint16_t *Ks = (uint16_t *)(smem + kPrepK);
    uint16_t *Vs = (uint16_t *)(smem + kPrepV);
    float *Lp = (float *)(smem + kPrepL);
    uint16_t *Ts = (uint16_t *)(smem + kPrepT);
    uint16_t *Ws = (uint16_t *)(smem + kPrepW);
    float *Gs = (float *)(smem + kPrepG);
    float *Es = Gs + kC;  // exp(G)
    float *Bs = Es + kC;  // beta

    const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int hk = h / (p.HV / p.HK);
    const int tbase = c * kC;

    // ---- K and V rows of the chunk (zeros past T), g and beta ----
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int piece = tid + i * kGdnThreads; // 64 rows x 16 pieces of 16 bytes
        const int r = piece >> 4, col = (piece & 15) * 8;
        const int t = tbase + r;
        u32x4 kv = {0u, 0u, 0u, 0u}, vv = {0u, 0u, 0u, 0u};
        if (t < p.T) {
            kv = *(const u32x4 *)(p.k + b * p.sbk + (long)t * p.ldk + hk * kDk + col);
            vv = *(const u32x4 *)(p.v + b * p.sbv + (long)t * p.ldv + h * kDv + col);
        }
        *(u32x4 *)(Ks + r * kRowP + col) = kv;
        *(u32x4 *)(Vs + r * kRowP + col) = vv;
    }
    float gval = 0.0f;
    if (tid < kC) {
        const int t = tbase + tid;
        float bv = 0.0f;
        if (t < p.T) {
            const long gi = ((long)b * p.T + t) * p.HV + h;
            gval = p.g[gi];
            bv = load_as_f32(p.beta, p.beta_dtype, gi);
        }
        Gs[tid] = gval;
        Bs[tid] = bv;
    }
    __syncthreads();
    // ---- G = in-chunk cumulative sum of g (wave 0: one token per lane, log-step scan) ----
    if (wave == 0) {
        float acc = gval;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const float n = __shfl_up(acc, off, 64);
            if (lane >= off) acc += n;
        }
        Gs[tid] = acc;
        Es[tid] = fexp(acc);
        p.gc[((long)b * p.HV + h) * p.NT * kC + tbase + tid] = acc;
    }
    __syncthreads();

    // ---- L = beta_i (k_i . k_j) exp(G_i - G_j) for j < i: one 32 x 32 tile per wave ----
    {
        const int ti = wave >> 1, tj = wave & 1;
        f32x16 acc = {};
        const int kh = (lane >> 5) * 8;
#pragma unroll
        for (int s = 0; s < kDk / 16; ++s) {
            const bf16x8 a = ld_frag(Ks + (ti * 32 + (lane & 31)) * kRowP + s * 16 + kh);
            const bf16x8 bb = ld_frag(Ks + (tj * 32 + (lane & 31)) * kRowP + s * 16 + kh);
            acc = mfma(a, bb, acc);
        }
        const int j = tj * 32 + (lane & 31);
        const float gj = Gs[j];
        // rows i = ti 32 + 8 r4 + 4 (lane / 32) + u: four consecutive G and beta values per r4, read
        // before any math (a masked select, not a branch, so the LDS reads are not serialised)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            const int i0 = ti * 32 + 8 * r4 + 4 * (lane >> 5);
            const float4 gi = *(const float4 *)(Gs + i0), bi = *(const float4 *)(Bs + i0);
            const float ga[4] = {gi.x, gi.y, gi.z, gi.w}, ba[4] = {bi.x, bi.y, bi.z, bi.w};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = i0 + u;
                const float lv = (ba[u] * acc[4 * r4 + u]) * fexp(ga[u] - gj);
                Lp[i * kLs + j] = j < i ? lv : 0.0f;
            }
        }
    }
    __syncthreads();

    // ---- T = (I + L)^-1 over 16 x 16 blocks (block (i, j) = rows 16 i.., columns 16 j..).  From
    // (I + L) T = I: the diagonal blocks D_i = (I + L_ii)^-1 by forward substitution, and below the
    // diagonal T_ij = -D_i sum_{k=j}^{i-1} L_ik T_kj, in three dependent stages of fp32 MFMA products:
    //   stage 1: T_10 (wave 0), T_21 (wave 1), T_32 (wave 2), L_30 D_0 (wave 3, kept)
    //   stage 2: T_20 (wave 0), T_31 (wave 1), + L_31 T_10 (wave 3)
    //   stage 3: T_30 = -D_3 (L_30 D_0 + L_31 T_10 + L_32 T_20) (wave 3)
    // D_i replaces L_ii in LDS, and T_10, T_21, T_32, T_20 go to the unused upper blocks (0, 1),
    // (1, 2), (2, 3), (0, 2) for the waves that read them.  Every wave keeps its own blocks in
    // registers and writes them as bf16 once no wave reads L any more. ----
    {
        const int jc = lane & 15, gq = lane >> 4;
        auto blk = [&](int bi, int bj) { return Lp + 16 * bi * kLs + 16 * bj; };
        // wave w: D_w, lane jc + 16 gq holding rows 4 gq .. 4 gq + 3 of column jc.  Four rows at a
        // time: the terms of earlier row groups are summed per lane (its own four rows m) and over
        // the four lane groups, then the 4 x 4 substitution is done redundantly in every lane
        f32x4 D = {0.0f, 0.0f, 0.0f, 0.0f};
        {
            const float *N = blk(wave, wave);
#pragma unroll
            for (int g2 = 0; g2 < 4; ++g2) {
                float S4[4];
#pragma unroll
                for (int a = 0; a < 4; ++a) {
                    float acc = 0.0f;
                    if (g2 > 0) {
                        const float4 nv = *(const float4 *)(N + (4 * g2 + a) * kLs + 4 * gq);
                        acc = __builtin_fmaf(nv.x, D[0], __builtin_fmaf(nv.y, D[1], __builtin_fmaf(nv.z, D[2], nv.w * D[3])));
                        acc = gq < g2 ? acc : 0.0f;
                        acc += __shfl_xor(acc, 16, 64);
                        acc += __shfl_xor(acc, 32, 64);
                    }
                    S4[a] = acc;
                }
                const float *nb = N + 4 * g2 * kLs + 4 * g2; // N[4 g2 + a][4 g2 + b] at nb[a * kLs + b]
                const float n10 = nb[kLs], n20 = nb[2 * kLs], n21 = nb[2 * kLs + 1];
                const float n30 = nb[3 * kLs], n31 = nb[3 * kLs + 1], n32 = nb[3 * kLs + 2];
                const int r0 = 4 * g2;
                const float x0 = (r0 == jc ? 1.0f : 0.0f) - S4[0];
                const float x1 = (r0 + 1 == jc ? 1.0f : 0.0f) - S4[1] - n10 * x0;
                const float x2 = (r0 + 2 == jc ? 1.0f : 0.0f) - S4[2] - n20 * x0 - n21 * x1;
                const float x3 = (r0 + 3 == jc ? 1.0f : 0.0f) - S4[3] - n30 * x0 - n31 * x1 - n32 * x2;
                if (gq == g2) D = f32x4{x0, x1, x2, x3};
            }
            blk_store(Lp, wave, wave, D, lane); // only this wave read L_ww
        }
        __syncthreads();
        const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
        f32x4 Ta = z, Tb = z; // this wave's off-diagonal blocks
        if (wave < 3) {
            // T_{w+1, w} = -D_{w+1} (L_{w+1, w} D_w)
            const f32x4 x = blk_mm(blk(wave + 1, wave), blk(wave, wave), z, lane);
            Ta = -blk_mm_reg(blk(wave + 1, wave + 1), x, z, lane);
            blk_store(Lp, wave, wave + 1, Ta, lane);
        } else {
            Tb = blk_mm(blk(3, 0), blk(0, 0), z, lane); // L_30 D_0, completed in stages 2 and 3
        }
        __syncthreads();
        if (wave == 0) {
            // T_20 = -D_2 (L_20 D_0 + L_21 T_10)
            const f32x4 x = blk_mm(blk(2, 1), blk(0, 1), blk_mm(blk(2, 0), blk(0, 0), z, lane), lane);
            Tb = -blk_mm_reg(blk(2, 2), x, z, lane);
            blk_store(Lp, 0, 2, Tb, lane);
        } else if (wave == 1) {
            // T_31 = -D_3 (L_31 D_1 + L_32 T_21)
            const f32x4 x = blk_mm(blk(3, 2), blk(1, 2), blk_mm(blk(3, 1), blk(1, 1), z, lane), lane);
            Tb = -blk_mm_reg(blk(3, 3), x, z, lane);
        } else if (wave == 3) {
            Tb = blk_mm(blk(3, 1), blk(0, 1), Tb, lane); // + L_31 T_10
        }
        __syncthreads();
        if (wave == 3) Ta = -blk_mm_reg(blk(3, 3), blk_mm(blk(3, 2), blk(0, 2), Tb, lane), z, lane); // T_30
        __syncthreads(); // no wave reads L or the fp32 blocks any more: T (bf16) takes their place
        // blocks as bf16: D_w on the diagonal, the off-diagonal blocks of each wave, zeros above
        blk_store_bf16(Ts, wave, wave, D, lane);
        if (wave < 3) blk_store_bf16(Ts, wave + 1, wave, Ta, lane);
        if (wave == 0) blk_store_bf16(Ts, 2, 0, Tb, lane);
        if (wave == 1) blk_store_bf16(Ts, 3, 1, Tb, lane);
        if (wave == 3) blk_store_bf16(Ts, 3, 0, Ta, lane);
        // the six zero blocks above the diagonal, two per wave 0-2
        if (wave == 0) { blk_store_bf16(Ts, 0, 1, z, lane); blk_store_bf16(Ts, 0, 2, z, lane); }
        if (wave == 1) { blk_store_bf16(Ts, 0, 3, z, lane); blk_store_bf16(Ts, 1, 2, z, lane); }
        if (wave == 2) { blk_store_bf16(Ts, 1, 3, z, lane); blk_store_bf16(Ts, 2, 3, z, lane); }
    }
    __syncthreads();

    // ---- W = T (beta exp(G) K), U = T (beta V): wave w computes the 32 columns 32 w .. 32 w + 31 of
    // both, for all 64 rows (two 32-row tiles); the B operands are columns of K / V, scaled per
    // token and rounded to bf16 ----
    {
        const int col = wave * 32 + (lane & 31);
        const int kh = (lane >> 5) * 8;
        f32x16 aw[2] = {}, au[2] = {};
#pragma unroll
        for (int s = 0; s < kC / 16; ++s) {
            const int m0 = s * 16 + kh;
            u32x4 kb, vb;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int m = m0 + 2 * e;
                const float k0 = bf16_to_f32(Ks[m * kRowP + col]) * Bs[m] * Es[m];
                const float k1 = bf16_to_f32(Ks[(m + 1) * kRowP + col]) * Bs[m + 1] * Es[m + 1];
                const float v0 = bf16_to_f32(Vs[m * kRowP + col]) * Bs[m];
                const float v1 = bf16_to_f32(Vs[(m + 1) * kRowP + col]) * Bs[m + 1];
                kb[e] = pack_bf16x2(k0, k1);
                vb[e] = pack_bf16x2(v0, v1);
            }
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                const bf16x8 a = ld_frag(Ts + (mt * 32 + (lane & 31)) * kRowC + m0);
                aw[mt] = mfma(a, as_bf16x8(kb), aw[mt]);
                au[mt] = mfma(a, as_bf16x8(vb), au[mt]);
            }
        }
        const long cid = chunk_id(p, b, h, c);
        // U: stored in the accumulator layout, tile (mt, dv tile = wave), 16 values per lane
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            u32x4 lo, hi;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                lo[e] = pack_bf16x2(au[mt][2 * e], au[mt][2 * e + 1]);
                hi[e] = pack_bf16x2(au[mt][8 + 2 * e], au[mt][8 + 2 * e + 1]);
            }
            uint16_t *dst = p.uf + cid * (kC * kDv) + ((mt * 4 + wave) * 64 + lane) * 16;
            *(u32x4 *)dst = lo;
            *(u32x4 *)(dst + 8) = hi;
        }
        __syncthreads(); // every wave is done reading K: the W staging takes its place
        // W: staged row-major, re-read below in the operand layout
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int r = 0; r < 16; ++r) Ws[(mt * 32 + acc_row(r, lane)) * kRowP + col] = f32_to_bf16(aw[mt][r]);
    }
    __syncthreads();
    // W in the MFMA A-operand layout: fragment f = (row tile mt, k-step s) of 64 lanes x 8 values,
    // lane l holding row 32 mt + l % 32, columns 16 s + 8 (l / 32) .. + 7
    {
        const long cid = chunk_id(p, b, h, c);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int piece = tid + i * kGdnThreads; // 16 fragments x 64 lanes
            const int f = piece >> 6, l = piece & 63;
            const int mt = f >> 3, s = f & 7;
            const u32x4 v = *(const u32x4 *)(Ws + (mt * 32 + (l & 31)) * kRowP + s * 16 + (l >> 5) * 8);
            *(u32x4 *)(p.wf + cid * (kC * kDk) + (long)piece * 8) = v;
        }
    }
}

// ---- scan: one workgroup of 8 waves per (value head, sequence) --------------------------------
// Wave w: row role wr = w % 4 and dv half hf = w / 4.  The state S [128 dk x 128 dv] is spread so
// that wave w holds dk rows 32 wr .. 32 wr + 31 of dv half hf (DVT = two 32 x 32 accumulator tiles).
// With fewer (sequence, head) pairs than CUs the dv columns are split over gridDim.z workgroups
// (the columns of S, v_new and o are independent; every workgroup recomputes the chunk's P): 2 of 8
// waves with one 32 x 32 tile each (DVT = 1), or 4 of 4 waves (wr only, DVT = 1).  The arithmetic of
// every output element is the same in each split.
// Per chunk, X = [W; Q] S (rows 0-63 from W for wr = 0, 1; rows 64-127 from Q for wr = 2, 3),
// P^T = K Q^T (waves 0-3, one tile each), v_new = U - W S (wr = 0, 1), o (wr = 2, 3) and the state
// update (all waves).  Each operand held in registers is re-loaded for the next chunk right after
// its last use in this one, so the loads overlap the rest of the chunk.
// LDS (bytes): S^T (128 dv rows x 128 dk, bf16, 272 B rows); K rows of the chunk, two buffers
// (alternate chunks); v_new^T and its decayed copy (128 dv x 64 tokens, 144 B rows); P = masked
// Q K^T (64 x 64, 144 B rows); output staging (32 x 64 per output wave); G, two buffers.
constexpr int kScanS = 0;
constexpr int kScanK = kScanS + kDv * kRowP * 2;
constexpr int kScanVn = kScanK + 2 * kC * kRowP * 2;
constexpr int kScanVd = kScanVn + kDv * kRowC * 2;
constexpr int kScanP = kScanVd + kDv * kRowC * 2;
constexpr int kScanO = kScanP + kC * kRowC * 2;
constexpr int kScanG = kScanO + 4 * 32 * kRowC * 2;
constexpr int kScanSmem = kScanG + 2 * 3 * kC * 4;  // per buffer: G, exp(G_63 - G), exp(G)
static_assert(kScanSmem <= 160 * 1024, "scan LDS");

template <int DVT, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void gdn_scan_kernel(GdnParams p) {
    constexpr int kThr = 64 * WAVES;
    constexpr int kPieces = kC * 16 / kThr; // 16-byte pieces of the chunk's K rows per thread
    __shared__ __attribute__((aligned(16))) int8_t smem[kScanSmem];
    uint16_t *Sst = (uint16_t *)(smem + kScanS);
    uint16_t *Vn = (uint16_t *)(smem + kScanVn);
    uint16_t *Vd = (uint16_t *)(smem + kScanVd);
    uint16_t *Ps = (uint16_t *)(smem + kScanP);

    const int h = blockIdx.x, b = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave & 3, hf = wave >> 2;
    const int hk = h / (p.HV / p.HK);
    const int l32 = lane & 31, kh = (lane >> 5) * 8;
    // this wave's first value column: the workgroup's dv range starts at blockIdx.z times its width
    const int dvw = blockIdx.z * ((WAVES / 4) * 32 * DVT) + hf * 32 * DVT;
    const long bh = (long)b * p.HV + h;
    const bool w_rows = wr < 2;                    // X rows from W (v_new); otherwise from Q (output)
    const bool needs_q = !w_rows;                  // Q tile for X (wr = 2, 3) and the P^T tile
    const int mq = wr - 2;                         // that Q tile (query rows 32 mq ..)
    // P^T tiles (key tile mk, query tile mq) on the Q-row waves, which have no v_new to form before
    // barrier (B): wave 2 (0, 0), wave 3 (0, 1), wave 7 (1, 1); with 4 waves, wave 3 takes (0, 1) and
    // (1, 1).  Tile (1, 0) -- keys 32-63 against queries 0-31 -- is wholly masked: its zeros are
    // written once, before the first chunk.
    const bool p_tile = wave == 2 || wave == 3 || wave == 7;
    const int mk_lo = wave == 7 ? 1 : 0, mk_hi = (wave == 7 || (WAVES == 4 && wave == 3)) ? 1 : 0;

    // state: S[dk = 32 wr + acc_row][dv = 64 hf + 32 dvt + l32]
    f32x16 S[DVT];
#pragma unroll
    for (int dvt = 0; dvt < DVT; ++dvt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int dk = wr * 32 + acc_row(r, lane), dv = dvw + dvt * 32 + l32;
            S[dvt][r] = p.h0 ? p.h0[(bh * kDk + dk) * kDv + dv] : 0.0f;
        }
    auto store_state_bf16 = [&]() {
#pragma unroll
        for (int dvt = 0; dvt < DVT; ++dvt)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const int dk = wr * 32 + 8 * r4 + 4 * (lane >> 5);
                u32x2 w2;
                w2[0] = pack_bf16x2(S[dvt][4 * r4], S[dvt][4 * r4 + 1]);
                w2[1] = pack_bf16x2(S[dvt][4 * r4 + 2], S[dvt][4 * r4 + 3]);
                *(u32x2 *)(Sst + (dvw + dvt * 32 + l32) * kRowP + dk) = w2;
            }
    };
    store_state_bf16();

    // ---- per-chunk operand loads into registers ----
    u32x4 kreg[kPieces];
    float gn = 0.0f;
    bf16x8 qf[8], wfr[8];
    u32x4 uf[DVT][2];
    auto load_k = [&](int c) {
#pragma unroll
        for (int i = 0; i < kPieces; ++i) {
            const int piece = tid + i * kThr; // 64 rows x 16 pieces of 16 bytes
            const int t = c * kC + (piece >> 4);
            kreg[i] = u32x4{0u, 0u, 0u, 0u};
            if (t < p.T) kreg[i] = *(const u32x4 *)(p.k + b * p.sbk + (long)t * p.ldk + hk * kDk + (piece & 15) * 8);
        }
        if (tid < kC) gn = p.gc[bh * p.NT * kC + c * kC + tid];
    };
    auto load_q = [&](int c) {
        const int t = c * kC + mq * 32 + l32;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            u32x4 v = {0u, 0u, 0u, 0u};
            if (t < p.T) v = *(const u32x4 *)(p.q + b * p.sbq + (long)t * p.ldq + hk * kDk + s * 16 + kh);
            qf[s] = as_bf16x8(v);
        }
    };
    auto load_w = [&](int c) {
        const uint16_t *src = p.wf + chunk_id(p, b, h, c) * (kC * kDk) + ((long)(wr * 8) * 64 + lane) * 8;
#pragma unroll
        for (int s = 0; s < 8; ++s) wfr[s] = ld_frag(src + s * 64 * 8);
    };
    auto load_u = [&](int c) {
#pragma unroll
        for (int dvt = 0; dvt < DVT; ++dvt) {
            const uint16_t *src = p.uf + chunk_id(p, b, h, c) * (kC * kDv) + ((wr * 4 + dvw / 32 + dvt) * 64 + lane) * 16;
            uf[dvt][0] = *(const u32x4 *)src;
            uf[dvt][1] = *(const u32x4 *)(src + 8);
        }
    };
    load_k(0);
    if (needs_q) load_q(0);
    if (w_rows) { load_w(0); load_u(0); }
    // the masked P tile: P[i][j] = 0 for queries i < 32 and keys j >= 32 (read after barrier (B))
    for (int e = tid; e < 32 * 4; e += kThr) {
        const int i = e >> 2, j = 32 + (e & 3) * 8;
        *(u32x4 *)(Ps + i * kRowC + j) = u32x4{0u, 0u, 0u, 0u};
    }

    for (int c = 0; c < p.NT; ++c) {
        const int tbase = c * kC;
        const bool more = c + 1 < p.NT;
        uint16_t *Ks = (uint16_t *)(smem + kScanK) + (c & 1) * kC * kRowP;
        float *Gs = (float *)(smem + kScanG) + (c & 1) * 3 * kC;
        float *Ed = Gs + kC;      // exp(G_63 - G_m): the decay of v_new row m into the state update
        float *Eg = Ed + kC;      // exp(G_i): the decay of the state into output row i
#pragma unroll
        for (int i = 0; i < kPieces; ++i) {
            const int piece = tid + i * kThr;
            *(u32x4 *)(Ks + (piece >> 4) * kRowP + (piece & 15) * 8) = kreg[i];
        }
        if (tid < kC) {
            // each token's two decays once per chunk, for every wave that applies them
            const float glast = __shfl(gn, kC - 1, 64);
            Gs[tid] = gn;
            Ed[tid] = fexp(glast - gn);
            Eg[tid] = fexp(gn);
        }
        // the next chunk's K rows and g into the registers just written out: a whole chunk to arrive
        if (more) load_k(c + 1);
        __syncthreads(); // (A) K rows, G and the state S^T visible to every wave

        // ---- X = [W; Q] S for this wave's 32 rows and dv half ----
        f32x16 X[DVT] = {};
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const bf16x8 a = w_rows ? wfr[s] : qf[s];
#pragma unroll
            for (int dvt = 0; dvt < DVT; ++dvt)
                X[dvt] = mfma(a, ld_frag(Sst + (dvw + dvt * 32 + l32) * kRowP + s * 16 + kh), X[dvt]);
        }
        if (w_rows && more) load_w(c + 1);
        // ---- P^T tile (K rows mk) x (Q rows mq): P[i][j] = (q_i . k_j) exp(G_i - G_j), j <= i ----
        if (p_tile) for (int mk = mk_lo; mk <= mk_hi; ++mk) {
            f32x16 pt = {};
#pragma unroll
            for (int s = 0; s < 8; ++s) pt = mfma(ld_frag(Ks + (mk * 32 + l32) * kRowP + s * 16 + kh), qf[s], pt);
            const int i = mq * 32 + l32; // query token (column of P^T)
            const float gi = Gs[i];
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const int j0 = mk * 32 + 8 * r4 + 4 * (lane >> 5); // key tokens j0 .. j0 + 3
                const float4 gj = *(const float4 *)(Gs + j0);
                const float ga[4] = {gj.x, gj.y, gj.z, gj.w};
                float e[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    // computed for every lane, then selected: a branch here would serialise the LDS reads
                    const float ev = pt[4 * r4 + u] * fexp(gi - ga[u]);
                    e[u] = (j0 + u <= i) ? ev : 0.0f;
                }
                u32x2 w2;
                w2[0] = pack_bf16x2(e[0], e[1]);
                w2[1] = pack_bf16x2(e[2], e[3]);
                *(u32x2 *)(Ps + i * kRowC + j0) = w2;
            }
        }
        if (needs_q && more) load_q(c + 1);
        // ---- v_new = U - W S (wr = 0, 1), stored transposed, plain and decayed by exp(G_63 - G_m) ----
        if (w_rows) {
#pragma unroll
            for (int dvt = 0; dvt < DVT; ++dvt) {
                const int dv = dvw + dvt * 32 + l32;
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    const int m0 = wr * 32 + 8 * r4 + 4 * (lane >> 5);
                    const uint32_t u01 = uf[dvt][r4 >> 1][(r4 & 1) * 2], u23 = uf[dvt][r4 >> 1][(r4 & 1) * 2 + 1];
                    float vn[4] = {bf16_lo(u01) - X[dvt][4 * r4], bf16_hi(u01) - X[dvt][4 * r4 + 1],
                                   bf16_lo(u23) - X[dvt][4 * r4 + 2], bf16_hi(u23) - X[dvt][4 * r4 + 3]};
                    u32x2 a2, d2;
                    a2[0] = pack_bf16x2(vn[0], vn[1]);
                    a2[1] = pack_bf16x2(vn[2], vn[3]);
                    const float4 ed = *(const float4 *)(Ed + m0);
                    const float dec[4] = {vn[0] * ed.x, vn[1] * ed.y, vn[2] * ed.z, vn[3] * ed.w};
                    d2[0] = pack_bf16x2(dec[0], dec[1]);
                    d2[1] = pack_bf16x2(dec[2], dec[3]);
                    *(u32x2 *)(Vn + dv * kRowC + m0) = a2;
                    *(u32x2 *)(Vd + dv * kRowC + m0) = d2;
                }
            }
            if (more) load_u(c + 1);
        }
        __syncthreads(); // (B) v_new, P visible; every wave is done reading S^T and the previous K buffer

        // ---- o = scale (exp(G_i) (Q S)_i + P v_new) for the rows of wr = 2, 3 ----
        if (!w_rows) {
            const int mo = wr - 2; // output row tile
            f32x16 O[DVT] = {};
#pragma unroll
            for (int s = 0; s < kC / 16; ++s) {
                if (mo == 0 && s >= 2) break; // keys 32-63 are masked for queries 0-31
                const bf16x8 a = ld_frag(Ps + (mo * 32 + l32) * kRowC + s * 16 + kh);
#pragma unroll
                for (int dvt = 0; dvt < DVT; ++dvt)
                    O[dvt] = mfma(a, ld_frag(Vn + (dvw + dvt * 32 + l32) * kRowC + s * 16 + kh), O[dvt]);
            }
            float eg[16]; // exp(G) of this lane's 16 output rows, read before the stores
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const float4 g4 = *(const float4 *)(Eg + mo * 32 + 8 * r4 + 4 * (lane >> 5));
                eg[4 * r4] = g4.x;
                eg[4 * r4 + 1] = g4.y;
                eg[4 * r4 + 2] = g4.z;
                eg[4 * r4 + 3] = g4.w;
            }
            uint16_t *ost = (uint16_t *)(smem + kScanO) + (hf * 2 + mo) * 32 * kRowC;
#pragma unroll
            for (int dvt = 0; dvt < DVT; ++dvt)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int ml = acc_row(r, lane);
                    const float y = X[dvt][r] * eg[r] * p.scale + O[dvt][r] * p.scale;
                    ost[ml * kRowC + dvt * 32 + l32] = f32_to_bf16(y);
                }
            // write out: 32 rows x 64 DVT bytes, 4 DVT lanes per row
            constexpr int kLpr = 4 * DVT, kRpi = 64 / kLpr;
#pragma unroll
            for (int it = 0; it < 32 / kRpi; ++it) {
                const int ml = it * kRpi + lane / kLpr, cc = (lane % kLpr) * 8;
                const int t = tbase + mo * 32 + ml;
                const u32x4 v = *(const u32x4 *)(ost + ml * kRowC + cc);
                if (t < p.T) __builtin_nontemporal_store(v, (u32x4 *)(p.o + (((long)b * p.T + t) * p.HV + h) * kDv + dvw + cc));
            }
        }
        // ---- S <- exp(G_63) S + K^T (decayed v_new) ----
        {
            const float dl = Eg[kC - 1];
#pragma unroll
            for (int dvt = 0; dvt < DVT; ++dvt) S[dvt] *= dl;
            const int dk = wr * 32 + l32;
#pragma unroll
            for (int s = 0; s < kC / 16; ++s) {
                const int m0 = s * 16 + kh;
                u32x4 kt;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    kt[e] = (uint32_t)Ks[(m0 + 2 * e) * kRowP + dk] | ((uint32_t)Ks[(m0 + 2 * e + 1) * kRowP + dk] << 16);
#pragma unroll
                for (int dvt = 0; dvt < DVT; ++dvt)
                    S[dvt] = mfma(as_bf16x8(kt), ld_frag(Vd + (dvw + dvt * 32 + l32) * kRowC + s * 16 + kh), S[dvt]);
            }
        }
        store_state_bf16(); // read after barrier (A) of the next chunk
    }
    if (p.hT) {
#pragma unroll
        for (int dvt = 0; dvt < DVT; ++dvt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int dk = wr * 32 + acc_row(r, lane), dv = dvw + dvt * 32 + l32;
                p.hT[(bh * kDk + dk) * kDv + dv] = S[dvt][r];
            }
    }
}

// ================================================================================================
// Gated RMSNorm over each 128-wide value head (attn.norm(out, z), fork.py:148) fused with the
// per-token INT8 quantisation of the normalised row for out_proj.  One wave per token row of
// HV x 128 values: h = bf16(x rsqrt(mean x^2 + eps)); h = bf16(w h); y = bf16(h silu(z));
// then s = max(amax(y), 1e-8) / 127 and q = round_half_even(y / s) (int8_quant.py:64-73).
constexpr int kGnWaves = 4;

struct GatedNormParams {
    const uint16_t *x; int ldx; const uint16_t *z; int ldz; const uint16_t *w; // w: bf16 [128]
    uint16_t *y; int ldy;       // optional bf16 output
    int8_t *q; int ldq; float *s;
    int M, N; float eps;        // N = HV * 128 <= 8192
};

// NI = N / 512 pieces of 8 columns per lane: lane l owns columns 8 l + 512 i, so the 16 lanes of
// one 128-wide head are 16 consecutive lanes.  All of a row's loads are issued before any math.
template <int NI>
__global__ __launch_bounds__(64 * kGnWaves) void gated_norm_quant_kernel(GatedNormParams p) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * kGnWaves + (threadIdx.x >> 6);
    if (row >= p.M) return;
    u32x4 xr[NI], zr[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        xr[i] = *(const u32x4 *)(p.x + (long)row * p.ldx + i * 512 + lane * 8);
        zr[i] = *(const u32x4 *)(p.z + (long)row * p.ldz + i * 512 + lane * 8);
    }
    float wv[8];
    {
        const u32x4 wr = *(const u32x4 *)(p.w + (lane & 15) * 8);
#pragma unroll
        for (int e = 0; e < 4; ++e) { wv[2 * e] = bf16_lo(wr[e]); wv[2 * e + 1] = bf16_hi(wr[e]); }
    }
    u32x4 yr[NI];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        float xv[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) { xv[2 * e] = bf16_lo(xr[i][e]); xv[2 * e + 1] = bf16_hi(xr[i][e]); }
        float ss = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += xv[e] * xv[e];
        ss = row16_sum(ss); // the head's 16 lanes: one DPP row
        const float rstd = 1.0f / sqrtf(ss / 128.0f + p.eps);
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float zv = (e & 1) ? bf16_hi(zr[i][e >> 1]) : bf16_lo(zr[i][e >> 1]);
            const float hn = round_bf16(xv[e] * rstd);
            const float hw = round_bf16(wv[e] * hn);
            v[e] = hw * fsilu(zv);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            yr[i][e] = pack_bf16x2(v[2 * e], v[2 * e + 1]);
            amax = fmaxf(amax, fmaxf(fabsf(bf16_lo(yr[i][e])), fabsf(bf16_hi(yr[i][e]))));
        }
    }
    amax = wave_max(amax);
    const float s = row_scale(amax);
    // bf16 y with a bf16 row maximum: the one-FMA half-even quantizer (exact against the IEEE
    // quotient for every such pair, tests/native/fma_quotient_check.c)
    const float r = fma_quant_recip(amax, s, 1.0f / s);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int col = i * 512 + lane * 8;
        if (p.y) __builtin_nontemporal_store(yr[i], (u32x4 *)(p.y + (long)row * p.ldy + col));
        float x[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = (e & 1) ? bf16_hi(yr[i][e >> 1]) : bf16_lo(yr[i][e >> 1]);
        __builtin_nontemporal_store(fma_quant8(x, r), (u32x2 *)(p.q + (long)row * p.ldq + col));
    }
    if (lane == 0) p.s[row] = s;
}

// The GDN layer's decay and write strength per token and value head (fork.py:124-125):
//   g = -exp(A_log[h]) * softplus(f32(a) + dt_bias[h])   (softplus(x) = x above 20, else log1p(exp(x)),
//                                                         torch's threshold), fp32
//   beta = bf16(sigmoid(f32(b)))                         (torch's bf16 sigmoid: fp32 math, one rounding)
// One thread per (token, head); a and b are the bf16 outputs of in_proj_a / in_proj_b.
__global__ __launch_bounds__(256) void gate_kernel(const uint16_t *a, int lda, const uint16_t *b, int ldb,
                                                   const float *A_log, const float *dt_bias, float *g,
                                                   uint16_t *beta, int M, int HV) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= (long)M * HV) return;
    const int m = (int)(i / HV), h = (int)(i - (long)m * HV);
    const float x = bf16_to_f32(a[(long)m * lda + h]) + dt_bias[h];
    const float sp = x > 20.0f ? x : log1pf(expf(x));
    g[i] = -expf(A_log[h]) * sp;
    beta[i] = f32_to_bf16(1.0f / (1.0f + expf(-bf16_to_f32(b[(long)m * ldb + h]))));
}

// dst = src (or zeros when src is null): the final state of an empty scan
__global__ void state_fill_kernel(const float *src, float *dst, long n) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = src ? src[i] : 0.0f;
}

// the same for the conv's bf16 state: an empty sequence leaves the initial state (or zeros) unchanged
__global__ void state_fill16_kernel(const uint16_t *src, uint16_t *dst, long n) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = src ? src[i] : (uint16_t)0;
}

long long gdn_ws_bytes(long long B, long long T, long long HV) {
    const long long NT = (T + kC - 1) / kC;
    return B * HV * NT * (2LL * kC * kDk * 2 + kC * 4);
}

}  // namespace

// ================================================================================================
extern "C" int mica_causal_conv1d(const void *x, long long sbx, int ldx, const void *w, const void *bias,
                                  int w_dtype, int width, const void *init_state, void *final_state, void *y,
                                  long long sby, int ldy, int B, int T, int C, int silu, int n_norm, float eps,
                                  mica_stream_t stream) {
    if (w == nullptr || (T > 0 && (x == nullptr || y == nullptr))) return MICA_MISS_ARG;
    if (w_dtype != MICA_BF16 && w_dtype != MICA_FP32) return MICA_MISS_DTYPE;
    if (width < 1 || width > 4 || B < 0 || T < 0 || C <= 0 || C % 8 != 0 || n_norm < 0 || n_norm * 128 > C)
        return MICA_MISS_SHAPE;
    if (ldx < C || ldy < C || ldx % 8 != 0 || ldy % 8 != 0 || sbx < (long long)T * ldx || sby < (long long)T * ldy ||
        sbx % 8 != 0 || sby % 8 != 0)
        return MICA_MISS_STRIDE;
    if (!mica_aligned16(x) || !mica_aligned16(y)) return MICA_MISS_ALIGN;
    if (B == 0) return 0;
    if (T == 0) {
        // no tokens: the final state is the initial one (zeros without one), as after the scan
        if (final_state == nullptr || width == 1) return 0;
        const long n = (long)B * C * (width - 1);
        hipLaunchKernelGGL(state_fill16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                           (const uint16_t *)init_state, (uint16_t *)final_state, n);
        return mica_err(hipGetLastError());
    }
    ConvParams p{};
    p.x = (const uint16_t *)x; p.sbx = sbx; p.ldx = ldx;
    p.w = w; p.bias = bias; p.w_dtype = w_dtype; p.width = width;
    p.w_vec = width == 4 && w_dtype == MICA_BF16 && mica_aligned16(w);
    p.init = (const uint16_t *)init_state; p.final_state = (uint16_t *)final_state;
    p.y = (uint16_t *)y; p.sby = sby; p.ldy = ldy;
    p.B = B; p.T = T; p.C = C; p.silu = silu != 0; p.n_norm = n_norm; p.eps = eps;
    if ((T + kConvT - 1) / kConvT > 65535 || B > 65535) return MICA_MISS_SHAPE;
    dim3 grid((C / 8 + kConvThreads - 1) / kConvThreads, (T + kConvT - 1) / kConvT, B);
    hipStream_t st = (hipStream_t)stream;
    switch (width) {
    case 1: hipLaunchKernelGGL(conv_kernel<1>, grid, dim3(kConvThreads), 0, st, p); break;
    case 2: hipLaunchKernelGGL(conv_kernel<2>, grid, dim3(kConvThreads), 0, st, p); break;
    case 3: hipLaunchKernelGGL(conv_kernel<3>, grid, dim3(kConvThreads), 0, st, p); break;
    default: hipLaunchKernelGGL(conv_kernel<4>, grid, dim3(kConvThreads), 0, st, p); break;
    }
    return mica_err(hipGetLastError());
}

extern "C" long long mica_gdn_workspace_bytes(int B, int T, int HV) {
    if (B < 0 || T < 0 || HV <= 0) return -1;
    return gdn_ws_bytes(B, T, HV);
}

extern "C" int mica_gdn_chunk(const void *q, long long sbq, int ldq, const void *k, long long sbk, int ldk,
                              const void *v, long long sbv, int ldv, const float *g, const void *beta,
                              int beta_dtype, const float *initial_state, float *final_state, void *o, float scale,
                              int B, int T, int HK, int HV, void *workspace, long long workspace_bytes,
                              mica_stream_t stream) {
    if (beta_dtype != MICA_BF16 && beta_dtype != MICA_FP32) return MICA_MISS_DTYPE;
    if (B < 0 || T < 0 || HK <= 0 || HV <= 0 || HV % HK != 0) return MICA_MISS_SHAPE;
    // empty inputs have no token data (their pointers may be NULL)
    if (B > 0 && T > 0 && (q == nullptr || k == nullptr || v == nullptr || g == nullptr || beta == nullptr || o == nullptr))
        return MICA_MISS_ARG;
    if (ldq < HK * kDk || ldk < HK * kDk || ldv < HV * kDv || ldq % 8 || ldk % 8 || ldv % 8 || sbq % 8 || sbk % 8 ||
        sbv % 8 || sbq < (long long)T * ldq || sbk < (long long)T * ldk || sbv < (long long)T * ldv)
        return MICA_MISS_STRIDE;
    if (!mica_aligned16(q) || !mica_aligned16(k) || !mica_aligned16(v) || !mica_aligned16(o) ||
        (initial_state && !mica_aligned16(initial_state)) || (final_state && !mica_aligned16(final_state)) ||
        (workspace && !mica_aligned16(workspace)))
        return MICA_MISS_ALIGN;
    if ((long long)B * T * HV * kDv >= (1LL << 31) || (long long)B * HV * kDk * kDv >= (1LL << 31))
        return MICA_MISS_RANGE;
    if (B == 0) return 0;
    if (T == 0) {
        // nothing to scan: the final state is the initial one (or zeros)
        if (final_state) {
            const long n = (long)B * HV * kDk * kDv;
            hipLaunchKernelGGL(state_fill_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                               initial_state, final_state, n);
            return mica_err(hipGetLastError());
        }
        return 0;
    }
    if (workspace == nullptr || workspace_bytes < gdn_ws_bytes(B, T, HV)) return MICA_MISS_ARG;
    GdnParams p{};
    p.q = (const uint16_t *)q; p.sbq = sbq; p.ldq = ldq;
    p.k = (const uint16_t *)k; p.sbk = sbk; p.ldk = ldk;
    p.v = (const uint16_t *)v; p.sbv = sbv; p.ldv = ldv;
    p.g = g; p.beta = beta; p.beta_dtype = beta_dtype;
    p.h0 = initial_state; p.hT = final_state; p.o = (uint16_t *)o; p.scale = scale;
    p.B = B; p.T = T; p.HK = HK; p.HV = HV; p.NT = (T + kC - 1) / kC;
    const long long blocks = (long long)B * HV * p.NT;
    p.wf = (uint16_t *)workspace;
    p.uf = p.wf + blocks * kC * kDk;
    p.gc = (float *)(p.uf + blocks * kC * kDv);
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(gdn_prep_kernel, dim3(p.NT, HV, B), dim3(kGdnThreads), 0, st, p);
    int rc = mica_err(hipGetLastError());
    if (rc) return rc;
    // dv split of the scan when (sequence, head) pairs leave CUs idle
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    const long long pairs = (long long)B * HV;
    if (pairs * 4 <= cus) hipLaunchKernelGGL((gdn_scan_kernel<1, 4>), dim3(HV, B, 4), dim3(256), 0, st, p);
    else if (pairs * 2 <= cus) hipLaunchKernelGGL((gdn_scan_kernel<1, 8>), dim3(HV, B, 2), dim3(512), 0, st, p);
    else hipLaunchKernelGGL((gdn_scan_kernel<2, 8>), dim3(HV, B, 1), dim3(512), 0, st, p);
    return mica_err(hipGetLastError());
}

extern "C" int mica_gated_rmsnorm_quant(const void *x, int ldx, const void *z, int ldz, const void *w, float eps,
                                        void *y, int ldy, int8_t *q, int ldq, float *s, int M, int N,
                                        mica_stream_t stream) {
    if (x == nullptr || z == nullptr || w == nullptr || q == nullptr || s == nullptr) return MICA_MISS_ARG;
    if (M < 0 || N <= 0 || N % 512 != 0 || N > 8192 || ((N / 512) & (N / 512 - 1)) != 0) return MICA_MISS_SHAPE;
    if (ldx < N || ldz < N || ldq < N || (y && ldy < N) || ldx % 8 || ldz % 8 || ldq % 8 || (y && ldy % 8))
        return MICA_MISS_STRIDE;
    if (!mica_aligned16(x) || !mica_aligned16(z) || !mica_aligned16(w) || !mica_aligned16(q) || (y && !mica_aligned16(y)))
        return MICA_MISS_ALIGN;
    if ((long long)M * ldx >= (1LL << 31) || (long long)M * ldz >= (1LL << 31) || (long long)M * ldq >= (1LL << 31))
        return MICA_MISS_RANGE;
    if (M == 0) return 0;
    GatedNormParams p{};
    p.x = (const uint16_t *)x; p.ldx = ldx; p.z = (const uint16_t *)z; p.ldz = ldz; p.w = (const uint16_t *)w;
    p.y = (uint16_t *)y; p.ldy = ldy; p.q = q; p.ldq = ldq; p.s = s; p.M = M; p.N = N; p.eps = eps;
    const dim3 grid((M + kGnWaves - 1) / kGnWaves), block(64 * kGnWaves);
    hipStream_t st = (hipStream_t)stream;
    switch (N / 512) {
    case 1: hipLaunchKernelGGL(gated_norm_quant_kernel<1>, grid, block, 0, st, p); break;
    case 2: hipLaunchKernelGGL(gated_norm_quant_kernel<2>, grid, block, 0, st, p); break;
    case 4: hipLaunchKernelGGL(gated_norm_quant_kernel<4>, grid, block, 0, st, p); break;
    case 8: hipLaunchKernelGGL(gated_norm_quant_kernel<8>, grid, block, 0, st, p); break;
    case 16: hipLaunchKernelGGL(gated_norm_quant_kernel<16>, grid, block, 0, st, p); break;
    default: return MICA_MISS_SHAPE;
    }
    return mica_err(hipGetLastError());
}

extern "C" int mica_gdn_gate(const void *a, int lda, const void *b, int ldb, const float *A_log,
                             const float *dt_bias, float *g, void *beta, int M, int HV, mica_stream_t stream) {
    if (a == nullptr || b == nullptr || A_log == nullptr || dt_bias == nullptr || g == nullptr || beta == nullptr)
        return MICA_MISS_ARG;
    if (M < 0 || HV <= 0) return MICA_MISS_SHAPE;
    if (lda < HV || ldb < HV) return MICA_MISS_STRIDE;
    if ((long long)M * lda >= (1LL << 31) || (long long)M * ldb >= (1LL << 31) || (long long)M * HV >= (1LL << 31))
        return MICA_MISS_RANGE;
    if (M == 0) return 0;
    const long long n = (long long)M * HV;
    hipLaunchKernelGGL(gate_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t *)a, lda, (const uint16_t *)b, ldb, A_log, dt_bias, g, (uint16_t *)beta, M, HV);
    return mica_err(hipGetLastError());
}
