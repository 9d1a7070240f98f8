/*
 * mica_amd.h -- C ABI of the MI355X (gfx950) W8A8 linear-layer hot path.
 *
 * Every entry point takes plain device pointers, element strides (in elements),
 * int sizes and a HIP stream handle passed as void*.  Nothing here allocates or
 * frees memory, synchronises the device or prints: the caller owns every buffer
 * (inputs borrowed, outputs pre-allocated), and the launch is enqueued on the
 * stream it is given, so the calls are safe inside HIP graph capture.
 *
 * Return value of every launcher:
 *      0                launched (or nothing to do: M == 0)
 *     >0  MICA_MISS_*   unsupported case, nothing launched; the Python layer turns
 *                       this into the reference's "return None + count a fallback
 *                       reason" convention (v0.5/serving/lib/int8_kernels.py:22-24)
 *     <0                -(hipError_t) of a failed launch; Python raises RuntimeError,
 *                       as the reference's driver check does (int8_kernels.py:60-64)
 */
#ifndef MICA_AMD_H
#define MICA_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *mica_stream_t; /* hipStream_t; NULL is the null stream */

/* element types (the reference's DT table, int8_kernels.py:13, plus int8 / int32) */
enum { MICA_BF16 = 0, MICA_FP16 = 1, MICA_FP32 = 2, MICA_INT8 = 3, MICA_INT32 = 4 };

/* rounding of the activation quantizer:
 *   EVEN  torch.round, half to even        (int8_quant.py:70, the CPU path)
 *   AWAY  trunc(v +- 0.5), half away from 0 (kernel_src/kernels.py:35, the Triton kernel) */
enum { MICA_ROUND_EVEN = 0, MICA_ROUND_AWAY = 1 };

/* GEMM epilogues */
enum {
    MICA_EPI_SCALE = 0,    /* C = cvt((f32(acc) * sa[m]) * sb[n] (+ bias[n])) (kernels.py:63-68)          */
    MICA_EPI_SILU_MUL = 1, /* gate/up interleaved in groups of 64 rows of B; C[m, n'] has N/2 columns:
                              g = bf16(y_gate), u = bf16(y_up), C = bf16(bf16(silu(g)) * u)
                              (fast_runtime.py:126-132 + fused_kernels.py:36-42, 85-87)                 */
};

/* reasons for a miss (>0 return) */
enum {
    MICA_MISS_SHAPE = 1,  /* a size is out of the supported range                 */
    MICA_MISS_DTYPE = 2,  /* dtype code not supported for this argument           */
    MICA_MISS_ALIGN = 3,  /* a pointer is not 16-byte aligned                      */
    MICA_MISS_STRIDE = 4, /* a leading dimension is too small or not a multiple of 16 */
    MICA_MISS_RANGE = 5,  /* an index product would overflow int32                 */
    MICA_MISS_ARG = 6,    /* a required pointer is NULL / invalid flag            */
    MICA_MISS_DEVICE = 7, /* the current device is not gfx950                       */
};

/* library version, (major << 16) | minor */
int mica_version(void);

/* short name of a miss code ("shape", "dtype", ...) or of an error */
const char *mica_status_name(int rc);

/* properties of a device that the rooflines are priced with:
 * compute units, peak engine clock (kHz), LDS bytes per workgroup, gfx arch number (950). */
int mica_device_info(int device, int *cu_count, int *clock_khz, int *lds_per_block, int *gfx_arch);

/*
 * Per-token symmetric INT8 activation quantizer.
 * Replaces int8_kernels.act_quant (v0.5/serving/lib/int8_kernels.py:325-353), which launches the
 * Triton act_quant (kernel_src/kernels.py:14-37); CPU semantics int8_quant.quant_act (int8_quant.py:64-73):
 *   xf = f32(x[m, :]) (* inv_smooth[:]);  s[m] = max(max|xf|, 1e-8) / 127
 *   q[m, k] = clamp(round(xf[k] / s[m]), -127, 127)
 * x: [M, K] of x_dtype (bf16 / fp16 / fp32) with row stride ldx; q: [M, K] int8, row stride ldq;
 * s: [M] fp32.  inv_smooth: [K] fp32 or NULL.
 * Requires K % 8 == 0, 8 <= K <= 16384, 16-byte aligned rows.
 */
int mica_act_quant(const void *x, int x_dtype, int ldx, const float *inv_smooth, int8_t *q, int ldq, float *s,
                   int M, int K, int rounding, mica_stream_t stream);

/*
 * Fused RMSNorm (+ optional residual add) + per-token INT8 quantizer, one read of x.
 * Replaces fused_kernels.rms_norm (v0.5/serving/lib/fused_kernels.py:50-82, Triton norm :10-34)
 * followed by int8_kernels.act_quant on its output (the QLinear call at int8_runtime.py:181):
 *   v = residual ? bf16(x + residual) : x            (stored to sum if sum != NULL)   (:27-30, :52)
 *   y = bf16((f32(v) * rsqrt(mean(f32(v)^2) + eps)) * (offset + f32(w)))           (:31-34, :54)
 *   (q, s) = act_quant(y, inv_smooth)                 if q != NULL
 *   y stored if y != NULL
 * offset = 1.0 gives the Qwen3.5 zero-centred weight ((1 + w), fused_kernels.py:34);
 * offset = 0.0 a plain gamma.  x, residual, y, sum: [M, K] of x_dtype (bf16 or fp16);
 * w: [K] of w_dtype (bf16 / fp16 / fp32).  At least one of q, y must be non-NULL;
 * with q != NULL, s must be non-NULL.
 */
int mica_rmsnorm_quant(const void *x, int x_dtype, int ldx, const void *residual, int ldr, const void *w, int w_dtype,
                       float offset, float eps, const float *inv_smooth, int8_t *q, int ldq, float *s, void *y, int ldy,
                       void *sum, int lds, int M, int K, int rounding, mica_stream_t stream);

/*
 * The same fused RMSNorm, with the normed row quantized for n_out (1 to 4) consumers at once: the
 * input projections that share one norm in the reference model (q/k/v, or the linear-attention
 * in_proj_qkv / in_proj_z / in_proj_a / in_proj_b, or gate/up), each with its own SmoothQuant
 * factors (int8_quant.py:64-73 with inv_smooth = that QLinear's buffer, int8_runtime.py:124-127),
 * so the row is read once instead of once per consumer.  inv_smooth, q, ldq and s are host arrays of
 * n_out entries (device pointers; an inv_smooth entry may be NULL: no smoothing for that consumer).
 * Output o is bit-identical to mica_rmsnorm_quant with inv_smooth[o], q[o], ldq[o], s[o].
 * No counterpart in the reference, whose QLinears each quantize the shared normed row themselves.
 */
int mica_rmsnorm_quant_multi(const void *x, int x_dtype, int ldx, const void *residual, int ldr, const void *w,
                             int w_dtype, float offset, float eps, int n_out, const float *const *inv_smooth,
                             int8_t *const *q, const int *ldq, float *const *s, void *y, int ldy, void *sum, int lds,
                             int M, int K, int rounding, mica_stream_t stream);

/*
 * W8A8 GEMM on the gfx950 i8 matrix cores: acc[m, n] = sum_k A[m, k] * B[n, k] (exact int32),
 * then the epilogue.  Replaces int8_kernels.mm_i8 (v0.5/serving/lib/int8_kernels.py:359-406),
 * Triton mm_i8 (kernel_src/kernels.py:40-68); CPU fallback int8_runtime.py:186-192.
 * A: [M, K] int8 (lda), B: [N, K] int8 (ldb, K-contiguous like QLinear.qweight), sa: [M] fp32,
 * sb: [N] fp32, bias: [N] fp32 or NULL.  residual: NULL or [M, Nout] of out_dtype, added after the
 * epilogue's rounding: C = cvt(f32(cvt(y)) + f32(residual)) (the "h + mlp(...)" of fork.py:419-422).
 * C: [M, Nout] of out_dtype (bf16 / fp16 / fp32), Nout = N (SCALE) or N / 2 (SILU_MUL, bf16 only).
 * out_dtype MICA_INT32 stores the raw accumulators acc[m, n] (SCALE only; scales, bias and
 * residual are ignored) -- the int32 matmul of int8_quant.torch_int_mm (int8_quant.py:92-96).
 * Requires K % 16 == 0, lda/ldb % 16 == 0, N % 128 == 0 for SILU_MUL.
 *
 * workspace: NULL, or workspace_bytes >= mica_mm_i8_workspace_bytes(device) bytes of device memory,
 * 16-byte aligned, whose first 4 KiB are zero before its first use (every launch leaves them zero
 * again).  With it, two schedules split tiles along K:
 *   - 16-bit outputs (SILU_MUL included), K % 256 == 0, K >= 8192: when the output fits at most CUs / 3
 *     tiles of 128 x 160 (SCALE) or 128 x 256 (SILU_MUL) -- a short request's down projection, e.g.
 *     M <= 512 at N = 2560 -- every tile is split into K / 2560 parts (at least 3), one workgroup per
 *     part, and each tile's last part adds the others' partial sums;
 *   - int32 / fp32 outputs: when the last round of 256 x 256 tiles would hold at most CUs / 4 tiles,
 *     K >= 8192 and M <= 256 (elsewhere 128 x 128 quarter tiles, which need no workspace, serve such
 *     a round better), those tiles are split along K over four workgroups each.
 * Partial int32 sums go through the workspace and are added exactly, so the result is bit-identical
 * to the unsplit schedule.  Launches that
 * share a workspace must be ordered (one stream); concurrent launches need one workspace each.
 * The workspace has no counterpart in the reference (its Triton GEMM has no split schedule).
 */
int mica_mm_i8(const int8_t *A, int lda, const int8_t *B, int ldb, const float *sa, const float *sb,
               const float *bias, const void *residual, int ldr, void *C, int ldc, int out_dtype, int M, int N, int K,
               int epilogue, void *workspace, long long workspace_bytes, mica_stream_t stream);

/* bytes of GEMM workspace for `device` (its CU count x 512 KiB + 4 KiB), or -(hipError_t) */
long long mica_mm_i8_workspace_bytes(int device);

/*
 * mica_mm_i8 for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  No counterpart in the reference.  Same
 * arguments, checks, schedule and bits as mica_mm_i8 with a workspace, but the split schedule's
 * workspace is a static device array of the library (mica_mm_i8_noalloc_scratch_bytes() = 32 MiB +
 * 4 KiB per device, held until the process ends), so the call allocates nothing.  Limit: a split
 * round of 256 x 256 tiles of at most 16 tiles (64 workgroups); a call whose such round would need
 * more returns MICA_MISS_RANGE (the split of few 128-row tiles takes fewer parts when the scratch
 * holds too few of them).  Every call on a device shares that device's scratch: calls that overlap on one
 * device (concurrent streams) race, so order them on one stream.  The first call on a device also
 * clears the scratch's counters on its stream.
 */
int mica_mm_i8_noalloc(const int8_t *A, int lda, const int8_t *B, int ldb, const float *sa, const float *sb,
                       const float *bias, const void *residual, int ldr, void *C, int ldc, int out_dtype, int M,
                       int N, int K, int epilogue, mica_stream_t stream);

/* bytes of the static scratch behind mica_mm_i8_noalloc (per device) */
long long mica_mm_i8_noalloc_scratch_bytes(void);

/*
 * Elementwise SwiGLU y = bf16(bf16(silu(f32(g))) * f32(u)) over n elements of bf16.
 * Replaces fused_kernels.swi_glu (v0.5/serving/lib/fused_kernels.py:85-96, Triton swiglu :36-42).
 */
int mica_swiglu(const void *g, const void *u, void *y, long long n, int dtype, mica_stream_t stream);

/*
 * Last-position readout over the allowed answer ids.
 * Replaces the label-row readout of release_runtime.py:298-306 applied to
 * body.norm(final_hidden(...)) (prefill_engine.py:280-304) and the slice + softmax of
 * release_runtime.py:509-517, so no full-vocabulary projection is ever formed.
 *   x_b    = h[rows[b], :]                                       (rows: int32 [B], the last token of request b)
 *   x_b    = bf16(rms_norm(x_b, norm_w, eps, offset)) if norm_w != NULL  (the final norm)
 *   logits[b, j] = sum_k f32(x_b[k]) * f32(W[ids ? ids[j] : j, k])      (fp32, j < L)
 *   probs[b, i]  = softmax_i(logits[b, lo[b] + i]), i < cnt[b]          (lo/cnt NULL: over all L)
 * h: [n_rows, K] bf16 (ldh); W: [w_rows, K] of w_dtype (fp32: the pre-gathered label rows, or bf16:
 * the full output embedding indexed through ids); logits: [B, L] fp32; probs: [B, ldp] fp32 or NULL.
 * rows / ids / lo / cnt live on the device: a row or id out of range gives NaN logits (and NaN probs
 * for a bad row) instead of an access; the softmax slice is clipped to [0, L) and to ldp.
 */
int mica_gather_logits(const void *h, int ldh, int n_rows, const int *rows, int B, const void *norm_w, int norm_dtype,
                       float offset, float eps, const void *W, int w_dtype, int ldw, int w_rows, const int *ids, int L,
                       int K, float *logits, const int *lo, const int *cnt, float *probs, int ldp,
                       mica_stream_t stream);

/*
 * Rotary position embedding in place on the first n_heads heads of each token row (the q and k heads
 * of a fused QKV projection output), in bf16 arithmetic as transformers' apply_rotary_pos_emb
 * computes it for the attention layers: for i < h = head_dim / 2,
 *   y[i] = bf16(bf16(x[i] cos[p][i]) + bf16(x[i + h] (-sin[p][i])))
 *   y[i + h] = bf16(bf16(x[i + h] cos[p][i]) + bf16(x[i] sin[p][i]))
 * x: bf16 rows of ldx elements (T rows); cos_tab / sin_tab: bf16 [n_pos][h]; position p of row t is
 * pos[t] (int32, device) or t % period when pos is NULL.  head_dim % 16 == 0.  Rows whose position
 * falls outside the tables are left unrotated.  No counterpart in the reference's W8A8 launchers: it
 * replaces the torch elementwise RoPE of the attention layers around them.
 */
int mica_rope_inplace(void *x, long long ldx, int n_heads, int head_dim, const void *cos_tab, const void *sin_tab,
                      int n_pos, const int *pos, int period, int T, mica_stream_t stream);

/*
 * The q / k head norm and partial rotary embedding of the full-attention layers, in place on the rows
 * of a fused QKV projection output (replaces the torch ops q_norm / k_norm and rope_one of the
 * reference's attention, fast_runtime.py:229-236, prefill_engine.py:83-89, 123-130).  Segment q holds
 * n_q heads at column q_off of each row, segment k n_k heads at k_off; head_dim is a power of two, 16 to
 * 512.  Each head is first normed when its segment's weight is given (bf16 [head_dim]; NULL: no norm):
 *   y = bf16((x * (1 / sqrt(sum(x^2) / head_dim + eps))) * (offset + w))
 * (the reference model's zero-centred RMSNorm: offset 1), then its first rot_dim dims (a power of two,
 * 16 .. head_dim; 0: none) are rotated as mica_rope_inplace rotates a head of rot_dim dims, the others
 * passed through: for i < h = rot_dim / 2,
 *   y[i] = bf16(bf16(y[i] cos[p][i]) + bf16(y[i + h] (-sin[p][i]))),
 *   y[i + h] = bf16(bf16(y[i + h] cos[p][i]) + bf16(y[i] sin[p][i])),
 * with cos_tab / sin_tab bf16 [n_pos][rot_dim / 2] and position p of row t = pos[t] (int32, device) or
 * t % period when pos is NULL (rows whose position is outside the tables: normed, not rotated).
 */
int mica_head_norm_rope(void *x, long long ldx, int T, int q_off, int n_q, int k_off, int n_k, int head_dim,
                        const void *q_norm_w, const void *k_norm_w, float offset, float eps, int rot_dim,
                        const void *cos_tab, const void *sin_tab, int n_pos, const int *pos, int period,
                        mica_stream_t stream);

/*
 * The attention output gate of the full-attention layers fused with o_proj's activation quantizer:
 *   y = bf16(a * bf16(sigmoid(g)))   (fast_runtime.py:240: o * torch.sigmoid(gate), bf16 ops; the sigmoid
 *                                     as torch's fp32 1 / (1 + exp(-g)) rounded to bf16)
 *   s[m] = max(max_k |y[m, k]|, 1e-8) / 127,  q[m, k] = round_half_even(y[m, k] / s[m])
 *                                    (int8_quant.quant_act, int8_quant.py:64-73)
 * a, g: bf16 [M, K] with row strides lda / ldg (elements); q int8 [M, K] (ldq), s fp32 [M]; y (optional,
 * bf16, ldy): the gated rows.  K a multiple of 512, 512 .. 8192; rounding must be MICA_ROUND_EVEN.
 * No counterpart in the reference's launchers (its gate and act_quant are two torch / Triton steps).
 */
int mica_gate_quant(const void *a, long long lda, const void *gate, long long ldg, int8_t *q, long long ldq,
                    float *s, void *y, long long ldy, int M, int K, int rounding, mica_stream_t stream);

/*
 * Causal grouped-query attention forward, head dim 256, HQ = 4 HK (query head h reads key/value head
 * h / 4), Sq queries over Sk >= Sq keys (the queries are the last Sq positions).  Replaces the
 * reference's attn_fwd (int8_kernels.py:409-481, Triton kernel kernel_src/kernels.py:71-124) and the
 * torch SDPA path of the full-attention layers.
 *   o[b, t, h] = sum_{u <= t + Sk - Sq} softmax_u(scale q[b, t, h] . k[b, u, h / 4]) v[b, u, h / 4]
 * q / k / v / o: bf16; head j of row t of sequence b at ptr + b sb + j sh + t ld (elements, all % 8).
 * fp32 softmax and accumulation, bf16 products.  causal must be 1.  workspace:
 * mica_attention_workspace_bytes(B, Sk, HK) bytes (V^T tile images), 16-byte aligned.
 */
int mica_attention_fwd(const void *q, long long sbq, long long shq, long long ldq, const void *k, long long sbk,
                       long long shk, long long ldk, const void *v, long long sbv, long long shv, long long ldv, void *o,
                       long long sbo, long long sho, long long ldo, int B, int Sq, int Sk, int HQ, int HK,
                       int head_dim, float scale, int causal, void *workspace, long long workspace_bytes,
                       mica_stream_t stream);

/* bytes of mica_attention_fwd workspace: B x HK x ceil(Sk / 32) x 16 KiB */
long long mica_attention_workspace_bytes(int B, int Sk, int HK);

/*
 * mica_attention_fwd with each query block's keys split over key_splits workgroups (1 to 64), for
 * few query blocks over many keys (a continuation batch over a long prefix: Sq << Sk).  Each
 * workgroup writes its partial softmax state (unnormalised O in fp32, running maximum and sum) to
 * the workspace and a merge kernel combines them:
 *   o = (sum_s 2^(m_s - M) O_s) / (sum_s 2^(m_s - M) l_s),  M = max_s m_s.
 * The reference's kernel walks all key blocks of a query block in one program
 * (kernel_src/kernels.py:71-124, the n_q < n_k shift at :92-98); this split changes only the fp32
 * summation order, so o matches mica_attention_fwd within bf16 rounding, not bit for bit.
 * key_splits = 1 is mica_attention_fwd itself.  workspace:
 * mica_attention_split_workspace_bytes(B, Sq, Sk, HQ, HK, key_splits) bytes, 16-byte aligned.
 */
int mica_attention_fwd_split(const void *q, long long sbq, long long shq, long long ldq, const void *k, long long sbk,
                             long long shk, long long ldk, const void *v, long long sbv, long long shv, long long ldv,
                             void *o, long long sbo, long long sho, long long ldo, int B, int Sq, int Sk, int HQ,
                             int HK, int head_dim, float scale, int causal, int key_splits, void *workspace,
                             long long workspace_bytes, mica_stream_t stream);

/*
 * mica_attention_fwd_split with a key count per sequence: kv_len (int32 [B], device memory) gives
 * sequence b's number of keys, clamped to Sq .. Sk; its queries are the last Sq positions of those
 * kv_len[b] keys, and keys kv_len[b] .. Sk - 1 are never read.  This is the key limit of the reference's
 * last-position pass over requests padded to a common width (prefill_engine.py:298-304, 332-336:
 * keys < limit); with one query per sequence it runs only the picked positions' attention.  Each
 * query's arithmetic is that of mica_attention_fwd for the same query over the same keys, so with
 * key_splits = 1 the result equals the unpadded run's row bit for bit.  workspace as for
 * mica_attention_fwd_split.
 */
int mica_attention_fwd_kvlen(const void *q, long long sbq, long long shq, long long ldq, const void *k, long long sbk,
                             long long shk, long long ldk, const void *v, long long sbv, long long shv, long long ldv,
                             void *o, long long sbo, long long sho, long long ldo, int B, int Sq, int Sk, int HQ,
                             int HK, int head_dim, float scale, int causal, int key_splits, const int *kv_len,
                             void *workspace, long long workspace_bytes, mica_stream_t stream);

/* bytes of mica_attention_fwd_split workspace: the V^T images, then B x HQ x key_splits x
 * 32 ceil(Sq / 32) rows of 1032 bytes (O, m, l); -1 for an invalid argument */
long long mica_attention_split_workspace_bytes(int B, int Sq, int Sk, int HQ, int HK, int key_splits);

/*
 * mica_attention_fwd_kvlen (kv_len may be NULL) over keys whose first Pk (a multiple of 32, at most
 * Sk - Sq) are one prefix shared by every sequence: kp / vp hold the prefix's rows (head j of row t at
 * ptr + j sh + t ld), k / v each sequence's Sk - Pk keys after it.  The result equals
 * mica_attention_fwd_kvlen on the concatenated keys bit for bit (same key tiles, same order); the
 * prefix is neither copied per sequence nor transposed more than once.  Serves several continuations
 * of one cached prefix (the reference's prefix reuse, prefill_engine.py:283-339 with a recorded
 * state) without expanding it to every row of the batch.  workspace:
 * mica_attention_prefix_workspace_bytes(B, Sq, Sk, Pk, HQ, HK, key_splits) bytes, 16-byte aligned.
 */
int mica_attention_fwd_prefix(const void *q, long long sbq, long long shq, long long ldq, const void *k, long long sbk,
                              long long shk, long long ldk, const void *v, long long sbv, long long shv, long long ldv,
                              const void *kp, long long shkp, long long ldkp, const void *vp, long long shvp,
                              long long ldvp, int Pk, void *o, long long sbo, long long sho, long long ldo, int B,
                              int Sq, int Sk, int HQ, int HK, int head_dim, float scale, int causal, int key_splits,
                              const int *kv_len, void *workspace, long long workspace_bytes, mica_stream_t stream);

/* bytes of mica_attention_fwd_prefix workspace: HK x Pk / 32 prefix V^T images of 16 KiB, the
 * sequences' own images for Sk - Pk keys, the split states as above; -1 for an invalid argument */
long long mica_attention_prefix_workspace_bytes(int B, int Sq, int Sk, int Pk, int HQ, int HK, int key_splits);

/*
 * mica_attention_fwd_prefix (kv_len NULL; Pk = 0: no prefix) with the new rows' q / k head norm and rotary
 * embedding folded in: the attention layers' q_norm / k_norm and apply_rotary_pos_emb before the attention
 * (the steps mica_head_norm_rope and mica_rope_inplace perform as passes of their own).  Requires
 * Sk = Pk + Sq: row r of sequence b is query r and key Pk + r.  Each head (256 dims) is first normed when
 * its weight is given (q_norm_w / k_norm_w, bf16 [256], 16-byte aligned; NULL: no norm):
 *   y = bf16((x * (1 / sqrt(sum(x^2) / 256 + eps))) * (norm_offset + w)),
 * then its first rot_dim dims (0, 64, 128 or 256) are rotated as mica_rope_inplace rotates a head of
 * rot_dim dims, at position pos[b Sq + r] (int32, device) or Pk + r when pos is NULL; cos_tab / sin_tab
 * are bf16 [n_pos][rot_dim / 2] (16-byte aligned), and a row whose position falls outside them is left
 * unrotated.  k is treated in place (bit for bit what mica_head_norm_rope writes) before the attention
 * reads it; q as it is loaded, left as it was in memory; the prefix's keys kp must already be treated.
 * The output equals mica_head_norm_rope over q and k followed by mica_attention_fwd_prefix bit for bit,
 * without the pass over q (its 16 heads are four fifths of the treated bytes).  At least one of the
 * norms or the rotation must be asked for.  Workspace as mica_attention_fwd_prefix.
 */
int mica_attention_fwd_rope(const void *q, long long sbq, long long shq, long long ldq, void *k, long long sbk,
                            long long shk, long long ldk, const void *v, long long sbv, long long shv, long long ldv,
                            const void *kp, long long shkp, long long ldkp, const void *vp, long long shvp,
                            long long ldvp, int Pk, void *o, long long sbo, long long sho, long long ldo, int B, int Sq,
                            int Sk, int HQ, int HK, int head_dim, float scale, int causal, int key_splits,
                            const void *q_norm_w, const void *k_norm_w, float norm_offset, float norm_eps, int rot_dim,
                            const void *cos_tab, const void *sin_tab, int n_pos, const int *pos, void *workspace,
                            long long workspace_bytes, mica_stream_t stream);

/* ---- gated delta net (GDN) token mixer ------------------------------------------------------- */

/*
 * Depthwise causal convolution over time + SiLU, optionally followed by an l2 normalisation of
 * each of the first n_norm 128-channel heads (the q / k heads of a GDN layer).
 * Replaces causal_conv1d_fn as the reference calls it on channel-last activations
 * (v0.5/serving/lib/fork.py:94-113, conv_channel_last :163-175) and, with n_norm > 0, the q / k
 * l2norm of use_qk_l2norm_in_kernel (fork.py:145).
 *   y[b, t, c] = bf16(act(bias[c] + sum_j w[c, j] x[b, t - width + 1 + j, c]))      (fp32 sums)
 *   y[b, t, head] = bf16(y / sqrt(sum_head y^2 + eps))                for the first n_norm heads
 * x, y: bf16 [B][T][C] with batch stride sbx / sby and token stride ldx / ldy (elements);
 * w: [C][width] of w_dtype (bf16 / fp32), bias: [C] of w_dtype or NULL; width <= 4.
 * init_state / final_state: bf16 [B][C][width - 1] (the inputs before t = 0 / the last width - 1
 * inputs, with history when T < width - 1), each optional; with T == 0 final_state receives
 * init_state (zeros without one).  C % 8 == 0, strides % 8 == 0.
 */
int mica_causal_conv1d(const void *x, long long sbx, int ldx, const void *w, const void *bias, int w_dtype, int width,
                       const void *init_state, void *final_state, void *y, long long sby, int ldy, int B, int T, int C,
                       int silu, int n_norm, float eps, mica_stream_t stream);

/*
 * Chunked gated delta rule (chunk length 64), head dims 128 x 128.
 * Replaces attn.chunk_gated_delta_rule(q, k, v, g=g, beta=beta, initial_state, output_final_state,
 * use_qk_l2norm_in_kernel) as called at fork.py:137-147 (flash-linear-attention 0.5.2's
 * chunk_gated_delta_rule), with q / k already l2-normalised (mica_causal_conv1d with n_norm) and
 * grouped value heads read in place (value head h uses key head h / (HV / HK), the
 * repeat_interleave of fork.py:134-136, without the copy).  Per sequence b and value head h:
 *   S <- exp(g_t) S;  S <- S + k_t (beta_t (v_t - S^T k_t))^T;  o_t = scale S^T q_t
 * q, k: bf16 [B][T][HK][128] (batch stride sbq / sbk, token stride ldq / ldk); v: bf16 [B][T][HV][128];
 * g: fp32 [B][T][HV] (log decays, <= 0); beta: [B][T][HV] of beta_dtype (bf16 / fp32);
 * initial_state / final_state: fp32 [B][HV][128][128] or NULL; o: bf16 [B][T][HV][128].
 * workspace: mica_gdn_workspace_bytes(B, T, HV) bytes, 16-byte aligned, no initialisation needed.
 */
int mica_gdn_chunk(const void *q, long long sbq, int ldq, const void *k, long long sbk, int ldk, const void *v,
                   long long sbv, int ldv, const float *g, const void *beta, int beta_dtype,
                   const float *initial_state, float *final_state, void *o, float scale, int B, int T, int HK, int HV,
                   void *workspace, long long workspace_bytes, mica_stream_t stream);

/* bytes of mica_gdn_chunk workspace: B x HV x ceil(T / 64) x 33 KiB (W, U and the in-chunk decays) */
long long mica_gdn_workspace_bytes(int B, int T, int HV);

/*
 * Gated RMSNorm over each 128-wide value head (attn.norm(out, z), fork.py:148; transformers
 * Qwen3_5RMSNormGated) fused with the per-token INT8 quantisation of out_proj's input
 * (int8_quant.quant_act, int8_quant.py:64-73):
 *   h = bf16(x rsqrt(mean_head x^2 + eps));  h = bf16(w h);  y = bf16(h silu(f32(z)))
 *   s[m] = max(amax_row |y|, 1e-8) / 127;  q = round_half_even(y / s[m])
 * x, z: bf16 [M][N] (ldx / ldz), w: bf16 [128], y: bf16 [M][N] or NULL; q int8 [M][N] (ldq), s fp32 [M].
 * N / 512 a power of two, N <= 8192.
 */
int mica_gated_rmsnorm_quant(const void *x, int ldx, const void *z, int ldz, const void *w, float eps, void *y,
                             int ldy, int8_t *q, int ldq, float *s, int M, int N, mica_stream_t stream);

/*
 * The GDN layer's gate (fork.py:124-125): per token m and value head h,
 *   g[m][h]    = -exp(A_log[h]) * softplus(f32(a[m][h]) + dt_bias[h])    fp32, softplus threshold 20
 *   beta[m][h] = bf16(sigmoid(f32(b[m][h])))
 * a, b: bf16 [M][HV] (lda / ldb, the in_proj_a / in_proj_b outputs); A_log, dt_bias: fp32 [HV];
 * g: fp32 [M][HV], beta: bf16 [M][HV], both contiguous.  Replaces the reference's torch expressions
 * (-self.A_log.float().exp() * F.softplus(a.float() + self.dt_bias), b.sigmoid()).
 */
int mica_gdn_gate(const void *a, int lda, const void *b, int ldb, const float *A_log, const float *dt_bias, float *g,
                  void *beta, int M, int HV, mica_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* MICA_AMD_H */
