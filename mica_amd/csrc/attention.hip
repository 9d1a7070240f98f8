// Causal grouped-query attention forward on gfx950, head dim 256 (the full-attention layers of the 4B
// model: 16 query heads sharing 4 key/value heads).  Replaces the reference's attention kernel
// (kernel_src/kernels.py:71-124, launched by int8_kernels.attn_fwd, int8_kernels.py:409-481) and the
// torch SDPA fallback the attention layers use without it.
//
//   o[t, h] = sum_{u <= t + Sk - Sq} softmax_u(scale q[t, h] . k[u, g(h)]) v[u, g(h)],  g(h) = h / (HQ / HK)
//
// (Sq queries over Sk >= Sq keys: the queries are the last Sq positions, as in the reference's kernel.
// With per-sequence key counts kv_len[b] (clamped to Sq .. Sk), sequence b's queries are the last Sq
// positions of its first kv_len[b] keys: Sk becomes kv_len[b] in the sum's bound, and the keys past it
// are never read -- the reference's key limit of the padded last-position pass, prefill_engine.py:332-336.)
//
// Work split: one workgroup of 4 waves per (sequence, key/value head, block of 32 query positions);
// wave w handles query head 4 g + w, so every K / V tile brought into LDS serves the 4 query heads of
// its group.  Per tile of 32 keys, each wave computes S^T = K Q^T (32 keys x 32 queries) with
// v_mfma_f32_32x32x16_bf16: a lane then holds 16 of the 32 scores of one query (its partner lane
// l ^ 32 the other 16), so the online softmax needs one cross-lane exchange.  P^T (bf16) is used as the
// B operand of O^T += V^T P^T directly from the accumulator layout: the contraction runs over the keys
// in the order the accumulator rows hold them, and the V^T fragments are read in that same order.
// O^T (256 x 32, fp32, 128 accumulators per lane) is rescaled only when a query's running maximum grows
// by more than 2^8 (the exponentials stay <= 256; the final division makes the result exact).
//
// Data movement: Q fragments stay in registers for the whole workgroup.  K tiles arrive by LDS DMA
// (buffer_load ... lds), 16-byte chunks XOR-swizzled by row so the operand reads are conflict-free;
// V^T tiles are DMA'd from an image that v_transpose_kernel writes beforehand in exactly the LDS
// layout.  Two LDS stages: the DMA of tile j + 1 overlaps the MFMAs of tile j.
//
// Optionally (mica_attention_fwd_rope) the new rows' q / k head RMSNorm and rotary embedding of the
// attention layers are folded in: each query as its fragments are loaded (the head's halves are a lane
// and its partner l ^ 32, the rotation pairs fragments of the same lane), each key in place by
// v_transpose_kernel before its V^T tile; the arithmetic is that of mica_head_norm_rope /
// mica_rope_inplace, element for element.

#include <type_traits>

#include "common.h"

namespace {

// Combine a value with the one held by lane l ^ 32 (v_permlane32_swap: no LDS round trip).  With the
// same register as both operands, the swap leaves (own, other) in lanes 0-31 and (other, own) in lanes
// 32-63, so max and sum come out bit-identical in every lane.
__device__ __forceinline__ float half_swap_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __builtin_fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_swap_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

constexpr int kD = 256;              // head dim
constexpr int kBQ = 32;              // query positions per workgroup
constexpr int kBK = 32;              // keys per tile
constexpr int kFaWaves = 4;          // = query heads per key/value head
constexpr int kFaThreads = 64 * kFaWaves;
constexpr int kKBytes = kBK * kD * 2;    // 16 KB: 32 key rows x 512 B
constexpr int kVBytes = kD * kBK * 2;    // 16 KB: 256 dim rows x 64 B
constexpr int kStage = kKBytes + kVBytes;
#ifndef MICA_FA_OCC
#define MICA_FA_OCC 2
#endif
constexpr int kNSt = 2;                  // LDS stages: tile j + 1 in flight while tile j is read
constexpr int kFaSmem = kNSt * kStage;   // also the output staging (4 waves x 32 x 512 B) after the loop
constexpr int kMaxKeySplits = 64;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kBufferFlags = 0x00020000;   // raw buffer, 32-bit data format (gfx9)

MICA_DEVICE f32x16 mfma_bf16(const bf16x8 &a, const bf16x8 &b, const f32x16 &c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
template <int N>
MICA_DEVICE void fa_wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// V^T tile image: dim d's 32 keys are a 64-byte row of four 16-byte chunks.  Chunk c = 2 s + h holds
// key units (4 keys each) 4 s + h and 4 s + 2 + h: the 8 keys that a lane in half h of the wave feeds
// to step s of O^T += V^T P^T (the order of the P^T accumulator rows), so each A operand is one
// ds_read_b128.  Chunk c sits at position c ^ vt_swz(d): the 16 lanes of a read quarter (16
// consecutive dims) then cover the 64 banks once.
MICA_DEVICE int vt_swz(int d) { return (d >> 2) & 3; }
// bf16 offset of key unit u (keys 4 u .. 4 u + 3) of dim d in the tile image
MICA_DEVICE int vt_pos(int d, int u) {
    const int c = 2 * (u >> 2) + (u & 1);
    return d * kBK + ((c ^ vt_swz(d)) * 2 + ((u >> 1) & 1)) * 4;
}

struct FaParams {
    const uint16_t *q; long long sbq, shq, ldq; // head h of row t of sequence b: q + b sbq + h shq + t ldq
    const uint16_t *k; long long sbk, shk, ldk;
    const uint16_t *v; long long sbv, shv, ldv;
    uint16_t *vt;                               // V^T images [B][HK][ntiles_k][256][32]
    uint16_t *o; long long sbo, sho, ldo;
    int B, Sq, Sk, HQ, HK, ntiles_q, ntiles_k;
    float scale_log2;                           // softmax scale x log2(e)
    // split keys: each query block's key tiles are divided over nsplit workgroups, which write their
    // unnormalised partial state (O fp32, running maximum m and sum l, all relative to m) for
    // fa_merge_kernel; part_* rows are (b, head, split, query), sq_pad = ntiles_q * 32 of them each
    int nsplit, sq_pad;
    float *part_o, *part_m, *part_l;
    const int *kv_len;                          // [B] per-sequence key counts, or null: Sk for every one
    // a prefix shared by every sequence: keys 0 .. 32 ntiles_p - 1 are row t of kp (head h at
    // kp + h shkp + t ldkp) with their V^T images at vtp [HK][ntiles_p][256][32]; keys from there on are
    // rows t - 32 ntiles_p of k / vt (vt [B][HK][ntiles_k - ntiles_p][256][32]).  ntiles_p = 0: no prefix.
    const uint16_t *kp; long long shkp, ldkp;
    const uint16_t *vtp;
    int ntiles_p;
    // the new rows' q / k head norm and rotary embedding, as mica_head_norm_rope computes them (rows of
    // sequence b: query r and key Pk + r, with Sk = Pk + Sq).  qnw / knw: bf16 [256] norm weights (null:
    // no norm), y = bf16((x rstd) (noff + w)); then the first rot_dim dims (0, 64, 128 or 256) rotated at
    // position rpos[b Sq + r], or Pk + r without rpos, tables bf16 [rn_pos][rot_dim / 2].
    const uint16_t *qnw, *knw;
    float noff, neps;
    int rot_dim;
    const uint16_t *rcos, *rsin;
    const int *rpos;
    int rn_pos;
};

// The head RMSNorm of mica_head_norm_rope on a head of 256 dims held as 32 pieces of 8 (piece i = dims
// 8 i .. 8 i + 7): each piece's sum of squares in order (piece_squares), then the pieces summed as its
// 32-lane butterfly adds them -- pieces i and i ^ m for m = 1, 2, 4, 8, 16 in turn, each level adding the
// same two values in either order, so every holder of the head gets the same bits.  The callers hold
// the pieces differently (a query: 16 per lane, the other 16 in lane l ^ 32; a key: 4 per thread over 8
// threads) and run the levels in-lane or across lanes accordingly.
MICA_DEVICE float piece_squares(const u32x4 &x) {
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float a = bf16_lo(x[e]), b = bf16_hi(x[e]);
        ss = __builtin_fmaf(a, a, ss);
        ss = __builtin_fmaf(b, b, ss);
    }
    return ss;
}
// y = bf16((x rstd) (off + w)) of 8 packed values
MICA_DEVICE u32x4 norm8(const u32x4 &x, float rstd, float off, const u32x4 &w) {
    u32x4 y;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        y[e] = pack_bf16x2((bf16_lo(x[e]) * rstd) * (off + bf16_lo(w[e])), (bf16_hi(x[e]) * rstd) * (off + bf16_hi(w[e])));
    return y;
}

// ---- V -> V^T tile images: one workgroup per (tile, sequence x head); thread = 8 dims x 4 keys ----
__global__ __launch_bounds__(256) void v_transpose_kernel(FaParams p) {
    const int tile = blockIdx.x, bh = blockIdx.y;
    const int b = bh / p.HK, hk = bh % p.HK;
    const int rh = p.rot_dim >> 1;    // rotated pairs per head
    if (p.knw != nullptr) {
        // the tile's K rows normed and rotated in place (as mica_head_norm_rope): 8 threads per key, thread
        // sub holding dims 32 sub .. 32 sub + 31 (pieces 4 sub .. 4 sub + 3); all lanes run the shuffles
        const int key = threadIdx.x >> 3, sub = threadIdx.x & 7, t = tile * kBK + key;
        const bool live = t < p.Sk;
        uint16_t *kr = (uint16_t *)p.k + b * p.sbk + hk * p.shk + (long long)(live ? t : 0) * p.ldk + 32 * sub;
        u32x4 x[4];
        float ps[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            x[j] = live ? *(const u32x4 *)(kr + 8 * j) : u32x4{0u, 0u, 0u, 0u};
            ps[j] = piece_squares(x[j]);
        }
        float ss = (ps[0] + ps[1]) + (ps[2] + ps[3]);                 // pieces ^ 1, then ^ 2
        ss += __shfl_xor(ss, 1, 64);                                  // pieces ^ 4
        ss += __shfl_xor(ss, 2, 64);                                  // ^ 8
        ss += __shfl_xor(ss, 4, 64);                                  // ^ 16
        const float rstd = 1.0f / __builtin_sqrtf(ss / (float)kD + p.neps);
#pragma unroll
        for (int j = 0; j < 4; ++j) x[j] = norm8(x[j], rstd, p.noff, *(const u32x4 *)(p.knw + 32 * sub + 8 * j));
        if (rh > 0) {
            // pairs (d, d + rh): the partner dims are held by thread sub ^ (rh / 32)
            const int pm = rh >> 5;
            u32x4 o[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) o[j][e] = __shfl_xor(x[j][e], pm, 64);
            const int pos = p.rpos ? p.rpos[b * p.Sk + (live ? t : 0)] : p.ntiles_p * kBK + t;
            if (32 * sub < p.rot_dim && pos >= 0 && pos < p.rn_pos) {
                const bool upper = (sub & pm) != 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int i0 = (32 * sub + 8 * j) & (rh - 1);        // index into cos / sin
                    const u32x4 c = *(const u32x4 *)(p.rcos + (long long)pos * rh + i0);
                    const u32x4 sn = *(const u32x4 *)(p.rsin + (long long)pos * rh + i0);
                    u32x4 ya, yb;
                    if (upper) {
                        rope_pairs8(o[j], x[j], c, sn, ya, yb);
                        x[j] = yb;
                    } else {
                        rope_pairs8(x[j], o[j], c, sn, ya, yb);
                        x[j] = ya;
                    }
                }
            }
        }
        if (live) {
#pragma unroll
            for (int j = 0; j < 4; ++j) *(u32x4 *)(kr + 8 * j) = x[j];
        }
    } else if (rh > 0) {
        // the tile's K rows rotated in place (rope_pairs8, as mica_rope_inplace): thread = 8 pairs of
        // one key.  Key t is new row t (its V^T image is built below).
        const int groups = rh >> 3;   // 8-pair groups per key
        for (int item = threadIdx.x; item < kBK * groups; item += 256) {
            const int t = tile * kBK + item / groups, i0 = (item % groups) * 8;
            if (t >= p.Sk) continue;
            const int pos = p.rpos ? p.rpos[b * p.Sk + t] : p.ntiles_p * kBK + t;
            if (pos < 0 || pos >= p.rn_pos) continue;       // out-of-table position: left unrotated
            uint16_t *kr = (uint16_t *)p.k + b * p.sbk + hk * p.shk + (long long)t * p.ldk;
            const u32x4 a = *(const u32x4 *)(kr + i0), bb = *(const u32x4 *)(kr + rh + i0);
            const u32x4 c = *(const u32x4 *)(p.rcos + (long long)pos * rh + i0);
            const u32x4 sn = *(const u32x4 *)(p.rsin + (long long)pos * rh + i0);
            u32x4 ya, yb;
            rope_pairs8(a, bb, c, sn, ya, yb);
            *(u32x4 *)(kr + i0) = ya;
            *(u32x4 *)(kr + rh + i0) = yb;
        }
    }
    const int d0 = (threadIdx.x >> 3) * 8, u = threadIdx.x & 7; // dims d0 .. d0 + 7, keys 4 u .. 4 u + 3
    u32x4 rows[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int t = tile * kBK + 4 * u + e;
        rows[e] = u32x4{0u, 0u, 0u, 0u};
        if (t < p.Sk) rows[e] = *(const u32x4 *)(p.v + b * p.sbv + hk * p.shv + (long long)t * p.ldv + d0);
    }
    uint16_t *dst = p.vt + (((long long)bh * p.ntiles_k + tile) * kD) * kBK;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int d = d0 + i;
        u32x2 w;
        const int sh = 16 * (i & 1);
        w[0] = ((rows[0][i >> 1] >> sh) & 0xffffu) | (((rows[1][i >> 1] >> sh) & 0xffffu) << 16);
        w[1] = ((rows[2][i >> 1] >> sh) & 0xffffu) | (((rows[3][i >> 1] >> sh) & 0xffffu) << 16);
        *(u32x2 *)(dst + vt_pos(d, u)) = w;
    }
}

template <bool SPLIT>
__global__ __launch_bounds__(kFaThreads, MICA_FA_OCC) void fa_fwd_kernel(FaParams p) {
    __shared__ __attribute__((aligned(1024))) int8_t smem[kFaSmem];
    // grid (HK, B, ntiles_q [x nsplit]): every (sequence, head) pair's longest query blocks are
    // dispatched first
    const int qblk = p.ntiles_q - 1 - (SPLIT ? (int)blockIdx.z / p.nsplit : (int)blockIdx.z);
    const int hk = blockIdx.x, b = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, hi = lane >> 5;
    const int head = hk * kFaWaves + wave;
    const int q0 = qblk * kBQ;
    // sequence b's key count (its queries are the last Sq of them); position of query row t: off + t
    const int skb = p.kv_len ? min(max(p.kv_len[b], p.Sq), p.Sk) : p.Sk;
    const int off = skb - p.Sq;
    // key tiles 0 .. last: the last one holds the block's last query position
    const int last = min(p.ntiles_k - 1, (off + q0 + kBQ - 1) / kBK);
    // this workgroup's tiles first .. last_own (all of them without a split)
    const int split = SPLIT ? (int)blockIdx.z % p.nsplit : 0;
    const int first = SPLIT ? (int)((long long)split * (last + 1) / p.nsplit) : 0;
    const int last_own = SPLIT ? (int)((long long)(split + 1) * (last + 1) / p.nsplit) - 1 : last;

    // operand buffers: K rows of (b, hk) past the prefix (rows past the keys read as zeros), their V^T
    // images, and the shared prefix's K rows and V^T images of head hk
    const int ntp = p.ntiles_p, ntn = p.ntiles_k - ntp, pk = ntp * kBK;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(p.k + b * p.sbk + hk * p.shk), 0, (int)((long long)(p.Sk - pk) * p.ldk * 2), kBufferFlags);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(p.vt + ((long long)(b * p.HK + hk) * ntn) * kD * kBK), 0, ntn * kVBytes, kBufferFlags);
    const __amdgpu_buffer_rsrc_t rkp = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(ntp ? p.kp + hk * p.shkp : p.k), 0, (int)((long long)pk * p.ldkp * 2), kBufferFlags);
    const __amdgpu_buffer_rsrc_t rvp = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(ntp ? p.vtp + ((long long)hk * ntp) * kD * kBK : p.vt), 0, ntp * kVBytes, kBufferFlags);
    // DMA of key tile j into stage ST.  K: 1 KB block (wave, i) = key rows 2 (4 wave + i) + lane / 32;
    // the lane writes physical chunk l % 32 of its row, which holds logical chunk (l % 32) ^ row.  V^T:
    // block (wave, i) of the tile image.  The per-lane offsets are recomputed at every call from an
    // opaque copy of the lane id: hoisted out of the key loop they stay live across it and push the
    // kernel's registers into scratch.  (The K offset carries the tile's rows: the per-lane offset is
    // what the buffer range check sees, which turns rows past Sk into zeros.)
    auto dma_tile = [&](int j, int st) {
        int8_t *ks = smem + st * kStage;
        int ln = lane;
        __asm__ volatile("" : "+v"(ln));
        const int hi_ = ln >> 5, l32_ = ln & 31;
        // the tile's segment: the shared prefix (tiles below ntp) or this sequence's own keys
        const bool pre = j < ntp;
        const __amdgpu_buffer_rsrc_t rks = pre ? rkp : rk, rvs = pre ? rvp : rv;
        const int jj = pre ? j : j - ntp;
        const long long ld = pre ? p.ldkp : p.ldk;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = (wave * 4 + i) * 2 + hi_;
            const int ko = (int)((long long)(jj * kBK + row) * ld * 2 + ((l32_ ^ row) << 4));
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rks, (lds_void *)(ks + (wave * 4 + i) * 1024), 16, ko, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rvs, (lds_void *)(ks + kKBytes + (wave * 4 + i) * 1024), 16,
                                                     ln * 16, jj * kVBytes + (wave * 4 + i) * 1024, 0, 0);
    };

    // Q fragments (B operand of S^T): lane holds query q0 + l % 32, dims 16 s + 8 (l / 32) .. + 7
    bf16x8 qf[kD / 16];
    {
        const int t = q0 + l32;
#pragma unroll
        for (int s = 0; s < kD / 16; ++s) {
            u32x4 v = {0u, 0u, 0u, 0u};
            if (t < p.Sq) v = *(const u32x4 *)(p.q + b * p.sbq + head * p.shq + (long long)t * p.ldq + s * 16 + hi * 8);
            qf[s] = __builtin_bit_cast(bf16x8, v);
        }
        // the query's head norm (as mica_head_norm_rope: fragment s is piece 2 s + hi of the head, its
        // level-1 partner piece in lane l ^ 32)
        if (p.qnw != nullptr) {
            float l1[kD / 16];
#pragma unroll
            for (int s = 0; s < kD / 16; ++s) {
                const float own = piece_squares(__builtin_bit_cast(u32x4, qf[s]));
                const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(own), __float_as_uint(own), false, false);
                l1[s] = own + __uint_as_float(hi ? r[0] : r[1]);     // pieces ^ 1
            }
#pragma unroll
            for (int m = 1; m < kD / 16; m <<= 1)                      // pieces ^ 2, ^ 4, ^ 8, ^ 16
#pragma unroll
                for (int s = 0; s < kD / 16; ++s)
                    if (!(s & m)) {
                        const float v = l1[s] + l1[s | m];
                        l1[s] = v;
                        l1[s | m] = v;
                    }
            const float rstd = 1.0f / __builtin_sqrtf(l1[0] / (float)kD + p.neps);
#pragma unroll
            for (int s = 0; s < kD / 16; ++s)
                qf[s] = __builtin_bit_cast(bf16x8, norm8(__builtin_bit_cast(u32x4, qf[s]), rstd, p.noff,
                                                         *(const u32x4 *)(p.qnw + s * 16 + hi * 8)));
        }
        // rotary embedding of the query's first rot_dim dims (rope_pairs8, as mica_rope_inplace): dims
        // d < rot_dim / 2 and d + rot_dim / 2 are fragments s and s + rot_dim / 32 of the same lane
        const int rq = p.rot_dim >> 1;
        const int rp = rq == 0 || t >= p.Sq ? -1 : p.rpos ? p.rpos[b * p.Sq + t] : p.ntiles_p * kBK + t;
        if (rp >= 0 && rp < p.rn_pos) {
            const uint16_t *cs = p.rcos + (long long)rp * rq + hi * 8;
            const uint16_t *sn = p.rsin + (long long)rp * rq + hi * 8;
            // one instance per rot_dim, so that the fragments are indexed by constants
            auto rotate = [&](auto rq_c) {
                constexpr int RQ = decltype(rq_c)::value;
#pragma unroll
                for (int s = 0; s < RQ / 16; ++s) {
                    u32x4 ya, yb;
                    rope_pairs8(__builtin_bit_cast(u32x4, qf[s]), __builtin_bit_cast(u32x4, qf[s + RQ / 16]),
                                *(const u32x4 *)(cs + s * 16), *(const u32x4 *)(sn + s * 16), ya, yb);
                    qf[s] = __builtin_bit_cast(bf16x8, ya);
                    qf[s + RQ / 16] = __builtin_bit_cast(bf16x8, yb);
                }
            };
            if (rq == kD / 2) rotate(std::integral_constant<int, kD / 2>{});
            else if (rq == kD / 4) rotate(std::integral_constant<int, kD / 4>{});
            else rotate(std::integral_constant<int, kD / 8>{});
        }
    }
    f32x16 O[kD / 32];
#pragma unroll
    for (int dt = 0; dt < kD / 32; ++dt) O[dt] = f32x16{};
    // a split's range may hold no key at or below some of its queries: with a finite start the
    // exponentials of their masked scores are exp2(-inf) = 0 (not NaN) and their state stays (m, 0, 0)
    float m_used = SPLIT ? -1e30f : -__builtin_inff(), lsum = 0.0f;
    const int query = off + q0 + l32; // position of this lane's query

    // K fragment s of a stage (A operand of S^T, read two steps ahead of its MFMA: left to itself the
    // compiler reads each fragment right before its MFMA and waits)
    const int kfoff = l32 * 512;
    // V^T operand (dims 32 dt + l % 32, step s) of a stage: vt_swz(d) does not depend on dt
    int vfoff[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) vfoff[s] = l32 * (kBK * 2) + (((2 * s + hi) ^ vt_swz(l32)) << 4);
    // tile j in stage (j - first) % 2, the other stage receiving tile j + 1
    if (first <= last_own) dma_tile(first, 0);
    for (int j = first; j <= last_own; ++j) {
        const int st = (j - first) & 1;
        // this wave's DMA of tile j landed; after the barrier every wave's has, and nobody reads
        // stage st ^ 1 (tile j - 1) any more
        fa_wait_vmcnt<0>();
        __syncthreads();
        if (j + 1 <= last_own) dma_tile(j + 1, st ^ 1);
        const int8_t *ks = smem + st * kStage;
        const int8_t *vs = ks + kKBytes;
        // ---- S^T = K Q^T: rows = keys j*32 + acc_row, column = query l % 32 ----
        f32x16 sacc = {};
        auto kfrag = [&](int s) {
            return __builtin_bit_cast(bf16x8, *(const u32x4 *)(ks + kfoff + (((2 * s + hi) ^ l32) * 16)));
        };
        bf16x8 ka = kfrag(0), kb = kfrag(1);
#pragma unroll
        for (int s = 0; s < kD / 16; ++s) {
            const bf16x8 a = (s & 1) ? kb : ka;
            if (s + 2 < kD / 16) {
                if (s & 1) kb = kfrag(s + 2);
                else ka = kfrag(s + 2);
            }
            __builtin_amdgcn_sched_barrier(0);
            sacc = mfma_bf16(a, qf[s], sacc);
        }
        // raw scores, masked above the diagonal; the maximum in log2 units (the scale is positive, so
        // it commutes with the maximum and its rounding)
        float mloc = -__builtin_inff();
        if (j * kBK + kBK - 1 <= off + q0) { // the whole tile lies at or below the block's diagonal
#pragma unroll
            for (int r = 0; r < 16; ++r) mloc = __builtin_fmaxf(mloc, sacc[r]);
        } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = j * kBK + 8 * (r >> 2) + 4 * hi + (r & 3);
                sacc[r] = key <= query ? sacc[r] : -__builtin_inff();
                mloc = __builtin_fmaxf(mloc, sacc[r]);
            }
        }
        mloc = half_swap_max(mloc) * p.scale_log2; // the other half of the wave holds the same queries' other keys
        // lazy rescale: move the reference maximum only when the new one exceeds it by more than 8
        const bool grow = mloc > m_used + 8.0f;
        const float alpha = grow ? __builtin_amdgcn_exp2f(m_used - mloc) : 1.0f;
        if (grow) m_used = mloc;
        if (__builtin_amdgcn_ballot_w64(grow)) {
#pragma unroll
            for (int dt = 0; dt < kD / 32; ++dt) O[dt] *= alpha;
            lsum *= alpha;
        }
        // p = 2^(scale s - m), the scaling fused into the exponent's argument
        bf16x8 pb[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            u32x4 w;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[8 * s + 2 * e], p.scale_log2, -m_used));
                const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[8 * s + 2 * e + 1], p.scale_log2, -m_used));
                lsum += p0 + p1;
                w[e] = pack_bf16x2(p0, p1);
            }
            pb[s] = __builtin_bit_cast(bf16x8, w);
        }
        // ---- O^T += V^T P^T: lane's keys for step s are rows 8 s .. 8 s + 7 of the accumulator, i.e.
        // key units 4 s + hi and 4 s + 2 + hi (4 keys each), one 16-byte chunk of the V^T image ----
        // Step m = 8 s + dt: every dim tile's step 0, then its step 1 (the two MFMAs on one accumulator
        // 8 apart, in the same order as before); the V^T fragments are read two steps ahead of their MFMA
        // (left to itself the compiler reads each into one register quad right before its MFMA and waits)
        auto vfrag = [&](int m) {
            return __builtin_bit_cast(bf16x8, *(const u32x4 *)(vs + vfoff[m >> 3] + (m & 7) * 32 * (kBK * 2)));
        };
        bf16x8 va = vfrag(0), vb = vfrag(1);
#pragma unroll
        for (int m = 0; m < kD / 16; ++m) {
            const bf16x8 a = (m & 1) ? vb : va;
            if (m + 2 < kD / 16) {
                if (m & 1) vb = vfrag(m + 2);
                else va = vfrag(m + 2);
            }
            __builtin_amdgcn_sched_barrier(0);
            O[m & 7] = mfma_bf16(a, pb[m >> 3], O[m & 7]);
        }
    }
    const float ltot = half_swap_sum(lsum);
    if constexpr (SPLIT) {
        // the partial state: O (fp32, 4 dims per 16-byte store) of query row q0 + l % 32, m and l;
        // rows past Sq (up to sq_pad) are written too and never read
        const long long prow = ((long long)(b * p.HQ + head) * p.nsplit + split) * p.sq_pad + q0 + l32;
        float *po = p.part_o + prow * kD;
#pragma unroll
        for (int dt = 0; dt < kD / 32; ++dt)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const int d = dt * 32 + 8 * r4 + 4 * hi;
                *(float4 *)(po + d) = float4{O[dt][4 * r4], O[dt][4 * r4 + 1], O[dt][4 * r4 + 2], O[dt][4 * r4 + 3]};
            }
        if (hi == 0) {
            p.part_m[prow] = m_used;
            p.part_l[prow] = ltot;
        }
        return;
    }
    // ---- normalise, stage per wave in LDS (32 queries x 512 B), write 16-byte row pieces ----
    const float inv = 1.0f / ltot;
    __syncthreads(); // every wave is done with the operand stages
    int8_t *ost = smem + wave * (kBQ * kD * 2);
#pragma unroll
    for (int dt = 0; dt < kD / 32; ++dt)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            const int d = dt * 32 + 8 * r4 + 4 * hi;
            u32x2 w;
            w[0] = pack_bf16x2(O[dt][4 * r4] * inv, O[dt][4 * r4 + 1] * inv);
            w[1] = pack_bf16x2(O[dt][4 * r4 + 2] * inv, O[dt][4 * r4 + 3] * inv);
            *(u32x2 *)(ost + l32 * (kD * 2) + d * 2) = w;
        }
#pragma unroll
    for (int it = 0; it < (kBQ * kD * 2) / (64 * 16); ++it) {
        const int piece = it * 64 + lane;
        const int row = piece >> 5, c = piece & 31; // 32 pieces of 16 B per 512 B row
        const int t = q0 + row;
        const u32x4 v = *(const u32x4 *)(ost + row * (kD * 2) + c * 16);
        if (t < p.Sq) __builtin_nontemporal_store(v, (u32x4 *)(p.o + b * p.sbo + head * p.sho + (long long)t * p.ldo + c * 8));
    }
}

// ---- merge of the split partial states: one wave per (sequence, query head, query row), 4 dims per
// lane.  With M = max_s m_s, w_s = exp2(m_s - M): o = (sum_s w_s O_s) / (sum_s w_s l_s), rounded to
// bf16 (a split whose keys are all masked for the row has l_s = 0 and O_s = 0) ----
__global__ __launch_bounds__(256) void fa_merge_kernel(FaParams p) {
    const long long r = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);  // (b * HQ + head) * Sq + t
    const int lane = threadIdx.x & 63;
    if (r >= (long long)p.B * p.HQ * p.Sq) return;
    const int t = (int)(r % p.Sq);
    const long long bh = r / p.Sq;
    const int b = (int)(bh / p.HQ), head = (int)(bh % p.HQ);
    const long long row0 = bh * p.nsplit * p.sq_pad + t;  // split s at row0 + s * sq_pad
    float mx = -__builtin_inff();
    for (int sp = 0; sp < p.nsplit; ++sp) mx = __builtin_fmaxf(mx, p.part_m[row0 + (long long)sp * p.sq_pad]);
    float4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    float l = 0.0f;
    for (int sp = 0; sp < p.nsplit; ++sp) {
        const long long pr = row0 + (long long)sp * p.sq_pad;
        const float w = __builtin_amdgcn_exp2f(p.part_m[pr] - mx);
        const float4 o = *(const float4 *)(p.part_o + pr * kD + lane * 4);
        l += w * p.part_l[pr];
        acc.x += w * o.x;
        acc.y += w * o.y;
        acc.z += w * o.z;
        acc.w += w * o.w;
    }
    const float inv = 1.0f / l;
    u32x2 out;
    out[0] = pack_bf16x2(acc.x * inv, acc.y * inv);
    out[1] = pack_bf16x2(acc.z * inv, acc.w * inv);
    *(u32x2 *)(p.o + b * p.sbo + head * p.sho + (long long)t * p.ldo + lane * 4) = out;
}

}  // namespace

extern "C" long long mica_attention_workspace_bytes(int B, int Sk, int HK) {
    if (B < 0 || Sk < 0 || HK <= 0) return -1;
    return (long long)B * HK * ((Sk + kBK - 1) / kBK) * kVBytes;
}

extern "C" long long mica_attention_prefix_workspace_bytes(int B, int Sq, int Sk, int Pk, int HQ, int HK, int key_splits) {
    if (B < 0 || Sq < 0 || Sk < 0 || Pk < 0 || Pk % kBK || Pk > Sk || HQ <= 0 || HK <= 0 || key_splits < 1 ||
        key_splits > kMaxKeySplits)
        return -1;
    // the prefix's V^T images (one set for every sequence), each sequence's own, the split states
    long long n = (long long)HK * (Pk / kBK) * kVBytes + mica_attention_workspace_bytes(B, Sk - Pk, HK);
    if (key_splits > 1) n += (long long)B * HQ * key_splits * ((Sq + kBQ - 1) / kBQ) * kBQ * (kD * 4 + 8);
    return n;
}

extern "C" long long mica_attention_split_workspace_bytes(int B, int Sq, int Sk, int HQ, int HK, int key_splits) {
    return mica_attention_prefix_workspace_bytes(B, Sq, Sk, 0, HQ, HK, key_splits);
}

namespace {

// kp / vp (optional, Pk > 0 keys, a multiple of 32): a key prefix shared by every sequence, read in
// place of each sequence's first Pk keys; k / v then hold each sequence's Sk - Pk keys after it.
int attention_launch(const void *q, long long sbq, long long shq, long long ldq, const void *k, long long sbk,
                     long long shk, long long ldk, const void *v, long long sbv, long long shv, long long ldv,
                     const void *kp, long long shkp, long long ldkp, const void *vp, long long shvp, long long ldvp,
                     int Pk, void *o, long long sbo, long long sho, long long ldo, int B, int Sq, int Sk, int HQ,
                     int HK, int head_dim, float scale, int causal, int key_splits, const int *kv_len, void *workspace,
                     long long workspace_bytes, mica_stream_t stream, const void *q_norm_w = nullptr,
                     const void *k_norm_w = nullptr, float norm_offset = 0.0f, float norm_eps = 0.0f,
                     int rot_dim = 0, const void *rope_cos = nullptr, const void *rope_sin = nullptr,
                     int rope_n_pos = 0, const int *rope_pos = nullptr) {
    if (head_dim != kD || HK <= 0 || HQ != HK * kFaWaves || B < 0 || Sq < 0 || Sk < Sq) return MICA_MISS_SHAPE;
    if (Pk < 0 || Pk % kBK || Pk > Sk - Sq) return MICA_MISS_SHAPE;
    if (!causal || key_splits < 1 || key_splits > kMaxKeySplits) return MICA_MISS_ARG;
    if (B == 0 || Sq == 0) return 0;
    if (q == nullptr || k == nullptr || v == nullptr || o == nullptr || workspace == nullptr) return MICA_MISS_ARG;
    if (Pk > 0 && (kp == nullptr || vp == nullptr)) return MICA_MISS_ARG;
    if (rot_dim != 0 || q_norm_w != nullptr || k_norm_w != nullptr) {
        // the treated rows are the new ones: every key past the prefix is one, none has its own count
        if (rot_dim != 0 && rot_dim != kD / 4 && rot_dim != kD / 2 && rot_dim != kD) return MICA_MISS_SHAPE;
        if (rot_dim != 0 && (rope_cos == nullptr || rope_sin == nullptr || rope_n_pos <= 0)) return MICA_MISS_ARG;
        if (kv_len != nullptr) return MICA_MISS_ARG;
        if (Sk != Pk + Sq) return MICA_MISS_SHAPE;
        if ((rot_dim && (!mica_aligned16(rope_cos) || !mica_aligned16(rope_sin))) ||
            (q_norm_w && !mica_aligned16(q_norm_w)) || (k_norm_w && !mica_aligned16(k_norm_w)))
            return MICA_MISS_ALIGN;
    }
    const long long st[16] = {sbq, shq, ldq, sbk, shk, ldk, sbv, shv, ldv, sbo, sho, ldo, shkp, ldkp, shvp, ldvp};
    for (long long x : st)
        if (x < 0 || x % 8) return MICA_MISS_STRIDE;
    if (ldq < kD && Sq > 1) return MICA_MISS_STRIDE;
    if (!mica_aligned16(q) || !mica_aligned16(k) || !mica_aligned16(v) || !mica_aligned16(o) ||
        !mica_aligned16(workspace) || (Pk > 0 && (!mica_aligned16(kp) || !mica_aligned16(vp))))
        return MICA_MISS_ALIGN;
    const int ntiles_q = (Sq + kBQ - 1) / kBQ, ntiles_k = (Sk + kBK - 1) / kBK, ntiles_p = Pk / kBK;
    if ((long long)ntiles_k * kBK * ldk * 2 >= (1LL << 31) || (long long)ntiles_k * kVBytes >= (1LL << 31) ||
        (long long)Pk * ldkp * 2 >= (1LL << 31) || (long long)ntiles_q * key_splits > 65535 || B > 65535)
        return MICA_MISS_RANGE;
    if (workspace_bytes < mica_attention_prefix_workspace_bytes(B, Sq, Sk, Pk, HQ, HK, key_splits)) return MICA_MISS_ARG;
    FaParams p{};
    p.q = (const uint16_t *)q; p.sbq = sbq; p.shq = shq; p.ldq = ldq;
    p.k = (const uint16_t *)k; p.sbk = sbk; p.shk = shk; p.ldk = ldk;
    p.v = (const uint16_t *)v; p.sbv = sbv; p.shv = shv; p.ldv = ldv;
    p.o = (uint16_t *)o; p.sbo = sbo; p.sho = sho; p.ldo = ldo;
    p.B = B; p.Sq = Sq; p.Sk = Sk; p.HQ = HQ; p.HK = HK; p.ntiles_q = ntiles_q; p.ntiles_k = ntiles_k;
    p.scale_log2 = scale * 1.44269504088896341f;
    p.nsplit = key_splits;
    p.sq_pad = ntiles_q * kBQ;
    p.kv_len = kv_len;
    p.qnw = (const uint16_t *)q_norm_w; p.knw = (const uint16_t *)k_norm_w;
    p.noff = norm_offset; p.neps = norm_eps; p.rot_dim = rot_dim;
    p.rcos = (const uint16_t *)rope_cos; p.rsin = (const uint16_t *)rope_sin; p.rpos = rope_pos;
    p.rn_pos = rope_n_pos;
    // workspace: the prefix's V^T images, then each sequence's, then the split states
    char *ws = (char *)workspace;
    p.kp = (const uint16_t *)kp; p.shkp = shkp; p.ldkp = ldkp;
    p.vtp = (uint16_t *)ws;
    p.ntiles_p = ntiles_p;
    ws += (long long)HK * ntiles_p * kVBytes;
    p.vt = (uint16_t *)ws;
    ws += mica_attention_workspace_bytes(B, Sk - Pk, HK);
    if (key_splits > 1) {
        // partial states: O rows (1 KiB each), then m, then l
        const long long rows = (long long)B * HQ * key_splits * p.sq_pad;
        p.part_o = (float *)ws;
        p.part_m = (float *)(ws + rows * kD * 4);
        p.part_l = p.part_m + rows;
    }
    hipStream_t stream_ = (hipStream_t)stream;
    // V^T images: each sequence's keys past the prefix, and the prefix's once (as one sequence)
    FaParams pv = p;
    pv.Sk = Sk - Pk;
    pv.ntiles_k = ntiles_k - ntiles_p;
    hipLaunchKernelGGL(v_transpose_kernel, dim3(pv.ntiles_k, B * HK), dim3(256), 0, stream_, pv);
    int rc = mica_err(hipGetLastError());
    if (rc) return rc;
    if (ntiles_p > 0) {
        FaParams pp = p;
        pp.v = (const uint16_t *)vp; pp.sbv = 0; pp.shv = shvp; pp.ldv = ldvp;
        pp.Sk = Pk;
        pp.ntiles_k = ntiles_p;
        pp.vt = (uint16_t *)p.vtp;  // the prefix images are written here, read-only in the attention kernel
        pp.knw = nullptr;           // the prefix's keys come normed and rotated
        pp.rot_dim = 0;
        hipLaunchKernelGGL(v_transpose_kernel, dim3(ntiles_p, HK), dim3(256), 0, stream_, pp);
        rc = mica_err(hipGetLastError());
        if (rc) return rc;
    }
    if (key_splits == 1) {
        hipLaunchKernelGGL(fa_fwd_kernel<false>, dim3(HK, B, ntiles_q), dim3(kFaThreads), 0, stream_, p);
        return mica_err(hipGetLastError());
    }
    hipLaunchKernelGGL(fa_fwd_kernel<true>, dim3(HK, B, ntiles_q * key_splits), dim3(kFaThreads), 0, stream_, p);
    rc = mica_err(hipGetLastError());
    if (rc) return rc;
    const long long rows = (long long)B * HQ * Sq;
    if ((rows + 3) / 4 >= (1LL << 31)) return MICA_MISS_RANGE;
    hipLaunchKernelGGL(fa_merge_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream_, p);
    return mica_err(hipGetLastError());
}

}  // namespace

extern "C" int mica_attention_fwd(const void *q, long long sbq, long long shq, long long ldq, const void *k, long long sbk,
                                  long long shk, long long ldk, const void *v, long long sbv, long long shv,
                                  long long ldv, void *o, long long sbo, long long sho, long long ldo, int B, int Sq,
                                  int Sk, int HQ, int HK, int head_dim, float scale, int causal, void *workspace,
                                  long long workspace_bytes, mica_stream_t stream) {
    return attention_launch(q, sbq, shq, ldq, k, sbk, shk, ldk, v, sbv, shv, ldv, nullptr, 0, 0, nullptr, 0, 0, 0, o,
                            sbo, sho, ldo, B, Sq, Sk, HQ, HK, head_dim, scale, causal, 1, nullptr, workspace,
                            workspace_bytes, stream);
}

extern "C" int mica_attention_fwd_split(const void *q, long long sbq, long long shq, long long ldq, const void *k,
                                        long long sbk, long long shk, long long ldk, const void *v, long long sbv,
                                        long long shv, long long ldv, void *o, long long sbo, long long sho,
                                        long long ldo, int B, int Sq, int Sk, int HQ, int HK, int head_dim, float scale,
                                        int causal, int key_splits, void *workspace, long long workspace_bytes,
                                        mica_stream_t stream) {
    return attention_launch(q, sbq, shq, ldq, k, sbk, shk, ldk, v, sbv, shv, ldv, nullptr, 0, 0, nullptr, 0, 0, 0, o,
                            sbo, sho, ldo, B, Sq, Sk, HQ, HK, head_dim, scale, causal, key_splits, nullptr, workspace,
                            workspace_bytes, stream);
}

extern "C" int mica_attention_fwd_kvlen(const void *q, long long sbq, long long shq, long long ldq, const void *k,
                                        long long sbk, long long shk, long long ldk, const void *v, long long sbv,
                                        long long shv, long long ldv, void *o, long long sbo, long long sho,
                                        long long ldo, int B, int Sq, int Sk, int HQ, int HK, int head_dim, float scale,
                                        int causal, int key_splits, const int *kv_len, void *workspace,
                                        long long workspace_bytes, mica_stream_t stream) {
    if (kv_len == nullptr) return MICA_MISS_ARG;
    return attention_launch(q, sbq, shq, ldq, k, sbk, shk, ldk, v, sbv, shv, ldv, nullptr, 0, 0, nullptr, 0, 0, 0, o,
                            sbo, sho, ldo, B, Sq, Sk, HQ, HK, head_dim, scale, causal, key_splits, kv_len, workspace,
                            workspace_bytes, stream);
}

extern "C" int mica_attention_fwd_prefix(const void *q, long long sbq, long long shq, long long ldq, const void *k,
                                         long long sbk, long long shk, long long ldk, const void *v, long long sbv,
                                         long long shv, long long ldv, const void *kp, long long shkp, long long ldkp,
                                         const void *vp, long long shvp, long long ldvp, int Pk, void *o,
                                         long long sbo, long long sho, long long ldo, int B, int Sq, int Sk, int HQ,
                                         int HK, int head_dim, float scale, int causal, int key_splits,
                                         const int *kv_len, void *workspace, long long workspace_bytes,
                                         mica_stream_t stream) {
    return attention_launch(q, sbq, shq, ldq, k, sbk, shk, ldk, v, sbv, shv, ldv, kp, shkp, ldkp, vp, shvp, ldvp, Pk,
                            o, sbo, sho, ldo, B, Sq, Sk, HQ, HK, head_dim, scale, causal, key_splits, kv_len,
                            workspace, workspace_bytes, stream);
}

extern "C" int mica_attention_fwd_rope(const void *q, long long sbq, long long shq, long long ldq, void *k,
                                       long long sbk, long long shk, long long ldk, const void *v, long long sbv,
                                       long long shv, long long ldv, const void *kp, long long shkp, long long ldkp,
                                       const void *vp, long long shvp, long long ldvp, int Pk, void *o,
                                       long long sbo, long long sho, long long ldo, int B, int Sq, int Sk, int HQ,
                                       int HK, int head_dim, float scale, int causal, int key_splits,
                                       const void *q_norm_w, const void *k_norm_w, float norm_offset, float norm_eps,
                                       int rot_dim, const void *cos_tab, const void *sin_tab, int n_pos,
                                       const int *pos, void *workspace, long long workspace_bytes,
                                       mica_stream_t stream) {
    if (rot_dim == 0 && q_norm_w == nullptr && k_norm_w == nullptr) return MICA_MISS_ARG;
    return attention_launch(q, sbq, shq, ldq, k, sbk, shk, ldk, v, sbv, shv, ldv, kp, shkp, ldkp, vp, shvp, ldvp, Pk,
                            o, sbo, sho, ldo, B, Sq, Sk, HQ, HK, head_dim, scale, causal, key_splits, nullptr,
                            workspace, workspace_bytes, stream, q_norm_w, k_norm_w, norm_offset, norm_eps, rot_dim,
                            cos_tab, sin_tab, n_pos, pos);
}
