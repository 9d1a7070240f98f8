// Rotary position embedding applied in place to the q and k heads of a fused QKV projection output,
// in bf16 arithmetic as the attention layers compute it (transformers apply_rotary_pos_emb:
// q * cos + rotate_half(q) * sin, each product rounded to bf16, then their sum rounded to bf16):
//     y[i]     = bf16(bf16(x[i] cos_i) + bf16(x[i + h] (-sin_i)))
//     y[i + h] = bf16(bf16(x[i + h] cos_i) + bf16(x[i] sin_i)),      i < h = head_dim / 2
// cos / sin are the model's bf16 tables [positions][h].  One thread rotates 8 pairs of one head of
// one token: two 16-byte loads of x, one of cos and one of sin, two 16-byte stores.

#include "common.h"

namespace {

constexpr int kRopeThreads = 256;

struct RopeParams {
    uint16_t *x; long long ldx;   // bf16 [T][...]: head j of token t at x + t ldx + j head_dim
    const uint16_t *cs, *sn;      // bf16 [n_pos][head_dim / 2]
    const int *pos;               // int32 [T] positions, or null: t % period
    int n_heads, head_dim, T, period, n_pos;
};

__global__ __launch_bounds__(kRopeThreads) void rope_kernel(RopeParams p) {
    const int h = p.head_dim >> 1;
    const int groups = h >> 3;                          // 8-pair groups per head
    const long gid = (long)blockIdx.x * kRopeThreads + threadIdx.x;
    const long per_token = (long)p.n_heads * groups;
    const long t = gid / per_token;
    if (t >= p.T) return;
    const int rem = (int)(gid - t * per_token);
    const int head = rem / groups, i0 = (rem - head * groups) * 8;
    const int pos = p.pos ? p.pos[t] : (int)(t % p.period);
    if (pos < 0 || pos >= p.n_pos) return;              // out-of-table position: left unrotated
    uint16_t *xh = p.x + t * p.ldx + (long)head * p.head_dim;
    const u32x4 a = *(const u32x4 *)(xh + i0), b = *(const u32x4 *)(xh + h + i0);
    const u32x4 c = *(const u32x4 *)(p.cs + (long)pos * h + i0), s = *(const u32x4 *)(p.sn + (long)pos * h + i0);
    u32x4 ya, yb;
    rope_pairs8(a, b, c, s, ya, yb);
    *(u32x4 *)(xh + i0) = ya;
    *(u32x4 *)(xh + h + i0) = yb;
}

}  // namespace

extern "C" int mica_rope_inplace(void *x, long long ldx, int n_heads, int head_dim, const void *cos_tab,
                                 const void *sin_tab, int n_pos, const int *pos, int period, int T,
                                 mica_stream_t stream) {
    if (x == nullptr || cos_tab == nullptr || sin_tab == nullptr) return MICA_MISS_ARG;
    if (T < 0 || n_heads <= 0 || head_dim <= 0 || head_dim % 16 != 0 || n_pos <= 0 || (pos == nullptr && period <= 0))
        return MICA_MISS_SHAPE;
    if (ldx < (long long)n_heads * head_dim || ldx % 8 != 0) return MICA_MISS_STRIDE;
    if (!mica_aligned16(x) || !mica_aligned16(cos_tab) || !mica_aligned16(sin_tab)) return MICA_MISS_ALIGN;
    if (T == 0) return 0;
    RopeParams p{};
    p.x = (uint16_t *)x; p.ldx = ldx; p.cs = (const uint16_t *)cos_tab; p.sn = (const uint16_t *)sin_tab;
    p.pos = pos; p.n_heads = n_heads; p.head_dim = head_dim; p.T = T; p.period = period; p.n_pos = n_pos;
    const long long threads = (long long)T * n_heads * (head_dim / 16);
    const long long blocks = (threads + kRopeThreads - 1) / kRopeThreads;
    if (blocks >= (1LL << 31)) return MICA_MISS_RANGE;
    hipLaunchKernelGGL(rope_kernel, dim3((unsigned)blocks), dim3(kRopeThreads), 0, (hipStream_t)stream, p);
    return mica_err(hipGetLastError());
}
