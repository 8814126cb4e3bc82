// attn.hip — decode attention for gfx950 over the paged fp16 K/V planes.
//
// K/V layout (MI355X-native): pages of 64 positions, head-major inside a
// page, so one kv head's 64 positions are one contiguous 64·hd·2-byte run:
//   element (pos, kvh, d) at ((pgtab[base + pos/64]·n_kv + kvh)·64 + pos%64)·hd + d
//
// Two forms, chosen by shape as the reference chooses (hd 128 with 4 or 8
// query heads per kv head takes the flash split-K; anything else the
// two-pass score/combine), each computing exactly the reference CPU
// backend's operation order:
//
// cj_attn_split_*: split-K (AttnKernel.attnDecodeCpuGqaKernel +
//   cpuDecodeHead, model/AttnKernel.cajeta:4216-4314). Splits per
//   cpuDecodeSplits (:4879-4889) for a given worker count; one workgroup per
//   (kv head, split slot), 16 lanes per query head; a split's positions run
//   in order through an online softmax whose scores are 16-lane partials
//   folded pairwise. K/V for a tile of positions is staged in LDS in a
//   lane-major layout. The last workgroup of a kv head merges the splits as
//   reducePackBlockCpu does (:5268-5400): four interleaved sub-sums.
// cj_attn_scores_* + cj_attn_combine_*: attnScoreKernel (:397-425) and
//   attnCombineKernel (:441-515): 32-lane strided dot + butterfly, then 128
//   lanes for max, exp and sum (stride-halving tree) and the ascending-t sum
//   of p·v per output dimension.
#include "common.h"

#define ATTN_MAX_SPLITS 64
#define ATTN_TILE 32

DEV int64_t kv_at(const int32_t *pgtab, int pg_base, int pos, int nkv, int kvh, int hd) {
    const int page = pgtab[pg_base + (pos >> 6)];
    return (((int64_t)page * nkv + kvh) * 64 + (pos & 63)) * hd;
}

// AttnKernel.cpuDecodeSplits: two work items a worker over the kv heads,
// within [1, min(64, count)].
DEV int decode_splits(int count, int nkv, int workers) {
    const int w = workers < 1 ? 1 : workers, rk = nkv < 1 ? 1 : nkv;
    int s = (2 * w + rk - 1) / rk;
    if (s > 64) s = 64;
    if (s > count) s = count;
    if (s < 1) s = 1;
    return s;
}

DEV void attn_window(const cj_attn_args &a, int &count, int &from) {
    if (a.state) { count = a.state->pos + 1; from = 0; } else { count = a.count; from = a.from; }
    if (a.window > 0 && count > a.window) { from += count - a.window; count = a.window; }
}

template <int HD, int G>
DEV void split_body(const cj_attn_args &a) {
    constexpr int VPL = HD / 16;                     // dims per lane: l, l+16, ...
    __shared__ uint16_t ks[ATTN_TILE][16][VPL], vs[ATTN_TILE][16][VPL];
    __shared__ int ticket;
    const int tid = threadIdx.x, nthr = G * 16;
    const int h = tid >> 4, l = tid & 15;
    const int kvh = blockIdx.x / ATTN_MAX_SPLITS, sp = blockIdx.x % ATTN_MAX_SPLITS;
    int count, from;
    attn_window(a, count, from);
    const int splits = decode_splits(count, a.n_kv, a.workers);
    const int qh = kvh * G + h;
    if (sp < splits) {
        const int chunk = (count + splits - 1) / splits;
        int t0 = sp * chunk, t1 = t0 + chunk;
        if (t1 > count) t1 = count;
        if (t0 > count) t0 = count;
        float q[VPL], acc[VPL];
#pragma unroll
        for (int v = 0; v < VPL; v++) { q[v] = a.q[(int64_t)qh * HD + 16 * v + l]; acc[v] = 0.0f; }
        float m = -3.0e38f, ls = 0.0f;
        for (int tb = t0; tb < t1; tb += ATTN_TILE) {
            const int n = t1 - tb < ATTN_TILE ? t1 - tb : ATTN_TILE;
            __syncthreads();
            // stage: 16-byte chunks (8 dims) of each position's K and V row,
            // all loads issued before the scatter of element d of position p
            // to [p][d % 16][d / 16]
            {
                constexpr int CPP = HD / 8;                      // chunks a position
                constexpr int CH = ATTN_TILE * CPP / (G * 16);   // chunks a thread
                uint4 kq[CH], vq[CH];
#pragma unroll
                for (int c = 0; c < CH; c++) {
                    const int e = tid + c * nthr, p = e / CPP, j = e % CPP;
                    if (p < n) {
                        const int64_t base = kv_at(a.pgtab, a.pg_base, from + tb + p, a.n_kv, kvh, HD) + 8 * j;
                        kq[c] = *(const uint4 *)(a.kc + base);
                        vq[c] = *(const uint4 *)(a.vc + base);
                    }
                }
#pragma unroll
                for (int c = 0; c < CH; c++) {
                    const int e = tid + c * nthr, p = e / CPP, j = e % CPP;
                    if (p < n) {
                        const uint32_t kw[4] = {kq[c].x, kq[c].y, kq[c].z, kq[c].w};
                        const uint32_t vw[4] = {vq[c].x, vq[c].y, vq[c].z, vq[c].w};
#pragma unroll
                        for (int i = 0; i < 8; i++) {
                            const int d = 8 * j + i;
                            ks[p][d & 15][d >> 4] = (uint16_t)(kw[i >> 1] >> (16 * (i & 1)));
                            vs[p][d & 15][d >> 4] = (uint16_t)(vw[i >> 1] >> (16 * (i & 1)));
                        }
                    }
                }
            }
            __syncthreads();
            for (int p = 0; p < n; p++) {
                float kf[VPL], vf[VPL];
#pragma unroll
                for (int v = 0; v < VPL; v++) { kf[v] = h2f(ks[p][l][v]); vf[v] = h2f(vs[p][l][v]); }
                float d = __fmul_rn(q[0], kf[0]);
#pragma unroll
                for (int v = 1; v < VPL; v++) d = __fadd_rn(d, __fmul_rn(q[v], kf[v]));
                d = __fadd_rn(d, __shfl_xor(d, 1));
                d = __fadd_rn(d, __shfl_xor(d, 2));
                d = __fadd_rn(d, __shfl_xor(d, 4));
                d = __fadd_rn(d, __shfl_xor(d, 8));
                const float sc = __fmul_rn(d, a.scale);
                if (sc > m) {
                    const float c = cj_expf(m - sc);
#pragma unroll
                    for (int v = 0; v < VPL; v++) acc[v] = __fmul_rn(acc[v], c);
                    ls = __fmul_rn(ls, c);
                    m = sc;
                }
                const float pr = cj_expf(sc - m);
                ls = __fadd_rn(ls, pr);
#pragma unroll
                for (int v = 0; v < VPL; v++) acc[v] = __fadd_rn(acc[v], __fmul_rn(vf[v], pr));
            }
        }
        float *pb = a.part + ((int64_t)qh * ATTN_MAX_SPLITS + sp) * (HD + 2);
#pragma unroll
        for (int v = 0; v < VPL; v++) pb[16 * v + l] = acc[v];
        if (l == 0) { pb[HD] = m; pb[HD + 1] = ls; }
    }
    if (!a.out) return;

    // the last workgroup of this kv head merges its splits
    __threadfence();
    __syncthreads();
    if (tid == 0) ticket = atomicAdd(&a.counters[kvh], 1);
    __syncthreads();
    if (ticket != ATTN_MAX_SPLITS - 1) return;
    __threadfence();
    for (int e = tid; e < G * HD; e += nthr) {
        const int hh = e / HD, dd = e % HD;
        const int qq = kvh * G + hh;
        const float *pb0 = a.part + (int64_t)qq * ATTN_MAX_SPLITS * (HD + 2);
        float gm = -3.0e38f;
        for (int s = 0; s < splits; s++) {
            const float mv = pb0[s * (HD + 2) + HD];
            if (mv > gm) gm = mv;
        }
        float tacc = 0.0f, gt = 0.0f;
        for (int sub = 0; sub < 4; sub++) {
            float gl = 0.0f, ac = 0.0f;
            for (int s = sub; s < splits; s += 4) {
                const float *pb = pb0 + s * (HD + 2);
                const float lsv = pb[HD + 1];
                if (lsv > 0.0f) {
                    const float wt = cj_expf(pb[HD] - gm);
                    gl = __fadd_rn(gl, __fmul_rn(wt, lsv));
                    ac = __fadd_rn(ac, __fmul_rn(pb[dd], wt));
                }
            }
            if (sub == 0) { tacc = ac; gt = gl; }
            else { tacc = __fadd_rn(tacc, ac); gt = __fadd_rn(gt, gl); }
        }
        a.out[(int64_t)qq * HD + dd] = __fmul_rn(tacc, __fdiv_rn(1.0f, gt));
    }
    if (tid == 0) a.counters[kvh] = 0;
}

#define SPLIT_KERNEL(HD, G) \
    extern "C" __global__ void __launch_bounds__(G * 16) cj_attn_split_h##HD##_g##G(cj_attn_args a) { split_body<HD, G>(a); }
SPLIT_KERNEL(128, 4)
SPLIT_KERNEL(128, 8)

// ------------------------------------------------------------ two-pass form

// scores[h][t] = scale · (q_h · K[from+t]): one 32-lane group per (h, t),
// lane i over d = i, i+32, ..., then a butterfly over the 32 lanes.
template <int HD>
DEV void scores_body(const cj_attn_args &a) {
    int count, from;
    attn_window(a, count, from);
    const int g = threadIdx.x >> 5, i = threadIdx.x & 31;
    const int64_t idx = (int64_t)blockIdx.x * 8 + g;
    const int grp = a.n_q / a.n_kv;
    const bool ok = idx < (int64_t)a.n_q * count;
    const int h = ok ? (int)(idx / count) : 0, t = ok ? (int)(idx % count) : 0;
    float s = 0.0f;
    if (ok) {
        const int64_t kb = kv_at(a.pgtab, a.pg_base, from + t, a.n_kv, h / grp, HD);
        for (int d = i; d < HD; d += 32) s = __fadd_rn(s, __fmul_rn(a.q[(int64_t)h * HD + d], h2f(a.kc[kb + d])));
    }
    s = __fadd_rn(s, __shfl_xor(s, 16, 32));
    s = __fadd_rn(s, __shfl_xor(s, 8, 32));
    s = __fadd_rn(s, __shfl_xor(s, 4, 32));
    s = __fadd_rn(s, __shfl_xor(s, 2, 32));
    s = __fadd_rn(s, __shfl_xor(s, 1, 32));
    if (ok && i == 0) a.part[(int64_t)h * a.splits + t] = __fmul_rn(s, a.scale);
}

// softmax over scores[h][0..count) in place and out[h] = Σ_t p_t·V_t / Σ p:
// one workgroup of 128 per query head.
template <int HD>
DEV void combine_body(const cj_attn_args &a) {
    __shared__ float red[128];
    int count, from;
    attn_window(a, count, from);
    const int h = blockIdx.x, l = threadIdx.x;
    const int grp = a.n_q / a.n_kv, kvh = h / grp;
    float *sc = a.part + (int64_t)h * a.splits;
    float mx = -3.0e38f;
    for (int t = l; t < count; t += 128) if (sc[t] > mx) mx = sc[t];
    red[l] = mx;
    __syncthreads();
    for (int r = 64; r > 0; r >>= 1) {
        if (l < r && red[l + r] > red[l]) red[l] = red[l + r];
        __syncthreads();
    }
    const float m = red[0];
    __syncthreads();
    float s = 0.0f;
    for (int t = l; t < count; t += 128) {
        const float e = cj_expf(sc[t] - m);
        sc[t] = e;
        s = __fadd_rn(s, e);
    }
    red[l] = s;
    __syncthreads();
    for (int r = 64; r > 0; r >>= 1) {
        if (l < r) red[l] = __fadd_rn(red[l], red[l + r]);
        __syncthreads();
    }
    const float rs = __fdiv_rn(1.0f, red[0]);
    for (int d = l; d < HD; d += 128) {
        float acc = 0.0f;
        for (int t = 0; t < count; t++) {
            const int64_t vb = kv_at(a.pgtab, a.pg_base, from + t, a.n_kv, kvh, HD);
            acc = __fadd_rn(acc, __fmul_rn(sc[t], h2f(a.vc[vb + d])));
        }
        a.out[(int64_t)h * HD + d] = __fmul_rn(acc, rs);
    }
}

extern "C" __global__ void __launch_bounds__(256) cj_attn_scores_h64(cj_attn_args a) { scores_body<64>(a); }
extern "C" __global__ void __launch_bounds__(256) cj_attn_scores_h128(cj_attn_args a) { scores_body<128>(a); }
extern "C" __global__ void __launch_bounds__(128) cj_attn_combine_h64(cj_attn_args a) { combine_body<64>(a); }
extern "C" __global__ void __launch_bounds__(128) cj_attn_combine_h128(cj_attn_args a) { combine_body<128>(a); }

// Merge split partials into f32 (+ the pack of the result): one workgroup of
// 256 per 256 output values (the reference's attnReducePackQ8Kernel
// contract), the merge in reducePackBlockCpu's order: the global max, then
// four interleaved sub-sums (splits s ≡ 0, 1, 2, 3 mod 4, each ascending) of
// w_s·l_s and of w_s·acc_s[d], w_s = exp(m_s − max), added in sub order;
// out = acc · (1 / l). The (head, split) weights are computed once in LDS.
extern "C" __global__ void __launch_bounds__(256) cj_attn_merge(cj_merge_args a) {
    __shared__ float wts[4][ATTN_MAX_SPLITS];     // per head of the block, per split (0: skipped)
    __shared__ int use[4][ATTN_MAX_SPLITS];
    __shared__ float gsum[4];
    const int t = threadIdx.x;
    const int64_t e = (int64_t)blockIdx.x * 256 + t;
    const int64_t n = (int64_t)a.n_q * a.head_dim;
    const int hd = a.head_dim;
    int splits = a.splits;
    if (a.state) {
        int count = a.state->pos + 1;
        if (a.window > 0 && count > a.window) count = a.window;
        splits = decode_splits(count, a.n_kv, a.workers);
    }
    const int h0 = (int)((int64_t)blockIdx.x * 256 / hd);     // first head of the block
    const int nh = 256 / hd < 1 ? 1 : 256 / hd;                 // heads a block (hd 64 or 128)
    // per (head, split): the weight, from the head's max over its splits
    {
        const int hh = t / ATTN_MAX_SPLITS, sp = t % ATTN_MAX_SPLITS;
        if (hh < nh && h0 + hh < a.n_q) {
            const float *pb0 = a.part + (int64_t)(h0 + hh) * ATTN_MAX_SPLITS * (hd + 2);
            float gm = -3.0e38f;
            for (int s2 = 0; s2 < splits; s2++) {
                const float mv = pb0[s2 * (hd + 2) + hd];
                if (mv > gm) gm = mv;
            }
            const bool on = sp < splits && pb0[sp * (hd + 2) + hd + 1] > 0.0f;
            use[hh][sp] = on;
            wts[hh][sp] = on ? cj_expf(pb0[sp * (hd + 2) + hd] - gm) : 0.0f;
        }
    }
    __syncthreads();
    if (t < nh && h0 + t < a.n_q) {
        const float *pb0 = a.part + (int64_t)(h0 + t) * ATTN_MAX_SPLITS * (hd + 2);
        float gt = 0.0f;
        for (int sub = 0; sub < 4; sub++) {
            float gl = 0.0f;
            for (int s2 = sub; s2 < splits; s2 += 4)
                if (use[t][s2]) gl = __fadd_rn(gl, __fmul_rn(wts[t][s2], pb0[s2 * (hd + 2) + hd + 1]));
            gt = sub == 0 ? gl : __fadd_rn(gt, gl);
        }
        gsum[t] = gt;
    }
    __syncthreads();
    float x = 0.0f;
    if (e < n) {
        const int h = (int)(e / hd), d = (int)(e % hd), hh = h - h0;
        const float *pb0 = a.part + (int64_t)h * ATTN_MAX_SPLITS * (hd + 2) + d;
        float ac[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int s0 = 0; s0 < splits; s0 += 4) {
#pragma unroll
            for (int sub = 0; sub < 4; sub++) {
                const int s2 = s0 + sub;
                if (s2 < splits && use[hh][s2]) ac[sub] = __fadd_rn(ac[sub], __fmul_rn(pb0[s2 * (hd + 2)], wts[hh][s2]));
            }
        }
        const float tacc = __fadd_rn(__fadd_rn(__fadd_rn(ac[0], ac[1]), ac[2]), ac[3]);
        x = __fmul_rn(tacc, __fdiv_rn(1.0f, gsum[hh]));
        if (a.out) a.out[e] = x;
    }
    if (!a.packed) return;
    // the block's pack: 256 values, one a thread
    __shared__ float bmax[8];
    const int lane = t & 63;
    const float av = fabsf(x);
    float am;
    if (a.per32) {
        const float mm = group_max<32>(av);
        if ((lane & 31) == 0) bmax[t >> 5] = mm;
        __syncthreads();
        am = bmax[t >> 5];
    } else {
        const float mm = group_max<64>(av);
        if (lane == 0) bmax[t >> 6] = mm;
        __syncthreads();
        am = fmaxf(fmaxf(bmax[0], bmax[1]), fmaxf(bmax[2], bmax[3]));
    }
    const float inv = am > 0.0f ? __fdiv_rn(127.0f, am) : 0.0f;
    const int q = round_away(__fmul_rn(x, inv));
    uint8_t *ob = a.packed + (int64_t)blockIdx.x * 320;
    ob[t] = (uint8_t)(int8_t)q;
    const int s = group_sum_i<32>(q);
    if ((lane & 31) == 0) *(int32_t *)(ob + 256 + 4 * (t >> 5)) = s;
    if (a.per32) {
        if ((lane & 31) == 0) *(float *)(ob + 288 + 4 * (t >> 5)) = __fdiv_rn(am, 127.0f);
    } else {
        if (t == 0) *(float *)(ob + 288) = __fdiv_rn(am, 127.0f);
        pack_zero_pad(ob, t);
    }
}

// QK-norm (optional) + split-half RoPE + fp16 K/V append, one workgroup of
// 64 per head, q heads first (AttnKernel.qkPrepKernel's contract).
extern "C" __global__ void __launch_bounds__(64) cj_qkprep(cj_qkprep_args a) {
    const int head = blockIdx.x, t = threadIdx.x;
    const bool isq = head < a.n_q;
    const int hd = a.head_dim, half = hd >> 1;
    const int kh = head - a.n_q;
    float *x = isq ? a.q + (int64_t)head * hd : a.k + (int64_t)kh * hd;
    const int pos = step_pos(a.state, a.pos);
    if (a.norm) {
        float ss = 0.0f;
        for (int i = t; i < hd; i += 64) ss = __fadd_rn(ss, __fmul_rn(x[i], x[i]));
        ss = group_sum<64>(ss);
        const float scale = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)hd), a.eps)));
        const float *w = isq ? a.qw : a.kw;
        for (int i = t; i < hd; i += 64) {
            const float wi = a.form == 1 ? __fadd_rn(1.0f, w[i]) : w[i];
            x[i] = __fmul_rn(__fmul_rn(x[i], scale), wi);
        }
        __syncthreads();
    }
    for (int d = t; d < half; d += 64) {
        const float2 cs = *(const float2 *)(a.rope_cs + 2 * ((int64_t)pos * half + d));
        const float x0 = x[d], x1 = x[d + half];
        const float ra = __fsub_rn(__fmul_rn(x0, cs.x), __fmul_rn(x1, cs.y));
        const float rb = __fadd_rn(__fmul_rn(x0, cs.y), __fmul_rn(x1, cs.x));
        x[d] = ra;
        x[d + half] = rb;
        if (!isq) {
            const int64_t ki = kv_at(a.pgtab, a.pg_base, pos, a.n_kv, kh, hd);
            a.kc[ki + d] = f2h(ra);
            a.kc[ki + d + half] = f2h(rb);
        }
    }
    if (!isq) {
        const int64_t vi = kv_at(a.pgtab, a.pg_base, pos, a.n_kv, kh, hd);
        for (int e = t; e < hd; e += 64) a.vc[vi + e] = f2h(a.v[(int64_t)kh * hd + e]);
    }
}
