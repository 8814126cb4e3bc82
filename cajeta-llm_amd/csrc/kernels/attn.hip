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
//   (kv head, split slot); a split's positions run in order through an
//   online softmax whose scores are the reference's 16 lane partials folded
//   pairwise. cj_attn_merge (or, with an output, the last workgroup of a kv
//   head) merges the splits as reducePackBlockCpu does (:5268-5400): four
//   interleaved sub-sums.
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

// One workgroup of 256 per (kv head, split slot). A split's positions go
// through LDS a tile at a time; per tile:
//   scores   thread (head, position): the reference's 16 lane partials
//            (lane l: Σ_v q[l+16v]·k[l+16v], v ascending) folded as the
//            xor-butterfly folds them — a fixed pairwise tree — so one thread
//            makes the same adds with no cross-lane traffic;
//   max      thread (head): the running max in position order, noting where
//            it rises (the reference rescales there);
//   exps     thread (head, position): the rescale factor exp(m_prev − s) and
//            the weight exp(s − m), all independent;
//   update   thread (head, dim): acc·c on a rise, then acc + v·p, in position
//            order; thread (head) does the same for the sum.
template <int HD, int G>
DEV void split_body(const cj_attn_args &a) {
    constexpr int TP = 64;                           // positions a tile
    constexpr int CK = 16;                           // positions a register chunk
    constexpr int PGMAX = 256;                       // page-table entries prefetched
    __shared__ __align__(16) uint16_t ks[TP][HD];
    __shared__ __align__(16) uint16_t vs[TP][HD];
    __shared__ __align__(16) float qs[G][HD];
    __shared__ __align__(16) float sc[G][TP], cf[G][TP], pr[G][TP], mb[G][TP], ma[G][TP];
    __shared__ int up[G][TP];
    __shared__ int pgs[PGMAX];
    __shared__ float mrun[G], lrun[G];
    const int t = threadIdx.x;
    const int kvh = blockIdx.x / ATTN_MAX_SPLITS, sp = blockIdx.x % ATTN_MAX_SPLITS;
    // q, the page table and the step state load together
    for (int e = t; e < G * HD; e += 256) qs[e / HD][e % HD] = a.q[(int64_t)(kvh * G) * HD + e];
    if (t < PGMAX) pgs[t] = t < a.pg_n ? a.pgtab[a.pg_base + t] : 0;
    int count, from;
    attn_window(a, count, from);
    const int splits = decode_splits(count, a.n_kv, a.workers);
    if (sp < splits) {
        const int chunk = (count + splits - 1) / splits;
        int t0 = sp * chunk, t1 = t0 + chunk;
        if (t1 > count) t1 = count;
        if (t0 > count) t0 = count;
        if (t < G) { mrun[t] = -3.0e38f; lrun[t] = 0.0f; }
        constexpr int PAIRS = G * HD / 256;          // (head, dim) pairs a thread
        float acc[PAIRS];
#pragma unroll
        for (int k = 0; k < PAIRS; k++) acc[k] = 0.0f;
        for (int tb = t0; tb < t1; tb += TP) {
            const int n = t1 - tb < TP ? t1 - tb : TP;
            __syncthreads();
            // stage the tile's K and V rows (16-byte chunks, natural layout)
            constexpr int CPP = HD / 8;
            for (int c = t; c < n * CPP; c += 256) {
                const int p = c / CPP, j = c % CPP;
                const int pos = from + tb + p, pi = pos >> 6;
                const int page = pi < PGMAX ? pgs[pi] : a.pgtab[a.pg_base + pi];
                const int64_t base = (((int64_t)page * a.n_kv + kvh) * 64 + (pos & 63)) * HD + 8 * j;
                *(uint4 *)&ks[p][8 * j] = *(const uint4 *)(a.kc + base);
                *(uint4 *)&vs[p][8 * j] = *(const uint4 *)(a.vc + base);
            }
            __syncthreads();
            // scores: thread (head, position)
            for (int hp = t; hp < G * TP; hp += 256) {
                const int h = hp / TP, p = hp % TP;
                if (p < n) {
                    float part[16];
#pragma unroll
                    for (int l = 0; l < 16; l++) part[l] = __fmul_rn(qs[h][l], h2f(ks[p][l]));
#pragma unroll
                    for (int v = 1; v < HD / 16; v++)
#pragma unroll
                        for (int l = 0; l < 16; l++)
                            part[l] = __fadd_rn(part[l], __fmul_rn(qs[h][l + 16 * v], h2f(ks[p][l + 16 * v])));
#pragma unroll
                    for (int w = 1; w < 16; w <<= 1)
#pragma unroll
                        for (int l = 0; l < 16; l += 2 * w) part[l] = __fadd_rn(part[l], part[l + w]);
                    sc[h][p] = __fmul_rn(part[0], a.scale);
                }
            }
            __syncthreads();
            // running max, in position order (scores read a chunk ahead)
            if (t < G) {
                float m = mrun[t];
                for (int p0 = 0; p0 < n; p0 += CK) {
                    float sv[CK];
#pragma unroll
                    for (int p = 0; p < CK; p += 4) {
                        const float4 f = *(const float4 *)&sc[t][p0 + p];
                        sv[p] = f.x; sv[p + 1] = f.y; sv[p + 2] = f.z; sv[p + 3] = f.w;
                    }
#pragma unroll
                    for (int p = 0; p < CK; p++) {
                        if (p0 + p < n) {
                            mb[t][p0 + p] = m;
                            up[t][p0 + p] = sv[p] > m;
                            if (sv[p] > m) m = sv[p];
                            ma[t][p0 + p] = m;
                        }
                    }
                }
                mrun[t] = m;
            }
            __syncthreads();
            // rescale factors (exactly 1 where the max holds: x·1 = x) and weights
            for (int hp = t; hp < G * TP; hp += 256) {
                const int h = hp / TP, p = hp % TP;
                if (p < n) {
                    cf[h][p] = up[h][p] ? cj_expf(mb[h][p] - sc[h][p]) : 1.0f;
                    pr[h][p] = cj_expf(sc[h][p] - ma[h][p]);
                }
            }
            __syncthreads();
            // the recurrences, in position order, operands a chunk ahead
#pragma unroll
            for (int k = 0; k < PAIRS; k++) {
                const int e = t + 256 * k, h = e / HD, d = e % HD;
                float x = acc[k];
                for (int p0 = 0; p0 < n; p0 += CK) {
                    float cv[CK], pv[CK], vv[CK];
#pragma unroll
                    for (int p = 0; p < CK; p += 4) {
                        const float4 c4 = *(const float4 *)&cf[h][p0 + p], p4 = *(const float4 *)&pr[h][p0 + p];
                        cv[p] = c4.x; cv[p + 1] = c4.y; cv[p + 2] = c4.z; cv[p + 3] = c4.w;
                        pv[p] = p4.x; pv[p + 1] = p4.y; pv[p + 2] = p4.z; pv[p + 3] = p4.w;
                    }
#pragma unroll
                    for (int p = 0; p < CK; p++) vv[p] = h2f(vs[p0 + p][d]);
#pragma unroll
                    for (int p = 0; p < CK; p++) {
                        if (p0 + p < n) {
                            x = __fmul_rn(x, cv[p]);
                            x = __fadd_rn(x, __fmul_rn(vv[p], pv[p]));
                        }
                    }
                }
                acc[k] = x;
            }
            if (t < G) {
                float ls = lrun[t];
                for (int p = 0; p < n; p++) {
                    ls = __fmul_rn(ls, cf[t][p]);
                    ls = __fadd_rn(ls, pr[t][p]);
                }
                lrun[t] = ls;
            }
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < PAIRS; k++) {
            const int e = t + 256 * k, h = e / HD, d = e % HD;
            a.part[((int64_t)(kvh * G + h) * ATTN_MAX_SPLITS + sp) * (HD + 2) + d] = acc[k];
        }
        if (t < G) {
            float *pb = a.part + ((int64_t)(kvh * G + t) * ATTN_MAX_SPLITS + sp) * (HD + 2);
            pb[HD] = mrun[t];
            pb[HD + 1] = lrun[t];
        }
    }
    if (!a.out) return;

    // the last workgroup of this kv head merges its splits
    __shared__ int ticket;
    __threadfence();
    __syncthreads();
    if (t == 0) ticket = atomicAdd(&a.counters[kvh], 1);
    __syncthreads();
    if (ticket != ATTN_MAX_SPLITS - 1) return;
    __threadfence();
    for (int e = t; e < G * HD; e += 256) {
        const int hh = e / HD, dd = e % HD;
        const int qq = kvh * G + hh;
        const float *pb0 = a.part + (int64_t)qq * ATTN_MAX_SPLITS * (HD + 2);
        float gm = -3.0e38f;
        for (int s2 = 0; s2 < splits; s2++) {
            const float mv = pb0[s2 * (HD + 2) + HD];
            if (mv > gm) gm = mv;
        }
        float tacc = 0.0f, gt = 0.0f;
        for (int sub = 0; sub < 4; sub++) {
            float gl = 0.0f, ac = 0.0f;
            for (int s2 = sub; s2 < splits; s2 += 4) {
                const float *pb = pb0 + s2 * (HD + 2);
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
    if (t == 0) a.counters[kvh] = 0;
}

#define SPLIT_KERNEL(HD, G) \
    extern "C" __global__ void __launch_bounds__(256) cj_attn_split_h##HD##_g##G(cj_attn_args a) { split_body<HD, G>(a); }
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
// out = acc · (1 / l).
extern "C" __global__ void __launch_bounds__(256) cj_attn_merge(cj_merge_args a) {
    const int t = threadIdx.x;
    const int64_t e = (int64_t)blockIdx.x * 256 + t;
    const int64_t n = (int64_t)a.n_q * a.head_dim;
    const int hd = a.head_dim;
    // thread t: output e (head h, dim d). Its 64 accumulators are loaded
    // first; meanwhile wave w (< heads in the block) reads head h0+w's
    // (max, sum) pairs, one split a lane, and leaves the weights in LDS.
    __shared__ float wts[4][ATTN_MAX_SPLITS], lsum[4][ATTN_MAX_SPLITS];
    __shared__ int use[4][ATTN_MAX_SPLITS];
    const int h0 = (int)((int64_t)blockIdx.x * 256 / hd), nh = hd >= 256 ? 1 : 256 / hd;
    // every slot of the partials is loaded (the buffer holds 64 a head); the
    // step's split count only masks the arithmetic, so no load waits on it
    float pv[ATTN_MAX_SPLITS];
    const int h = (int)(e / hd), d = (int)(e % hd);
    {
        const float *pb0 = a.part + (int64_t)(e < n ? h : 0) * ATTN_MAX_SPLITS * (hd + 2) + d;
#pragma unroll
        for (int s2 = 0; s2 < ATTN_MAX_SPLITS; s2++) pv[s2] = pb0[s2 * (hd + 2)];
    }
    int splits = a.splits;
    if (a.state) {
        int count = a.state->pos + 1;
        if (a.window > 0 && count > a.window) count = a.window;
        splits = decode_splits(count, a.n_kv, a.workers);
    }
    {
        const int w = t >> 6, sl = t & 63;
        if (w < nh) {
            const int hw = h0 + w < a.n_q ? h0 + w : 0;
            const float *pb = a.part + ((int64_t)hw * ATTN_MAX_SPLITS + sl) * (hd + 2) + hd;
            const float m0 = pb[0], l0 = pb[1];
            const bool in = h0 + w < a.n_q && sl < splits;
            const float mv = in ? m0 : -3.0e38f, lv = in ? l0 : 0.0f;
            const float gm = group_max<64>(mv);
            const bool on = in && lv > 0.0f;
            use[w][sl] = on;
            wts[w][sl] = on ? cj_expf(mv - gm) : 0.0f;
            lsum[w][sl] = lv;
        }
    }
    __syncthreads();
    float x = 0.0f;
    if (e < n) {
        const int hh = h - h0;
        float gl[4] = {0.0f, 0.0f, 0.0f, 0.0f}, ac[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s2 = 0; s2 < ATTN_MAX_SPLITS; s2++) {
            if (s2 < splits && use[hh][s2]) {
                const float w = wts[hh][s2];
                gl[s2 & 3] = __fadd_rn(gl[s2 & 3], __fmul_rn(w, lsum[hh][s2]));
                ac[s2 & 3] = __fadd_rn(ac[s2 & 3], __fmul_rn(pv[s2], w));
            }
        }
        const float gt = __fadd_rn(__fadd_rn(__fadd_rn(gl[0], gl[1]), gl[2]), gl[3]);
        const float tacc = __fadd_rn(__fadd_rn(__fadd_rn(ac[0], ac[1]), ac[2]), ac[3]);
        x = __fmul_rn(tacc, __fdiv_rn(1.0f, gt));
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
