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
//   lanes for exp and sum (stride-halving tree) and the ascending-t sum of
//   p·v per output dimension, its products staged through LDS.
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

// One workgroup of 256 per (kv head, split slot); wave w owns query heads
// w, w+4 of the kv head's group (one for G = 4, two for G = 8). A split's
// positions go through LDS a tile of 64 at a time. After the staging barrier
// every step is wave-local:
//   scores   lane p, position p: the reference's 16 lane partials (partial j:
//            Σ_v q[16v+j]·k[16v+j], v ascending) folded as the xor-butterfly
//            folds them — the fixed pairwise tree — K rows read from LDS
//            rows padded to 272 bytes (16-byte reads, no bank conflicts);
//   max      a wave prefix-max scan: lane p learns the running max before and
//            after its position (max is exact, so the scan order is free);
//   exps     lane p: the rescale exp(m_before − s) where s is a new maximum
//            (the reference rescales only there) and the weight exp(s − m);
//   update   lane d: acc·c (only where the maximum rose) then + v·w, in
//            position order, each position's c and w read from its lane.
// The last workgroup of a kv head to finish merges the head's splits and
// writes the merged output and its q8 pack.
template <int G>
DEV void split_body(const cj_attn_args &a) {
    constexpr int HD = 128, TP = 64, KS = HD + 8, PGMAX = 256, HW = G / 4;
    __shared__ __align__(16) uint16_t ks[TP][KS];
    __shared__ __align__(16) uint16_t vs[TP][HD];
    __shared__ __align__(16) float qs[G][HD];
    __shared__ int pgs[PGMAX];
    __shared__ float bmax[8];
    __shared__ int ticket;
    __shared__ uint64_t etab[32];
    cj_exp_table(etab);   // visible after the tile loop's first barrier
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    // id mod n_kv = kv head: a kv head's splits run on one XCD (workgroups are
    // dealt to the eight round-robin by id), whose L2 then holds the
    // partials its query heads' merges read
    const int kvh = blockIdx.x % a.n_kv, sp = blockIdx.x / a.n_kv;
    // q, the page table and the step state load together
    for (int e = 4 * t; e < G * HD; e += 1024) *(float4 *)&qs[0][e] = *(const float4 *)(a.q + (int64_t)kvh * G * HD + e);
    if (t < PGMAX) pgs[t] = t < a.pg_n ? a.pgtab[a.pg_base + t] : 0;
    int count, from;
    attn_window(a, count, from);
    const int splits = decode_splits(count, a.n_kv, a.workers);
    if (sp < splits) {
        const int chunk = (count + splits - 1) / splits;
        int t0 = sp * chunk, t1 = t0 + chunk;
        if (t1 > count) t1 = count;
        if (t0 > count) t0 = count;
        float m[HW], l[HW], acc0[HW], acc1[HW];
#pragma unroll
        for (int hh = 0; hh < HW; hh++) { m[hh] = -3.0e38f; l[hh] = 0.0f; acc0[hh] = 0.0f; acc1[hh] = 0.0f; }
        for (int tb = t0; tb < t1; tb += TP) {
            const int n = t1 - tb < TP ? t1 - tb : TP;
            __syncthreads();   // the previous tile's reads are done (first tile: q and pages visible)
            // stage the tile's K and V rows: 16-byte chunks, every load issued
            // before the first store (rows past the tile repeat its last row)
            {
                uint4 kr[4], vr[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int c = t + 256 * i, j = c & 15;
                    const int p = (c >> 4) < n ? (c >> 4) : n - 1;
                    const int pos = from + tb + p, pi = pos >> 6;
                    const int page = pi < PGMAX ? pgs[pi] : a.pgtab[a.pg_base + pi];
                    const int64_t base = (((int64_t)page * a.n_kv + kvh) * 64 + (pos & 63)) * HD + 8 * j;
                    kr[i] = *(const uint4 *)(a.kc + base);
                    vr[i] = *(const uint4 *)(a.vc + base);
                }
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int c = t + 256 * i;
                    *(uint4 *)&ks[c >> 4][8 * (c & 15)] = kr[i];
                    *(uint4 *)&vs[c >> 4][8 * (c & 15)] = vr[i];
                }
            }
            __syncthreads();
            // scores of position `lane` for this wave's heads, one head at a time
            float s[HW];
#pragma unroll
            for (int hh = 0; hh < HW; hh++) {
                const float *qh = &qs[wave + 4 * hh][0];
                float part[16];
#pragma unroll
                for (int c = 0; c < 16; c++) {
                    const uint4 kk = *(const uint4 *)&ks[lane][8 * c];
                    const float4 qa = *(const float4 *)(qh + 8 * c), qb = *(const float4 *)(qh + 8 * c + 4);
                    const uint32_t kw[4] = {kk.x, kk.y, kk.z, kk.w};
                    const float qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        const int j = 8 * (c & 1) + i;
                        const float pr = (i & 1) ? mul_h16hi(kw[i >> 1], qv[i]) : mul_h16lo(kw[i >> 1], qv[i]);
                        part[j] = c < 2 ? pr : __fadd_rn(part[j], pr);
                    }
                }
#pragma unroll
                for (int w = 1; w < 16; w <<= 1)
#pragma unroll
                    for (int j = 0; j < 16; j += 2 * w) part[j] = __fadd_rn(part[j], part[j + w]);
                s[hh] = __fmul_rn(part[0], a.scale);
            }
            const bool live = lane < n;
#pragma unroll 1
            for (int hh = 0; hh < HW; hh++) {
                // running max before (exc) and after (inc) each position
                const float inc = fmaxf(m[hh], wave_prefix_max(live ? s[hh] : -3.0e38f));
                const float exc = wave_shr1(inc, m[hh]);
                const bool up = live && s[hh] > exc;
                const uint64_t ups = __ballot(up);
                // the rescale's exp only where a position raises the maximum
                // (after the first tiles, rarely: the wave skips it)
                float cf = 1.0f;
                if (ups) cf = up ? cj_expf(exc - s[hh], etab) : 1.0f;
                const float pw = live ? cj_expf(s[hh] - inc, etab) : 0.0f;
                m[hh] = lane_f(inc, n - 1);
                // the lane's V pair of every position of the tile first (all
                // reads in flight at once), then the recurrence in position
                // order with each position's weight (and rescale, where the
                // maximum rose) read from its lane
                uint32_t vv[TP];
#pragma unroll
                for (int p = 0; p < TP; p++) vv[p] = *(const uint32_t *)&vs[p][2 * lane];
                float x0 = acc0[hh], x1 = acc1[hh], ls = l[hh];
#pragma unroll
                for (int p = 0; p < TP; p++) {
                    if (p < n) {
                        const float w = lane_f(pw, p);
                        if ((ups >> p) & 1) {
                            const float c = lane_f(cf, p);
                            x0 = __fmul_rn(x0, c);
                            x1 = __fmul_rn(x1, c);
                            ls = __fmul_rn(ls, c);
                        }
                        ls = __fadd_rn(ls, w);
                        x0 = __fadd_rn(x0, mul_h16lo(vv[p], w));
                        x1 = __fadd_rn(x1, mul_h16hi(vv[p], w));
                    }
                }
                acc0[hh] = x0; acc1[hh] = x1; l[hh] = ls;
            }
        }
#pragma unroll
        for (int hh = 0; hh < HW; hh++) {
            float *pb = a.part + ((int64_t)(kvh * G + wave + 4 * hh) * ATTN_MAX_SPLITS + sp) * (HD + 2);
            *(float2 *)(pb + 2 * lane) = make_float2(acc0[hh], acc1[hh]);
            if (lane == 0) *(float2 *)(pb + HD) = make_float2(m[hh], l[hh]);
        }
    }
    if (!a.out && !a.packed) return;

    // the last workgroup of this kv head merges its splits
    __threadfence();
    __syncthreads();
    if (t == 0) ticket = atomicAdd(&a.counters[kvh], 1);
    __syncthreads();
    if (ticket != ATTN_MAX_SPLITS - 1) return;
    __threadfence();
    float *ob = (float *)&vs[0][0];                  // G·HD merged values (LDS reuse)
#pragma unroll 1
    for (int hh = 0; hh < HW; hh++) {
        const int qq = kvh * G + wave + 4 * hh;
        const float *pb0 = a.part + (int64_t)qq * ATTN_MAX_SPLITS * (HD + 2);
        // lane s: split s's (max, sum); the weights of the merge
        const float2 ml = *(const float2 *)(pb0 + lane * (HD + 2) + HD);
        const bool in = lane < splits;
        const float mv = in ? ml.x : -3.0e38f;
        const float gm = group_max<64>(mv);
        const bool on = in && ml.y > 0.0f;
        const float wt = on ? cj_expf(mv - gm, etab) : 0.0f;
        const uint64_t ons = __ballot(on);
        float gl[4] = {0.0f, 0.0f, 0.0f, 0.0f}, ac0[4] = {0.0f, 0.0f, 0.0f, 0.0f}, ac1[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int s0 = 0; s0 < splits; s0 += 16) {
            float2 av[16];
#pragma unroll
            for (int k = 0; k < 16; k++) av[k] = *(const float2 *)(pb0 + (s0 + k) * (HD + 2) + 2 * lane);
#pragma unroll
            for (int k = 0; k < 16; k++) {
                const int s2 = s0 + k;
                if (s2 < splits && ((ons >> s2) & 1)) {
                    const float w = lane_f(wt, s2), lsv = lane_f(ml.y, s2);
                    gl[k & 3] = __fadd_rn(gl[k & 3], __fmul_rn(w, lsv));
                    ac0[k & 3] = __fadd_rn(ac0[k & 3], __fmul_rn(av[k].x, w));
                    ac1[k & 3] = __fadd_rn(ac1[k & 3], __fmul_rn(av[k].y, w));
                }
            }
        }
        const float gt = __fadd_rn(__fadd_rn(__fadd_rn(gl[0], gl[1]), gl[2]), gl[3]);
        const float rs = __fdiv_rn(1.0f, gt);
        const float o0 = __fmul_rn(__fadd_rn(__fadd_rn(__fadd_rn(ac0[0], ac0[1]), ac0[2]), ac0[3]), rs);
        const float o1 = __fmul_rn(__fadd_rn(__fadd_rn(__fadd_rn(ac1[0], ac1[1]), ac1[2]), ac1[3]), rs);
        if (a.out) *(float2 *)(a.out + (int64_t)qq * HD + 2 * lane) = make_float2(o0, o1);
        *(float2 *)(ob + (wave + 4 * hh) * HD + 2 * lane) = make_float2(o0, o1);
    }
    if (a.packed) {
        __syncthreads();
        // the kv head's G·HD outputs are G·HD/256 whole pack blocks
#pragma unroll
        for (int b = 0; b < G * HD / 256; b++)
            pack256(ob[256 * b + t], a.per32, a.packed + ((int64_t)kvh * (G * HD / 256) + b) * 320, bmax);
    }
    if (t == 0) a.counters[kvh] = 0;
}

// The many-row form (batched decode): workgroup (row, kv head, split slot);
// row r's sequence, position and q from the row table, the split rule over
// all rows' kv heads (AttnKernel.attnDecodeCpuGqaBatchKernel,
// model/AttnKernel.cajeta:4316-4350); a long split's next tile is requested
// during the current one.
template <int G>
DEV void split_rows_body(const cj_attn_args &a) {
    constexpr int HD = 128, TP = 64, KS = HD + 8, PGMAX = 256, HW = G / 4;
    __shared__ __align__(16) uint16_t ks[TP][KS];
    __shared__ __align__(16) uint16_t vs[TP][HD];
    __shared__ __align__(16) float qs[G][HD];
    __shared__ int pgs[PGMAX];
    __shared__ uint64_t etab[32];
    cj_exp_table(etab);   // visible after the "q and pages" barrier
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int per = a.n_kv * a.spl, r = blockIdx.x / per, rem = blockIdx.x % per;
    const int kvh = rem / a.spl, sp = rem % a.spl;
    const int slot = a.rowtab[2 * r];
    int count = a.states[slot].pos + a.rowtab[2 * r + 1] + 1, from = 0;
    if (a.window > 0 && count > a.window) { from = count - a.window; count = a.window; }
    const int pg_base = slot * a.pg_n, rows_kv = a.nrows * a.n_kv;
    const float *qrow = a.q + (int64_t)r * a.q_stride;
    float *part = a.part + (int64_t)r * a.part_stride;
    // q, the page table and the step state load together
    for (int e = 4 * t; e < G * HD; e += 1024) *(float4 *)&qs[0][e] = *(const float4 *)(qrow + (int64_t)kvh * G * HD + e);
    if (t < PGMAX) pgs[t] = t < a.pg_n ? a.pgtab[pg_base + t] : 0;
    const int splits = decode_splits(count, rows_kv, a.workers);
    if (sp < splits) {
        const int chunk = (count + splits - 1) / splits;
        int t0 = sp * chunk, t1 = t0 + chunk;
        if (t1 > count) t1 = count;
        if (t0 > count) t0 = count;
        float m[HW], l[HW], acc0[HW], acc1[HW];
#pragma unroll
        for (int hh = 0; hh < HW; hh++) { m[hh] = -3.0e38f; l[hh] = 0.0f; acc0[hh] = 0.0f; acc1[hh] = 0.0f; }
        // a tile's K and V rows as 16-byte chunks (rows past the split's end
        // repeat its last row); the next tile's are requested before this
        // tile's arithmetic, so a long split streams without a gap. The four
        // chunks' pages are resolved before any K/V load is issued: a page
        // read from global memory (past the staged table) waits for every
        // load in flight, so resolving it between loads would serialize them.
        // (Measured and rejected for this VALU-bound form: widening K and V
        // to f32 once at staging — twice the LDS, half the workgroups a CU,
        // 12.8 ms a C4 step against 11.0; each position's weight from an LDS
        // row instead of its lane — 129 VGPRs, one wave a SIMD fewer, 12.1.)
        u32x4 kr[4], vr[4];   // native vectors: stay in registers across the loop
#define SPLIT_FETCH(TB)                                                                                   \
    do {                                                                                                  \
        const int n_ = t1 - (TB) < TP ? t1 - (TB) : TP;                                                   \
        int64_t base_[4];                                                                                 \
        _Pragma("unroll") for (int i = 0; i < 4; i++) {                                                  \
            const int c = t + 256 * i, j = c & 15;                                                        \
            const int p = (c >> 4) < n_ ? (c >> 4) : n_ - 1;                                              \
            const int pos = from + (TB) + p, pi = pos >> 6;                                               \
            const int page = pi < PGMAX ? pgs[pi] : a.pgtab[pg_base + pi];                                \
            base_[i] = (((int64_t)page * a.n_kv + kvh) * 64 + (pos & 63)) * HD + 8 * j;                   \
        }                                                                                                 \
        _Pragma("unroll") for (int i = 0; i < 4; i++) {                                                  \
            kr[i] = *(const u32x4 *)(a.kc + base_[i]);                                                    \
            vr[i] = *(const u32x4 *)(a.vc + base_[i]);                                                    \
        }                                                                                                 \
    } while (0)
        __syncthreads();   // q and pages visible
        if (t0 < t1) SPLIT_FETCH(t0);
        for (int tb = t0; tb < t1; tb += TP) {
            const int n = t1 - tb < TP ? t1 - tb : TP;
            __syncthreads();   // the previous tile's reads are done
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int c = t + 256 * i;
                *(u32x4 *)&ks[c >> 4][8 * (c & 15)] = kr[i];
                *(u32x4 *)&vs[c >> 4][8 * (c & 15)] = vr[i];
            }
            __syncthreads();
            if (tb + TP < t1) SPLIT_FETCH(tb + TP);
            // scores of position `lane` for this wave's heads, one head at a time
            float s[HW];
#pragma unroll
            for (int hh = 0; hh < HW; hh++) {
                const float *qh = &qs[wave + 4 * hh][0];
                float part[16];
#pragma unroll
                for (int c = 0; c < 16; c++) {
                    const uint4 kk = *(const uint4 *)&ks[lane][8 * c];
                    const float4 qa = *(const float4 *)(qh + 8 * c), qb = *(const float4 *)(qh + 8 * c + 4);
                    const uint32_t kw[4] = {kk.x, kk.y, kk.z, kk.w};
                    const float qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        const int j = 8 * (c & 1) + i;
                        // q·k with k's f16 read in place (the product's bits unchanged)
                        const float pr = (i & 1) ? mul_h16hi(kw[i >> 1], qv[i]) : mul_h16lo(kw[i >> 1], qv[i]);
                        part[j] = c < 2 ? pr : __fadd_rn(part[j], pr);
                    }
                }
#pragma unroll
                for (int w = 1; w < 16; w <<= 1)
#pragma unroll
                    for (int j = 0; j < 16; j += 2 * w) part[j] = __fadd_rn(part[j], part[j + w]);
                s[hh] = __fmul_rn(part[0], a.scale);
            }
            const bool live = lane < n;
#pragma unroll 1
            for (int hh = 0; hh < HW; hh++) {
                // running max before (exc) and after (inc) each position
                const float inc = fmaxf(m[hh], wave_prefix_max(live ? s[hh] : -3.0e38f));
                const float exc = wave_shr1(inc, m[hh]);
                const bool up = live && s[hh] > exc;
                const uint64_t ups = __ballot(up);
                // the rescale's exp only where a position raises the maximum
                // (after the first tiles, rarely: the wave skips it)
                float cf = 1.0f;
                if (ups) cf = up ? cj_expf(exc - s[hh], etab) : 1.0f;
                const float pw = live ? cj_expf(s[hh] - inc, etab) : 0.0f;
                m[hh] = lane_f(inc, n - 1);
                // the lane's V pair of every position of the tile first (all
                // reads in flight at once), then the recurrence in position
                // order with each position's weight (and rescale, where the
                // maximum rose) read from its lane
                uint32_t vv[TP];
#pragma unroll
                for (int p = 0; p < TP; p++) vv[p] = *(const uint32_t *)&vs[p][2 * lane];
                float x0 = acc0[hh], x1 = acc1[hh], ls = l[hh];
#pragma unroll
                for (int p = 0; p < TP; p++) {
                    if (p < n) {
                        const float w = lane_f(pw, p);
                        if ((ups >> p) & 1) {
                            const float c = lane_f(cf, p);
                            x0 = __fmul_rn(x0, c);
                            x1 = __fmul_rn(x1, c);
                            ls = __fmul_rn(ls, c);
                        }
                        ls = __fadd_rn(ls, w);
                        x0 = __fadd_rn(x0, mul_h16lo(vv[p], w));
                        x1 = __fadd_rn(x1, mul_h16hi(vv[p], w));
                    }
                }
                acc0[hh] = x0; acc1[hh] = x1; l[hh] = ls;
            }
        }
#pragma unroll
        for (int hh = 0; hh < HW; hh++) {
            float *pb = part + ((int64_t)(kvh * G + wave + 4 * hh) * ATTN_MAX_SPLITS + sp) * (HD + 2);
            *(float2 *)(pb + 2 * lane) = make_float2(acc0[hh], acc1[hh]);
            if (lane == 0) *(float2 *)(pb + HD) = make_float2(m[hh], l[hh]);
        }
    }
}

#undef SPLIT_FETCH

// Register budget of the four-heads-a-group forms: four waves a SIMD (128
// VGPRs; the f64 steps of the exp had pushed them to 132 and three waves —
// the rows form 132 -> 165 µs a C4 layer). The eight-heads forms hold two
// heads a wave and would spill at that budget.
#define SPLIT_KERNEL(G, ATTR)                                                                                  \
    extern "C" __global__ void __launch_bounds__(256) ATTR cj_attn_split_h128_g##G(cj_attn_args a) {           \
        split_body<G>(a);                                                                                      \
    }                                                                                                          \
    extern "C" __global__ void __launch_bounds__(256) ATTR cj_attn_split_rows_h128_g##G(cj_attn_args a) {      \
        split_rows_body<G>(a);                                                                                 \
    }
SPLIT_KERNEL(4, __attribute__((amdgpu_waves_per_eu(4))))
SPLIT_KERNEL(8, )

// ------------------------------------------------------------ two-pass form

// scores[h][t] = scale · (q_h · K[from+t]) in the reference's sum order:
// partial i (i < 32) adds q[d]·k[d] for d = i, i+32, ... from 0, then the
// xor-butterfly's pairs (16, 8, 4, 2, 1) fold the partials — a fixed tree, so
// one lane can form all of it. Lane = position: a workgroup takes 256
// positions of one query head (grid: position blocks × query heads; the
// group's heads read the same K rows, from L2 after the first), q in LDS
// read as broadcasts. A head a workgroup keeps each lane's chain of
// products short: the scores of a 4096-position span take 8× fewer
// dependent steps than a workgroup per kv head.
template <int HD, bool KF32 = false>
DEV void scores_body(const cj_attn_args &a, int bx, int h) {
    __shared__ __align__(16) float qs[HD];
    int count, from;
    attn_window(a, count, from);
    const int grp = a.n_q / a.n_kv, kvh = h / grp;
    const int t = bx * 256 + threadIdx.x;
    if (bx * 256 >= count) return;      // the whole workgroup idles past count
    // the page entry is requested with q (the K row's address waits on it)
    const int pos = from + min(t, count - 1);
    const int page = a.pgtab[a.pg_base + (pos >> 6)];
    for (int i = threadIdx.x; i < HD; i += 256) qs[i] = a.q[(int64_t)h * HD + i];
    __syncthreads();
    if (t >= count) return;
    const int64_t koff = (((int64_t)page * a.n_kv + kvh) * 64 + (pos & 63)) * HD;
    float k[HD];
    if constexpr (KF32) {
        const float *kr = (const float *)a.kc + koff;
#pragma unroll
        for (int j = 0; j < HD / 4; j++) {
            const float4 v = *(const float4 *)(kr + 4 * j);
            k[4 * j + 0] = v.x; k[4 * j + 1] = v.y; k[4 * j + 2] = v.z; k[4 * j + 3] = v.w;
        }
    } else {
        const uint16_t *kr = a.kc + koff;
#pragma unroll
        for (int j = 0; j < HD / 8; j++) {
            const u32x4 v = *(const u32x4 *)(kr + 8 * j);
            k[8 * j + 0] = h2f(v.x); k[8 * j + 1] = h2f(v.x >> 16);
            k[8 * j + 2] = h2f(v.y); k[8 * j + 3] = h2f(v.y >> 16);
            k[8 * j + 4] = h2f(v.z); k[8 * j + 5] = h2f(v.z >> 16);
            k[8 * j + 6] = h2f(v.w); k[8 * j + 7] = h2f(v.w >> 16);
        }
    }
    float p[32];
#pragma unroll
    for (int i = 0; i < 32; i++) p[i] = 0.0f;
#pragma unroll
    for (int d0 = 0; d0 < HD; d0 += 32) {
#pragma unroll
        for (int i = 0; i < 32; i += 4) {
            const float4 qv = *(const float4 *)(qs + d0 + i);
            p[i] = __fadd_rn(p[i], __fmul_rn(qv.x, k[d0 + i]));
            p[i + 1] = __fadd_rn(p[i + 1], __fmul_rn(qv.y, k[d0 + i + 1]));
            p[i + 2] = __fadd_rn(p[i + 2], __fmul_rn(qv.z, k[d0 + i + 2]));
            p[i + 3] = __fadd_rn(p[i + 3], __fmul_rn(qv.w, k[d0 + i + 3]));
        }
    }
#pragma unroll
    for (int m = 16; m > 0; m >>= 1) {
#pragma unroll
        for (int i = 0; i < m; i++) p[i] = __fadd_rn(p[i], p[i + m]);
    }
    a.part[(int64_t)h * a.splits + t] = __fmul_rn(p[0], a.scale);
}

// The scores of all the query heads of one kv head (at most 16): a lane a
// position whose K row is read once and kept in registers while it is dotted
// with each head's q (staged in LDS) in scores_body's order — the 32 lane
// partials p_i = Σ q[d]·k[d] over d = i, i+32, ... from 0, the fixed
// pairwise tree, ·scale. Grid y is row · n_kv + kv head.
template <int HD>
DEV void scores_grp_body(const cj_attn_args &a, int bx, int kvh) {
    __shared__ __align__(16) float qs[16][HD];
    int count, from;
    attn_window(a, count, from);
    const int grp = a.n_q / a.n_kv;
    const int t = bx * 256 + threadIdx.x;
    if (bx * 256 >= count) return;      // the whole workgroup idles past count
    const int pos = from + min(t, count - 1);
    const int page = a.pgtab[a.pg_base + (pos >> 6)];
    for (int i = threadIdx.x; i < grp * HD; i += 256) qs[i / HD][i % HD] = a.q[(int64_t)kvh * grp * HD + i];
    __syncthreads();
    if (t >= count) return;
    const uint16_t *kr = a.kc + (((int64_t)page * a.n_kv + kvh) * 64 + (pos & 63)) * HD;
    float k[HD];
#pragma unroll
    for (int j = 0; j < HD / 8; j++) {
        const u32x4 v = *(const u32x4 *)(kr + 8 * j);
        k[8 * j + 0] = h2f(v.x); k[8 * j + 1] = h2f(v.x >> 16);
        k[8 * j + 2] = h2f(v.y); k[8 * j + 3] = h2f(v.y >> 16);
        k[8 * j + 4] = h2f(v.z); k[8 * j + 5] = h2f(v.z >> 16);
        k[8 * j + 6] = h2f(v.w); k[8 * j + 7] = h2f(v.w >> 16);
    }
#pragma unroll 1
    for (int hh = 0; hh < grp; hh++) {
        const float *qh = qs[hh];
        float p[32];
#pragma unroll
        for (int i = 0; i < 32; i++) p[i] = 0.0f;
#pragma unroll
        for (int d0 = 0; d0 < HD; d0 += 32) {
#pragma unroll
            for (int i = 0; i < 32; i += 4) {
                const float4 qv = *(const float4 *)(qh + d0 + i);
                p[i] = __fadd_rn(p[i], __fmul_rn(qv.x, k[d0 + i]));
                p[i + 1] = __fadd_rn(p[i + 1], __fmul_rn(qv.y, k[d0 + i + 1]));
                p[i + 2] = __fadd_rn(p[i + 2], __fmul_rn(qv.z, k[d0 + i + 2]));
                p[i + 3] = __fadd_rn(p[i + 3], __fmul_rn(qv.w, k[d0 + i + 3]));
            }
        }
#pragma unroll
        for (int m = 16; m > 0; m >>= 1) {
#pragma unroll
            for (int i = 0; i < m; i++) p[i] = __fadd_rn(p[i], p[i + m]);
        }
        a.part[(int64_t)(kvh * grp + hh) * a.splits + t] = __fmul_rn(p[0], a.scale);
    }
}

#define COMBINE_PAGES 2048   // K/V pages a two-pass span covers (131072 positions)

// A combine producer's item of tile I: positions I·T + 4·tq + k (k < 4),
// dimensions 8·dg..+7 of V and the positions' weights e from `ev` (past
// count: the last position, loaded but staged as +0).
struct CombineItem {
    u32x4 v[4];
    float e[4];
};

// Pages are read from `pgs`, the sequence's page-table entries staged in LDS
// (entry j for page from/64 + j), so no V load waits on a page-table load.
// EXP: `ev` holds the scores and e_t = exp(s_t − m) is formed here (the same
// operation on the same operands as the sum pass, so the same bits): spans
// longer than the LDS weight buffer never write the score row, which the
// head's sibling workgroups read concurrently.
// The item's four consecutive positions lie in at most two pages: the page
// entries of its first and last position (two LDS reads, not four).
struct CombinePages {
    int first, last;
};
template <int T>
DEV CombinePages combine_pages(const int *pgs, int count, int from, int tq, int I) {
    const int t0 = I * T + 4 * tq;
    const int pa = from + min(t0, count - 1), pb = from + min(t0 + 3, count - 1);
    return CombinePages{pgs[(pa >> 6) - (from >> 6)], pgs[(pb >> 6) - (from >> 6)]};
}
template <int HD, int T>
DEV void combine_fetch_v(CombineItem &it, const CombinePages &pg, const cj_attn_args &a, int count, int from, int kvh,
                         int d0, int dg, int tq, int I) {
    const int t0 = I * T + 4 * tq;
    const int seg0 = (from + min(t0, count - 1)) >> 6;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int t = min(t0 + k, count - 1), pos = from + t;
        const int page = (pos >> 6) == seg0 ? pg.first : pg.last;
        it.v[k] = *(const u32x4 *)(a.vc + (((int64_t)page * a.n_kv + kvh) * 64 + (pos & 63)) * HD + d0 + 8 * dg);
    }
}
template <int HD, int T>
DEV void combine_fetch_v(CombineItem &it, const cj_attn_args &a, const int *pgs, int count, int from, int kvh, int d0,
                         int dg, int tq, int I) {
    combine_fetch_v<HD, T>(it, combine_pages<T>(pgs, count, from, tq, I), a, count, from, kvh, d0, dg, tq, I);
}
template <int T, bool EXP>
DEV void combine_fetch_e(CombineItem &it, const float *ev, float m, int count, int tq, int I, const uint64_t *et) {
    const int t0 = I * T + 4 * tq;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int t = min(t0 + k, count - 1);
        it.e[k] = EXP ? cj_expf(ev[t] - m, et) : ev[t];
    }
}
template <int HD, int T, bool EXP>
DEV CombineItem combine_fetch(const cj_attn_args &a, const int *pgs, const float *ev, float m, int count, int from,
                              int kvh, int d0, int dg, int tq, int I, const uint64_t *et) {
    CombineItem it;
    combine_fetch_v<HD, T>(it, a, pgs, count, from, kvh, d0, dg, tq, I);
    combine_fetch_e<T, EXP>(it, ev, m, count, tq, I, et);
    return it;
}

// The item's 32 rounded products e_t·v_t[d] into the tile's rows d (row
// stride S), four positions a 16-byte store.
template <int T, int S>
DEV void combine_store(float *pb, const CombineItem &it, int I, int count, int tq) {
    const int t0 = I * T + 4 * tq;
    const bool ok0 = t0 < count, ok1 = t0 + 1 < count, ok2 = t0 + 2 < count, ok3 = t0 + 3 < count;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int sh = 16 * (j & 1);
        float4 o;
        o.x = ok0 ? __fmul_rn(it.e[0], h2f(it.v[0][j >> 1] >> sh)) : 0.0f;
        o.y = ok1 ? __fmul_rn(it.e[1], h2f(it.v[1][j >> 1] >> sh)) : 0.0f;
        o.z = ok2 ? __fmul_rn(it.e[2], h2f(it.v[2][j >> 1] >> sh)) : 0.0f;
        o.w = ok3 ? __fmul_rn(it.e[3], h2f(it.v[3][j >> 1] >> sh)) : 0.0f;
        *(float4 *)(pb + j * S) = o;
    }
}

// softmax over scores[h][0..count) in place and out[h] = Σ_t p_t·V_t / Σ p:
// one workgroup of 256 per query head and 32 output dimensions, spans of up
// to COMBINE_PAGES pages.
//   max   lanes 0..127 (max is exact, so any grouping gives the same value);
//   sum   lanes 0..127 as the reference's 128: lane l adds e_t for t = l,
//         l+128, ... in order (e_t kept in LDS, or past COMBINE_ES positions
//         written over the score), then the stride-halving tree;
//   p·V   each output dimension's ascending-t sum is one lane's chain. A
//         span of up to 2048 16-byte V chunks (256 positions at HD 64, 128 at
//         128) stages V whole in LDS and each chain lane forms its own
//         products. Longer spans put the chains in the first HD/64 waves (the
//         adders). The other waves (producers) stage
//         the rounded products e_t·v_t[d] through LDS a tile ahead, their V
//         rows loaded CD tiles ahead, so an adder spends 1.25 instructions a
//         position: a 16-byte LDS read of four positions' products, then four
//         adds. Positions past count are staged as +0, which leaves the sum's
//         bits unchanged (the sum starts at +0 and so is never -0); their
//         loads read position count-1.
#define COMBINE_ES 6144   // positions whose weights stay in LDS (one 48-a-lane load round)

template <int HD>
struct CombineDims {
    static constexpr int DH = CJ_COMBINE_DH;        // output dimensions a workgroup (HD/DH workgroups a head)
    static constexpr int NSPLIT = HD / DH;
    static constexpr int A = 1;                     // adder wave (DH lanes)
    static constexpr int P = 256 - 64 * A;          // producer lanes
    static constexpr int DG = DH / 8;               // 8-dimension groups of the workgroup's slice of a V row
    static constexpr int TQ = P / DG;               // 4-position groups a tile: one 4 × 8 item a producer lane
    static constexpr int T = 4 * TQ;                // positions a tile
    static constexpr int S = T + 4;                 // product row stride (floats): 16 lanes' 16-byte reads, distinct banks
    static constexpr int PB = DH * S;               // a product buffer (floats)
};

// p·V of the combine: returns the adder lane's sum (0 on producers). `ev` is
// the weights e_t in LDS or (EXP, spans past COMBINE_ES positions) the scores
// with their maximum m. CD (even) tiles of V are in flight per producer; both
// roles run a whole number of CD-tile rounds.
template <int HD, int CD, bool EXP, class Exps, class Sums>
DEV float combine_pv(const cj_attn_args &a, const int *pgs, const float *ev, float m, float *prod, int count, int from,
                     int kvh, int d0, const uint64_t *et, Exps &&exps, Sums &&sums) {
    using D = CombineDims<HD>;
    constexpr int T = D::T, S = D::S;
    const int l = threadIdx.x, w = l >> 6, ntiles = (count + T - 1) / T;
    const int pl = l - 64 * D::A, tq = pl % D::TQ, dg = pl / D::TQ;
    // both loops run a whole number of CD-tile rounds, so the producer's
    // body has no branch (tiles past the end go to the idle buffer, unread)
    const int nit = (ntiles + CD - 1) / CD * CD;
    float acc = 0.0f;
    // CD tiles of V rows in flight, ring slot = tile mod CD: the first CD
    // tiles' rows are requested between the softmax's exps and its sums,
    // which need none of them
    CombineItem ring[CD];
    exps();
    if (w >= D::A) {
        // every page entry first, then the rows: no load waits on an LDS read
        // issued after an earlier load
        CombinePages pg[CD];
#pragma unroll
        for (int j = 0; j < CD; j++) pg[j] = combine_pages<T>(pgs, count, from, tq, j);
#pragma unroll
        for (int j = 0; j < CD; j++) combine_fetch_v<HD, T>(ring[j], pg[j], a, count, from, kvh, d0, dg, tq, j);
    }
    sums();
    if (w < D::A) {
        lds_barrier();
        const float *pr = prod + min(l, D::DH - 1) * S;
        for (int i = 0; i < nit; i++) {
            const float *pt = pr + (i & 1) * D::PB;
            const int n = i < ntiles ? min(T, count - i * T) : 0;
            if (n == T) {
                // every read of a half tile issued before its first add (the
                // scheduler would otherwise keep two in flight and wait out
                // each one's latency)
                constexpr int HQ = T / 8;
#pragma unroll
                for (int hh = 0; hh < 2; hh++) {
                    float4 p[HQ];
#pragma unroll
                    for (int q = 0; q < HQ; q++) p[q] = *(const float4 *)(pt + 4 * (hh * HQ + q));
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int q = 0; q < HQ; q++) {
                        acc = __fadd_rn(acc, p[q].x);
                        acc = __fadd_rn(acc, p[q].y);
                        acc = __fadd_rn(acc, p[q].z);
                        acc = __fadd_rn(acc, p[q].w);
                    }
                }
            } else {
                for (int q = 0; q < n; q += 4) {
                    const float4 p = *(const float4 *)(pt + q);
                    acc = __fadd_rn(acc, p.x);
                    acc = __fadd_rn(acc, p.y);
                    acc = __fadd_rn(acc, p.z);
                    acc = __fadd_rn(acc, p.w);
                }
            }
            lds_barrier();
        }
    } else {
#pragma unroll
        for (int j = 0; j < CD; j++) combine_fetch_e<T, EXP>(ring[j], ev, m, count, tq, j, et);
        float *pb = prod + 8 * dg * S + 4 * tq;
        combine_store<T, S>(pb, ring[0], 0, count, tq);
        ring[0] = combine_fetch<HD, T, EXP>(a, pgs, ev, m, count, from, kvh, d0, dg, tq, CD, et);
        lds_barrier();
        for (int i0 = 0; i0 < nit; i0 += CD) {
#pragma unroll
            for (int j = 0; j < CD; j++) {
                const int i = i0 + j, r = (j + 1) % CD;
                combine_store<T, S>(pb + ((j + 1) & 1) * D::PB, ring[r], i + 1, count, tq);
                ring[r] = combine_fetch<HD, T, EXP>(a, pgs, ev, m, count, from, kvh, d0, dg, tq, i + 1 + CD, et);
                lds_barrier();
            }
        }
    }
    return acc;
}

template <int HD>
DEV void combine_body(const cj_attn_args &a, int bx) {
    using D = CombineDims<HD>;
    __shared__ float red[4 + 128];
    __shared__ __align__(16) float prod[2 * D::PB];   // also V of a short span: 2048 chunks of 16 bytes
    __shared__ int pgs[COMBINE_PAGES];
    __shared__ __align__(16) float es[COMBINE_ES];
    __shared__ uint64_t etab[32];
    cj_exp_table(etab);   // visible after the max's barrier
    int count, from;
    attn_window(a, count, from);
    // workgroups are dealt to the eight XCDs round-robin by id, so taking
    // the kv head as id mod n_kv keeps the grp·NSPLIT workgroups that read one
    // kv head's V rows on one XCD, whose L2 serves the repeats
    const int grp = a.n_q / a.n_kv, kvh = bx % a.n_kv, r = bx / a.n_kv, l = threadIdx.x;
    const int h = kvh * grp + r / D::NSPLIT, d0 = D::DH * (r % D::NSPLIT);
    const float *sc = a.part + (int64_t)h * a.splits;
    const int npg = ((from + count - 1) >> 6) - (from >> 6) + 1;
    // the page entries and the first round of scores are requested together
    // (one memory round trip). The max and the exps of the span's first
    // COMBINE_ES positions are spread over the four waves: lane l holds the
    // slots k = 2i + l/128 of reference lane l mod 128 (positions
    // (l mod 128) + 128k)
    constexpr int PK = COMBINE_ES / 128, PH = PK / 2;
    const int j128 = l & 127, half = l >> 7;
    const int pg0 = l < npg ? a.pgtab[a.pg_base + (from >> 6) + l] : 0;
    float v[PH];
#pragma unroll
    for (int i = 0; i < PH; i++) v[i] = sc[min(j128 + 128 * (2 * i + half), count - 1)];
    if (l < npg) pgs[l] = pg0;
    for (int j = l + 256; j < npg; j += 256) pgs[j] = a.pgtab[a.pg_base + (from >> 6) + j];
    float mx = -3.0e38f;
#pragma unroll
    for (int i = 0; i < PH; i++) if (j128 + 128 * (2 * i + half) < count && v[i] > mx) mx = v[i];
    if (l < 128) {
        for (int base = COMBINE_ES; base < count; base += COMBINE_ES) {
            float u[PK];
#pragma unroll
            for (int k = 0; k < PK; k++) u[k] = sc[min(base + l + 128 * k, count - 1)];
#pragma unroll
            for (int k = 0; k < PK; k++) if (base + l + 128 * k < count && u[k] > mx) mx = u[k];
        }
    }
    // max is exact, so a wave reduction and then the waves' maxima (no lane
    // holds a NaN here, so fmaxf agrees with the comparison; a tie of -0 and
    // +0 changes no exp(s - m))
    mx = xmax64(mx);
    if ((l & 63) == 0) red[l >> 6] = mx;
    __syncthreads();
    const float m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    // short spans take V whole into LDS: the rows are requested here (their
    // page entries are visible after the barrier above) while the weights
    // form, and each adder lane then runs its chain from LDS
    constexpr int DCH = 8;                                  // 16-byte chunks a thread
    const bool direct = count * (HD / 8) <= 256 * DCH;
    u32x4 vst[DCH];
    if (direct) {
#pragma unroll
        for (int k = 0; k < DCH; k++) {
            const int c = l + 256 * k, j = c % (HD / 8), pos = from + min(c / (HD / 8), count - 1);
            const int page = pgs[(pos >> 6) - (from >> 6)];
            vst[k] = *(const u32x4 *)(a.vc + (((int64_t)page * a.n_kv + kvh) * 64 + (pos & 63)) * HD + 8 * j);
        }
    }
    // e_t of the first COMBINE_ES positions in LDS (past them, formed again
    // from the scores where the sum and p·V need it: the score row is shared
    // by the head's HD/32 workgroups and stays read-only)
    const bool elds = count <= COMBINE_ES;
    auto exps = [&] {
#pragma unroll
        for (int i = 0; i < PH; i++) {
            const int k = 2 * i + half, t = j128 + 128 * k;
            if (128 * k < count) {   // the same for the wave: a slot some lane needs
                const float e = cj_expf(v[i] - m, etab);
                if (t < count) es[t] = e;
            }
        }
    };
    float rs = 0.0f;
    // lane l < 128 adds its positions l, l + 128, ... in order, as the
    // reference's lane l does, then the 128 sums fold
    auto sums = [&] {
        lds_barrier();                 // the exps in LDS; red[0..3] read by every lane above
        float s = 0.0f;
        if (l < 128) {
            // every read issued before the first add (kept two in flight, each
            // pair's latency is waited out in turn)
            float e[PK];
#pragma unroll
            for (int k = 0; k < PK; k++)
                if (128 * k < count) e[k] = es[min(l + 128 * k, COMBINE_ES - 1)];
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int k = 0; k < PK; k++)
                if (128 * k < count) s = l + 128 * k < count ? __fadd_rn(s, e[k]) : s;
            for (int base = COMBINE_ES; base < count; base += COMBINE_ES) {
                float u[PK];
#pragma unroll
                for (int k = 0; k < PK; k++) u[k] = sc[min(base + l + 128 * k, count - 1)];
#pragma unroll
                for (int k = 0; k < PK; k++) {
                    const int t = base + l + 128 * k;
                    if (t < count) {
                        const float e = cj_expf(u[k] - m, etab);
                        s = __fadd_rn(s, e);
                    }
                }
            }
        }
        // the reference's 128-lane stride-halving tree: the 64 stride crosses
        // waves through LDS, the strides 32..1 are wave 0's lanes
        if (l < 128) red[4 + l] = s;
        lds_barrier();
        if (l < 64) {
            const float v2 = fold64_lane0(__fadd_rn(red[4 + l], red[4 + l + 64]));
            if (l == 0) red[2] = v2;
        }
        lds_barrier();
        rs = __fdiv_rn(1.0f, red[2]);
    };
    if (direct) {
        exps();
        sums();
        uint16_t *vs = (uint16_t *)prod;                    // [t][HD] halves
#pragma unroll
        for (int k = 0; k < DCH; k++) {
            const int c = l + 256 * k;
            if (c < count * (HD / 8)) *(u32x4 *)(vs + 8 * c) = vst[k];
        }
        __syncthreads();
        if (l < D::DH) {
            float acc = 0.0f;
            int t = 0;
            for (; t + 4 <= count; t += 4) {
                const float4 e4 = *(const float4 *)(es + t);
                const float v0 = h2f(vs[t * HD + d0 + l]), v1 = h2f(vs[(t + 1) * HD + d0 + l]);
                const float v2 = h2f(vs[(t + 2) * HD + d0 + l]), v3 = h2f(vs[(t + 3) * HD + d0 + l]);
                acc = __fadd_rn(acc, __fmul_rn(e4.x, v0));
                acc = __fadd_rn(acc, __fmul_rn(e4.y, v1));
                acc = __fadd_rn(acc, __fmul_rn(e4.z, v2));
                acc = __fadd_rn(acc, __fmul_rn(e4.w, v3));
            }
            for (; t < count; t++) acc = __fadd_rn(acc, __fmul_rn(es[t], h2f(vs[t * HD + d0 + l])));
            a.out[(int64_t)h * HD + d0 + l] = __fmul_rn(acc, rs);
        }
        return;
    }
    // two tiles of V rows in flight where the weights sit in LDS (a tile is
    // ~3,000 cycles of the adder's chain, so two cover the rows' latency; a
    // deeper ring's first burst from every workgroup at once only delays the
    // softmax), six where the producers form the exps themselves
    const float acc = !elds ? combine_pv<HD, 6, true>(a, pgs, sc, m, prod, count, from, kvh, d0, etab, exps, sums)
                            : combine_pv<HD, 2, false>(a, pgs, es, m, prod, count, from, kvh, d0, etab, exps, sums);
    if (l < D::DH) a.out[(int64_t)h * HD + d0 + l] = __fmul_rn(acc, rs);
}

// The combine over f32 K/V planes (the reference's PagedKvCache mode, where
// the host path keeps f32 K/V): the same operations in the same order as
// combine_body — the max, e_t = exp(s_t − max) with lane l of 128 adding its
// positions t = l, l+128, ... in order and the 128 sums folded by the
// stride-halving tree, then each output dimension's ascending-t sum of the
// rounded products e_t·v_t[d], scaled once by 1/Σ — a workgroup of 256 per
// query head and 32 output dimensions, V staged through LDS 64 positions at
// a time (coalesced 128-byte rows) for the 32 chain lanes. Spans up to
// COMBINE_ES positions (the engine's f32 mode caps its context there).
template <int HD>
DEV void combine_f32_body(const cj_attn_args &a, int bx) {
    constexpr int DH = 32, NSPLIT = HD / DH, TV = 64;
    __shared__ float red[4 + 128];
    __shared__ __align__(16) float es[COMBINE_ES];
    __shared__ __align__(16) float vt[TV][DH];
    __shared__ int pgs[COMBINE_ES / 64];
    __shared__ uint64_t etab[32];
    cj_exp_table(etab);   // visible after the max's barrier
    int count, from;
    attn_window(a, count, from);
    const int h = bx / NSPLIT, d0 = DH * (bx % NSPLIT), l = threadIdx.x;
    const int grp = a.n_q / a.n_kv, kvh = h / grp;
    const float *sc = a.part + (int64_t)h * a.splits;
    const int npg = ((from + count - 1) >> 6) - (from >> 6) + 1;
    for (int j = l; j < npg; j += 256) pgs[j] = a.pgtab[a.pg_base + (from >> 6) + j];
    float mx = -3.0e38f;
    if (l < 128)
        for (int t = l; t < count; t += 128) mx = fmaxf(mx, sc[t]);
    mx = xmax64(mx);
    if ((l & 63) == 0) red[l >> 6] = mx;
    __syncthreads();
    const float m = fmaxf(red[0], red[1]);
    float s = 0.0f;
    if (l < 128)
        for (int t = l; t < count; t += 128) {
            const float e = cj_expf(__fsub_rn(sc[t], m), etab);
            es[t] = e;
            s = __fadd_rn(s, e);
        }
    __syncthreads();                 // red[0..1] read by every lane above
    if (l < 128) red[4 + l] = s;
    __syncthreads();
    if (l < 64) {
        const float v2 = fold64_lane0(__fadd_rn(red[4 + l], red[4 + l + 64]));
        if (l == 0) red[2] = v2;
    }
    __syncthreads();
    const float rs = __fdiv_rn(1.0f, red[2]);
    const float *vp = (const float *)a.vc;
    float acc = 0.0f;
    for (int t0 = 0; t0 < count; t0 += TV) {
        // 64 positions × 32 dimensions: thread l loads 8 of them
#pragma unroll
        for (int k = 0; k < TV * DH / 256; k++) {
            const int c = l + 256 * k, p = c / DH, d = c % DH;
            const int pos = from + min(t0 + p, count - 1);
            const int page = pgs[(pos >> 6) - (from >> 6)];
            vt[p][d] = vp[(((int64_t)page * a.n_kv + kvh) * 64 + (pos & 63)) * HD + d0 + d];
        }
        __syncthreads();
        if (l < DH) {
            const int n = min(TV, count - t0);
            for (int p = 0; p < n; p++) acc = __fadd_rn(acc, __fmul_rn(es[t0 + p], vt[p][l]));
        }
        __syncthreads();
    }
    if (l < DH) a.out[(int64_t)h * HD + d0 + l] = __fmul_rn(acc, rs);
}

// The combine for a group of query heads sharing a kv head: a workgroup of
// 256 per 256/HD query heads (all HD output dimensions of each), so the
// group's V rows are staged once for all its heads. The operations and their
// order are combine_body's:
//   softmax  two heads at a time, lanes 0..127 and 128..255 each the
//            reference's 128: the max (exact in any grouping), then lane l
//            forms e_t = exp(s_t − max) for t = l, l+128, ... in order, adds
//            them in that order and writes e_t over s_t (each score row is
//            this workgroup's alone), the 128 sums folded by the
//            stride-halving tree;
//   p·V      lane (head j, dimension d) runs its ascending-t chain
//            acc + e_t·v_t[d] (the product rounded, then added) over tiles of
//            CGT positions whose weights and V rows are staged in LDS, the
//            next tile's loads in flight during the current tile's chain;
//            out = acc·(1/Σ).
#define CGT(HD) (16384 / (HD))   // positions a tile: 32 KB of V rows

template <int HD>
DEV void combine_grp_body(const cj_attn_args &a, int hq) {
    constexpr int HPW = 256 / HD, T = CGT(HD), VCH = T * HD / 8 / 256;   // 16-byte V chunks a thread a tile
    __shared__ float tree[256];
    __shared__ float gmax[4];
    __shared__ float rsum[HPW];
    __shared__ int pgs[COMBINE_PAGES];
    __shared__ __align__(16) float es[2][HPW][T];
    // V of a tile transposed, [dimension][position], rows VR halves apart
    // (16 bytes past a multiple of 256: 16 lanes' 16-byte reads of 16 rows
    // cover the 64 banks once)
    constexpr int VR = T + 8;
    __shared__ __align__(16) uint16_t vs[2][HD * VR];
    __shared__ uint64_t etab[32];
    cj_exp_table(etab);   // visible after the first max's barrier
    int count, from;
    attn_window(a, count, from);
    const int t = threadIdx.x, l = t & 127, g = t >> 7;
    const int grp = a.n_q / a.n_kv, h0 = hq * HPW, kvh = h0 / grp;
    const int npg = ((from + count - 1) >> 6) - (from >> 6) + 1;
    for (int j = t; j < npg; j += 256) pgs[j] = a.pgtab[a.pg_base + (from >> 6) + j];
    for (int j0 = 0; j0 < HPW; j0 += 2) {
        float *sc = a.part + (int64_t)(h0 + j0 + g) * a.splits;
        // a lane's scores in one round of loads where the span allows
        // (128·PK positions), else in rounds of 8 a lane
        constexpr int PK = 36;
        const bool one = count <= 128 * PK;
        float v[PK];
        float mx = -3.0e38f;
        if (one) {
#pragma unroll
            for (int k = 0; k < PK; k++) v[k] = sc[min(l + 128 * k, count - 1)];
#pragma unroll
            for (int k = 0; k < PK; k++) if (l + 128 * k < count && v[k] > mx) mx = v[k];
        } else {
            for (int b = 0; b < count; b += 128 * 8) {
                float u[8];
#pragma unroll
                for (int k = 0; k < 8; k++) u[k] = sc[min(b + l + 128 * k, count - 1)];
#pragma unroll
                for (int k = 0; k < 8; k++) if (b + l + 128 * k < count && u[k] > mx) mx = u[k];
            }
        }
        // the wave's maximum (no lane holds a NaN here, so fmaxf agrees with the
        // comparison; a tie of -0 and +0 changes no exp(s - m))
        mx = xmax64(mx);
        if ((t & 63) == 0) gmax[t >> 6] = mx;
        __syncthreads();
        const float m = gmax[2 * g + 1] > gmax[2 * g] ? gmax[2 * g + 1] : gmax[2 * g];
        float s = 0.0f;
        if (one) {
            // every slot's exp formed (past count a repeat, unused), then the
            // ordered sum and the stores
#pragma unroll
            for (int k = 0; k < PK; k++) v[k] = cj_expf(v[k] - m, etab);
#pragma unroll
            for (int k = 0; k < PK; k++) {
                const int p = l + 128 * k;
                if (p < count) {
                    sc[p] = v[k];
                    s = __fadd_rn(s, v[k]);
                }
            }
        } else {
            for (int b = 0; b < count; b += 128 * 8) {
                float u[8];
#pragma unroll
                for (int k = 0; k < 8; k++) u[k] = sc[min(b + l + 128 * k, count - 1)];
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const int p = b + l + 128 * k;
                    if (p < count) {
                        const float e = cj_expf(u[k] - m, etab);
                        sc[p] = e;
                        s = __fadd_rn(s, e);
                    }
                }
            }
        }
        tree[t] = s;
        __syncthreads();
        if (l < 64) {
            const float v2 = fold64_lane0(__fadd_rn(tree[128 * g + l], tree[128 * g + l + 64]));
            if (l == 0) rsum[j0 + g] = __fdiv_rn(1.0f, v2);
        }
        __syncthreads();   // the weights written over the scores are visible to the workgroup
    }

    // p·V over tiles: the weights of the HPW heads (a float4 a thread) and the
    // V rows (VCH 16-byte chunks a thread); two tiles' loads in flight in two
    // register sets while the chain runs over a third in LDS
    const int ntiles = (count + T - 1) / T;
    // HPW·T weights a tile, four a thread for the first HPW·T/4 threads (the
    // rest repeat the last head's, unstored); the score rows are only
    // 4-byte aligned, so four word loads
    constexpr int EF = HPW * T / 4;
    struct Tile {
        float4 e;
        u32x4 v[VCH];
    };
    auto load = [&](Tile &R, int i) {
        const int jj = min(t / (T / 4), HPW - 1), o = 4 * (t % (T / 4));
        const float *er0 = a.part + (int64_t)(h0 + jj) * a.splits;
        const int q0 = i * T + o;
        R.e.x = er0[min(q0, a.splits - 1)];
        R.e.y = er0[min(q0 + 1, a.splits - 1)];
        R.e.z = er0[min(q0 + 2, a.splits - 1)];
        R.e.w = er0[min(q0 + 3, a.splits - 1)];
        // thread t: the VCH consecutive positions VCH·(t / (HD/8)) + k of the
        // 8-dimension group t mod (HD/8) (a position past count reads position
        // count − 1); they span at most two pages, whose entries are read once
        const int lastpos = from + count - 1;
        const int p0 = from + i * T + VCH * (t / (HD / 8)), j = t % (HD / 8);
        const int f0 = min(p0, lastpos), f7 = min(p0 + VCH - 1, lastpos);
        const uint16_t *b0 = a.vc + ((int64_t)pgs[(f0 >> 6) - (from >> 6)] * a.n_kv + kvh) * 64 * HD + 8 * j;
        const uint16_t *b1 = a.vc + ((int64_t)pgs[(f7 >> 6) - (from >> 6)] * a.n_kv + kvh) * 64 * HD + 8 * j;
#pragma unroll
        for (int k = 0; k < VCH; k++) {
            const int q = min(p0 + k, lastpos);
            const uint16_t *b = (q >> 6) == (f0 >> 6) ? b0 : b1;
            R.v[k] = *(const u32x4 *)(b + (q & 63) * HD);
        }
    };
    // the thread's 8 positions × 8 dimensions transposed: dimension 8j + i's
    // 8 halves are one 16-byte row segment
    static_assert(VCH == 8, "eight positions a thread");
    auto store = [&](const Tile &R, int buf) {
        const int jj = min(t / (T / 4), HPW - 1), o = 4 * (t % (T / 4));
        if (t < EF) *(float4 *)&es[buf][jj][o] = R.e;
        const int j = t % (HD / 8), p0 = VCH * (t / (HD / 8));
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int w = i >> 1;
            const uint32_t sel = (i & 1) ? 0x07060302u : 0x05040100u;   // the high or the low halves
            u32x4 o4;
            o4.x = __builtin_amdgcn_perm(R.v[1][w], R.v[0][w], sel);
            o4.y = __builtin_amdgcn_perm(R.v[3][w], R.v[2][w], sel);
            o4.z = __builtin_amdgcn_perm(R.v[5][w], R.v[4][w], sel);
            o4.w = __builtin_amdgcn_perm(R.v[7][w], R.v[6][w], sel);
            *(u32x4 *)&vs[buf][(8 * j + i) * VR + p0] = o4;
        }
    };
    const int jj = t / HD, d = t % HD;
    float acc = 0.0f;
    // steps of 8 positions: one 16-byte read of the dimension's V row and two
    // of the head's weights, the next step's three issued before the current
    // step's adds (at most 15 LDS reads may be outstanding); the product
    // e_t·v_t[d] by the mixed multiply with a −0 addend (the rounded
    // product), then the add
    auto chain = [&](int buf, int n) {
        const float *ew = &es[buf][jj][0];
        const uint16_t *vrow = &vs[buf][d * VR];
        const int n8 = n / 8;
        struct Step {
            u32x4 v;
            float4 e0, e1;
        };
        auto rd = [&](Step &S, int st) {
            const int p0 = 8 * min(st, n8 - 1);
            S.v = *(const u32x4 *)(vrow + p0);
            S.e0 = *(const float4 *)(ew + p0);
            S.e1 = *(const float4 *)(ew + p0 + 4);
        };
        auto run = [&](const Step &S) {
            acc = __fadd_rn(acc, mul_h16lo(S.v.x, S.e0.x));
            acc = __fadd_rn(acc, mul_h16hi(S.v.x, S.e0.y));
            acc = __fadd_rn(acc, mul_h16lo(S.v.y, S.e0.z));
            acc = __fadd_rn(acc, mul_h16hi(S.v.y, S.e0.w));
            acc = __fadd_rn(acc, mul_h16lo(S.v.z, S.e1.x));
            acc = __fadd_rn(acc, mul_h16hi(S.v.z, S.e1.y));
            acc = __fadd_rn(acc, mul_h16lo(S.v.w, S.e1.z));
            acc = __fadd_rn(acc, mul_h16hi(S.v.w, S.e1.w));
        };
        if (n8 > 0) {
            Step sa, sb;
            rd(sa, 0);
            for (int st = 0; st < n8; st += 2) {
                rd(sb, st + 1);
                __builtin_amdgcn_sched_barrier(0);
                run(sa);
                if (st + 1 >= n8) break;
                rd(sa, st + 2);
                __builtin_amdgcn_sched_barrier(0);
                run(sb);
            }
        }
        for (int p = 8 * n8; p < n; p++) acc = __fadd_rn(acc, __fmul_rn(ew[p], h2f(vrow[p])));
    };
    // tile i is in LDS buffer i mod 2; at its chain, register set (i+1) mod 2
    // holds tile i+1 in flight and set i mod 2 takes tile i+2's loads (past
    // the last tile: the last again, never stored)
    Tile ra, rb;
    load(ra, 0);
    load(rb, min(1, ntiles - 1));
    store(ra, 0);
    __syncthreads();
    for (int i = 0; i < ntiles; i += 2) {
        load(ra, min(i + 2, ntiles - 1));
        chain(0, min(T, count - i * T));
        if (i + 1 >= ntiles) break;
        store(rb, 1);
        __syncthreads();
        load(rb, min(i + 3, ntiles - 1));
        chain(1, min(T, count - (i + 1) * T));
        if (i + 2 >= ntiles) break;
        store(ra, 0);
        __syncthreads();
    }
    a.out[(int64_t)(h0 + jj) * HD + d] = __fmul_rn(acc, rsum[jj]);
}

// Row r of a many-row launch as the one-row kernels see it: its sequence
// slot's pages and position, its q, output and score rows.
DEV cj_attn_args attn_row_args(const cj_attn_args &a, int r) {
    cj_attn_args b = a;
    const int slot = a.rowtab[2 * r];
    b.state = nullptr;
    b.count = a.states[slot].pos + a.rowtab[2 * r + 1] + 1;
    b.from = 0;
    b.pg_base = slot * a.pg_n;
    b.q = a.q + (int64_t)r * a.q_stride;
    b.out = a.out + (int64_t)r * a.q_stride;
    b.part = a.part + (int64_t)r * a.part_stride;
    return b;
}

// Workgroups are dealt to the eight XCDs round-robin by linear id. The
// one-row scores grid (position chunk x, query head y) is renumbered so that
// the grp query heads reading one chunk of one kv head's K rows share an XCD
// (id mod 8), whose L2 serves the repeats: id = 8·grp·(g/8) + 8·i + g mod 8
// for (chunk, kv head) pair g and member i. A grid whose pair count is not a
// multiple of 8 keeps the plain numbering.
DEV void scores_xcd(const cj_attn_args &a, int &bx, int &h) {
    const int nx = gridDim.x, grp = a.n_q / a.n_kv, ng = nx * a.n_kv;
    if (ng % 8 != 0 || (int)gridDim.y != a.n_q) {
        bx = blockIdx.x;
        h = blockIdx.y;
        return;
    }
    const int id = blockIdx.y * nx + blockIdx.x;
    const int q = id >> 3, i = q % grp, g = (q / grp) * 8 + (id & 7);
    bx = g / a.n_kv;
    h = (g % a.n_kv) * grp + i;
}
extern "C" __global__ void __launch_bounds__(256) cj_attn_scores_h64(cj_attn_args a) {
    int bx, h;
    scores_xcd(a, bx, h);
    scores_body<64>(a, bx, h);
}
extern "C" __global__ void __launch_bounds__(256) cj_attn_scores_h128(cj_attn_args a) {
    int bx, h;
    scores_xcd(a, bx, h);
    scores_body<128>(a, bx, h);
}
extern "C" __global__ void __launch_bounds__(256) cj_attn_combine_h64(cj_attn_args a) { combine_body<64>(a, blockIdx.x); }
extern "C" __global__ void __launch_bounds__(256) cj_attn_combine_h128(cj_attn_args a) { combine_body<128>(a, blockIdx.x); }
// f32 K/V planes: the two-pass pair, one row and many rows
#define TWO_PASS_F32(HD)                                                                                    \
    extern "C" __global__ void __launch_bounds__(256) cj_attn_scores_f32_h##HD(cj_attn_args a) {           \
        int bx, h;                                                                                         \
        scores_xcd(a, bx, h);                                                                              \
        scores_body<HD, true>(a, bx, h);                                                                   \
    }                                                                                                       \
    extern "C" __global__ void __launch_bounds__(256) cj_attn_combine_f32_h##HD(cj_attn_args a) {          \
        combine_f32_body<HD>(a, blockIdx.x);                                                                \
    }                                                                                                       \
    extern "C" __global__ void __launch_bounds__(256) cj_attn_scores_rows_f32_h##HD(cj_attn_args a) {      \
        scores_body<HD, true>(attn_row_args(a, blockIdx.y / a.n_q), blockIdx.x, blockIdx.y % a.n_q);       \
    }                                                                                                       \
    extern "C" __global__ void __launch_bounds__(256) cj_attn_combine_rows_f32_h##HD(cj_attn_args a) {     \
        combine_f32_body<HD>(attn_row_args(a, blockIdx.y), blockIdx.x);                                     \
    }
TWO_PASS_F32(64)
TWO_PASS_F32(128)
// The many-row forms (batched decode, and prefill chunks of the models that
// prefill a decode step a position): grid y is row · n_q + query head for
// the scores, the row for the combine.
#define TWO_PASS_ROWS(HD)                                                                                   \
    extern "C" __global__ void __launch_bounds__(256) cj_attn_scores_rows_h##HD(cj_attn_args a) {          \
        scores_body<HD>(attn_row_args(a, blockIdx.y / a.n_q), blockIdx.x, blockIdx.y % a.n_q);             \
    }                                                                                                       \
    extern "C" __global__ void __launch_bounds__(256) cj_attn_combine_rows_h##HD(cj_attn_args a) {         \
        combine_body<HD>(attn_row_args(a, blockIdx.y), blockIdx.x);                                         \
    }
TWO_PASS_ROWS(64)
TWO_PASS_ROWS(128)
extern "C" __global__ void __launch_bounds__(256) cj_attn_scores_grp_rows_h64(cj_attn_args a) {
    scores_grp_body<64>(attn_row_args(a, blockIdx.y / a.n_kv), blockIdx.x, blockIdx.y % a.n_kv);
}
extern "C" __global__ void __launch_bounds__(256) cj_attn_scores_grp_rows_h128(cj_attn_args a) {
    scores_grp_body<128>(attn_row_args(a, blockIdx.y / a.n_kv), blockIdx.x, blockIdx.y % a.n_kv);
}
// the grouped combine: grid x is the head group (256/HD query heads of one
// kv head), y the row. The m head groups of a kv head read the same V rows:
// x = j·n_kv + kv head puts them on one XCD (id mod 8 is x mod 8 while the
// row's n_q/(256/HD) groups are a multiple of 8) for its L2 to serve.
template <int HD>
DEV int combine_grp_head(const cj_attn_args &a) {
    const int m = (a.n_q / a.n_kv) / (256 / HD), x = blockIdx.x;
    return m > 0 ? (x % a.n_kv) * m + x / a.n_kv : x;
}
extern "C" __global__ void __launch_bounds__(256) cj_attn_combine_grp_rows_h64(cj_attn_args a) {
    combine_grp_body<64>(attn_row_args(a, blockIdx.y), combine_grp_head<64>(a));
}
extern "C" __global__ void __launch_bounds__(256) cj_attn_combine_grp_rows_h128(cj_attn_args a) {
    combine_grp_body<128>(attn_row_args(a, blockIdx.y), combine_grp_head<128>(a));
}

// The two-pass form in one launch for spans of at most FUSED_SPAN(HD)
// positions (sliding windows, small contexts): a workgroup per query head
// stages q, K and V of the span in LDS, then forms the head's scores,
// softmax and p·V with exactly the two kernels' operations — a score per
// lane (the butterfly's fixed tree of 32 strided partials, then ·scale), the
// max, the 128-lane ordered sums and their stride-halving tree, and each
// output dimension's ascending-t sum — so its results are theirs bit for bit.
#define FUSED_SPAN(HD) ((HD) == 64 ? 256 : 128)
template <int HD>
DEV void fused_body(const cj_attn_args &a, int h) {
    constexpr int SPAN = FUSED_SPAN(HD);
    __shared__ __align__(16) uint16_t ks[SPAN * HD], vs[SPAN * HD];
    __shared__ __align__(16) float qs[HD];
    __shared__ float sc[SPAN];
    __shared__ float red[128], mred[2];
    __shared__ float rsv;
    __shared__ uint64_t etab[32];
    cj_exp_table(etab);   // visible after the staging barrier
    int count, from;
    attn_window(a, count, from);
    const int l = threadIdx.x, grp = a.n_q / a.n_kv, kvh = h / grp;
    // q, then K and V rows of the span (chunk c of row t: the page entry of
    // the row, then its 16 bytes), all loads issued together
    for (int i = l; i < HD; i += 256) qs[i] = a.q[(int64_t)h * HD + i];
    constexpr int CH = HD / 8, NC = SPAN * CH / 256;
    u32x4 kr[NC], vr[NC];
#pragma unroll
    for (int k = 0; k < NC; k++) {
        const int c = l + 256 * k, t = min(c / CH, count - 1), pos = from + t;
        const int page = a.pgtab[a.pg_base + (pos >> 6)];
        const int64_t off = (((int64_t)page * a.n_kv + kvh) * 64 + (pos & 63)) * HD + 8 * (c % CH);
        kr[k] = *(const u32x4 *)(a.kc + off);
        vr[k] = *(const u32x4 *)(a.vc + off);
    }
#pragma unroll
    for (int k = 0; k < NC; k++) {
        const int c = l + 256 * k;
        *(u32x4 *)(ks + 8 * c) = kr[k];
        *(u32x4 *)(vs + 8 * c) = vr[k];
    }
    __syncthreads();
    // scores: lane t
    if (l < count) {
        float k[HD];
#pragma unroll
        for (int d = 0; d < HD; d++) k[d] = h2f(ks[l * HD + d]);
        float p[32];
#pragma unroll
        for (int i = 0; i < 32; i++) p[i] = 0.0f;
#pragma unroll
        for (int d0 = 0; d0 < HD; d0 += 32) {
#pragma unroll
            for (int i = 0; i < 32; i++) p[i] = __fadd_rn(p[i], __fmul_rn(qs[d0 + i], k[d0 + i]));
        }
#pragma unroll
        for (int m = 16; m > 0; m >>= 1) {
#pragma unroll
            for (int i = 0; i < m; i++) p[i] = __fadd_rn(p[i], p[i + m]);
        }
        sc[l] = __fmul_rn(p[0], a.scale);
    }
    __syncthreads();
    // softmax over lanes 0..127 (lane j takes t = j, j + 128)
    const int j = l & 127;
    float mx = -3.0e38f;
    if (l < 128) {
        for (int t = j; t < count; t += 128) if (sc[t] > mx) mx = sc[t];
    }
    // the wave's maximum (no lane holds a NaN here, so fmaxf agrees with the
    // comparison; a tie of -0 and +0 changes no exp(s - m))
    mx = xmax64(mx);
    if (l < 128 && (l & 63) == 0) mred[l >> 6] = mx;
    __syncthreads();
    const float m = mred[1] > mred[0] ? mred[1] : mred[0];
    float s = 0.0f;
    if (l < 128) {
        for (int t = j; t < count; t += 128) {
            const float e = cj_expf(sc[t] - m, etab);
            sc[t] = e;
            s = __fadd_rn(s, e);
        }
        red[j] = s;
    }
    __syncthreads();
    if (l < 64) {
        const float v2 = fold64_lane0(__fadd_rn(red[l], red[l + 64]));
        if (l == 0) rsv = __fdiv_rn(1.0f, v2);
    }
    __syncthreads();
    // p·V: output dimension d's ascending-t chain on lane d
    if (l < HD) {
        float acc = 0.0f;
        for (int t = 0; t < count; t++) acc = __fadd_rn(acc, __fmul_rn(sc[t], h2f(vs[t * HD + l])));
        a.out[(int64_t)h * HD + l] = __fmul_rn(acc, rsv);
    }
}

// a query head a workgroup, numbered kv head = id mod n_kv so the heads that
// read one kv head's K and V rows share an XCD's L2
DEV int fused_head(const cj_attn_args &a, int id) { return (id % a.n_kv) * (a.n_q / a.n_kv) + id / a.n_kv; }
extern "C" __global__ void __launch_bounds__(256) cj_attn_fused_h64(cj_attn_args a) {
    fused_body<64>(a, fused_head(a, blockIdx.x));
}
extern "C" __global__ void __launch_bounds__(256) cj_attn_fused_h128(cj_attn_args a) {
    fused_body<128>(a, fused_head(a, blockIdx.x));
}
// many rows: grid (n_q, rows)
extern "C" __global__ void __launch_bounds__(256) cj_attn_fused_rows_h64(cj_attn_args a) {
    fused_body<64>(attn_row_args(a, blockIdx.y), fused_head(a, blockIdx.x));
}
extern "C" __global__ void __launch_bounds__(256) cj_attn_fused_rows_h128(cj_attn_args a) {
    fused_body<128>(attn_row_args(a, blockIdx.y), fused_head(a, blockIdx.x));
}

// Merge split partials into f32 (+ the pack of the result): one workgroup of
// 256 per 256 output values (the reference's attnReducePackQ8Kernel
// contract), the merge in reducePackBlockCpu's order: the global max, then
// four interleaved sub-sums (splits s ≡ 0, 1, 2, 3 mod 4, each ascending) of
// w_s·l_s and of w_s·acc_s[d], w_s = exp(m_s − max), added in sub order;
// out = acc · (1 / l). Thread t owns output e (head h, dim d) and loads its
// 64 accumulators at once; lane s of its wave holds split s's (max, sum) and
// weight, read by every lane in split order — no LDS, no barrier before the
// pack.
extern "C" __global__ void __launch_bounds__(256) cj_attn_merge(cj_merge_args a) {
    __shared__ float bmax[8];
    __shared__ __align__(16) float sw[4][ATTN_MAX_SPLITS], sl[4][ATTN_MAX_SPLITS];
    __shared__ uint64_t etab[32];
    cj_exp_table(etab);
    const int t = threadIdx.x, lane = t & 63;
    const int64_t e = (int64_t)blockIdx.x * 256 + t;
    const int64_t n = (int64_t)a.n_q * a.head_dim;
    const int hd = a.head_dim;
    // the wave's head (hd ≥ 64: a wave's 64 outputs share one head)
    const int64_t ew = min((int64_t)blockIdx.x * 256 + (t & ~63), n - 1);
    const int h = (int)(ew / hd), d = (int)(min(e, n - 1) % hd);
    const float *pb0 = a.part + (int64_t)h * ATTN_MAX_SPLITS * (hd + 2);
    float pv[ATTN_MAX_SPLITS];
#pragma unroll
    for (int s2 = 0; s2 < ATTN_MAX_SPLITS; s2++) pv[s2] = pb0[s2 * (hd + 2) + d];
    const float2 ml = *(const float2 *)(pb0 + lane * (hd + 2) + hd);
    int splits = a.splits;
    if (a.state) {
        int count = a.state->pos + 1;
        if (a.window > 0 && count > a.window) count = a.window;
        splits = decode_splits(count, a.n_kv, a.workers);
    }
    const bool in = lane < splits;
    const float mv = in ? ml.x : -3.0e38f;
    const float gm = group_max<64>(mv);
    const bool on = in && ml.y > 0.0f;
    __syncthreads();   // the exp table
    const float wt = on ? cj_expf(mv - gm, etab) : 0.0f;
    const uint64_t ons = __ballot(on);
    // split weights and sums through the wave's LDS row, back as broadcast
    // 16-byte reads, 16 splits a chunk; selects (not branches): a split that
    // takes no part leaves the sums as they were
    const int wave = t >> 6;
    sw[wave][lane] = wt;
    sl[wave][lane] = ml.y;
    __builtin_amdgcn_wave_barrier();
    float gl[4] = {0.0f, 0.0f, 0.0f, 0.0f}, ac[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s0 = 0; s0 < ATTN_MAX_SPLITS; s0 += 16) {
        float w[16], lv[16];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float4 w4 = *(const float4 *)&sw[wave][s0 + 4 * k];
            const float4 l4 = *(const float4 *)&sl[wave][s0 + 4 * k];
            w[4 * k] = w4.x; w[4 * k + 1] = w4.y; w[4 * k + 2] = w4.z; w[4 * k + 3] = w4.w;
            lv[4 * k] = l4.x; lv[4 * k + 1] = l4.y; lv[4 * k + 2] = l4.z; lv[4 * k + 3] = l4.w;
        }
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const int s2 = s0 + j;
            const bool use = (ons >> s2) & 1;
            const float g2 = __fadd_rn(gl[s2 & 3], __fmul_rn(w[j], lv[j]));
            const float a2 = __fadd_rn(ac[s2 & 3], __fmul_rn(pv[s2], w[j]));
            gl[s2 & 3] = use ? g2 : gl[s2 & 3];
            ac[s2 & 3] = use ? a2 : ac[s2 & 3];
        }
    }
    const float gt = __fadd_rn(__fadd_rn(__fadd_rn(gl[0], gl[1]), gl[2]), gl[3]);
    const float tacc = __fadd_rn(__fadd_rn(__fadd_rn(ac[0], ac[1]), ac[2]), ac[3]);
    const float x = e < n ? __fmul_rn(tacc, __fdiv_rn(1.0f, gt)) : 0.0f;
    if (a.out && e < n) a.out[e] = x;
    if (a.packed) pack256(x, a.per32, a.packed + (int64_t)blockIdx.x * 320, bmax);
}

// The merge with its four sub-sums on four lanes: a workgroup of two waves
// per (query head, 32 output dimensions); lane (j, i) of a wave, j = lane/16,
// forms sub-sum j of dimension i — splits j, j+4, j+8, ... in ascending
// order, the chain cj_attn_merge's sub j runs — and lane (0, i) adds the four
// in sub order and scales by 1/Σ. A lane loads 16 partials and runs a chain
// of 16 where the wave-per-64-dimensions form runs all 64 splits on every
// lane; the splits' weights and sums come from LDS ordered sub-major, so a
// lane's 16 are four 16-byte reads.
extern "C" __global__ void __launch_bounds__(128) cj_attn_merge_q(cj_merge_args a) {
    __shared__ uint64_t etab[32];
    cj_exp_table(etab);
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, hd = a.head_dim, per = hd / 32;
    // id mod n_kv = kv head, as the split kernel numbers its workgroups: the
    // merges of a kv head's query heads read its partials on the same XCD
    const int kv = (int)(blockIdx.x % a.n_kv), rest = (int)(blockIdx.x / a.n_kv);
    const int h = kv * (a.n_q / a.n_kv) + rest / per, j = lane >> 4, i = lane & 15;
    const int d = (rest % per) * 32 + 16 * wave + i;
    const float *pb0 = a.part + (int64_t)h * ATTN_MAX_SPLITS * (hd + 2);
    float pv[16];
#pragma unroll
    for (int k = 0; k < 16; k++) pv[k] = pb0[(4 * k + j) * (hd + 2) + d];
    const float2 ml = *(const float2 *)(pb0 + lane * (hd + 2) + hd);
    int splits = a.splits;
    if (a.state) {
        int count = a.state->pos + 1;
        if (a.window > 0 && count > a.window) count = a.window;
        splits = decode_splits(count, a.n_kv, a.workers);
    }
    const bool in = lane < splits;
    const float mv = in ? ml.x : -3.0e38f;
    const float gm = group_max<64>(mv);
    const bool on = in && ml.y > 0.0f;
    __syncthreads();   // the exp table
    const float wt = on ? cj_expf(mv - gm, etab) : 0.0f;
    const uint64_t mine = __ballot(on) >> j;   // bit 4k: split 4k + j takes part
    __shared__ __align__(16) float sw[2][ATTN_MAX_SPLITS], sl[2][ATTN_MAX_SPLITS];
    const int si = (lane & 3) * 16 + (lane >> 2);   // split s at (s mod 4)·16 + s/4
    sw[wave][si] = wt;
    sl[wave][si] = ml.y;
    __builtin_amdgcn_wave_barrier();
    float g = 0.0f, ac = 0.0f;
#pragma unroll
    for (int k4 = 0; k4 < 4; k4++) {
        const float4 w4 = *(const float4 *)&sw[wave][16 * j + 4 * k4];
        const float4 l4 = *(const float4 *)&sl[wave][16 * j + 4 * k4];
        const float w[4] = {w4.x, w4.y, w4.z, w4.w}, lv[4] = {l4.x, l4.y, l4.z, l4.w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int k = 4 * k4 + q;
            const bool use = (mine >> (4 * k)) & 1;
            const float g2 = __fadd_rn(g, __fmul_rn(w[q], lv[q]));
            const float a2 = __fadd_rn(ac, __fmul_rn(pv[k], w[q]));
            g = use ? g2 : g;
            ac = use ? a2 : ac;
        }
    }
    // lane i's partners i + 16, i + 32, i + 48 (rows 1, 2, 3 of the wave) by
    // row swaps: the second half of a 16-row swap holds rows 1,1,3,3 and of a
    // 32-lane swap rows 2,3,2,3; a 32-lane swap of the former brings row 3
    auto rows123 = [](float v, float &v1, float &v2, float &v3) {
        int a0, a1, b0, b1, c0, c1;
        swap16(__float_as_int(v), a0, a1);
        swap32(__float_as_int(v), b0, b1);
        swap32(a1, c0, c1);
        v1 = __int_as_float(a1);
        v2 = __int_as_float(b1);
        v3 = __int_as_float(c1);
    };
    float g1, g2, g3, a1, a2, a3;
    rows123(g, g1, g2, g3);
    rows123(ac, a1, a2, a3);
    if (j == 0) {
        const float gt = __fadd_rn(__fadd_rn(__fadd_rn(g, g1), g2), g3);
        const float tacc = __fadd_rn(__fadd_rn(__fadd_rn(ac, a1), a2), a3);
        a.out[(int64_t)h * hd + d] = __fmul_rn(tacc, __fdiv_rn(1.0f, gt));
    }
}

// The many-row form: row r's blocks (a row is whole blocks of 256), its
// partials and split count from the row table, its output and pack at the
// row strides.
// The merge of one output of a batch row over its first NS splits (the row
// takes at most NS; the rest hold no part).
template <int NS>
DEV void merge_rows_fold(const cj_merge_args &a, const float *pb0, int lane, int d, int splits, int64_t e, int64_t n,
                         float *out, uint8_t *packed, int64_t blk, float *bmax, float (*sw)[ATTN_MAX_SPLITS],
                         float (*sl)[ATTN_MAX_SPLITS], const uint64_t *et) {
    const int hd = a.head_dim, t = threadIdx.x;
    float pv[NS];
#pragma unroll
    for (int s2 = 0; s2 < NS; s2++) pv[s2] = pb0[s2 * (hd + 2) + d];
    const float2 ml = *(const float2 *)(pb0 + lane * (hd + 2) + hd);
    const bool in = lane < splits;
    const float mv = in ? ml.x : -3.0e38f;
    const float gm = group_max<64>(mv);
    const bool on = in && ml.y > 0.0f;
    const float wt = on ? cj_expf(mv - gm, et) : 0.0f;
    const uint64_t ons = __ballot(on);
    // split weights and sums through the wave's LDS row, back as broadcast
    // 16-byte reads, 16 splits a chunk; selects (not branches): a split that
    // takes no part leaves the sums as they were
    const int wave = t >> 6;
    sw[wave][lane] = wt;
    sl[wave][lane] = ml.y;
    __builtin_amdgcn_wave_barrier();
    float gl[4] = {0.0f, 0.0f, 0.0f, 0.0f}, ac[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s0 = 0; s0 < NS; s0 += 16) {
        float w[16], lv[16];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float4 w4 = *(const float4 *)&sw[wave][s0 + 4 * k];
            const float4 l4 = *(const float4 *)&sl[wave][s0 + 4 * k];
            w[4 * k] = w4.x; w[4 * k + 1] = w4.y; w[4 * k + 2] = w4.z; w[4 * k + 3] = w4.w;
            lv[4 * k] = l4.x; lv[4 * k + 1] = l4.y; lv[4 * k + 2] = l4.z; lv[4 * k + 3] = l4.w;
        }
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const int s2 = s0 + j;
            const bool use = (ons >> s2) & 1;
            const float g2 = __fadd_rn(gl[s2 & 3], __fmul_rn(w[j], lv[j]));
            const float a2 = __fadd_rn(ac[s2 & 3], __fmul_rn(pv[s2], w[j]));
            gl[s2 & 3] = use ? g2 : gl[s2 & 3];
            ac[s2 & 3] = use ? a2 : ac[s2 & 3];
        }
    }
    const float gt = __fadd_rn(__fadd_rn(__fadd_rn(gl[0], gl[1]), gl[2]), gl[3]);
    const float tacc = __fadd_rn(__fadd_rn(__fadd_rn(ac[0], ac[1]), ac[2]), ac[3]);
    const float x = e < n ? __fmul_rn(tacc, __fdiv_rn(1.0f, gt)) : 0.0f;
    if (out && e < n) out[e] = x;
    if (packed) pack256(x, a.per32, packed + blk * 320, bmax);
}

extern "C" __global__ void __launch_bounds__(256) cj_attn_merge_rows(cj_merge_args a) {
    __shared__ float bmax[8];
    __shared__ __align__(16) float sw[4][ATTN_MAX_SPLITS], sl[4][ATTN_MAX_SPLITS];
    __shared__ uint64_t etab[32];
    cj_exp_table(etab);
    const int t = threadIdx.x, lane = t & 63;
    const int64_t n = (int64_t)a.n_q * a.head_dim;
    const int hd = a.head_dim;
    const int64_t per = n / 256, r = blockIdx.x / per, blk = blockIdx.x % per;
    const float *part = a.part + r * a.part_stride;
    float *out = a.out ? a.out + r * a.out_stride : nullptr;
    uint8_t *packed = a.packed ? a.packed + r * a.pack_stride : nullptr;
    int count = a.states[a.rowtab[2 * r]].pos + a.rowtab[2 * r + 1] + 1;
    const int64_t e = blk * 256 + t;
    // the wave's head (hd ≥ 64: a wave's 64 outputs share one head)
    const int64_t ew = min(blk * 256 + (t & ~63), n - 1);
    const int h = (int)(ew / hd), d = (int)(min(e, n - 1) % hd);
    const float *pb0 = part + (int64_t)h * ATTN_MAX_SPLITS * (hd + 2);
    if (a.window > 0 && count > a.window) count = a.window;
    const int splits = decode_splits(count, a.nrows * a.n_kv, a.workers);
    // a batch's rows take few splits (4 at 32 rows of 8 kv heads): read and
    // fold only the first 16 where that covers them
    __syncthreads();   // the exp table
    if (splits <= 16) merge_rows_fold<16>(a, pb0, lane, d, splits, e, n, out, packed, blk, bmax, sw, sl, etab);
    else merge_rows_fold<ATTN_MAX_SPLITS>(a, pb0, lane, d, splits, e, n, out, packed, blk, bmax, sw, sl, etab);
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
        if (hd == 128) {
            // AttnKernel.cpuHeadNorm's order: thread t squares the pair
            // (2t, 2t+1); pairs fold as a tree within each 16 (xor 1, 2, 4),
            // two 16s make a 32 (xor 8), the four 32s add in order
            ss = __fadd_rn(__fmul_rn(x[2 * t], x[2 * t]), __fmul_rn(x[2 * t + 1], x[2 * t + 1]));
#pragma unroll
            for (int m = 1; m <= 8; m <<= 1) ss = __fadd_rn(ss, __shfl_xor(ss, m));
            ss = __fadd_rn(__fadd_rn(__fadd_rn(__shfl(ss, 0), __shfl(ss, 16)), __shfl(ss, 32)), __shfl(ss, 48));
        } else {
            // the generic qkPrepKernel's order: reference lane l (of 128)
            // sums x[l]², x[l+128]², ...; Workgroup.reduce folds each 32-lane
            // wave by the butterfly from the adjacent lane up (1, 2, 4, 8,
            // 16) and adds the four wave sums in order. Lane t holds
            // reference lanes t (a) and t + 64 (b): lanes 0-31 end with waves
            // 0 and 2, lanes 32-63 with waves 1 and 3.
            float a = 0.0f, b = 0.0f;
            for (int i = t; i < hd; i += 128) a = __fadd_rn(a, __fmul_rn(x[i], x[i]));
            for (int i = t + 64; i < hd; i += 128) b = __fadd_rn(b, __fmul_rn(x[i], x[i]));
#pragma unroll
            for (int m = 1; m <= 16; m <<= 1) {
                a = __fadd_rn(a, __shfl_xor(a, m));
                b = __fadd_rn(b, __shfl_xor(b, m));
            }
            ss = __fadd_rn(__fadd_rn(__fadd_rn(__shfl(a, 0), __shfl(a, 32)), __shfl(b, 0)), __shfl(b, 32));
        }
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
            kv_store2(a.kc, a.kv_f32, ki + d, ra, ki + d + half, rb);
        }
    }
    if (!isq) {
        const int64_t vi = kv_at(a.pgtab, a.pg_base, pos, a.n_kv, kh, hd);
        for (int e = t; e < hd; e += 64) {
            const float x = a.v[(int64_t)kh * hd + e];
            if (a.kv_f32) ((float *)a.vc)[vi + e] = x;
            else a.vc[vi + e] = f2h(x);
        }
    }
}

// ------------------------------------------------------------ prefill form

// Prefill attention over rows of one sequence at head size 128 — the CPU
// backend's prefill attend (AttnKernel.attnPrefillCpuGqaKernel,
// model/AttnKernel.cajeta:3916-4004): one pass per (row, query head) over
// its positions [t0, count) in order, an online softmax with q scaled first
// (q·scale rounded, then the dot), the running max from -1e30, a rescale
// only where the maximum rises, out = acc·(1/l).
//
// Sixteen lanes own one (row, head): lane j holds q[16v+j]·scale and the
// accumulators of dims 16v+j (v < 8) and forms the partial
// Σ_v q[16v+j]·k[16v+j] in v order; the 16 partials fold by the fixed
// pairwise tree in four DPP steps within the 16-lane row (quad xor 1, quad
// xor 2, half-row mirror, row mirror: pairs, quads, halves, the whole — fp
// addition commutes, so all 16 lanes end with the tree's bits). A workgroup
// of 4 waves takes RB rows of one kv head, 16·NS (row, head) pairs (NS a
// wave; a wave's four pairs share a row for G ≥ 4); each tile of TK
// positions is staged once for all of them, as f32 in lane order
// ([t][j][v], so a lane's 8 values are two 16-byte reads that all of a
// wave's pairs share). The heaviest row blocks are dispatched first.
template <int CTRL>
DEV float dpp_rowf(float v) { return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false)); }

template <int G>
DEV void prefill_body(const cj_attn_args &a) {
    constexpr int HD = 128, TK = 32, NS = G >= 8 ? G / 4 : 1, RB = 16 * NS / G;
    __shared__ __align__(16) float kl[TK][16][8];
    __shared__ __align__(16) float vl[TK][16][8];
    __shared__ uint64_t etab[32];
    cj_exp_table(etab);   // visible after the first tile's barrier
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, j = lane & 15, grp = lane >> 4;
    const int nblk = (a.nrows + RB - 1) / RB;
    const int kvh = (int)(blockIdx.x % a.n_kv), rb = nblk - 1 - (int)(blockIdx.x / a.n_kv);
    const int slot = a.rowtab[0];
    const int pg_base = slot * a.pg_n, base_pos = a.states[slot].pos;
    // the workgroup's position range: the union of its rows' ranges
    int lo = 0x7fffffff, hi = 0;
    for (int i = 0; i < RB; i++) {
        const int r = rb * RB + i;
        if (r >= a.nrows) break;
        const int count = base_pos + a.rowtab[2 * r + 1] + 1;
        const int t0 = a.window > 0 && count > a.window ? count - a.window : 0;
        lo = min(lo, t0);
        hi = max(hi, count);
    }
    float qv[NS][8], acc[NS][8], m[NS], l[NS];
    int c0[NS], c1[NS], row[NS], head[NS];
#pragma unroll
    for (int s = 0; s < NS; s++) {
        const int p = 16 * s + 4 * wave + grp;
        row[s] = rb * RB + p / G;
        head[s] = kvh * G + p % G;
        const int rr = min(row[s], a.nrows - 1);
        const int count = base_pos + a.rowtab[2 * rr + 1] + 1;
        c0[s] = a.window > 0 && count > a.window ? count - a.window : 0;
        c1[s] = row[s] < a.nrows ? count : c0[s];
        const float *qr = a.q + (int64_t)rr * a.q_stride + (int64_t)head[s] * HD + j;
#pragma unroll
        for (int v = 0; v < 8; v++) {
            qv[s][v] = __fmul_rn(qr[16 * v], a.scale);
            acc[s][v] = 0.0f;
        }
        m[s] = -1.0e30f;
        l[s] = 0.0f;
    }
    for (int tb = lo; tb < hi; tb += TK) {
        const int nt = hi - tb < TK ? hi - tb : TK;
        __syncthreads();   // the previous tile's reads are done
        // stage: chunk c = 8 halves (dims 8m .. 8m+7) of key c/16; dim d goes
        // to lane d & 15, slot d >> 4
        uint4 kr[2], vr[2];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int c = t + 256 * i, kk = c >> 4, mp = c & 15;
            const int pos = tb + (kk < nt ? kk : nt - 1);
            const int page = a.pgtab[pg_base + (pos >> 6)];
            const int64_t off = (((int64_t)page * a.n_kv + kvh) * 64 + (pos & 63)) * HD + 8 * mp;
            kr[i] = *(const uint4 *)(a.kc + off);
            vr[i] = *(const uint4 *)(a.vc + off);
        }
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const int c = t + 256 * i, kk = c >> 4, mp = c & 15;
            const int j0 = (mp & 1) * 8, v0 = mp >> 1;
            const uint32_t kw[4] = {kr[i].x, kr[i].y, kr[i].z, kr[i].w}, vw[4] = {vr[i].x, vr[i].y, vr[i].z, vr[i].w};
#pragma unroll
            for (int e = 0; e < 8; e++) {
                kl[kk][j0 + e][v0] = h2f(kw[e >> 1] >> (16 * (e & 1)));
                vl[kk][j0 + e][v0] = h2f(vw[e >> 1] >> (16 * (e & 1)));
            }
        }
        __syncthreads();
        for (int tt = 0; tt < nt; tt++) {
            const int tp = tb + tt;
            const float4 ka = *(const float4 *)&kl[tt][j][0], kb = *(const float4 *)&kl[tt][j][4];
            const float4 va = *(const float4 *)&vl[tt][j][0], vb = *(const float4 *)&vl[tt][j][4];
            const float kf[8] = {ka.x, ka.y, ka.z, ka.w, kb.x, kb.y, kb.z, kb.w};
            const float vf[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
#pragma unroll
            for (int s = 0; s < NS; s++) {
                if (tp >= c0[s] && tp < c1[s]) {
                    float d = __fmul_rn(qv[s][0], kf[0]);
#pragma unroll
                    for (int v = 1; v < 8; v++) d = __fadd_rn(d, __fmul_rn(qv[s][v], kf[v]));
                    d = __fadd_rn(d, dpp_rowf<0xB1>(d));    // quad xor 1: the pairs
                    d = __fadd_rn(d, dpp_rowf<0x4E>(d));    // quad xor 2: the quads
                    d = __fadd_rn(d, dpp_rowf<0x141>(d));   // half-row mirror: the halves of 8
                    d = __fadd_rn(d, dpp_rowf<0x140>(d));   // row mirror: the 16
                    if (d > m[s]) {
                        const float c = cj_expf(m[s] - d, etab);
#pragma unroll
                        for (int v = 0; v < 8; v++) acc[s][v] = __fmul_rn(acc[s][v], c);
                        l[s] = __fmul_rn(l[s], c);
                        m[s] = d;
                    }
                    const float pw = cj_expf(d - m[s], etab);
                    l[s] = __fadd_rn(l[s], pw);
#pragma unroll
                    for (int v = 0; v < 8; v++) acc[s][v] = __fadd_rn(acc[s][v], __fmul_rn(vf[v], pw));
                }
            }
        }
    }
#pragma unroll
    for (int s = 0; s < NS; s++) {
        if (row[s] >= a.nrows) continue;
        const float inv = __fdiv_rn(1.0f, l[s]);
        float *o = a.out + (int64_t)row[s] * a.q_stride + (int64_t)head[s] * HD + j;
#pragma unroll
        for (int v = 0; v < 8; v++) o[16 * v] = __fmul_rn(acc[s][v], inv);
    }
}

#define PREFILL_KERNEL(G) \
    extern "C" __global__ void __launch_bounds__(256) cj_attn_prefill_h128_g##G(cj_attn_args a) { prefill_body<G>(a); }
PREFILL_KERNEL(1)
PREFILL_KERNEL(2)
PREFILL_KERNEL(4)
PREFILL_KERNEL(8)
