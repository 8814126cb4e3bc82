// rows.hip — the many-row forms of the step's small kernels for gfx950:
// batched decode (one row a sequence, CausalLM.decodeBatchRows,
// model/CausalLM.cajeta:4133-4360) and prefill chunks (one row a position of
// one sequence, forwardRowsBatched, :2873). Row r of a launch is sequence
// slot rowtab[2r] at position states[slot].pos + rowtab[2r+1]; every row
// computes exactly what the one-row kernel computes for it.
#include "common.h"

DEV int row_slot(const cj_rows_args &a, int r) { return a.rowtab[2 * r]; }
DEV int row_pos(const cj_rows_args &a, int r) { return a.states[a.rowtab[2 * r]].pos + a.rowtab[2 * r + 1]; }

// Embedding rows: row r's token from its sequence's history at its position,
// decoded to f32 (grid: width blocks × rows).
extern "C" __global__ void __launch_bounds__(256) cj_rows_embed(cj_rows_args a) {
    const int r = blockIdx.y;
    const int slot = row_slot(a, r), pos = row_pos(a, r);
    const int token = a.tokens[(int64_t)slot * a.hist + pos];
    const uint8_t *row = a.table + (int64_t)token * a.row_bytes;
    float *o = a.out + (int64_t)r * a.out_stride;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < a.n; e += (int64_t)gridDim.x * 256)
        o[e] = decode_file(a.type, row, e);
}

// q|k|v rows (GGUF pair order, the projection's stored output) through the
// one-row epilogue: RoPE of each (2b, 2b+1) pair of q and k at the row's
// position, q out in HF order, k and v appended to the fp16 pages of the
// row's sequence (grid: 512-value blocks of the row × rows, a pair a thread;
// a workgroup a row looped over the row with its stores between the loads).
extern "C" __global__ void __launch_bounds__(256) cj_rows_qkv(cj_rows_args a) {
    const int r = blockIdx.y;
    const int slot = row_slot(a, r), pos = row_pos(a, r);
    const int page = a.pgtab[(int64_t)slot * a.pg_n + (pos >> 6)];
    const int hd = a.head_dim, half = hd >> 1;
    const int64_t qrows = (int64_t)a.n_q * hd, krows = (int64_t)a.n_kv * hd, total = qrows + 2 * krows;
    const float *y = a.in + (int64_t)r * a.in_stride;
    float *qo = a.q_out + (int64_t)r * a.out_stride;
    const int64_t i = 512 * (int64_t)blockIdx.x + 2 * (int64_t)threadIdx.x;
    if (i < total) {
        const float2 vv = *(const float2 *)(y + i);
        const float v = vv.x, vp = vv.y;
        if (i < qrows + krows) {
            const int64_t rr = i < qrows ? i : i - qrows;
            const int h = (int)(rr / hd), bb = (int)(rr % hd) >> 1;
            const float2 cs = *(const float2 *)(a.rope_cs + 2 * ((int64_t)pos * half + bb));
            const float ra = __fsub_rn(__fmul_rn(v, cs.x), __fmul_rn(vp, cs.y));
            const float rb = __fadd_rn(__fmul_rn(v, cs.y), __fmul_rn(vp, cs.x));
            if (i < qrows) {
                qo[(int64_t)h * hd + bb] = ra;
                qo[(int64_t)h * hd + half + bb] = rb;
            } else {
                const int64_t ki = (((int64_t)page * a.n_kv + h) * 64 + (pos & 63)) * hd;
                kv_store2(a.kc, a.kv_f32, ki + bb, ra, ki + half + bb, rb);
            }
        } else {
            const int64_t rr = i - qrows - krows;
            const int h = (int)(rr / hd), d = (int)(rr % hd);
            const int64_t vi = (((int64_t)page * a.n_kv + h) * 64 + (pos & 63)) * hd;
            kv_store2(a.vc, a.kv_f32, vi + d, v, vi + d + 1, vp);
        }
    }
}

// SiLU(gate)·up of interleaved gate/up rows (row 2e gate, 2e+1 up: the fused
// projection's layout), then the q8 pack of each 256-wide block for the down
// projection (grid: groups of four blocks × rows). A wave packs one block,
// four consecutive values a lane (two 16-byte loads of gate/up pairs, one
// 4-byte store of codes): the block and 32-group maxima, the codes, sums and
// scales of pack256, reduced across lanes without LDS. The f32 result is kept
// when `out` is set.
extern "C" __global__ void __launch_bounds__(256) cj_rows_glu(cj_rows_args a) {
    const int r = blockIdx.y, lane = threadIdx.x & 63;
    const int64_t blk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= a.npad / 256) return;   // whole waves past the last block
    const int64_t e0 = blk * 256 + 4 * lane;
    const float *y = a.in + (int64_t)r * a.in_stride;
    float v[4];
    if (e0 + 4 <= a.n && ((uintptr_t)y & 15) == 0) {
        const float4 p0 = *(const float4 *)(y + 2 * e0), p1 = *(const float4 *)(y + 2 * e0 + 4);
        v[0] = glu_value(a.form, e0, a.n, p0.x, p0.y);
        v[1] = glu_value(a.form, e0 + 1, a.n, p0.z, p0.w);
        v[2] = glu_value(a.form, e0 + 2, a.n, p1.x, p1.y);
        v[3] = glu_value(a.form, e0 + 3, a.n, p1.z, p1.w);
    } else {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int64_t e = e0 + k;
            v[k] = 0.0f;
            if (e < a.n) {
                const float2 gu = *(const float2 *)(y + 2 * e);
                v[k] = glu_value(a.form, e, a.n, gu.x, gu.y);
            }
        }
    }
    if (a.out) {
        float *o = a.out + (int64_t)r * a.out_stride;
#pragma unroll
        for (int k = 0; k < 4; k++) if (e0 + k < a.n) o[e0 + k] = v[k];
    }
    float m = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    m = fmaxf(m, __shfl_xor(m, 1));
    m = fmaxf(m, __shfl_xor(m, 2));
    m = fmaxf(m, __shfl_xor(m, 4));    // the 32-group (eight lanes)
    if (!a.per32) {
        m = fmaxf(m, __shfl_xor(m, 8));
        m = fmaxf(m, __shfl_xor(m, 16));
        m = fmaxf(m, __shfl_xor(m, 32));
    }
    const float inv = m > 0.0f ? __fdiv_rn(127.0f, m) : 0.0f;
    uint32_t w = 0u;
    int s = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int q = round_away(__fmul_rn(v[k], inv));
        s += q;
        w |= ((uint32_t)q & 255u) << (8 * k);
    }
    uint8_t *ob = a.packed + (int64_t)r * a.pack_stride + blk * 320;
    *(uint32_t *)(ob + 4 * lane) = w;
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 4);
    if ((lane & 7) == 0) *(int32_t *)(ob + 256 + 4 * (lane >> 3)) = s;
    if (a.per32) {
        if ((lane & 7) == 0) *(float *)(ob + 288 + 4 * (lane >> 3)) = __fdiv_rn(m, 127.0f);
    } else {
        if (lane == 0) *(float *)(ob + 288) = __fdiv_rn(m, 127.0f);
        pack_zero_pad(ob, lane);
    }
}

// First-occurrence argmax partials: chunk c (1024 wide) of row r's logits →
// (value, index) at [r][c] (grid: chunks × rows).
extern "C" __global__ void __launch_bounds__(256) cj_rows_argmax(cj_rows_args a) {
    __shared__ float bv[256];
    __shared__ int bi[256];
    const int t = threadIdx.x, r = blockIdx.y;
    const float *v = a.in + (int64_t)r * a.in_stride;
    const int64_t lo = (int64_t)blockIdx.x * 1024, hi = min(lo + 1024, a.n);
    float best = 0.0f;
    int besti = -1;
    for (int64_t i = lo + t; i < hi; i += 256) {
        const float x = v[i];
        if (besti < 0 || x > best) { best = x; besti = (int)i; }
    }
    bv[t] = best;
    bi[t] = besti;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (t < s && argmax_take(bv[t + s], bi[t + s], bv[t], bi[t])) { bv[t] = bv[t + s]; bi[t] = bi[t + s]; }
        __syncthreads();
    }
    if (t == 0) {
        a.pv[(int64_t)r * a.nchunks + blockIdx.x] = bv[0];
        a.pi[(int64_t)r * a.nchunks + blockIdx.x] = bi[0];
    }
}

// Row r's greedy pick from its partials (the smallest index of the largest
// value), written as preds[pos+1] and, past the prompt, tokens[pos+1] of the
// row's sequence; advances that sequence's position (one workgroup a row,
// one row a sequence).
extern "C" __global__ void __launch_bounds__(256) cj_rows_pick(cj_rows_args a) {
    __shared__ float bv[256];
    __shared__ int bi[256];
    const int t = threadIdx.x, r = blockIdx.x;
    float gb = 0.0f;
    int gi = -1;
    for (int g = t; g < a.nchunks; g += 256) {
        const float x = a.pv[(int64_t)r * a.nchunks + g];
        const int xi = a.pi[(int64_t)r * a.nchunks + g];
        if (argmax_take(x, xi, gb, gi)) { gb = x; gi = xi; }
    }
    bv[t] = gb;
    bi[t] = gi;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (t < s && argmax_take(bv[t + s], bi[t + s], bv[t], bi[t])) { bv[t] = bv[t + s]; bi[t] = bi[t + s]; }
        __syncthreads();
    }
    if (t == 0) {
        const int slot = row_slot(a, r), pos = row_pos(a, r);
        cj_step_state *st = a.states + slot;
        int32_t *hist_t = a.tokens + (int64_t)slot * a.hist, *hist_p = a.preds + (int64_t)slot * a.hist;
        hist_p[pos + 1] = bi[0];
        if (pos + 1 >= st->fixed_until) hist_t[pos + 1] = bi[0];
        st->pos = pos + 1;
    }
}
