// prim.hip — the small decode primitives for gfx950: activation packs
// (with and without the RMSNorm), SwiGLU (+ pack), residual add, embedding
// row decode, first-occurrence argmax, block dequant and the load-time
// re-layout of weight rows.
#include "common.h"

// ---------------------------------------------------------------- packs

// One workgroup per row: optional RMSNorm, optional f32 out, then the pack
// (Prim.rmsnormPackDevice / QuantKernel.q8kPackRowsLaunchNoSync contracts).
extern "C" __global__ void __launch_bounds__(256) cj_pack(cj_pack_args a) {
    __shared__ float red[256];
    extern __shared__ __align__(16) uint8_t sx[];
    const int64_t row = blockIdx.x;
    const float *x = a.x + row * a.n;
    const int nblk = (int)(a.npad / 256);
    const float scale = a.do_norm ? stage_norm_scale(x, a.n, a.eps, red) : 1.0f;
    float *xo = a.xout ? a.xout + row * a.n : nullptr;
    if (!a.out) {
        for (int64_t e = threadIdx.x; e < a.n; e += 256) xo[e] = stage_value(x, a.n, e, a.do_norm, scale, a.w, a.form);
        return;
    }
    stage_pack(x, a.n, nblk, a.do_norm, scale, a.w, a.form, a.per32, sx, xo);
    uint8_t *o = a.out + row * (int64_t)nblk * 320;
    for (int i = threadIdx.x; i < nblk * 20; i += 256) ((uint4 *)o)[i] = ((const uint4 *)sx)[i];
}

// RMSNorm + pack of one row, one workgroup per 256-wide block. Every
// workgroup forms the row's sum of squares itself in the reference order
// (thread t: x[t + 256k], k ascending, ragged past the width, then the
// 128..1 tree) from loads it issues at once, then packs its own block: no
// workgroup waits on another.
DEV void norm_pack_block(const cj_pack_args &a, const float *x) {
    __shared__ float red[256];
    __shared__ float bmax[8];
    const int t = threadIdx.x, lane = t & 63;
    const int64_t blk = blockIdx.x, e = blk * 256 + t;
    const float xe = e < a.n ? x[e] : 0.0f;
    const float we = e < a.n ? a.w[e] : 0.0f;
    const float scale = stage_norm_scale(x, a.n, a.eps, red);
    const float wi = a.form == 1 ? __fadd_rn(1.0f, we) : we;
    const float v = e < a.n ? __fmul_rn(__fmul_rn(xe, scale), wi) : 0.0f;
    if (a.xout && e < a.n) a.xout[e] = v;
    if (!a.out) return;
    const float av = fabsf(v);
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
    const int q = round_away(__fmul_rn(v, inv));
    uint8_t *ob = a.out + blk * 320;
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
extern "C" __global__ void __launch_bounds__(256) cj_norm_pack(cj_pack_args a) { norm_pack_block(a, a.x); }

// The same for many rows: workgroup (256-block, row), row r of x, out and
// xout a.n floats / npad/256 blocks / a.n floats apart. (A workgroup a row
// puts a batch of 32 rows on 32 CUs.)
extern "C" __global__ void __launch_bounds__(256) cj_norm_pack_rows(cj_pack_args a) {
    const int64_t row = blockIdx.y;
    cj_pack_args r = a;
    r.x = a.x + row * a.n;
    r.out = a.out ? a.out + row * (a.npad / 256) * 320 : nullptr;
    r.xout = a.xout ? a.xout + row * a.n : nullptr;
    norm_pack_block(r, r.x);
}

// The MoE combine (MoeFfn.forwardRow, model/MoeFfn.cajeta:1896-1901: the
// selected experts' rows weighted and summed in k order, then onto the
// residual) and the RMSNorm + pack that follows it (the next layer's
// attention norm or the final norm) in one launch, one workgroup per 256
// outputs as cj_norm_pack: every workgroup forms the whole combined row in
// LDS (each value as cj_moe_combine forms it), writes its own block of it
// to hs_out — a buffer other than hs_in, so no workgroup reads a value
// another has already replaced — and norms and packs its block from the LDS
// row exactly as cj_norm_pack does from global memory. Dynamic LDS: n floats.
// Thread t takes the 4-value groups t, t+256, t+512, t+768 (n ≤ 4096, n a
// multiple of 4, up to 8 experts a row: the host checks), every load of
// the row issued before the first sum and none under a branch of its own
// (NU, 4 or 8, bounds the experts read; past n_used the last expert's row
// is read again and never added).
template <int NU>
DEV void combine_norm_body(const cj_combine_norm_args &a, float *xs) {
    const int t = threadIdx.x, nu = a.n_used;
    const int64_t n4 = a.n / 4;
    float wk[NU];
#pragma unroll
    for (int k = 0; k < NU; k++) wk[k] = a.w[min(k, nu - 1)];
    float4 hv[4], yv[4][NU];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int64_t g = min((int64_t)t + 256 * j, n4 - 1);
        hv[j] = ((const float4 *)a.hs_in)[g];
#pragma unroll
        for (int k = 0; k < NU; k++) yv[j][k] = ((const float4 *)(a.y + min(k, nu - 1) * a.n))[g];
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int64_t g = (int64_t)t + 256 * j;
        if (g >= n4) continue;
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int k = 0; k < NU; k++) {
            const bool on = k < nu;
            acc.x = on ? __fadd_rn(acc.x, __fmul_rn(wk[k], yv[j][k].x)) : acc.x;
            acc.y = on ? __fadd_rn(acc.y, __fmul_rn(wk[k], yv[j][k].y)) : acc.y;
            acc.z = on ? __fadd_rn(acc.z, __fmul_rn(wk[k], yv[j][k].z)) : acc.z;
            acc.w = on ? __fadd_rn(acc.w, __fmul_rn(wk[k], yv[j][k].w)) : acc.w;
        }
        const float4 h = make_float4(__fadd_rn(hv[j].x, acc.x), __fadd_rn(hv[j].y, acc.y),
                                     __fadd_rn(hv[j].z, acc.z), __fadd_rn(hv[j].w, acc.w));
        ((float4 *)xs)[g] = h;
        if (((4 * g) >> 8) == (int64_t)blockIdx.x) ((float4 *)a.hs_out)[g] = h;
    }
}

extern "C" __global__ void __launch_bounds__(256) cj_moe_combine_norm(cj_combine_norm_args a) {
    extern __shared__ __align__(16) float xs[];
    if (a.n_used <= 4) combine_norm_body<4>(a, xs);
    else combine_norm_body<8>(a, xs);
    __syncthreads();
    norm_pack_block(a.p, xs);
}

// Device copy of n16 16-byte words (grid-stride, one uint4 a thread a step).
extern "C" __global__ void __launch_bounds__(256) cj_copy(cj_copy_args a) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < a.n16; i += stride)
        ((uint4 *)a.dst)[i] = ((const uint4 *)a.src)[i];
}

// ------------------------------------------------------------------ glu

// One workgroup per 256-wide block: out = act(g)·u, then (optionally) that
// block's pack — the block is local, so no other workgroup is waited on.
extern "C" __global__ void __launch_bounds__(256) cj_glu(cj_glu_args a) {
    __shared__ float bmax[8];
    const int t = threadIdx.x, lane = t & 63;
    const int64_t e = (int64_t)blockIdx.x * 256 + t;
    float v = 0.0f;
    if (e < a.n) {
        v = glu_value(a.form, e, a.n, a.g[e], a.u[e]);
        a.out[e] = v;
    }
    if (!a.packed) return;
    float am;
    const float av = fabsf(v);
    if (a.per32) {
        float m = group_max<32>(av);
        if ((lane & 31) == 0) bmax[t >> 5] = m;
        __syncthreads();
        am = bmax[t >> 5];
    } else {
        float m = group_max<64>(av);
        if (lane == 0) bmax[t >> 6] = m;
        __syncthreads();
        am = fmaxf(fmaxf(bmax[0], bmax[1]), fmaxf(bmax[2], bmax[3]));
    }
    const float inv = am > 0.0f ? __fdiv_rn(127.0f, am) : 0.0f;
    const int q = round_away(__fmul_rn(v, inv));
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

extern "C" __global__ void __launch_bounds__(256) cj_add(cj_add_args a) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < a.n) a.a[i] = __fadd_rn(a.a[i], a.b[i]);
}

// --------------------------------------------------------- block decode


// Element e of a FILE-layout row (GGUF blocks), the reference block bodies
// (Quant.q80Block / q40Block / q4kBlock / q6kBlock / mxfp4Block).
DEV float decode_file(int type, const uint8_t *row, int64_t e) {
    switch (type) {
    case CJ_F32: return ((const float *)row)[e];
    case CJ_F16: return h2f(((const uint16_t *)row)[e]);
    case CJ_Q8_0: {
        const uint8_t *b = row + (e >> 5) * 34;
        return __fmul_rn(h2f(*(const uint16_t *)b), (float)(int8_t)b[2 + (e & 31)]);
    }
    case CJ_Q4_0: {
        const uint8_t *b = row + (e >> 5) * 18;
        const int j = e & 31;
        const int q = b[2 + (j & 15)];
        const int v = j < 16 ? (q & 15) - 8 : (q >> 4) - 8;
        return __fmul_rn(h2f(*(const uint16_t *)b), (float)v);
    }
    case CJ_MXFP4: {
        const uint8_t *b = row + (e >> 5) * 17;
        const int j = e & 31;
        const int byv = b[1 + (j & 15)];
        return __fmul_rn(mxfp4_val(j < 16 ? (byv & 15) : (byv >> 4)), mxfp4_scale(b[0]));
    }
    case CJ_Q4_K: {
        const uint8_t *b = row + (e >> 8) * 144;
        const int el = e & 255, g = el / 64, r = el % 64, s = r / 32, l = r % 32, sb = el / 32;
        const int q = (b[16 + 32 * g + l] >> (4 * s)) & 15;
        const uint8_t *sc = b + 4;
        int scv, mnv;
        if (sb < 4) { scv = sc[sb] & 63; mnv = sc[sb + 4] & 63; }
        else { scv = (sc[sb + 4] & 15) | ((sc[sb - 4] >> 2) & 48); mnv = (sc[sb + 4] >> 4) | ((sc[sb] >> 2) & 48); }
        const float d = h2f(*(const uint16_t *)b), dmin = h2f(*(const uint16_t *)(b + 2));
        return __fsub_rn(__fmul_rn(__fmul_rn(d, (float)scv), (float)q), __fmul_rn(dmin, (float)mnv));
    }
    case CJ_Q6_K: {
        const uint8_t *b = row + (e >> 8) * 210;
        const int el = e & 255, g = el / 128, r = el % 128, sl = r / 64, l64 = r % 64, sh = r / 32, l32 = r % 32;
        const int ql = (b[64 * g + l64] >> (4 * sl)) & 15;
        const int qh = (b[128 + 32 * g + l32] >> (2 * sh)) & 3;
        const int q = (ql | (qh << 4)) - 32;
        return __fmul_rn(__fmul_rn(h2f(*(const uint16_t *)(b + 208)), (float)(int8_t)b[192 + el / 16]), (float)q);
    }
    }
    return 0.0f;
}

// Element e of a PREPARED row (the gemv layouts), for the layout's own check.
DEV float decode_prepared(int type, const uint8_t *row, int64_t cols, int64_t e) {
    const int64_t nb = cols / 256, nb32 = cols / 32;
    switch (type) {
    case CJ_Q8_0: {
        const int64_t b = e >> 5;
        return __fmul_rn(h2f(*(const uint16_t *)(row + nb32 * 32 + 2 * b)), (float)(int8_t)row[b * 32 + (e & 31)]);
    }
    case CJ_Q4_0: {
        const int64_t b = e >> 5;
        const int j = e & 31;
        const int q = row[b * 16 + (j & 15)];
        const int v = j < 16 ? (q & 15) - 8 : (q >> 4) - 8;
        return __fmul_rn(h2f(*(const uint16_t *)(row + nb32 * 16 + 2 * b)), (float)v);
    }
    case CJ_MXFP4: {
        const int64_t b = e >> 5;
        const int j = e & 31;
        const int byv = row[b * 16 + (j & 15)];
        return __fmul_rn(mxfp4_val(j < 16 ? (byv & 15) : (byv >> 4)), mxfp4_scale(row[nb32 * 16 + b]));
    }
    case CJ_Q4_K: {
        // qs byte k of block b at ((k / 16)·nb + b)·16 + k % 16; the header at 128·nb + 16·b
        const int64_t b = e >> 8;
        const int el = e & 255, g = el / 64, r = el % 64, s = r / 32, l = r % 32, sb = el / 32;
        const int k = 32 * g + l;
        const int q = (row[((int64_t)(k >> 4) * nb + b) * 16 + (k & 15)] >> (4 * s)) & 15;
        const uint8_t *hb = row + nb * 128 + b * 16;
        const uint8_t *sc = hb + 4;
        int scv, mnv;
        if (sb < 4) { scv = sc[sb] & 63; mnv = sc[sb + 4] & 63; }
        else { scv = (sc[sb + 4] & 15) | ((sc[sb - 4] >> 2) & 48); mnv = (sc[sb + 4] >> 4) | ((sc[sb] >> 2) & 48); }
        const float d = h2f(*(const uint16_t *)hb), dmin = h2f(*(const uint16_t *)(hb + 2));
        return __fsub_rn(__fmul_rn(__fmul_rn(d, (float)scv), (float)q), __fmul_rn(dmin, (float)mnv));
    }
    case CJ_Q6_K: {
        const int64_t b = e >> 8;
        const int el = e & 255, g = el / 128, r = el % 128, sl = r / 64, l64 = r % 64, sh = r / 32, l32 = r % 32;
        const int ql = (row[b * 128 + 64 * g + l64] >> (4 * sl)) & 15;
        const int qh = (row[nb * 128 + b * 64 + 32 * g + l32] >> (2 * sh)) & 3;
        const int q = (ql | (qh << 4)) - 32;
        const float d = h2f(*(const uint16_t *)(row + nb * 208 + 2 * b));
        return __fmul_rn(__fmul_rn(d, (float)(int8_t)row[nb * 192 + b * 16 + el / 16]), (float)q);
    }
    default: return decode_file(type, row, e);
    }
}

// Dequantize rows (Quant.dequantize): grid-stride over elements, from the
// file layout or the prepared layout.
extern "C" __global__ void __launch_bounds__(256) cj_dequant(cj_dequant_args a) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < a.elems; i += (int64_t)gridDim.x * 256) {
        const int64_t r = i / a.cols, c = i % a.cols;
        const uint8_t *row = a.raw + r * a.row_bytes;
        a.out[i] = a.prepared ? decode_prepared(a.type, row, a.cols, c) : decode_file(a.type, row, c);
    }
}

// Load-time re-layout of FILE rows into the prepared gemv layout: one thread
// per block. `src` rows are the GGUF bytes, `dst` rows the prepared ones.

extern "C" __global__ void __launch_bounds__(256) cj_prepare(cj_prepare_args a) {
    const int64_t bpr = (a.type == CJ_Q6_K || a.type == CJ_Q4_K) ? a.cols / 256 : a.cols / 32;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= a.rows * bpr) return;
    const int64_t r = i / bpr, b = i % bpr;
    const uint8_t *s = a.src + r * a.src_row_bytes;
    uint8_t *d = a.dst + r * a.dst_row_bytes;
    switch (a.type) {
    case CJ_Q4_K: {
        // piece c of the qs to ((c·bpr) + b)·16, the 16-byte header to 128·bpr + 16·b
        const uint8_t *blk = s + b * 144;
        for (int c = 0; c < 8; c++)
            for (int k = 0; k < 16; k++) d[(c * bpr + b) * 16 + k] = blk[16 + 16 * c + k];
        for (int k = 0; k < 16; k++) d[bpr * 128 + b * 16 + k] = blk[k];
    } break;
    case CJ_Q6_K: {
        const uint8_t *blk = s + b * 210;
        for (int k = 0; k < 128; k++) d[b * 128 + k] = blk[k];
        for (int k = 0; k < 64; k++) d[bpr * 128 + b * 64 + k] = blk[128 + k];
        for (int k = 0; k < 16; k++) d[bpr * 192 + b * 16 + k] = blk[192 + k];
        d[bpr * 208 + 2 * b] = blk[208];
        d[bpr * 208 + 2 * b + 1] = blk[209];
    } break;
    case CJ_Q8_0: {
        const uint8_t *blk = s + b * 34;
        for (int k = 0; k < 32; k++) d[b * 32 + k] = blk[2 + k];
        d[bpr * 32 + 2 * b] = blk[0];
        d[bpr * 32 + 2 * b + 1] = blk[1];
    } break;
    case CJ_Q4_0: {
        const uint8_t *blk = s + b * 18;
        for (int k = 0; k < 16; k++) d[b * 16 + k] = blk[2 + k];
        d[bpr * 16 + 2 * b] = blk[0];
        d[bpr * 16 + 2 * b + 1] = blk[1];
    } break;
    case CJ_MXFP4: {
        const uint8_t *blk = s + b * 17;
        for (int k = 0; k < 16; k++) d[b * 16 + k] = blk[1 + k];
        d[bpr * 16 + b] = blk[0];
    } break;
    }
}

// ------------------------------------------------------------ embedding

// The token's row of the table decoded to f32 (EmbedKernel.embedRow*):
// the token comes from the device token history at the step position.
extern "C" __global__ void __launch_bounds__(256) cj_embed(cj_embed_args a) {
    const int token = a.tokens ? a.tokens[step_pos(a.state, a.token)] : a.token;
    if (a.vocab > 0 && (token < 0 || token >= a.vocab)) {
        // an id read from device memory that names no row: no read past the table
        for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < a.hidden; e += (int64_t)gridDim.x * 256) a.out[e] = 0.0f;
        if (a.status && blockIdx.x == 0 && threadIdx.x == 0) a.status[0] = 1;
        return;
    }
    const uint8_t *row = a.table + (int64_t)token * a.row_bytes;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < a.hidden; e += (int64_t)gridDim.x * 256)
        a.out[e] = decode_file(a.type, row, e);
}

// --------------------------------------------------------------- argmax

// QuantKernel.argmaxRowKernel's contract: the smallest index of the largest
// value; 1024 elements a workgroup, the last workgroup reduces the partials.
// The step's greedy pick: first-occurrence argmax over per-workgroup
// (value, index) partials (HostOps.argmaxRow's order), written as
// preds[pos+1] and, past the prompt, tokens[pos+1]; advances the position.
extern "C" __global__ void __launch_bounds__(256) cj_argmax_pick(cj_pick_args a) {
    __shared__ float bv[256];
    __shared__ int bi[256];
    const int t = threadIdx.x;
    float gb = 0.0f;
    int gi = -1;
    for (int g = t; g < a.n; g += 256) {
        const float x = a.pv[g];
        const int xi = a.pi[g];
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
        const int pos = a.state ? a.state->pos : a.pos;
        if (a.preds) a.preds[pos + 1] = bi[0];
        if (a.tokens && (!a.state || pos + 1 >= a.state->fixed_until)) a.tokens[pos + 1] = bi[0];
        if (a.host_tok) __hip_atomic_store(a.host_tok + pos + 1, bi[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        if (a.state) a.state->pos = pos + 1;
    }
}

extern "C" __global__ void __launch_bounds__(256) cj_argmax(cj_argmax_args a) {
    __shared__ float bv[256];
    __shared__ int bi[256];
    __shared__ int ticket;
    const int t = threadIdx.x;
    const int64_t end0 = ((int64_t)blockIdx.x + 1) * 1024;
    const int64_t end = end0 < a.n ? end0 : a.n;
    float best = 0.0f; int besti = -1;
    for (int64_t i = (int64_t)blockIdx.x * 1024 + t; i < end; i += 256) {
        const float x = a.v[i];
        if (besti < 0 || x > best) { best = x; besti = (int)i; }
    }
    bv[t] = best; bi[t] = besti;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (t < s) {
            float ov = bv[t + s]; int oi = bi[t + s]; float mv = bv[t]; int mi = bi[t];
            if (mi < 0 || (oi >= 0 && (ov > mv || (ov == mv && oi < mi)))) { bv[t] = ov; bi[t] = oi; }
        }
        __syncthreads();
    }
    if (t == 0) {
        a.pv[blockIdx.x] = bv[0];
        a.pi[blockIdx.x] = bi[0];
        __threadfence();
        ticket = atomicAdd(a.counter, 1);
    }
    __syncthreads();
    if (ticket != (int)gridDim.x - 1) return;
    __threadfence();
    float gb = 0.0f; int gi = -1;
    for (int g = t; g < (int)gridDim.x; g += 256) {
        const float x = a.pv[g]; const int xi = a.pi[g];
        if (xi >= 0 && (gi < 0 || x > gb || (x == gb && xi < gi))) { gb = x; gi = xi; }
    }
    bv[t] = gb; bi[t] = gi;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (t < s) {
            float ov = bv[t + s]; int oi = bi[t + s]; float mv = bv[t]; int mi = bi[t];
            if (mi < 0 || (oi >= 0 && (ov > mv || (ov == mv && oi < mi)))) { bv[t] = ov; bi[t] = oi; }
        }
        __syncthreads();
    }
    if (t == 0) { a.counter[0] = 0; a.tok[a.row] = bi[0]; }
}

// ------------------------------------------------------------------ misc

// Word fill with zero: the graph-safe clear (no memset node in a graph).
typedef struct { uint32_t *p; int64_t words; } cj_zero_args;
extern "C" __global__ void __launch_bounds__(256) cj_zero(cj_zero_args a) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < a.words; i += (int64_t)gridDim.x * 256) a.p[i] = 0u;
}

// MoeFfn.routeFromLogits per row (route_row, common.h): a workgroup of one
// wave a row.
extern "C" __global__ void __launch_bounds__(64) cj_moe_route(cj_route_args a) {
    __shared__ RouteLds rl;
    const int row = blockIdx.x, t = threadIdx.x;
    route_row(a.logits + (int64_t)row * a.n_experts, a.n_experts, a.n_used, a.norm_topk, a.w_scale, a.status, rl);
    if (t < a.n_used) {
        a.sel[row * a.n_used + t] = rl.sel[t];
        a.w[row * a.n_used + t] = rl.w[t];
    }
}

// routerTopKKernel (io/QuantKernel.cajeta:39850-39960): the router mat-vec
// and its top-k in one launch, for models whose router takes the device
// route. Workgroup e forms logit e: thread l adds the rounded products
// w[e][j]·x[j] for j = l, l+256, ... in order, and the 256 partials fold
// 128, 64, ..., 1 (the reference's recorded e128h2048k8 logits fix that
// order). It publishes the logit (device-scope release) and takes a ticket
// on `counter`; the workgroup taking the last one selects in 32 lanes of its
// first wave, the reference's wave width: lane l's experts l, l+32, ...; the
// maximum; each lane's sum of exp(logit − max) in expert order, the 32 sums
// by the butterfly (lane distance 16, 8, 4, 2, 1 — Wave.reduceSumF32's
// order, fixed by the recorded two-pass scores); `used` picks, each the
// largest probability below the previous pick (an equal probability: the
// next index up), w = p/sum; the renormalisation by Σw in pick order clamped
// at 2^-14, then ×w_scale unless it is 0 or 1; the counter back to zero.
extern "C" __global__ void __launch_bounds__(256) cj_router_topk(cj_router_topk_args a) {
    __shared__ float red[256];
    __shared__ int last;
    const int t = threadIdx.x, e = blockIdx.x;
    float acc = 0.0f;
    if (e < a.experts)
        for (int j = t; j < a.cols; j += 256) acc = __fadd_rn(acc, __fmul_rn(a.w_router[(int64_t)e * a.cols + j], a.x[j]));
    red[t] = acc;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if (t < s) red[t] = __fadd_rn(red[t], red[t + s]);
        __syncthreads();
    }
    if (t == 0) {
        if (e < a.experts) a.logits[e] = red[0];
        __threadfence();
        last = atomicAdd(a.counter, 1) == (int)gridDim.x - 1;
    }
    __syncthreads();
    if (!last || t >= 32) return;
    __threadfence();
    const int ne = a.experts;
    float lm = -3.4028234663852886e38f;
    for (int x = t; x < ne; x += 32) lm = fmaxf(lm, __hip_atomic_load(a.logits + x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
#pragma unroll
    for (int m = 16; m > 0; m >>= 1) lm = fmaxf(lm, __shfl_xor(lm, m));
    const float mx = lm;
    float ls = 0.0f;
    for (int x = t; x < ne; x += 32)
        ls = __fadd_rn(ls, cj_expf(__fsub_rn(__hip_atomic_load(a.logits + x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), mx)));
#pragma unroll
    for (int m = 16; m > 0; m >>= 1) ls = __fadd_rn(ls, __shfl_xor(ls, m));
    const float sum = ls;
    float vlast = 3.4028234663852886e38f;
    int ilast = ne;
    for (int k = 0; k < a.used; k++) {
        float bv = -1.0f;
        int bi = ne;
        for (int x = t; x < ne; x += 32) {
            const float p = cj_expf(__fsub_rn(__hip_atomic_load(a.logits + x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), mx));
            const bool ok = p < vlast || (p == vlast && x > ilast);
            if (ok && (p > bv || (p == bv && x < bi))) { bv = p; bi = x; }
        }
        // the wave's largest probability, then the lowest index holding it
        float vk = bv;
#pragma unroll
        for (int m = 16; m > 0; m >>= 1) vk = fmaxf(vk, __shfl_xor(vk, m));
        int ik = bv == vk ? bi : ne;
#pragma unroll
        for (int m = 16; m > 0; m >>= 1) ik = min(ik, __shfl_xor(ik, m));
        if (t == 0) {
            a.sel[k] = ik;
            a.w[k] = __fdiv_rn(vk, sum);
        }
        vlast = vk;
        ilast = ik;
    }
    if (t == 0) {
        if (a.norm_topk) {
            float ws = 0.0f;
            for (int k = 0; k < a.used; k++) ws = __fadd_rn(ws, a.w[k]);
            if (ws < 0.00006103515625f) ws = 0.00006103515625f;
            for (int k = 0; k < a.used; k++) a.w[k] = __fdiv_rn(a.w[k], ws);
        }
        if (a.w_scale != 0.0f && a.w_scale != 1.0f)
            for (int k = 0; k < a.used; k++) a.w[k] = __fmul_rn(a.w[k], a.w_scale);
        a.counter[0] = 0;
    }
}

// MoE combine (MoeFfn.forwardRow, model/MoeFfn.cajeta:1849-1913): the
// selected experts' rows weighted and summed in k order, then onto hs.
// Grid y is the row of a many-row step: row r's hs, its n_used outputs and
// weights follow row r − 1's.
extern "C" __global__ void __launch_bounds__(256) cj_moe_combine(cj_combine_args a) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x, r = blockIdx.y;
    if (i >= a.n) return;
    const float *w = a.w + r * a.n_used, *y = a.y + r * a.n_used * a.n;
    float acc = 0.0f;
    for (int k = 0; k < a.n_used; k++) acc = __fadd_rn(acc, __fmul_rn(w[k], y[k * a.n + i]));
    float *hs = a.hs + r * a.n;
    hs[i] = __fadd_rn(hs[i], acc);
}
