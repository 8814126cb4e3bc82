// gemv.hip — quantised mat-vec family for gfx950 (wave64).
//
// One body serves every decode projection. A prologue stages the activation
// in LDS (a copied pack, the pack of an f32 vector, or RMSNorm + pack). Then:
//
//   phase A  lanes stream the weight rows with 128-bit loads — lanes across a
//            row's blocks, LPR lanes a row, NR (4 or 2) rows in flight — and compute
//            each block's exact terms: integer dot4s for the quants, the
//            6-bit scales and mins in integer space, the quad of lanes that
//            shares a block summed exactly, then the block's f32 terms as the
//            reference forms them. The terms go to LDS per (row, block).
//   phase B  one thread per row folds its row's terms in block order — the
//            order Quant.q4kMatVecIntoQ8 / q6kMatVecIntoQ8 / q80MatVecIntoQ8Sub
//            add them (io/Quant.cajeta:3079-3110, :3374-3486) — and runs the
//            epilogue: store, residual accumulate, RoPE + the fp16 K/V append,
//            SiLU·up + the pack of the result, or the greedy argmax.
//
// The f32-activation formats (Q4_0, MXFP4, the f32 router) are summed by one
// thread a row in the reference's element order.
//
// Prepared row layouts (HBM, 16-byte aligned rows):
//   Q4_K : the GGUF blocks as they are: {f16 d, f16 dmin, 12 B scales, 128 B qs}
//   Q6_K : [ql nb·128][qh nb·64][scales nb·16][d nb·2, padded to 16]
//   Q8_0 : [qs nb·32][d nb·2, padded to 16]
//   Q4_0 : [qs nb·16][d nb·2, padded to 16]
//   MXFP4: [qs nb·16][e nb, padded to 16]
//   F32  : the f32 row
#include "common.h"

#define LDS_SCRATCH 3072   // red[256] + bmax[512] floats

// Terms each row leaves in LDS, by format.
DEV int terms_per_row(int fmt, int64_t cols) {
    switch (fmt) {
    case CJ_Q4_K: return (int)(cols / 256) * 2;
    case CJ_Q6_K: return (int)(cols / 256);
    case CJ_Q8_0: return (int)((cols / 32 + 7) / 8);
    default: return 1;
    }
}

// ----------------------------------------------------------------- phase A

// Q4_K × q8_K. Unit (block b, 64-element chunk j): the two sub-blocks' int
// dots × their 6-bit scales and the mins × the pack's sub-block sums, summed
// over the quad exactly; the leader writes (d·xs·sumi, dmin·xs·dmins).
template <int NR, int LPR>
DEV void terms_q4k(const uint8_t *const (&wr)[NR], float *const (&tr)[NR], const uint8_t *sx, int nb, int slot) {
    const int units = nb * 4;
    for (int u = slot; u < units; u += LPR) {
        const int b = u >> 2, j = u & 3;
        uint4 hd[NR], q0[NR], q1[NR];
#pragma unroll
        for (int r = 0; r < NR; r++) {
            const uint8_t *blk = wr[r] + (int64_t)b * 144;
            hd[r] = *(const uint4 *)blk;
            q0[r] = *(const uint4 *)(blk + 16 + 32 * j);
            q1[r] = *(const uint4 *)(blk + 32 + 32 * j);
        }
        const uint8_t *ax = sx + b * 320 + 64 * j;
        const uint4 a0 = *(const uint4 *)(ax), a1 = *(const uint4 *)(ax + 16);
        const uint4 a2 = *(const uint4 *)(ax + 32), a3 = *(const uint4 *)(ax + 48);
        const int2 bs = *(const int2 *)(sx + b * 320 + 256 + 8 * j);
        const float xs = *(const float *)(sx + b * 320 + 288);
        const int hi = j >= 2;
        const int t0 = (2 * j) & 3;
#pragma unroll
        for (int r = 0; r < NR; r++) {
            const uint32_t M = 0x0F0F0F0Fu;
            int dlo = 0, dhi = 0;
            dlo = sdot4(q0[r].x & M, a0.x, dlo); dlo = sdot4(q0[r].y & M, a0.y, dlo);
            dlo = sdot4(q0[r].z & M, a0.z, dlo); dlo = sdot4(q0[r].w & M, a0.w, dlo);
            dlo = sdot4(q1[r].x & M, a1.x, dlo); dlo = sdot4(q1[r].y & M, a1.y, dlo);
            dlo = sdot4(q1[r].z & M, a1.z, dlo); dlo = sdot4(q1[r].w & M, a1.w, dlo);
            dhi = sdot4((q0[r].x >> 4) & M, a2.x, dhi); dhi = sdot4((q0[r].y >> 4) & M, a2.y, dhi);
            dhi = sdot4((q0[r].z >> 4) & M, a2.z, dhi); dhi = sdot4((q0[r].w >> 4) & M, a2.w, dhi);
            dhi = sdot4((q1[r].x >> 4) & M, a3.x, dhi); dhi = sdot4((q1[r].y >> 4) & M, a3.y, dhi);
            dhi = sdot4((q1[r].z >> 4) & M, a3.z, dhi); dhi = sdot4((q1[r].w >> 4) & M, a3.w, dhi);
            // 6-bit scales/mins of sub-blocks 2j, 2j+1 (the headK4 unpacking)
            const uint32_t sy = hd[r].y, sz = hd[r].z, sw = hd[r].w;
            const uint32_t A0 = (sy >> (8 * t0)) & 255, B0 = (sz >> (8 * t0)) & 255, C0 = (sw >> (8 * t0)) & 255;
            const uint32_t A1 = (sy >> (8 * t0 + 8)) & 255, B1 = (sz >> (8 * t0 + 8)) & 255, C1 = (sw >> (8 * t0 + 8)) & 255;
            int sc0, mn0, sc1, mn1;
            if (hi) {
                sc0 = (C0 & 15) | ((A0 >> 2) & 48); mn0 = (C0 >> 4) | ((B0 >> 2) & 48);
                sc1 = (C1 & 15) | ((A1 >> 2) & 48); mn1 = (C1 >> 4) | ((B1 >> 2) & 48);
            } else {
                sc0 = A0 & 63; mn0 = B0 & 63; sc1 = A1 & 63; mn1 = B1 & 63;
            }
            int sumi = dlo * sc0 + dhi * sc1;
            int dmins = mn0 * bs.x + mn1 * bs.y;
            sumi += quad_xor1(sumi); sumi += quad_xor2(sumi);
            dmins += quad_xor1(dmins); dmins += quad_xor2(dmins);
            if (j == 0) {
                const float d = h2f(hd[r].x), dmin = h2f(hd[r].x >> 16);
                *(float2 *)(tr[r] + 2 * b) = make_float2(__fmul_rn(__fmul_rn(d, xs), (float)sumi),
                                                         __fmul_rn(__fmul_rn(dmin, xs), (float)dmins));
            }
        }
    }
}

// Q6_K × q8_K. Unit (block b, 64 elements): half g, lane half hl; four
// 16-element scale groups; the 6-bit values 0..63 dot the int8 activation
// and 32·Σa comes off per group. The leader writes d·xs·sumi.
template <int NR, int LPR>
DEV void terms_q6k(const uint8_t *const (&wr)[NR], float *const (&tr)[NR], const uint8_t *sx, int nb, int slot) {
    const int units = nb * 4;
    for (int u = slot; u < units; u += LPR) {
        const int b = u >> 2, j = u & 3, g = j >> 1, hl = j & 1;
        uint4 qa[NR], qb[NR], qh[NR];
        uint2 sc[NR];
        uint32_t dh[NR];
#pragma unroll
        for (int r = 0; r < NR; r++) {
            const uint8_t *row = wr[r];
            qa[r] = *(const uint4 *)(row + (int64_t)b * 128 + 64 * g + 16 * hl);
            qb[r] = *(const uint4 *)(row + (int64_t)b * 128 + 64 * g + 32 + 16 * hl);
            qh[r] = *(const uint4 *)(row + (int64_t)nb * 128 + (int64_t)b * 64 + 32 * g + 16 * hl);
            sc[r] = *(const uint2 *)(row + (int64_t)nb * 192 + (int64_t)b * 16 + 8 * g);
            dh[r] = *(const uint16_t *)(row + (int64_t)nb * 208 + 2 * b);
        }
        const uint8_t *ab = sx + b * 320 + 128 * g + 16 * hl;
        uint4 a[4];
        int S[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            a[k] = *(const uint4 *)(ab + 32 * k);
            int s = 0;
            s = sdot4(0x01010101u, a[k].x, s); s = sdot4(0x01010101u, a[k].y, s);
            s = sdot4(0x01010101u, a[k].z, s); s = sdot4(0x01010101u, a[k].w, s);
            S[k] = s;
        }
        const float xs = *(const float *)(sx + b * 320 + 288);
#pragma unroll
        for (int r = 0; r < NR; r++) {
            int sumi = 0;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint4 ql = (k & 1) ? qb[r] : qa[r];
                const int sh = (k >> 1) * 4;
                const uint32_t M = 0x0F0F0F0Fu, H = 0x03030303u;
                const uint32_t vx = ((ql.x >> sh) & M) | (((qh[r].x >> (2 * k)) & H) << 4);
                const uint32_t vy = ((ql.y >> sh) & M) | (((qh[r].y >> (2 * k)) & H) << 4);
                const uint32_t vz = ((ql.z >> sh) & M) | (((qh[r].z >> (2 * k)) & H) << 4);
                const uint32_t vw = ((ql.w >> sh) & M) | (((qh[r].w >> (2 * k)) & H) << 4);
                int dt = 0;
                dt = sdot4(vx, a[k].x, dt); dt = sdot4(vy, a[k].y, dt);
                dt = sdot4(vz, a[k].z, dt); dt = sdot4(vw, a[k].w, dt);
                const int byte_i = 2 * k + hl;
                const uint32_t word = byte_i < 4 ? sc[r].x : sc[r].y;
                const int scv = (int)(int8_t)((word >> (8 * (byte_i & 3))) & 255);
                sumi += scv * (dt - 32 * S[k]);
            }
            sumi += quad_xor1(sumi); sumi += quad_xor2(sumi);
            if (j == 0) tr[r][b] = __fmul_rn(__fmul_rn(h2f(dh[r]), xs), (float)sumi);
        }
    }
}

// Q8_0 × per-32 int8. One 32-element block a lane, term (d·xs)·isum; the 8
// lanes of a 256-wide group then sum their terms in block order (the
// reference's fs) and the group's first lane writes it.
template <int NR, int LPR>
DEV void terms_q80(const uint8_t *const (&wr)[NR], float *const (&tr)[NR], const uint8_t *sx, int nb32, int slot) {
    const int lane = threadIdx.x & 63;
    const int base = lane & ~7;
    const int iters = (nb32 + LPR - 1) / LPR;
    for (int it = 0; it < iters; it++) {
        const int u = slot + it * LPR;
        const bool ok = u < nb32;
        const int uu = ok ? u : nb32 - 1;
        uint4 w0[NR], w1[NR];
        uint32_t dh[NR];
#pragma unroll
        for (int r = 0; r < NR; r++) {
            w0[r] = *(const uint4 *)(wr[r] + (int64_t)uu * 32);
            w1[r] = *(const uint4 *)(wr[r] + (int64_t)uu * 32 + 16);
            dh[r] = *(const uint16_t *)(wr[r] + (int64_t)nb32 * 32 + 2 * uu);
        }
        const uint8_t *ab = sx + (uu >> 3) * 320;
        const uint4 a0 = *(const uint4 *)(ab + 32 * (uu & 7)), a1 = *(const uint4 *)(ab + 32 * (uu & 7) + 16);
        const float xs = *(const float *)(ab + 288 + 4 * (uu & 7));
        const int left = nb32 - (u & ~7);          // real blocks in this group of 8
#pragma unroll
        for (int r = 0; r < NR; r++) {
            int s = 0;
            s = sdot4(w0[r].x, a0.x, s); s = sdot4(w0[r].y, a0.y, s);
            s = sdot4(w0[r].z, a0.z, s); s = sdot4(w0[r].w, a0.w, s);
            s = sdot4(w1[r].x, a1.x, s); s = sdot4(w1[r].y, a1.y, s);
            s = sdot4(w1[r].z, a1.z, s); s = sdot4(w1[r].w, a1.w, s);
            const float t = __fmul_rn(__fmul_rn(h2f(dh[r]), xs), (float)s);
            float fs = __shfl(t, base);
#pragma unroll
            for (int k = 1; k < 8; k++) {
                const float o = __shfl(t, base + k);
                if (k < left) fs = __fadd_rn(fs, o);
            }
            if (ok && (u & 7) == 0) tr[r][u >> 3] = fs;
        }
    }
}

// f32-activation formats: one thread a row, the row summed in the
// reference's element order, x from LDS.
//   Q4_0  : Quant.q40MatVecIntoAt (io/Quant.cajeta:1516-1545): per block, dot over the
//           16 byte pairs (low nibble then high), then acc + d·dot.
//   MXFP4 : Quant.mxfp4MatVecIntoScalar (io/Quant.cajeta:1146-1182):
//           acc + code·d·x element by element.
//   F32   : the router's plain row dot in column order.
template <int FMT>
DEV float seq_row(const uint8_t *wr, const float *xs, int64_t cols, const float *lut) {
    float acc = 0.0f;
    if (FMT == CJ_F32) {
        const float4 *w4 = (const float4 *)wr;
        for (int64_t u = 0; u < cols / 4; u++) {
            const float4 w = w4[u];
            const float4 x = *(const float4 *)(xs + 4 * u);
            acc = __fadd_rn(acc, __fmul_rn(w.x, x.x));
            acc = __fadd_rn(acc, __fmul_rn(w.y, x.y));
            acc = __fadd_rn(acc, __fmul_rn(w.z, x.z));
            acc = __fadd_rn(acc, __fmul_rn(w.w, x.w));
        }
        return acc;
    }
    const int nb32 = (int)(cols / 32);
    for (int u = 0; u < nb32; u++) {
        const uint4 q = *(const uint4 *)(wr + (int64_t)u * 16);
        const uint32_t ws[4] = {q.x, q.y, q.z, q.w};
        const float *xb = xs + u * 32;
        if (FMT == CJ_Q4_0) {
            const float dv = h2f(*(const uint16_t *)(wr + (int64_t)nb32 * 16 + 2 * u));
            float dot = 0.0f;
#pragma unroll
            for (int jj = 0; jj < 16; jj++) {
                const int b = (ws[jj >> 2] >> (8 * (jj & 3))) & 255;
                dot = __fadd_rn(dot, __fmul_rn((float)((b & 15) - 8), xb[jj]));
                dot = __fadd_rn(dot, __fmul_rn((float)((b >> 4) - 8), xb[jj + 16]));
            }
            acc = __fadd_rn(acc, __fmul_rn(dv, dot));
        } else {
            const float d = mxfp4_scale(wr[(int64_t)nb32 * 16 + u]);
#pragma unroll
            for (int k = 0; k < 32; k++) {
                const int jj = k & 15;
                const uint32_t b = (ws[jj >> 2] >> (8 * (jj & 3))) & 255;
                const uint32_t nib = k < 16 ? (b & 15) : (b >> 4);
                acc = __fadd_rn(acc, __fmul_rn(__fmul_rn(lut[nib], d), xb[k]));
            }
        }
    }
    return acc;
}

// ------------------------------------------------------------- epilogues

DEV int64_t kv_index(const int32_t *pgtab, int pg_base, int pos, int nkv, int kvh, int hd) {
    const int page = pgtab[pg_base + (pos >> 6)];
    return (((int64_t)page * nkv + kvh) * 64 + (pos & 63)) * hd;
}

// Pack one 256-wide block of an f32 vector (values past n are zero) from
// HBM into the 320-byte layout, by the whole workgroup.
DEV void pack_block_global(const float *x, int64_t n, int64_t blk, int per32, uint8_t *out, float *bmax) {
    const int t = threadIdx.x, lane = t & 63;
    const int64_t e = blk * 256 + t;
    const float v = e < n ? x[e] : 0.0f;
    const float a = fabsf(v);
    if (per32) {
        const float m = group_max<32>(a);
        if ((lane & 31) == 0) bmax[t >> 5] = m;
    } else {
        const float m = group_max<64>(a);
        if (lane == 0) bmax[t >> 6] = m;
    }
    __syncthreads();
    const float am = per32 ? bmax[t >> 5] : fmaxf(fmaxf(bmax[0], bmax[1]), fmaxf(bmax[2], bmax[3]));
    const float inv = am > 0.0f ? __fdiv_rn(127.0f, am) : 0.0f;
    const int q = round_away(__fmul_rn(v, inv));
    uint8_t *ob = out + blk * 320;
    ob[t] = (uint8_t)(int8_t)q;
    const int s = group_sum_i<32>(q);
    if ((lane & 31) == 0) *(int32_t *)(ob + 256 + 4 * (t >> 5)) = s;
    if (per32) {
        if ((lane & 31) == 0) *(float *)(ob + 288 + 4 * (t >> 5)) = __fdiv_rn(am, 127.0f);
    } else {
        if (t == 0) *(float *)(ob + 288) = __fdiv_rn(am, 127.0f);
        pack_zero_pad(ob, t);
    }
    __syncthreads();
}

DEV bool argmax_take(float ov, int oi, float mv, int mi) {
    return mi < 0 || (oi >= 0 && (ov > mv || (ov == mv && oi < mi)));
}

// ------------------------------------------------------------------ body

template <int FMT, int LPR, int NR>
DEV void gemv_body(const cj_gemv_args &a) {
    extern __shared__ __align__(16) uint8_t smem[];
    float *red = (float *)smem;
    float *bmax = red + 256;
    uint8_t *sx = smem + LDS_SCRATCH;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int64_t cols = a.cols;
    constexpr bool f32act = (FMT == CJ_Q4_0 || FMT == CJ_MXFP4 || FMT == CJ_F32);
    const int nblk = (int)((cols + 255) / 256);
    const int act_bytes = f32act ? nblk * 1024 : nblk * 320;
    float *terms = (float *)(sx + act_bytes);
    const int TB = terms_per_row(FMT, cols);
    const int R = a.rows_per_wg;

    // MoE indirection: copy k of the rows reads expert sel[k]
    int64_t wg = blockIdx.x;
    int kidx = 0;
    if (a.sel) {
        const int64_t wpk = (a.rows + R - 1) / R;
        kidx = (int)(wg / wpk);
        wg = wg % wpk;
    }
    const uint8_t *W = a.w + (a.sel ? (int64_t)a.sel[kidx] * a.expert_bytes : 0);
    const float *X = a.x ? a.x + kidx * a.x_stride : nullptr;
    float *Y = a.y ? a.y + kidx * a.y_stride : nullptr;
    float *ACT = a.act ? a.act + kidx * a.y_stride : nullptr;
    const int64_t row0 = wg * R;

    // ---- prologue: the activation into LDS
    if (a.pro == CJ_PRO_PACKED) {
        stage_copy(a.xp + kidx * a.xp_stride, nblk, sx);
    } else {
        const bool norm = a.pro == CJ_PRO_NORM_PACK || a.pro == CJ_PRO_NORM_F32;
        const float scale = norm ? stage_norm_scale(X, cols, a.eps, red) : 1.0f;
        if (f32act) stage_f32(X, cols, nblk, norm, scale, a.nw, a.norm_form, (float *)sx);
        else stage_pack(X, cols, nblk, norm, scale, a.nw, a.norm_form, a.per32, sx, nullptr);
    }

    float v = 0.0f;
    const int64_t r = row0 + t;
    const bool live = t < R && r < a.rows;
    if constexpr (f32act) {
        // ---- one thread a row, in element order
        __shared__ float lut[16];
        if (t < 16) lut[t] = mxfp4_val(t);
        __syncthreads();
        if (live) v = seq_row<FMT>(W + r * a.row_bytes, (const float *)sx, cols, lut);
    } else {
    // ---- phase A: block terms of the workgroup's R rows, NR rows a group in flight
    {
        constexpr int G = 64 / LPR;
        const int group = lane / LPR, slot = lane % LPR;
        const int lanes_groups = 4 * G;                      // row groups across the workgroup
        const int nb = (int)(cols / 256), nb32 = (int)(cols / 32);
        for (int i = 0; i < R; i += NR * lanes_groups) {
            const int rl0 = i + NR * (wave * G + group);
            if (rl0 >= R) continue;     // uniform per LPR group
            const uint8_t *wr[NR];
            float *tr[NR];
#pragma unroll
            for (int k = 0; k < NR; k++) {
                const int64_t rk = row0 + rl0 + k;
                wr[k] = W + (rk < a.rows ? rk : a.rows - 1) * a.row_bytes;
                tr[k] = terms + (rl0 + k) * TB;
            }
            if (FMT == CJ_Q4_K) terms_q4k<NR, LPR>(wr, tr, sx, nb, slot);
            else if (FMT == CJ_Q6_K) terms_q6k<NR, LPR>(wr, tr, sx, nb, slot);
            else terms_q80<NR, LPR>(wr, tr, sx, nb32, slot);
        }
    }
    __syncthreads();

    // ---- phase B: thread t folds row t's terms in block order
    if (t < R) {
        const float *tp = terms + t * TB;
        if (FMT == CJ_Q4_K) {
            for (int b = 0; b < TB; b += 2) v = __fsub_rn(__fadd_rn(v, tp[b]), tp[b + 1]);
        } else {
            for (int b = 0; b < TB; b++) v = __fadd_rn(v, tp[b]);
        }
    }
    }
    const float vp = __shfl_xor(v, 1);      // the paired row (RoPE pair, gate/up pair)
    const int pos = (a.epi == CJ_EPI_QKV_ROPE || a.epi == CJ_EPI_ARGMAX) ? step_pos(a.state, a.pos) : 0;

    switch (a.epi) {
    case CJ_EPI_STORE:
        if (live) Y[a.y_off + r] = v;
        break;
    case CJ_EPI_ACCUM:
        if (live) Y[a.y_off + r] = __fadd_rn(Y[a.y_off + r], v);
        break;
    case CJ_EPI_QKV_ROPE: {
        if (!live || (t & 1)) break;
        const int hd = a.head_dim, half = hd >> 1;
        const int64_t qrows = (int64_t)a.n_q * hd, krows = (int64_t)a.n_kv * hd;
        if (r < qrows + krows) {
            // GGUF pair order: row h·hd + 2b + a holds HF dim a·half + b
            const int64_t rr = r < qrows ? r : r - qrows;
            const int h = (int)(rr / hd), bb = (int)(rr % hd) >> 1;
            const float2 cs = *(const float2 *)(a.rope_cs + 2 * ((int64_t)pos * half + bb));
            const float ra = __fsub_rn(__fmul_rn(v, cs.x), __fmul_rn(vp, cs.y));
            const float rb = __fadd_rn(__fmul_rn(v, cs.y), __fmul_rn(vp, cs.x));
            if (r < qrows) {
                a.q_out[(int64_t)h * hd + bb] = ra;
                a.q_out[(int64_t)h * hd + half + bb] = rb;
            } else {
                const int64_t ki = kv_index(a.pgtab, a.pg_base, pos, a.n_kv, h, hd);
                a.kc[ki + bb] = f2h(ra);
                a.kc[ki + half + bb] = f2h(rb);
            }
        } else {
            const int64_t rr = r - qrows - krows;
            const int h = (int)(rr / hd), d = (int)(rr % hd);
            const int64_t vi = kv_index(a.pgtab, a.pg_base, pos, a.n_kv, h, hd);
            a.vc[vi + d] = f2h(v);
            a.vc[vi + d + 1] = f2h(vp);
        }
    } break;
    case CJ_EPI_GLU:
        if (live && !(t & 1)) ACT[r >> 1] = glu_value(a.glu_form, r >> 1, a.act_n, v, vp);
        break;
    default:
        break;
    }

    if (a.epi == CJ_EPI_GLU && a.act_pack) {
        // The last workgroup to finish a 256-wide block of the activation
        // packs it for the down projection.
        __shared__ int last_blocks[4];
        __shared__ int n_last;
        __threadfence();
        __syncthreads();
        const int64_t a0 = row0 >> 1;
        int64_t a1 = a0 + (R >> 1);
        if (a1 > (a.rows >> 1)) a1 = a.rows >> 1;
        if (t == 0) {
            n_last = 0;
            for (int64_t blk = a0 / 256; blk * 256 < a1; blk++) {
                const int64_t lo = blk * 256 > a0 ? blk * 256 : a0;
                const int64_t hi = (blk + 1) * 256 < a1 ? (blk + 1) * 256 : a1;
                const int64_t real = ((blk + 1) * 256 < a.act_n ? (blk + 1) * 256 : a.act_n) - blk * 256;
                const int mine = (int)(hi - lo);
                const int old = atomicAdd(&a.counters[blk], mine);
                if (old + mine == real) last_blocks[n_last++] = (int)blk;
            }
        }
        __syncthreads();
        const int nl = n_last;
        if (nl > 0) {
            __threadfence();
            for (int k = 0; k < nl; k++) {
                const int blk = last_blocks[k];
                pack_block_global(ACT, a.act_n, blk, a.act_per32, a.act_pack, bmax);
                if (t == 0) a.counters[blk] = 0;
            }
        }
    } else if (a.epi == CJ_EPI_ARGMAX) {
        // first occurrence across the workgroup, then the last workgroup
        // reduces every workgroup's partial and advances the step
        __shared__ float bv[256];
        __shared__ int bi[256];
        __shared__ int ticket;
        if (live) Y[r] = v;
        bv[t] = v;
        bi[t] = live ? (int)r : -1;
        __syncthreads();
        for (int s = 128; s > 0; s >>= 1) {
            if (t < s && argmax_take(bv[t + s], bi[t + s], bv[t], bi[t])) { bv[t] = bv[t + s]; bi[t] = bi[t + s]; }
            __syncthreads();
        }
        if (t == 0) {
            a.part_v[blockIdx.x] = bv[0];
            a.part_i[blockIdx.x] = bi[0];
        }
        if (!a.counters) return;      // the pick runs as its own launch
        if (t == 0) {
            __threadfence();
            ticket = atomicAdd(a.counters, 1);
        }
        __syncthreads();
        if (ticket != (int)gridDim.x - 1) return;
        __threadfence();
        float gb = 0.0f;
        int gi = -1;
        for (int gg = t; gg < (int)gridDim.x; gg += 256) {
            const float x = a.part_v[gg];
            const int xi = a.part_i[gg];
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
            a.counters[0] = 0;
            if (a.preds) a.preds[pos + 1] = bi[0];
            if (a.tokens && (!a.state || pos + 1 >= a.state->fixed_until)) a.tokens[pos + 1] = bi[0];
            if (a.state) a.state->pos = pos + 1;
        }
    }
}

#define GEMV_KERNEL(NAME, FMT, LPR, NR)                                                \
    extern "C" __global__ void __launch_bounds__(256) NAME(cj_gemv_args a) {            \
        gemv_body<FMT, LPR, NR>(a);                                                     \
    }

#define GEMV_FAMILY(PFX, FMT, NR)               \
    GEMV_KERNEL(PFX##_l64, FMT, 64, NR)         \
    GEMV_KERNEL(PFX##_l32, FMT, 32, NR)         \
    GEMV_KERNEL(PFX##_l16, FMT, 16, NR)         \
    GEMV_KERNEL(PFX##_l8, FMT, 8, NR)

// cj_gemv_<fmt>_l<LPR>[_n2]: LPR lanes a row, 4 (or 2: _n2, and Q6_K) rows
// in flight per lane group
#define GEMV_FAMILY_N2(PFX, FMT)                    \
    GEMV_KERNEL(PFX##_l64_n2, FMT, 64, 2)           \
    GEMV_KERNEL(PFX##_l32_n2, FMT, 32, 2)           \
    GEMV_KERNEL(PFX##_l16_n2, FMT, 16, 2)           \
    GEMV_KERNEL(PFX##_l8_n2, FMT, 8, 2)

GEMV_FAMILY(cj_gemv_q4k, CJ_Q4_K, 4)
GEMV_FAMILY_N2(cj_gemv_q4k, CJ_Q4_K)
GEMV_FAMILY(cj_gemv_q6k, CJ_Q6_K, 2)
GEMV_FAMILY(cj_gemv_q80, CJ_Q8_0, 4)
GEMV_FAMILY_N2(cj_gemv_q80, CJ_Q8_0)
GEMV_KERNEL(cj_gemv_q40, CJ_Q4_0, 64, 1)
GEMV_KERNEL(cj_gemv_mxfp4, CJ_MXFP4, 64, 1)
GEMV_KERNEL(cj_gemv_f32, CJ_F32, 64, 1)
