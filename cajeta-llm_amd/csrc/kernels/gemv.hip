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
// The f32-activation formats are summed in the reference's orders: Q4_0
// block by block (its block dots are independent until the row's fold, so
// lanes form them in parallel: q40_rows), MXFP4 in its scalar form and the
// f32 router element by element, one adder lane a row fed products through
// LDS (seq_body).
//
// Q4_K has its own body (gemv_q4k_body): one lane a whole 256-element block,
// the first weight block of every lane in flight before the prologue, and
// workgroups that sweep several passes of rows with a one-block prefetch.
//
// Prepared row layouts (HBM, 16-byte aligned rows):
//   Q4_K : [c 0..7][b 0..nb-1] 16-byte pieces of the blocks' qs (piece c of
//          block b = qs bytes 16c..16c+15), then [b] the 16-byte block
//          headers {f16 d, f16 dmin, 12 B scales}: lanes holding consecutive
//          blocks load consecutive 16-byte words
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

// Q4_K × q8_K, one lane a whole block. The 16 sub-block halves' int dots
// (low nibbles: sub-block 2g, high: 2g+1 of each 64-element group g), the
// 6-bit scales and mins (Quant.headK4) and the pack's 32-sums stay in
// integers; the block's f32 terms are formed as Quant.q4kMatVecIntoQ8 forms
// them (io/Quant.cajeta:3374-3445): (d·xs)·sumi and (dmin·xs)·dmins.
#define Q4K_LDS_STRIDE 336   // pack blocks in LDS: 16 lanes on 16 blocks hit distinct banks
struct Q4kBlock { uint4 q[8]; uint4 h; };

DEV void q4k_fetch(Q4kBlock &x, const uint8_t *row, int nb, int b) {
#pragma unroll
    for (int c = 0; c < 8; c++) x.q[c] = ld_stream16(row + ((int64_t)c * nb + b) * 16);
    x.h = ld_stream16(row + (int64_t)nb * 128 + (int64_t)b * 16);
}

// The activation a lane needs for one block: the 256 int8 codes, the eight
// 32-sums and the scale of one 320-byte pack block.
struct Q4kAct { uint4 a[16]; int4 s0, s1; float xs; };

DEV void q4k_act_load(Q4kAct &v, const uint8_t *ax) {
#pragma unroll
    for (int k = 0; k < 16; k++) v.a[k] = *(const uint4 *)(ax + 16 * k);
    v.s0 = *(const int4 *)(ax + 256);
    v.s1 = *(const int4 *)(ax + 272);
    v.xs = *(const float *)(ax + 288);
}

DEV float2 q4k_block_terms(const Q4kBlock &x, const Q4kAct &v) {
    const uint32_t M = 0x0F0F0F0Fu;
    int dot[8];
#pragma unroll
    for (int g = 0; g < 4; g++) {
        int lo = 0, hi = 0;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint4 q = x.q[2 * g + h];
            const uint4 al = v.a[4 * g + h];        // elements 64g + 16h ..
            const uint4 ah = v.a[4 * g + 2 + h];    // elements 64g + 32 + 16h ..
            lo = sdot4(q.x & M, al.x, lo); lo = sdot4(q.y & M, al.y, lo);
            lo = sdot4(q.z & M, al.z, lo); lo = sdot4(q.w & M, al.w, lo);
            hi = sdot4((q.x >> 4) & M, ah.x, hi); hi = sdot4((q.y >> 4) & M, ah.y, hi);
            hi = sdot4((q.z >> 4) & M, ah.z, hi); hi = sdot4((q.w >> 4) & M, ah.w, hi);
        }
        dot[2 * g] = lo;
        dot[2 * g + 1] = hi;
    }
    // scales[0..3] = A, [4..7] = B, [8..11] = C: sub-block j < 4 takes the
    // low 6 bits of A_j (scale) and B_j (min); j + 4 takes the nibbles of C_j
    // with the top two bits of A_j (scale) and B_j (min) above them. Every
    // factor fits in 24 bits (|dot| ≤ 32·15·127, |32-sum| ≤ 32·127, scales
    // and mins ≤ 63), so the 24-bit multiplies are exact.
    const uint32_t A = x.h.y, B = x.h.z, C = x.h.w;
    const int bs[8] = {v.s0.x, v.s0.y, v.s0.z, v.s0.w, v.s1.x, v.s1.y, v.s1.z, v.s1.w};
    int sumi = 0, dmins = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const uint32_t a8 = (A >> (8 * j)) & 255, b8 = (B >> (8 * j)) & 255, c8 = (C >> (8 * j)) & 255;
        const int sc_lo = (int)(a8 & 63), mn_lo = (int)(b8 & 63);
        const int sc_hi = (int)((c8 & 15) | ((a8 >> 2) & 48)), mn_hi = (int)((c8 >> 4) | ((b8 >> 2) & 48));
        sumi += __mul24(dot[j], sc_lo) + __mul24(dot[j + 4], sc_hi);
        dmins += __mul24(bs[j], mn_lo) + __mul24(bs[j + 4], mn_hi);
    }
    const float d = h2f(x.h.x), dmin = h2f(x.h.x >> 16);
    return make_float2(__fmul_rn(__fmul_rn(d, v.xs), (float)sumi), __fmul_rn(__fmul_rn(dmin, v.xs), (float)dmins));
}

// Q6_K × q8_K. Unit (block b, 64 elements): half g, lane half hl; four
// 16-element scale groups; the 6-bit values 0..63 dot the int8 activation
// and 32·Σa comes off per group. The leader writes d·xs·sumi.
template <int NR>
struct Q6kItem {
    uint4 qa[NR], qb[NR], qh[NR];
    uint2 sc[NR];
    uint32_t dh[NR];
};

template <int NR>
DEV void q6k_item(Q6kItem<NR> &x, const uint8_t *const (&wr)[NR], int nb, int u) {
    const int b = u >> 2, j = u & 3, g = j >> 1, hl = j & 1;
#pragma unroll
    for (int r = 0; r < NR; r++) {
        const uint8_t *row = wr[r];
        x.qa[r] = ld_stream16(row + (int64_t)b * 128 + 64 * g + 16 * hl);
        x.qb[r] = ld_stream16(row + (int64_t)b * 128 + 64 * g + 32 + 16 * hl);
        x.qh[r] = ld_stream16(row + (int64_t)nb * 128 + (int64_t)b * 64 + 32 * g + 16 * hl);
        x.sc[r] = *(const uint2 *)(row + (int64_t)nb * 192 + (int64_t)b * 16 + 8 * g);
        x.dh[r] = *(const uint16_t *)(row + (int64_t)nb * 208 + 2 * b);
    }
}

// Sweeps of LPR units (64-element quarter blocks); the next sweep's weights
// are requested before this one's arithmetic, as in terms_q80. A quad of
// lanes past the row's units (all four or none: units and LPR are multiples
// of 4) re-reads the last unit and writes nothing.
template <int NR, int LPR>
DEV void terms_q6k(const uint8_t *const (&wr)[NR], float *const (&tr)[NR], const uint8_t *sx, int nb, int slot) {
    const int units = nb * 4, iters = (units + LPR - 1) / LPR;
    auto u_of = [&](int it) { const int u = slot + it * LPR; return u < units ? u : units - 1; };
    auto body = [&](const Q6kItem<NR> &x, int it) {
        const bool ok = slot + it * LPR < units;
        const int u = u_of(it);
        const int b = u >> 2, j = u & 3, g = j >> 1, hl = j & 1;
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
                const uint4 ql = (k & 1) ? x.qb[r] : x.qa[r];
                const int sh = (k >> 1) * 4;
                const uint32_t M = 0x0F0F0F0Fu, H = 0x03030303u;
                const uint32_t vx = ((ql.x >> sh) & M) | (((x.qh[r].x >> (2 * k)) & H) << 4);
                const uint32_t vy = ((ql.y >> sh) & M) | (((x.qh[r].y >> (2 * k)) & H) << 4);
                const uint32_t vz = ((ql.z >> sh) & M) | (((x.qh[r].z >> (2 * k)) & H) << 4);
                const uint32_t vw = ((ql.w >> sh) & M) | (((x.qh[r].w >> (2 * k)) & H) << 4);
                int dt = 0;
                dt = sdot4(vx, a[k].x, dt); dt = sdot4(vy, a[k].y, dt);
                dt = sdot4(vz, a[k].z, dt); dt = sdot4(vw, a[k].w, dt);
                const int byte_i = 2 * k + hl;
                const uint32_t word = byte_i < 4 ? x.sc[r].x : x.sc[r].y;
                const int scv = (int)(int8_t)((word >> (8 * (byte_i & 3))) & 255);
                sumi += scv * (dt - 32 * S[k]);
            }
            sumi += quad_xor1(sumi); sumi += quad_xor2(sumi);
            if (ok && j == 0) tr[r][b] = __fmul_rn(__fmul_rn(h2f(x.dh[r]), xs), (float)sumi);
        }
    };
    Q6kItem<NR> cur, nxt;
    q6k_item(cur, wr, nb, u_of(0));
    for (int it = 0; it + 1 < iters; it++) {
        q6k_item(nxt, wr, nb, u_of(it + 1));
        body(cur, it);
        cur = nxt;
    }
    body(cur, iters - 1);
}

// Q6_K without the next sweep's prefetch, for rows that fit one sweep
// (fewer registers: the one-sweep kernels keep their occupancy).
template <int NR, int LPR>
DEV void terms_q6k_1(const uint8_t *const (&wr)[NR], float *const (&tr)[NR], const uint8_t *sx, int nb, int slot) {
    const int units = nb * 4;
    for (int u = slot; u < units; u += LPR) {
        const int b = u >> 2, j = u & 3, g = j >> 1, hl = j & 1;
        uint4 qa[NR], qb[NR], qh[NR];
        uint2 sc[NR];
        uint32_t dh[NR];
#pragma unroll
        for (int r = 0; r < NR; r++) {
            const uint8_t *row = wr[r];
            qa[r] = ld_stream16(row + (int64_t)b * 128 + 64 * g + 16 * hl);
            qb[r] = ld_stream16(row + (int64_t)b * 128 + 64 * g + 32 + 16 * hl);
            qh[r] = ld_stream16(row + (int64_t)nb * 128 + (int64_t)b * 64 + 32 * g + 16 * hl);
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
template <int NR>
struct Q80Sweep {
    uint4 w0[NR], w1[NR];
    uint32_t dh[NR];
};
// sweep `it` of the lane's block (slot + it·LPR; past the row, the last block)
template <int NR, int LPR>
DEV void q80_load(const uint8_t *const (&wr)[NR], int nb32, int slot, int it, Q80Sweep<NR> &sw) {
    const int u = slot + it * LPR, uu = u < nb32 ? u : nb32 - 1;
#pragma unroll
    for (int r = 0; r < NR; r++) {
        sw.w0[r] = ld_stream16(wr[r] + (int64_t)uu * 32);
        sw.w1[r] = ld_stream16(wr[r] + (int64_t)uu * 32 + 16);
        sw.dh[r] = *(const uint16_t *)(wr[r] + (int64_t)nb32 * 32 + 2 * uu);
    }
}
template <int NR, int LPR>
DEV void q80_compute(float *const (&tr)[NR], const uint8_t *sx, int nb32, int slot, int it, const Q80Sweep<NR> &sw) {
    const int u = slot + it * LPR;
    const bool ok = u < nb32;
    const int uu = ok ? u : nb32 - 1;
    const uint8_t *ab = sx + (uu >> 3) * 320;
    const uint4 a0 = *(const uint4 *)(ab + 32 * (uu & 7)), a1 = *(const uint4 *)(ab + 32 * (uu & 7) + 16);
    const float xs = *(const float *)(ab + 288 + 4 * (uu & 7));
    const int left = nb32 - (u & ~7);          // real blocks in this group of 8
#pragma unroll
    for (int r = 0; r < NR; r++) {
        int s = 0;
        s = sdot4(sw.w0[r].x, a0.x, s); s = sdot4(sw.w0[r].y, a0.y, s);
        s = sdot4(sw.w0[r].z, a0.z, s); s = sdot4(sw.w0[r].w, a0.w, s);
        s = sdot4(sw.w1[r].x, a1.x, s); s = sdot4(sw.w1[r].y, a1.y, s);
        s = sdot4(sw.w1[r].z, a1.z, s); s = sdot4(sw.w1[r].w, a1.w, s);
        const float t = __fmul_rn(__fmul_rn(h2f(sw.dh[r]), xs), (float)s);
        // lane base + k's term reaches lane base by row_shl:k (base is a
        // multiple of 8, so the eight stay inside one 16-lane row)
        const float o[7] = {dpp_shl<1>(t), dpp_shl<2>(t), dpp_shl<3>(t), dpp_shl<4>(t),
                            dpp_shl<5>(t), dpp_shl<6>(t), dpp_shl<7>(t)};
        float fs = t;
#pragma unroll
        for (int k = 1; k < 8; k++)
            if (k < left) fs = __fadd_rn(fs, o[k - 1]);
        if (ok && (u & 7) == 0) tr[r][u >> 3] = fs;
    }
}
template <int NR, int LPR>
DEV void terms_q80(const uint8_t *const (&wr)[NR], float *const (&tr)[NR], const uint8_t *sx, int nb32, int slot) {
    const int iters = (nb32 + LPR - 1) / LPR;
    if (iters == 2) {
        // rows of two sweeps: both sweeps' weights requested before either's
        // arithmetic (one memory round trip, not two)
        Q80Sweep<NR> s0, s1;
        q80_load<NR, LPR>(wr, nb32, slot, 0, s0);
        q80_load<NR, LPR>(wr, nb32, slot, 1, s1);
        q80_compute<NR, LPR>(tr, sx, nb32, slot, 0, s0);
        q80_compute<NR, LPR>(tr, sx, nb32, slot, 1, s1);
        return;
    }
    for (int it = 0; it < iters; it++) {
        Q80Sweep<NR> sw;
        q80_load<NR, LPR>(wr, nb32, slot, it, sw);
        q80_compute<NR, LPR>(tr, sx, nb32, slot, it, sw);
    }
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

// Where a workgroup's rows come from: with MoE indirection (`sel`), copy k
// of the rows reads expert sel[k]'s weight, activation k / sel_per_x (k
// where sel_per_x ≤ 1: many rows' selections share their row's activation)
// and writes output k.
struct GemvSlice {
    const uint8_t *W;
    const float *X;
    float *Y, *ACT;
    int64_t row0;
    int kidx, xidx;
};

DEV GemvSlice gemv_slice(const cj_gemv_args &a) {
    GemvSlice s;
    const int R = a.rows_per_wg;
    int64_t wg = blockIdx.x;
    s.kidx = 0;
    if (a.sel || a.route_logits) {
        const int64_t wpk = (a.rows + R - 1) / R;
        s.kidx = (int)(wg / wpk);
        wg = wg % wpk;
    }
    s.W = a.w + (a.sel ? (int64_t)a.sel[s.kidx] * a.expert_bytes : 0);
    s.xidx = a.sel_per_x > 1 ? s.kidx / a.sel_per_x : s.kidx;
    s.X = a.x ? a.x + s.xidx * a.x_stride : nullptr;
    s.Y = a.y ? a.y + s.kidx * a.y_stride : nullptr;
    s.ACT = a.act ? a.act + s.kidx * a.y_stride : nullptr;
    s.row0 = wg * R;
    return s;
}

// The activation into LDS: a copied pack, the pack of an f32 vector, RMSNorm
// + pack, or (f32-activation formats) the f32 values, normed or not. Ends on
// a barrier.
template <class Mid = NoMid>
DEV void gemv_prologue(const cj_gemv_args &a, const GemvSlice &sl, bool f32act, uint8_t *sx, float *red, int bstride,
                       bool swz = false, Mid &&mid = Mid{}) {
    const int64_t cols = a.cols;
    const int nblk = (int)((cols + 255) / 256);
    if (a.pro == CJ_PRO_PACKED) {
        mid();
        stage_copy(a.xp + sl.xidx * a.xp_stride, nblk, sx, bstride);
    } else {
        const bool norm = a.pro == CJ_PRO_NORM_PACK || a.pro == CJ_PRO_NORM_F32;
        float scale = 1.0f;
        if (norm) scale = stage_norm_scale(sl.X, cols, a.eps, red, mid);
        else mid();
        if (f32act) {
            stage_f32(sl.X, cols, nblk, norm, scale, a.nw, a.norm_form, (float *)sx, swz);
            if (a.xout && norm && !swz && blockIdx.x == 0) {   // the staged values (stage_f32 ends on a barrier)
                for (int64_t e = threadIdx.x; e < cols; e += 256) a.xout[e] = ((const float *)sx)[e];
            }
        } else {
            stage_pack(sl.X, cols, nblk, norm, scale, a.nw, a.norm_form, a.per32, sx, nullptr, bstride);
        }
    }
}

// Operands the epilogue reads from global memory, loaded early (after the
// weight stream is requested) so they have arrived when the rows finish:
// the residual of an accumulating row, and for q|k|v the RoPE (cos, sin) of
// the row's pair and the K/V page of the step position.
struct EpiPre {
    float y;
    float2 cs;
    int page;
    int pos;
};

template <int EPI>
DEV EpiPre epi_prefetch_t(const cj_gemv_args &a, const GemvSlice &sl) {
    EpiPre e{0.0f, make_float2(0.0f, 0.0f), 0, 0};
    const int64_t r = min(sl.row0 + (int64_t)threadIdx.x, a.rows - 1);
    if constexpr (EPI == CJ_EPI_ACCUM) {
        e.y = sl.Y[a.y_off + r];
    } else if constexpr (EPI == CJ_EPI_QKV_ROPE) {
        e.pos = step_pos(a.state, a.pos);
        e.page = a.pgtab[a.pg_base + (e.pos >> 6)];
        const int hd = a.head_dim, half = hd >> 1;
        const int bb = (int)(r % hd) >> 1;
        e.cs = *(const float2 *)(a.rope_cs + 2 * ((int64_t)e.pos * half + bb));
    }
    return e;
}

// The epilogue chosen at run time (the generic body).
DEV EpiPre epi_prefetch(const cj_gemv_args &a, const GemvSlice &sl) {
    switch (a.epi) {
    case CJ_EPI_ACCUM: return epi_prefetch_t<CJ_EPI_ACCUM>(a, sl);
    case CJ_EPI_QKV_ROPE: return epi_prefetch_t<CJ_EPI_QKV_ROPE>(a, sl);
    default: return epi_prefetch_t<CJ_EPI_STORE>(a, sl);
    }
}

// Row r's value v (thread t = r − row0; the paired row r^1 sits on thread
// t^1) through the epilogue: store, residual accumulate, RoPE + the fp16 K/V
// append, SiLU·up (+ the pack of the result), or the greedy argmax.
template <int EPI>
DEV void gemv_epilogue_t(const cj_gemv_args &a, const GemvSlice &sl, float v, float *bmax, const EpiPre &pre) {
    const int t = threadIdx.x;
    const int R = a.rows_per_wg;
    const int64_t r = sl.row0 + t;
    const bool live = t < R && r < a.rows;
    float *Y = sl.Y, *ACT = sl.ACT;
    const int64_t row0 = sl.row0;
    const float vp = dpp_f<DPP_XOR1>(v);    // the paired row (RoPE pair, gate/up pair)
    const int pos = EPI == CJ_EPI_QKV_ROPE ? pre.pos : EPI == CJ_EPI_ARGMAX ? step_pos(a.state, a.pos) : 0;

    switch (EPI) {
    case CJ_EPI_STORE:
        if (live) Y[a.y_off + r] = v;
        break;
    case CJ_EPI_ACCUM:
        if (live) Y[a.y_off + r] = __fadd_rn(pre.y, v);
        break;
    case CJ_EPI_QKV_ROPE: {
        if (!live || (t & 1)) break;
        const int hd = a.head_dim, half = hd >> 1;
        const int64_t qrows = (int64_t)a.n_q * hd, krows = (int64_t)a.n_kv * hd;
        if (r < qrows + krows) {
            // GGUF pair order: row h·hd + 2b + a holds HF dim a·half + b
            const int64_t rr = r < qrows ? r : r - qrows;
            const int h = (int)(rr / hd), bb = (int)(rr % hd) >> 1;
            const float2 cs = pre.cs;
            const float ra = __fsub_rn(__fmul_rn(v, cs.x), __fmul_rn(vp, cs.y));
            const float rb = __fadd_rn(__fmul_rn(v, cs.y), __fmul_rn(vp, cs.x));
            if (r < qrows) {
                a.q_out[(int64_t)h * hd + bb] = ra;
                a.q_out[(int64_t)h * hd + half + bb] = rb;
            } else {
                const int64_t ki = (((int64_t)pre.page * a.n_kv + h) * 64 + (pos & 63)) * hd;
                kv_store2(a.kc, a.kv_f32, ki + bb, ra, ki + half + bb, rb);
            }
        } else {
            const int64_t rr = r - qrows - krows;
            const int h = (int)(rr / hd), d = (int)(rr % hd);
            const int64_t vi = (((int64_t)pre.page * a.n_kv + h) * 64 + (pos & 63)) * hd;
            kv_store2(a.vc, a.kv_f32, vi + d, v, vi + d + 1, vp);
        }
    } break;
    case CJ_EPI_GLU:
        if (live && !(t & 1)) ACT[r >> 1] = glu_value(a.glu_form, r >> 1, a.act_n, v, vp);
        break;
    default:
        break;
    }

    if (EPI == CJ_EPI_GLU && a.act_pack) {
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
                if (old + mine == real && n_last < 4) last_blocks[n_last++] = (int)blk;
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
    } else if (EPI == CJ_EPI_ARGMAX) {
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

// The epilogue chosen at run time (the generic body).
DEV void gemv_epilogue(const cj_gemv_args &a, const GemvSlice &sl, float v, float *bmax, const EpiPre &pre) {
    switch (a.epi) {
    case CJ_EPI_ACCUM: gemv_epilogue_t<CJ_EPI_ACCUM>(a, sl, v, bmax, pre); break;
    case CJ_EPI_QKV_ROPE: gemv_epilogue_t<CJ_EPI_QKV_ROPE>(a, sl, v, bmax, pre); break;
    case CJ_EPI_GLU: gemv_epilogue_t<CJ_EPI_GLU>(a, sl, v, bmax, pre); break;
    case CJ_EPI_ARGMAX: gemv_epilogue_t<CJ_EPI_ARGMAX>(a, sl, v, bmax, pre); break;
    default: gemv_epilogue_t<CJ_EPI_STORE>(a, sl, v, bmax, pre); break;
    }
}

// The element-order chains:
//   MXFP4 : Quant.mxfp4MatVecIntoScalar (io/Quant.cajeta:1146-1182):
//           acc + (code·d)·x element by element;
//   F32   : the router's plain row dot in column order.
// Each row's sum is one dependent chain, so the work splits by role. Lane r
// of the first wave (the adder) owns row r of the workgroup's 64 and only
// adds: its row's rounded products arrive through LDS in the order it adds
// them, a 16-byte read of four, so the chain costs 1.25 instructions an
// element. The other three waves (producers) form the products one tile
// ahead: in a tile of SEQ_TB 32-element blocks, producer wave p + 1 owns
// block p of all 64 rows (one row a lane, x a broadcast from LDS), its next
// tile's weights already loaded into registers.
#define SEQ_TB 3                   // blocks a tile: one a producer wave
#define SEQ_S (32 * SEQ_TB + 4)    // product row stride (floats): 16-byte reads by 16 lanes hit distinct banks

template <int FMT>
struct SeqItem {
    u32x4 q[FMT == CJ_F32 ? 8 : 1];
    uint32_t s;
};

// One row block's weights: 32 f32, or the 16 code bytes and the block scale.
template <int FMT>
DEV SeqItem<FMT> seq_fetch(const uint8_t *wr, int nb32, int blk) {
    SeqItem<FMT> it;
    blk = min(blk, nb32 - 1);     // a block past the row is formed but never added
    if constexpr (FMT == CJ_F32) {
#pragma unroll
        for (int j = 0; j < 8; j++) it.q[j] = *(const u32x4 *)(wr + (int64_t)blk * 128 + 16 * j);
        it.s = 0;
    } else {
        it.q[0] = *(const u32x4 *)(wr + (int64_t)blk * 16);
        it.s = wr[(int64_t)nb32 * 16 + blk];
    }
    return it;
}

// The block's 32 x values from LDS into registers.
DEV void seq_xload(const float *xs, int blk, float4 (&x)[8]) {
#pragma unroll
    for (int j = 0; j < 8; j++) x[j] = *(const float4 *)(xs + 32 * blk + 4 * j);
}

// The block's 32 rounded products in add order into dst.
template <int FMT>
DEV void seq_products(const SeqItem<FMT> &it, const float4 (&xr)[8], float *dst) {
    if constexpr (FMT == CJ_F32) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float4 x = xr[j];
            float4 o;
            o.x = __fmul_rn(__uint_as_float(it.q[j].x), x.x);
            o.y = __fmul_rn(__uint_as_float(it.q[j].y), x.y);
            o.z = __fmul_rn(__uint_as_float(it.q[j].z), x.z);
            o.w = __fmul_rn(__uint_as_float(it.q[j].w), x.w);
            *(float4 *)(dst + 4 * j) = o;
        }
    } else {
        // element k: code byte k & 15, low nibble for k < 16, high after;
        // |code| from the low three bits by a byte permute of {0,1,2,3,4,6,8,12},
        // the sign from bit 3. Code 8 comes out as -0 where the reference has
        // +0: its product is a zero either way, and a zero added to the sum
        // (which starts at +0, so is never -0) changes no bit.
        const float d = mxfp4_scale(it.s);
        const uint32_t ws[4] = {it.q[0].x, it.q[0].y, it.q[0].z, it.q[0].w};
#pragma unroll
        for (int g = 0; g < 8; g++) {
            const uint32_t nibs = g < 4 ? (ws[g & 3] & 0x0f0f0f0fu) : ((ws[g & 3] >> 4) & 0x0f0f0f0fu);
            const uint32_t mag = __builtin_amdgcn_perm(0x0c080604u, 0x03020100u, nibs & 0x07070707u);
            const float4 x = xr[g];
            const float xv[4] = {x.x, x.y, x.z, x.w};
            float ov[4];
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                const float c = __uint_as_float(__float_as_uint((float)((mag >> (8 * kk)) & 255u)) ^
                                                (((nibs >> (8 * kk + 3)) & 1u) << 31));
                ov[kk] = __fmul_rn(__fmul_rn(c, d), xv[kk]);
            }
            *(float4 *)(dst + 4 * g) = make_float4(ov[0], ov[1], ov[2], ov[3]);
        }
    }
}

// Row threadIdx.x (< 64) of the workgroup's rows summed; x staged in LDS by
// `pro`, the prologue, which every thread calls first. Every thread of the
// workgroup must call it (it holds barriers). A producer lane keeps D tiles
// of its weights in flight (a ring indexed at compile time: the tile loop is
// unrolled by D) and reads its next block of x from LDS a tile ahead, so its
// products wait on neither; the adder reads three blocks' products (24
// 16-byte reads) before their 96 adds: measured against reads kept a fixed
// distance ahead of the adds, each read then waited for in turn, the batch
// is faster (a lone wave's chain: 6.9 against 8.3 cycles an add, 4.6 with
// the operands in registers).
#ifndef SEQ_D
#define SEQ_D 8
#endif
template <int FMT, int ROWS, class Pro>
DEV float seq_body(const cj_gemv_args &a, const GemvSlice &sl, const float *xs, Pro &&pro) {
    // one row a workgroup: a tile is 192 blocks, so two in flight suffice
    constexpr int D = ROWS == 1 ? 2 : SEQ_D;
    static_assert(D % 2 == 0, "the ring depth must be even");
    static_assert(ROWS == 64 || ROWS == 32 || ROWS == 1, "64, 32 or 1 rows a workgroup");
    static_assert(ROWS != 1 || 96 * 64 <= 32 * (192 / ROWS) + 4, "a one-row tile's products fit 96 a lane");
    constexpr int TB = 192 / ROWS;            // blocks a tile: the 192 producer lanes, one (row, block) each
    constexpr int TU = TB <= 6 ? TB / 3 : 2;  // the adder's unroll over a whole tile's triples
    constexpr int S = 32 * TB + 4;            // product row stride (floats): 16-byte reads by 16 lanes, distinct banks
    __shared__ __align__(16) float prod[2][64 * SEQ_S];   // ROWS·S ≤ 64·SEQ_S floats a buffer
    const int t = threadIdx.x, w = t >> 6, lane = t & 63;
    const int nb32 = (int)(a.cols / 32), ntiles = (nb32 + TB - 1) / TB;
    const int pl = max(t - 64, 0), prow = pl % ROWS, pb = pl / ROWS;   // (the adder wave as producer 0)
    const uint8_t *wr = sl.W + min(sl.row0 + prow, a.rows - 1) * a.row_bytes;
    float *pdst = prod[0] + prow * S + 32 * pb;
    constexpr int PBUF = 64 * SEQ_S;
    // both loops run a whole number of D-tile rounds: the producer's body
    // is then free of branches (tiles past the end are formed into the idle
    // buffer and never read)
    // (a one-row workgroup whose row is one tile — the router — runs that
    // tile alone: one barrier each side, no idle tile formed or read)
    const bool one = ROWS == 1 && ntiles == 1;
    const int nit = one ? 0 : (ntiles + D - 1) / D * D;
    float acc = 0.0f;
    // the first D tiles' weights are requested inside the prologue, after its
    // own loads (every wave, so no load sits under a branch; the adder wave's
    // are never used)
    SeqItem<FMT> ring[D];
    pro([&] {
#pragma unroll
        for (int j = 0; j < D; j++) ring[j] = seq_fetch<FMT>(wr, nb32, j * TB + pb);
    });
    if (w == 0 && ROWS == 1) {
        // one row: the chain walks the wave's lanes. Lane L holds products
        // 96·L .. 96·L + 95 of the tile in registers (one batch of LDS reads a
        // tile); the lanes add their own in lockstep, and after lane L's 96
        // its sum is broadcast to every lane (readlane), so each of the
        // chain's adds reads its operand from a register
        __syncthreads();
        for (int i = 0; i < max(nit, (int)one); i++) {
            const float *pr = prod[0] + (i & 1) * PBUF + 96 * lane;   // within the row: 96·64 ≤ S
            const int n = (i < ntiles ? min(TB, nb32 - i * TB) : 0) * 32;
            f32x4 p[24];
#pragma unroll
            for (int q = 0; q < 24; q++) p[q] = *(const f32x4 *)(pr + 4 * q);
            for (int L = 0; 96 * L < n; L++) {
                const int cnt = n - 96 * L;                            // a multiple of 32
#pragma unroll
                for (int c = 0; c < 3; c++) {
                    if (c == 0 || cnt > 32 * c) {
#pragma unroll
                        for (int q = 8 * c; q < 8 * c + 8; q++) {
                            acc = __fadd_rn(acc, p[q].x);
                            acc = __fadd_rn(acc, p[q].y);
                            acc = __fadd_rn(acc, p[q].z);
                            acc = __fadd_rn(acc, p[q].w);
                        }
                    }
                }
                acc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), L));
            }
            if (!one) __syncthreads();
        }
    } else if (w == 0) {
        __syncthreads();
        const float *pr0 = prod[0] + min(lane, ROWS - 1) * S;
        auto add3 = [&](const float *pr, int b0) {
            float4 p[24];
#pragma unroll
            for (int q = 0; q < 24; q++) p[q] = *(const float4 *)(pr + 32 * b0 + 4 * q);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int q = 0; q < 24; q++) {
                acc = __fadd_rn(acc, p[q].x);
                acc = __fadd_rn(acc, p[q].y);
                acc = __fadd_rn(acc, p[q].z);
                acc = __fadd_rn(acc, p[q].w);
            }
        };
        auto add1 = [&](const float *pr, int b) {
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const float4 p = *(const float4 *)(pr + 32 * b + 4 * q);
                acc = __fadd_rn(acc, p.x);
                acc = __fadd_rn(acc, p.y);
                acc = __fadd_rn(acc, p.z);
                acc = __fadd_rn(acc, p.w);
            }
        };
        for (int i = 0; i < nit; i++) {
            const float *pr = pr0 + (i & 1) * PBUF;
            const int nb = i < ntiles ? min(TB, nb32 - i * TB) : 0;
            if (nb == TB) {
#pragma unroll TU
                for (int b0 = 0; b0 < TB; b0 += 3) add3(pr, b0);
            } else {
                int b0 = 0;
                for (; b0 + 3 <= nb; b0 += 3) add3(pr, b0);
                for (int b = b0; b < nb; b++) add1(pr, b);
            }
            __syncthreads();
        }
    } else {
        float4 xr[2][8];
        seq_xload(xs, min(pb, nb32 - 1), xr[0]);
        seq_xload(xs, min(TB + pb, nb32 - 1), xr[1]);
        seq_products<FMT>(ring[0], xr[0], pdst);
        ring[0] = seq_fetch<FMT>(wr, nb32, D * TB + pb);
        __syncthreads();
        // round j of an iteration forms tile i + 1 from ring[(j + 1) % D] and
        // x registers xr[(j + 1) & 1], then loads x of tile i + 2 into xr[j & 1]
        for (int i0 = 0; i0 < nit; i0 += D) {
#pragma unroll
            for (int j = 0; j < D; j++) {
                const int i = i0 + j;
                const int r = (j + 1) % D;
                const int nbuf = (j + 1) & 1;      // D is even, so (i + 1) & 1
                seq_xload(xs, min((i + 2) * TB + pb, nb32 - 1), xr[j & 1]);
                seq_products<FMT>(ring[r], xr[nbuf], pdst + nbuf * PBUF);
                ring[r] = seq_fetch<FMT>(wr, nb32, (i + 1 + D) * TB + pb);
                __syncthreads();
            }
        }
    }
    return acc;
}

// Q4_0, block-parallel: wave w owns RW rows of the workgroup's 4·RW, and
// lane L forms the block terms d·dot of blocks L, L + 64, … (a sweep of 64
// blocks at a time) for all RW rows from one read of each x block; lane k <
// RW folds row k's terms in block order from the wave's LDS rows, a sweep
// behind, in the same straight-line code as the next sweep's products so the
// fold's dependent adds fill their gaps. (Before the first sweep it folds a
// zeroed row: +0 added to the +0 start changes no bit. Lanes past RW fold a
// copy of the last row and drop it.) The next sweep's codes and scales are in
// flight while a sweep is formed; x comes from LDS, so the two never wait on
// each other. Returns row t's sum on thread t < 4·RW.
template <int RW>
DEV float q40_rows(const cj_gemv_args &a, const GemvSlice &sl, const float *xs) {
    __shared__ __align__(16) float tb[4][2][RW][Q40_TS];
    __shared__ float rv[4 * RW];
    const int t = threadIdx.x, w = t >> 6, lane = t & 63;
    const int nb = (int)(a.cols / 32), sweeps = (nb + 63) >> 6;
    const int fr = min(lane, RW - 1);
#pragma unroll
    for (int k = 0; k < RW; k++) tb[w][1][k][lane] = 0.0f;
    const uint8_t *wr[RW];
#pragma unroll
    for (int k = 0; k < RW; k++) wr[k] = sl.W + min(sl.row0 + w * RW + k, a.rows - 1) * a.row_bytes;
    uint4 qn[RW];
    uint32_t dn[RW];
    // a sweep's codes and scales (blocks past the row re-read the last one, never folded)
    auto fetch = [&](int j) {
        const int b = min(64 * j + lane, nb - 1);
#pragma unroll
        for (int k = 0; k < RW; k++) {
            qn[k] = ld_stream16(wr[k] + 16 * (int64_t)b);
            dn[k] = *(const uint16_t *)(wr[k] + 16 * (int64_t)nb + 2 * b);
        }
    };
    fetch(0);
    __builtin_amdgcn_wave_barrier();
    float acc = 0.0f;
    for (int j = 0; j < sweeps; j++) {
        uint4 q[RW];
        uint32_t d[RW];
#pragma unroll
        for (int k = 0; k < RW; k++) { q[k] = qn[k]; d[k] = dn[k]; }
        fetch(j + 1);
        float4 x[8];
        q40_xblock(xs, min(64 * j + lane, nb - 1), x);
#pragma unroll
        for (int k = 0; k < RW; k++) {
            float v[32];
            q40_decode(q[k], v);
            tb[w][j & 1][k][lane] = __fmul_rn(h2f(d[k]), q40_dot(v, x));
        }
        acc = q40_fold64(tb[w][(j + 1) & 1][fr], acc);   // sweep j − 1: whole (only the last can be short)
        __builtin_amdgcn_wave_barrier();
    }
    acc = q40_fold(tb[w][(sweeps - 1) & 1][fr], nb - 64 * (sweeps - 1), acc);
    if (lane < RW) rv[w * RW + lane] = acc;
    __syncthreads();
    return t < 4 * RW ? rv[t] : 0.0f;
}

// The Q4_0 GEMV: prologue (x, or its RMSNorm, staged swizzled), the rows,
// and the common epilogues.
template <int RW>
DEV void q40_gemv(const cj_gemv_args &a) {
    extern __shared__ __align__(16) uint8_t smem[];
    float *red = (float *)smem;
    float *bmax = red + 256;
    uint8_t *sx = smem + LDS_SCRATCH;
    const GemvSlice sl = gemv_slice(a);
    gemv_prologue(a, sl, true, sx, red, 320, true);
    const EpiPre pre = epi_prefetch(a, sl);
    const float v = q40_rows<RW>(a, sl, (const float *)sx);
    gemv_epilogue(a, sl, v, bmax, pre);
}

// Generic body (Q6_K, Q8_0 and the f32-activation formats).
template <int FMT, int LPR, int NR, bool MULTI = false>
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
    const GemvSlice sl = gemv_slice(a);
    const int64_t row0 = sl.row0;

    // one row a workgroup over plain f32 x: no two producer lanes share a
    // block of x, so each reads its block from global memory beside its
    // weights rather than after x is staged in LDS (one round trip fewer)
    const bool xdirect = f32act && LPR == 1 && a.pro == CJ_PRO_F32 && ((uintptr_t)sl.X & 15) == 0;
    if constexpr (FMT == CJ_Q8_0 && !MULTI) {
        // Q8_0 over a packed activation, the workgroup's rows one pass of at
        // most two sweeps: the activation's words are requested first, then
        // both sweeps' weights, then the epilogue's operands, and only then
        // are the words written to LDS — loads retire in issue order, so the
        // staging waits for the activation alone and the weight stream's
        // latency overlaps it (a round trip, not two)
        constexpr int G = 64 / LPR, XW = 2;
        const int nb32 = (int)(cols / 32), nwords = nblk * 20;
        if (a.pro == CJ_PRO_PACKED && R <= NR * 4 * G && nb32 <= 2 * LPR && nwords <= 256 * XW) {
            const uint8_t *xsrc = a.xp + sl.xidx * a.xp_stride;
            u32x4 xw[XW];
#pragma unroll
            for (int k = 0; k < XW; k++) xw[k] = *(const u32x4 *)(xsrc + 16 * min(t + 256 * k, nwords - 1));
            const int group = lane / LPR, slot = lane % LPR;
            const int rl0 = NR * (wave * G + group);   // rows past R: loaded (clamped), never stored
            const uint8_t *wr[NR];
            float *tr[NR];
#pragma unroll
            for (int k = 0; k < NR; k++) {
                const int64_t rk = row0 + rl0 + k;
                wr[k] = sl.W + (rk < a.rows ? rk : a.rows - 1) * a.row_bytes;
                tr[k] = terms + (rl0 + k) * TB;
            }
            Q80Sweep<NR> s0, s1;
            q80_load<NR, LPR>(wr, nb32, slot, 0, s0);
            q80_load<NR, LPR>(wr, nb32, slot, 1, s1);
            const EpiPre pre = epi_prefetch(a, sl);
#pragma unroll
            for (int k = 0; k < XW; k++) {
                const int idx = t + 256 * k;
                if (idx < nwords) *(u32x4 *)(sx + (idx / 20) * 320 + 16 * (idx % 20)) = xw[k];
            }
            lds_barrier();
            if (rl0 < R) {
                q80_compute<NR, LPR>(tr, sx, nb32, slot, 0, s0);
                if (nb32 > LPR) q80_compute<NR, LPR>(tr, sx, nb32, slot, 1, s1);
            }
            __syncthreads();
            float v = 0.0f;
            if (t < R) {
                const float *tp = terms + t * TB;
                for (int b = 0; b < TB; b++) v = __fadd_rn(v, tp[b]);
            }
            gemv_epilogue(a, sl, v, bmax, pre);
            return;
        }
    }
    // (the f32-activation formats stage x inside seq_body, after a one-row
    // workgroup's weights are requested)
    if (!f32act && !xdirect) gemv_prologue(a, sl, f32act, sx, red, 320);
    const EpiPre pre = epi_prefetch(a, sl);

    float v = 0.0f;
    const int64_t r = row0 + t;
    const bool live = t < R && r < a.rows;
    if constexpr (f32act) {
        // ---- one adder lane a row, in element order (64 rows a workgroup)
        // (for these formats LPR is the rows a workgroup: 64, or 32 / 1
        // where the matrix is short and more workgroups fill the chip)
        const float sv = seq_body<FMT, LPR>(a, sl, xdirect ? sl.X : (const float *)sx, [&](auto &&mid) {
            if (!xdirect) gemv_prologue(a, sl, f32act, sx, red, 320, false, mid);
            else mid();
        });
        if (live) v = sv;
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
                wr[k] = sl.W + (rk < a.rows ? rk : a.rows - 1) * a.row_bytes;
                tr[k] = terms + (rl0 + k) * TB;
            }
            if constexpr (MULTI) {
                static_assert(FMT == CJ_Q6_K, "the multi-sweep form is Q6_K's");
                terms_q6k<NR, LPR>(wr, tr, sx, nb, slot);
            } else {
                if (FMT == CJ_Q6_K) terms_q6k_1<NR, LPR>(wr, tr, sx, nb, slot);
                else terms_q80<NR, LPR>(wr, tr, sx, nb32, slot);
            }
        }
    }
    __syncthreads();

    // ---- phase B: thread t folds row t's terms in block order
    if (t < R) {
        const float *tp = terms + t * TB;
        for (int b = 0; b < TB; b++) v = __fadd_rn(v, tp[b]);
    }
    }
    gemv_epilogue(a, sl, v, bmax, pre);
}

// The Q4_K prologue in two halves, so its global loads can be issued before
// the weight stream and its arithmetic run after: loads retire in issue
// order, so anything the prologue loaded after the weights would wait for
// HBM. PRO is the prologue (PACKED, PACK or NORM_PACK); RND bounds the
// activation to RND·4096 columns. The register arrays are plain locals of
// fixed size so they stay in registers; every load is unconditional (indices
// clamped into range, the surplus masked where it is used) because a load
// under a branch makes the compiler wait for every load in flight at the
// join, the weight stream included.

template <int PRO, int RND>
struct Q4kProDims {
    static constexpr int NPK = PRO == CJ_PRO_PACKED ? (RND * 16 * 20 + 255) / 256 : 1;
    static constexpr int NX = PRO == CJ_PRO_PACKED ? 1 : RND;
    static constexpr int NW = PRO == CJ_PRO_NORM_PACK ? RND : 1;
    static constexpr int NS = PRO == CJ_PRO_NORM_PACK ? RND * 16 : 1;
};

template <int PRO, int RND>
DEV void q4k_pro_load(const cj_gemv_args &a, const GemvSlice &sl, float4 (&px)[Q4kProDims<PRO, RND>::NX][4],
                      float4 (&pw)[Q4kProDims<PRO, RND>::NW][4], float (&pxs)[Q4kProDims<PRO, RND>::NS],
                      u32x4 (&ppk)[Q4kProDims<PRO, RND>::NPK]) {
    using D = Q4kProDims<PRO, RND>;
    const int t = threadIdx.x;
    const int64_t n = a.cols;
    if constexpr (PRO == CJ_PRO_PACKED) {
        const u32x4 *src = (const u32x4 *)(a.xp + sl.xidx * a.xp_stride);
        const int n16 = (int)(n / 256) * 20;
#pragma unroll
        for (int i = 0; i < D::NPK; i++) ppk[i] = src[min(t + 256 * i, n16 - 1)];
    } else {
        const float *X = sl.X;
#pragma unroll
        for (int r = 0; r < RND; r++) {
            const int64_t e0 = min((int64_t)(4096 * r + 16 * t), n - 16);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                px[r][j] = *(const float4 *)(X + e0 + 4 * j);
                if constexpr (PRO == CJ_PRO_NORM_PACK) pw[r][j] = *(const float4 *)(a.nw + e0 + 4 * j);
            }
        }
        if constexpr (PRO == CJ_PRO_NORM_PACK) {
#pragma unroll
            for (int k = 0; k < RND * 16; k++) pxs[k] = X[min((int64_t)(t + 256 * k), n - 1)];
        }
    }
}

// Pack one 16-value slice per thread into the LDS blocks (stage_pack's
// arithmetic: the 32-group or block maximum over lane neighbours, codes
// round-half-away(v·127/amax), 32-sums, scale).
DEV void q4k_pack_slice(const float (&v)[16], int64_t e0, int per32, uint8_t *sx, int bstride) {
    float am = 0.0f;
#pragma unroll
    for (int k = 0; k < 16; k++) am = fmaxf(am, fabsf(v[k]));
    am = per32 ? fmaxf(am, dpp_f<DPP_XOR1>(am)) : xmax16(am);
    const float inv = am > 0.0f ? __fdiv_rn(127.0f, am) : 0.0f;
    uint32_t wd[4] = {0u, 0u, 0u, 0u};
    int sum = 0;
#pragma unroll
    for (int k = 0; k < 16; k++) {
        const int q = round_away(__fmul_rn(v[k], inv));
        sum += q;
        wd[k >> 2] |= ((uint32_t)q & 255u) << (8 * (k & 3));
    }
    sum += quad_xor1(sum);
    const int64_t blk = e0 >> 8;
    const int in = (int)(e0 & 255);
    uint8_t *b = sx + blk * bstride;
    *(uint4 *)(b + in) = make_uint4(wd[0], wd[1], wd[2], wd[3]);
    const int g = in >> 5, j = (in >> 4) & 15;
    if (!(j & 1)) *(int32_t *)(b + 256 + 4 * g) = sum;
    if (per32) {
        if (!(j & 1)) *(float *)(b + 288 + 4 * g) = __fdiv_rn(am, 127.0f);
    } else {
        if (j == 0) *(float *)(b + 288) = __fdiv_rn(am, 127.0f);
        else if (j < 8) *(uint32_t *)(b + 288 + 4 * j) = 0u;
    }
}

template <int PRO, int RND>
DEV void q4k_pro_compute(const cj_gemv_args &a, const float4 (&px)[Q4kProDims<PRO, RND>::NX][4],
                         const float4 (&pw)[Q4kProDims<PRO, RND>::NW][4], const float (&pxs)[Q4kProDims<PRO, RND>::NS],
                         const u32x4 (&ppk)[Q4kProDims<PRO, RND>::NPK], uint8_t *sx, float *red) {
    using D = Q4kProDims<PRO, RND>;
    const int t = threadIdx.x;
    const int64_t n = a.cols;
    if constexpr (PRO == CJ_PRO_PACKED) {
        // words past the pack go to a dummy slot in the (here unused) scratch
        const int n16 = (int)(n / 256) * 20;
#pragma unroll
        for (int i = 0; i < D::NPK; i++) {
            const int idx = t + 256 * i;
            uint8_t *dst = idx < n16 ? sx + (idx / 20) * Q4K_LDS_STRIDE + (idx % 20) * 16 : (uint8_t *)red + 16 * (t & 63);
            *(u32x4 *)dst = ppk[i];
        }
    } else {
        float scale = 1.0f;
        if constexpr (PRO == CJ_PRO_NORM_PACK) {
            // RMSNorm scale in the CPU row form's order (Prim.rmsnormPackRowCpuKernel):
            // thread t sums x[t + 256k]^2 over k, the partials fold 128, 64, ..., 1
            float s = 0.0f;
#pragma unroll
            for (int k = 0; k < RND * 16; k++)
                if (t + 256 * k < n) s = __fadd_rn(s, __fmul_rn(pxs[k], pxs[k]));
            red[t] = s;
            lds_barrier();
            if (t < 128) red[t] = __fadd_rn(red[t], red[t + 128]);
            lds_barrier();
            if (t < 64) {
                const float v = fold64_lane0(__fadd_rn(red[t], red[t + 64]));
                if (t == 0) red[0] = v;
            }
            lds_barrier();
            scale = __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fdiv_rn(red[0], (float)n), a.eps)));
        }
#pragma unroll
        for (int r = 0; r < RND; r++) {
            const int64_t e0 = 4096 * r + 16 * t;
            if (e0 < n) {
                const float xv[16] = {px[r][0].x, px[r][0].y, px[r][0].z, px[r][0].w, px[r][1].x, px[r][1].y,
                                      px[r][1].z, px[r][1].w, px[r][2].x, px[r][2].y, px[r][2].z, px[r][2].w,
                                      px[r][3].x, px[r][3].y, px[r][3].z, px[r][3].w};
                float v[16];
                if constexpr (PRO == CJ_PRO_NORM_PACK) {
                    const float wv[16] = {pw[r][0].x, pw[r][0].y, pw[r][0].z, pw[r][0].w, pw[r][1].x, pw[r][1].y,
                                          pw[r][1].z, pw[r][1].w, pw[r][2].x, pw[r][2].y, pw[r][2].z, pw[r][2].w,
                                          pw[r][3].x, pw[r][3].y, pw[r][3].z, pw[r][3].w};
#pragma unroll
                    for (int k = 0; k < 16; k++) {
                        const float wi = a.norm_form == 1 ? __fadd_rn(1.0f, wv[k]) : wv[k];
                        v[k] = __fmul_rn(__fmul_rn(xv[k], scale), wi);
                    }
                } else {
#pragma unroll
                    for (int k = 0; k < 16; k++) v[k] = xv[k];
                }
                q4k_pack_slice(v, e0, a.per32, sx, Q4K_LDS_STRIDE);
            }
        }
    }
    lds_barrier();
}

// Q4_K body. Lane (wave w, lane l) owns row group l / LPR of each pass and
// blocks b = l % LPR + LPR·k of its row. The items (pass, k) run in order
// through a ring of four 144-byte blocks: item i computes while items
// i+1..i+3 load. Issue order: the prologue's loads, the first four items,
// the epilogue's operands, then the prologue's arithmetic — so the norm and
// pack run while the weight stream is in flight. The block terms go to LDS;
// thread t then folds row t's in block order, acc = (acc + A_b) − B_b
// (Quant.q4kMatVecIntoQ8), and runs the epilogue.
// IT > 0: the workgroup's items a lane are exactly IT (the planner's
// choice), and the item loop is fully unrolled with every weight load
// unconditional (clamped addresses): the compiler then knows at each use
// exactly which loads are younger, and waits only for the item it consumes
// — in the runtime loop (IT = 0) its waits are conservative and the ring
// drains to one item in flight.
template <int LPR, int PRO, int RND, int EPI, int RING, int IT = 0>
DEV void gemv_q4k_body(const cj_gemv_args &a) {
    extern __shared__ __align__(16) uint8_t smem[];
    float *red = (float *)smem;
    float *bmax = red + 256;
    uint8_t *sx = smem + LDS_SCRATCH;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int nb = (int)(a.cols / 256);
    float *terms = (float *)(sx + nb * Q4K_LDS_STRIDE);
    const int R = a.rows_per_wg;
    const GemvSlice sl = gemv_slice(a);
    const int64_t row0 = sl.row0;

    constexpr int RG = 64 / LPR;                 // rows a wave covers in one pass
    const int rg = lane / LPR, li = lane % LPR;
    const int K = (nb + LPR - 1) / LPR;          // items a pass (the last may leave lanes idle)
    const int items = IT > 0 ? IT : (R / (4 * RG)) * K;   // R is a multiple of 4·RG
    auto row_of = [&](int it) { return (it / K) * (4 * RG) + wave * RG + rg; };
    auto blk_of = [&](int it) { return li + LPR * (it % K); };
    auto fetch = [&](Q4kBlock &x, int it) {
        const int64_t rr = row0 + row_of(it);
        const int b = blk_of(it);
        q4k_fetch(x, sl.W + (rr < a.rows ? rr : a.rows - 1) * a.row_bytes, nb, b < nb ? b : nb - 1);
    };
    // a lane whose row has no more blocks than LPR keeps the one block it
    // owns for the whole kernel: its activation is read from LDS once
    const bool fixed = K == 1;
    Q4kAct act;
    auto consume = [&](const Q4kBlock &x, int it) {
        const int rl = row_of(it), b = blk_of(it);
        if (!fixed) q4k_act_load(act, sx + min(b, nb - 1) * Q4K_LDS_STRIDE);
        if (b < nb) *(float2 *)(terms + ((int64_t)rl * nb + b) * 2) = q4k_block_terms(x, act);
    };

    // issue order: f32 prologues load before the weights; a copied pack
    // loads after the first weight item (its words are stored to LDS as soon
    // as they arrive, which is before that item is consumed)
    using PD = Q4kProDims<PRO, RND>;
    float4 px[PD::NX][4], pw[PD::NW][4];
    float pxs[PD::NS];
    u32x4 ppk[PD::NPK];
    Q4kBlock ring[RING];
    if constexpr (PRO != CJ_PRO_PACKED) {
        q4k_pro_load<PRO, RND>(a, sl, px, pw, pxs, ppk);
        __builtin_amdgcn_sched_barrier(0);
    }
    fetch(ring[0], 0);
    if constexpr (PRO == CJ_PRO_PACKED) {
        __builtin_amdgcn_sched_barrier(0);
        q4k_pro_load<PRO, RND>(a, sl, px, pw, pxs, ppk);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 1; j < RING; j++) fetch(ring[j], min(j, items - 1));
    __builtin_amdgcn_sched_barrier(0);
    const EpiPre pre = epi_prefetch_t<EPI>(a, sl);
    __builtin_amdgcn_sched_barrier(0);
    q4k_pro_compute<PRO, RND>(a, px, pw, pxs, ppk, sx, red);
    if (fixed) q4k_act_load(act, sx + min(li, nb - 1) * Q4K_LDS_STRIDE);
    if constexpr (IT > 0) {
#pragma unroll
        for (int it = 0; it < IT; it++) {
            consume(ring[it % RING], it);
            if (it + RING < IT) fetch(ring[it % RING], it + RING);
        }
    } else {
        for (int it0 = 0; it0 < items; it0 += RING) {
#pragma unroll
            for (int j = 0; j < RING; j++) {
                const int it = it0 + j;
                if (it < items) {
                    consume(ring[j], it);
                    if (it + RING < items) fetch(ring[j], it + RING);
                }
            }
        }
    }
    __syncthreads();

    float v = 0.0f;
    if (t < R) {
        const float4 *tp = (const float4 *)(terms + (int64_t)t * nb * 2);
        int b = 0;
        for (; b + 1 < nb; b += 2) {
            const float4 q = tp[b >> 1];
            v = __fsub_rn(__fadd_rn(v, q.x), q.y);
            v = __fsub_rn(__fadd_rn(v, q.z), q.w);
        }
        if (b < nb) {
            const float2 q = *(const float2 *)(terms + ((int64_t)t * nb + b) * 2);
            v = __fsub_rn(__fadd_rn(v, q.x), q.y);
        }
    }
    gemv_epilogue_t<EPI>(a, sl, v, bmax, pre);
}

#define GEMV_KERNEL(NAME, FMT, LPR, NR)                                                \
    extern "C" __global__ void __launch_bounds__(256) NAME(cj_gemv_args a) {            \
        gemv_body<FMT, LPR, NR>(a);                                                     \
    }

// _s: Q6_K rows wider than one sweep of 64 lanes, the next sweep's weights
// requested before the current sweep's arithmetic
#define GEMV_KERNEL_S(NAME, FMT, NR)                                                   \
    extern "C" __global__ void __launch_bounds__(256) NAME(cj_gemv_args a) {            \
        gemv_body<FMT, 64, NR, true>(a);                                                \
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

// cj_gemv_q4k_<prologue><epilogue>_b<LPR>[_w]: LPR lanes a row, one lane a
// block; prologue c (copied pack), p (pack of f32) or n (RMSNorm + pack);
// epilogue s (store), a (accumulate), q (q|k|v RoPE + K/V), g (SiLU·up) or
// m (argmax); activations up to 4096 columns (_w: up to 16384, no norm). The
// prologue and epilogue are compile-time so no load waits on a branch.
#ifndef Q4K_RING
#define Q4K_RING 2   // weight blocks in flight per lane (deeper rings delay the first block)
#endif
#define Q4K_KERNEL(NAME, LPR, PRO, RND, EPI) \
    extern "C" __global__ void __launch_bounds__(256) NAME(cj_gemv_args a) { gemv_q4k_body<LPR, PRO, RND, EPI, Q4K_RING>(a); }
#define Q4K_EPIS(P, LPR, PRO)                                                    \
    Q4K_KERNEL(cj_gemv_q4k_##P##s_b##LPR, LPR, PRO, 1, CJ_EPI_STORE)             \
    Q4K_KERNEL(cj_gemv_q4k_##P##a_b##LPR, LPR, PRO, 1, CJ_EPI_ACCUM)             \
    Q4K_KERNEL(cj_gemv_q4k_##P##q_b##LPR, LPR, PRO, 1, CJ_EPI_QKV_ROPE)          \
    Q4K_KERNEL(cj_gemv_q4k_##P##g_b##LPR, LPR, PRO, 1, CJ_EPI_GLU)               \
    Q4K_KERNEL(cj_gemv_q4k_##P##m_b##LPR, LPR, PRO, 1, CJ_EPI_ARGMAX)
Q4K_EPIS(c, 16, CJ_PRO_PACKED)
Q4K_EPIS(p, 16, CJ_PRO_PACK)
Q4K_EPIS(n, 16, CJ_PRO_NORM_PACK)
Q4K_EPIS(c, 8, CJ_PRO_PACKED)
Q4K_EPIS(p, 8, CJ_PRO_PACK)
Q4K_EPIS(n, 8, CJ_PRO_NORM_PACK)
#define Q4K_EPIS_W(P, PRO)                                                       \
    Q4K_KERNEL(cj_gemv_q4k_##P##s_b16_w, 16, PRO, 4, CJ_EPI_STORE)               \
    Q4K_KERNEL(cj_gemv_q4k_##P##a_b16_w, 16, PRO, 4, CJ_EPI_ACCUM)               \
    Q4K_KERNEL(cj_gemv_q4k_##P##q_b16_w, 16, PRO, 4, CJ_EPI_QKV_ROPE)            \
    Q4K_KERNEL(cj_gemv_q4k_##P##g_b16_w, 16, PRO, 4, CJ_EPI_GLU)                 \
    Q4K_KERNEL(cj_gemv_q4k_##P##m_b16_w, 16, PRO, 4, CJ_EPI_ARGMAX)
Q4K_EPIS_W(c, CJ_PRO_PACKED)
Q4K_EPIS_W(p, CJ_PRO_PACK)
// _b64_w: 64 lanes a row for wide rows (56 blocks at 14336 columns: one
// wave instruction reads 896 contiguous bytes of a row, and each lane keeps
// one block's activation in registers)
#define Q4K_EPIS_W64(P, PRO)                                                     \
    Q4K_KERNEL(cj_gemv_q4k_##P##s_b64_w, 64, PRO, 4, CJ_EPI_STORE)               \
    Q4K_KERNEL(cj_gemv_q4k_##P##a_b64_w, 64, PRO, 4, CJ_EPI_ACCUM)               \
    Q4K_KERNEL(cj_gemv_q4k_##P##q_b64_w, 64, PRO, 4, CJ_EPI_QKV_ROPE)            \
    Q4K_KERNEL(cj_gemv_q4k_##P##g_b64_w, 64, PRO, 4, CJ_EPI_GLU)                 \
    Q4K_KERNEL(cj_gemv_q4k_##P##m_b64_w, 64, PRO, 4, CJ_EPI_ARGMAX)
Q4K_EPIS_W64(c, CJ_PRO_PACKED)
Q4K_EPIS_W64(p, CJ_PRO_PACK)
// _i<IT>: exactly IT items a lane, fully unrolled (ring min(IT, 3))
#define Q4KI_KERNEL(NAME, LPR, PRO, RND, EPI, IT) \
    extern "C" __global__ void __launch_bounds__(256) NAME(cj_gemv_args a) { \
        gemv_q4k_body<LPR, PRO, RND, EPI, (IT < 3 ? IT : 3), IT>(a); }
#define Q4KI_EPIS(P, PRO, LPR, SFX, RND, IT)                                                      \
    Q4KI_KERNEL(cj_gemv_q4k_##P##s_b##LPR##SFX##_i##IT, LPR, PRO, RND, CJ_EPI_STORE, IT)           \
    Q4KI_KERNEL(cj_gemv_q4k_##P##a_b##LPR##SFX##_i##IT, LPR, PRO, RND, CJ_EPI_ACCUM, IT)           \
    Q4KI_KERNEL(cj_gemv_q4k_##P##q_b##LPR##SFX##_i##IT, LPR, PRO, RND, CJ_EPI_QKV_ROPE, IT)        \
    Q4KI_KERNEL(cj_gemv_q4k_##P##g_b##LPR##SFX##_i##IT, LPR, PRO, RND, CJ_EPI_GLU, IT)             \
    Q4KI_KERNEL(cj_gemv_q4k_##P##m_b##LPR##SFX##_i##IT, LPR, PRO, RND, CJ_EPI_ARGMAX, IT)
#define Q4KI_ITS(P, PRO)                                                                               \
    Q4KI_EPIS(P, PRO, 16, , 1, 1) Q4KI_EPIS(P, PRO, 16, , 1, 2) Q4KI_EPIS(P, PRO, 16, , 1, 4)            \
    Q4KI_EPIS(P, PRO, 16, , 1, 7)
Q4KI_ITS(c, CJ_PRO_PACKED)
Q4KI_ITS(p, CJ_PRO_PACK)
Q4KI_ITS(n, CJ_PRO_NORM_PACK)
Q4KI_EPIS(c, CJ_PRO_PACKED, 64, _w, 4, 4)
Q4KI_EPIS(p, CJ_PRO_PACK, 64, _w, 4, 4)

// ------------------------------------------------------------ MXFP4 × q8

// MXFP4 in the reference's device Q8 form (QuantKernel.mxfp4MatVecCoopQ8Launch,
// io/QuantKernel.cajeta:43699-43713). Every workgroup quantizes the f32
// activation per 32 elements into LDS (mxfp4QuantActKernel, :43614-43636:
// bmax = max|x|, q = round-half-away(x · 127/bmax), d = bmax/127), then a
// 32-lane half-wave takes a row (mxfp4MatVecKernelCoopQ8, :43660-43697):
// lane L the blocks L, L+32, ..., each block's 32 E2M1 codes decoded to int8
// and dotted with the q8 codes in v_dot4 steps (an exact integer s), then
// acc = acc + s·d_w·d_x; the half-wave's xor butterfly (strides 16..1) sums
// the lanes. Row values go through LDS to the common epilogue (thread t =
// row t). The weight rows are the prepared [codes nb·16][scales nb] layout:
// a half-wave's 16-byte code loads are one 512-byte sweep.

// Four E2M1 codes (the low nibbles of v's bytes) as four int8 values of the
// reference's table {0, 1, 2, 3, 4, 6, 8, 12} with the sign bit (Quant.mxfp4Kv):
// the magnitude through a byte permute of the positive and of the negated
// table, then a third permute takes byte j from the negated result where the
// code's sign bit (bit 3) is set — selector byte j + 4·sign — six operations
// for four codes.
DEV uint32_t e2m1_x4(uint32_t v) {
    const uint32_t idx = v & 0x07070707u;
    const uint32_t pos = __builtin_amdgcn_perm(0x0C080604u, 0x03020100u, idx);
    const uint32_t neg = __builtin_amdgcn_perm(0xF4F8FAFCu, 0xFDFEFF00u, idx);
    const uint32_t sel = ((v >> 1) & 0x04040404u) | 0x03020100u;
    return __builtin_amdgcn_perm(neg, pos, sel);
}

// The LDS layout after the scratch: codes [cols], scales [nb], row values [R].
DEV int mxq8_xd_off(int64_t cols) { return (int)((cols + 15) & ~15); }

template <int EPI, int KB, int RW>
DEV void mxq8_body(const cj_gemv_args &a) {
    extern __shared__ __align__(16) uint8_t smem[];
    float *red = (float *)smem;
    float *bmax = red + 256;
    int8_t *xq = (int8_t *)(smem + LDS_SCRATCH);
    const int64_t cols = a.cols;
    const int nb = (int)(cols / 32);
    float *xd = (float *)(smem + LDS_SCRATCH + mxq8_xd_off(cols));
    float *res = xd + ((nb + 3) & ~3);
    const int t = threadIdx.x, hw = t >> 5, hl = t & 31;
    const int R = a.rows_per_wg;
    GemvSlice sl = gemv_slice(a);
    // the activation's first round of blocks (below) requested before the
    // route: it does not depend on the expert, so its latency overlaps the
    // route's own load and arithmetic
    constexpr int PR = 3;    // rounds of 32 blocks whose loads are issued together
    float4 f0[PR];
#pragma unroll
    for (int k = 0; k < PR; k++)
        f0[k] = *(const float4 *)(sl.X + 32 * (int64_t)min(32 * k + (t >> 3), nb - 1) + 4 * (t & 7));
    if (a.route_logits) {
        // the route of this copy's row, then its expert (the row's first
        // workgroup publishes the row's selections and weights)
        __shared__ RouteLds rl;
        const int nu = a.route_used, r = sl.kidx / nu, k = sl.kidx % nu;
        route_row(a.route_logits + (int64_t)r * a.route_experts, a.route_experts, nu, a.route_norm_topk,
                  a.route_scale, a.route_status, rl);
        sl.W = a.w + (int64_t)rl.sel[k] * a.expert_bytes;
        if (k == 0 && sl.row0 == 0 && t < nu) {
            a.route_sel[r * nu + t] = rl.sel[t];
            a.route_w[r * nu + t] = rl.w[t];
        }
    }
    const EpiPre pre = epi_prefetch_t<EPI>(a, sl);
    (void)red;
    u32x4 wv[RW][KB];
    uint32_t sc[RW][KB];
    auto fetch = [&](int i0, int c0) {
#pragma unroll
        for (int i = 0; i < RW; i++) {
            const int64_t r = min(sl.row0 + i0 + i, a.rows - 1);
            const uint8_t *wr = sl.W + r * a.row_bytes;
#pragma unroll
            for (int k = 0; k < KB; k++) {
                const int b = min(c0 + hl + 32 * k, nb - 1);
                wv[i][k] = __builtin_nontemporal_load((const u32x4 *)(wr + 16 * b));
                sc[i][k] = wr[16 * nb + b];
            }
        }
    };
    // the activation's codes: eight lanes a 32-block, four values a lane;
    // the block maximum by an xor exchange over the eight (max is exact)
    {
        auto quant = [&](int b0, const float4 (&f)[PR]) {
#pragma unroll
            for (int k = 0; k < PR; k++) {
                const int b = b0 + 32 * k + (t >> 3);
                const float bm = xmax8(fmaxf(fmaxf(fabsf(f[k].x), fabsf(f[k].y)), fmaxf(fabsf(f[k].z), fabsf(f[k].w))));
                const float inv = bm > 0.0f ? __fdiv_rn(127.0f, bm) : 0.0f;
                const uint32_t q = ((uint32_t)round_away(__fmul_rn(f[k].x, inv)) & 0xFFu) |
                                   (((uint32_t)round_away(__fmul_rn(f[k].y, inv)) & 0xFFu) << 8) |
                                   (((uint32_t)round_away(__fmul_rn(f[k].z, inv)) & 0xFFu) << 16) |
                                   (((uint32_t)round_away(__fmul_rn(f[k].w, inv)) & 0xFFu) << 24);
                if (b < nb) {
                    *(uint32_t *)(xq + 32 * b + 4 * (t & 7)) = q;
                    if ((t & 7) == 0) xd[b] = __fdiv_rn(bm, 127.0f);
                }
            }
        };
        quant(0, f0);
        for (int b0 = 32 * PR; b0 < nb; b0 += 32 * PR) {
            float4 f[PR];
#pragma unroll
            for (int k = 0; k < PR; k++) {
                const int b = min(b0 + 32 * k + (t >> 3), nb - 1);
                f[k] = *(const float4 *)(sl.X + 32 * (int64_t)b + 4 * (t & 7));
            }
            quant(b0, f);
        }
    }
    __syncthreads();
    // rows: half-wave hw takes rows hw·RW .. +RW−1 of each 8·RW-row pass;
    // every load of a sweep is issued (clamped into range) before the first
    // is used
    for (int i0 = hw * RW; i0 < R; i0 += 8 * RW) {
        float acc[RW];
#pragma unroll
        for (int i = 0; i < RW; i++) acc[i] = 0.0f;
        for (int c0 = 0; c0 < nb; c0 += 32 * KB) {
            fetch(i0, c0);
            // keep the sweep's loads ahead of its arithmetic (the scheduler
            // otherwise sinks them between the decodes, each then waited for
            // in turn)
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < RW; i++) {
#pragma unroll
                for (int k = 0; k < KB; k++) {
                    const int b = c0 + hl + 32 * k, bc = min(b, nb - 1);
                    const u32x4 w = wv[i][k];
                    const u32x4 x0 = *(const u32x4 *)(xq + 32 * bc), x1 = *(const u32x4 *)(xq + 32 * bc + 16);
                    int sd = 0;
                    sd = __builtin_amdgcn_sdot4((int)e2m1_x4(w.x), (int)x0.x, sd, false);
                    sd = __builtin_amdgcn_sdot4((int)e2m1_x4(w.y), (int)x0.y, sd, false);
                    sd = __builtin_amdgcn_sdot4((int)e2m1_x4(w.z), (int)x0.z, sd, false);
                    sd = __builtin_amdgcn_sdot4((int)e2m1_x4(w.w), (int)x0.w, sd, false);
                    sd = __builtin_amdgcn_sdot4((int)e2m1_x4(w.x >> 4), (int)x1.x, sd, false);
                    sd = __builtin_amdgcn_sdot4((int)e2m1_x4(w.y >> 4), (int)x1.y, sd, false);
                    sd = __builtin_amdgcn_sdot4((int)e2m1_x4(w.z >> 4), (int)x1.z, sd, false);
                    sd = __builtin_amdgcn_sdot4((int)e2m1_x4(w.w >> 4), (int)x1.w, sd, false);
                    const float term = __fmul_rn(__fmul_rn((float)sd, mxfp4_scale(sc[i][k])), xd[bc]);
                    if (b < nb) acc[i] = __fadd_rn(acc[i], term);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < RW; i++) {
            const float v = xsum32(acc[i]);
            if (hl == 0 && i0 + i < R) res[i0 + i] = v;
        }
    }
    __syncthreads();
    gemv_epilogue_t<EPI>(a, sl, t < R ? res[t] : 0.0f, bmax, pre);
}

#define MXQ8_KERNEL(E, EPI, KB, RW)                                                                    \
    extern "C" __global__ void __launch_bounds__(256) cj_gemv_mxq8_##E##_k##KB##_r##RW(cj_gemv_args a) {  \
        mxq8_body<EPI, KB, RW>(a);                                                                        \
    }
#define MXQ8_KBS(E, EPI, RW) \
    MXQ8_KERNEL(E, EPI, 1, RW) MXQ8_KERNEL(E, EPI, 2, RW) MXQ8_KERNEL(E, EPI, 3, RW) MXQ8_KERNEL(E, EPI, 4, RW)
MXQ8_KBS(s, CJ_EPI_STORE, 2)
MXQ8_KBS(s, CJ_EPI_STORE, 4)
MXQ8_KBS(a, CJ_EPI_ACCUM, 2)
MXQ8_KBS(a, CJ_EPI_ACCUM, 4)
MXQ8_KBS(g, CJ_EPI_GLU, 2)
MXQ8_KBS(g, CJ_EPI_GLU, 4)

// ------------------------------------------- MXFP4 experts grouped by expert

// The rows' selections by expert: a counter an expert in LDS, each selection
// appended to its expert's list (the order inside a list changes no result:
// every selection's products and epilogue are its own).
extern "C" __global__ void __launch_bounds__(256) cj_moe_group(cj_moe_group_args a) {
    __shared__ int c[256];
    const int t = threadIdx.x;
    for (int e = t; e < a.n_experts; e += 256) c[e] = 0;
    __syncthreads();
    for (int i = t; i < a.n_sel; i += 256) {
        const int e = a.sel[i];
        if (e >= 0 && e < a.n_experts) {
            const int p = atomicAdd(&c[e], 1);
            if (p < a.cap) a.mem[(int64_t)e * a.cap + p] = i;
        }
    }
    __syncthreads();
    for (int e = t; e < a.n_experts; e += 256) a.cnt[e] = min(c[e], a.cap);
}

#define GRP_CC 16   // member selections a column chunk
#define GRP_RS (GRP_CC + 1)

// Workgroup (row tile, expert e): the 64 rows run as four passes of 16 (a
// 32-lane half-wave two rows, as cj_gemv_mxq8_*; rows of at most 32·KB
// blocks, one sweep), the next pass's weights in flight during the current
// one's arithmetic. Each 32-block's E2M1 codes are
// decoded once and dotted with every member's q8 codes, so a member's row
// value is cj_gemv_mxq8_*'s bit for bit: acc = acc + (s·d_w)·d_x over the
// lane's blocks in order, the half-wave's xor butterfly. Members run in
// chunks of 16 (their codes staged in LDS); a chunk past the first re-reads
// the tile (L2). EPI: CJ_EPI_GLU — SiLU·up of each gate/up row pair, then
// the member's 32 activation values quantized per 32 (mxfp4QuantActKernel's
// arithmetic) into its pack; CJ_EPI_STORE — the row values.
template <int EPI, int KB, int GRT, int RW = 2, int CC = GRP_CC>
DEV void moe_grp_body(const cj_moe_grp_args &a) {
    constexpr int PASSES = GRT / (8 * RW), RS = CC + 1;
    static_assert(PASSES % 2 == 0, "an even number of passes");
    static_assert(EPI != CJ_EPI_GLU || GRT == 64, "the SiLU·up form: one 32-block of the activation a workgroup");
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int mi[CC];
    const int e = blockIdx.y;
    const int c = a.cnt[e];
    if (c == 0) return;
    const int t = threadIdx.x, hw = t >> 5, hl = t & 31;
    const int nb = (int)(a.cols / 32);
    const int cpad = (int)((a.cols + 15) & ~15), nbp = (nb + 3) & ~3;
    int8_t *xq = (int8_t *)smem;
    float *xd = (float *)(smem + CC * cpad);
    float *res = xd + CC * nbp;
    const uint8_t *W = a.w + (int64_t)e * a.expert_bytes;
    const int64_t row0 = (int64_t)blockIdx.x * GRT;

    auto fetch = [&](u32x4 (&wv)[RW][KB], uint32_t (&sc)[RW][KB], int p) {
#pragma unroll
        for (int i = 0; i < RW; i++) {
            const int64_t r = min(row0 + p * 8 * RW + hw * RW + i, a.rows - 1);
            const uint8_t *wr = W + r * a.row_bytes;
#pragma unroll
            for (int k = 0; k < KB; k++) {
                const int b = min(hl + 32 * k, nb - 1);
                wv[i][k] = __builtin_nontemporal_load((const u32x4 *)(wr + 16 * b));
                sc[i][k] = wr[16 * nb + b];
            }
        }
    };
    for (int j0 = 0; j0 < c; j0 += CC) {
        const int nc = min(CC, c - j0);
        __syncthreads();   // the previous chunk's LDS reads are done
        if (t < nc) mi[t] = a.mem[(int64_t)e * a.cap + j0 + t];
        __syncthreads();
        // the chunk's codes and scales: 32-block b of a pack row at
        // (b/8)·320 + (b%8)·32, its scale at (b/8)·320 + 288 + 4·(b%8)
        for (int idx = t; idx < nc * nb * 2; idx += 256) {
            const int jj = idx / (nb * 2), b = (idx % (nb * 2)) >> 1, h = idx & 1;
            const uint8_t *row = a.xp + (int64_t)(mi[jj] / a.x_per) * a.xp_stride + (b >> 3) * 320;
            *(u32x4 *)(xq + jj * cpad + 32 * b + 16 * h) = *(const u32x4 *)(row + (b & 7) * 32 + 16 * h);
            if (!h) xd[jj * nbp + b] = *(const float *)(row + 288 + 4 * (b & 7));
        }
        __syncthreads();

        // one pass: its blocks decoded once, then the members one at a time
        // (a member's two row values finish before the next member starts)
        auto compute = [&](const u32x4 (&wv)[RW][KB], const uint32_t (&sc)[RW][KB], int p) {
            int dw[RW][KB][8];
            float ws[RW][KB];
#pragma unroll
            for (int i = 0; i < RW; i++)
#pragma unroll
                for (int k = 0; k < KB; k++) {
                    const u32x4 w = wv[i][k];
                    dw[i][k][0] = (int)e2m1_x4(w.x); dw[i][k][1] = (int)e2m1_x4(w.y);
                    dw[i][k][2] = (int)e2m1_x4(w.z); dw[i][k][3] = (int)e2m1_x4(w.w);
                    dw[i][k][4] = (int)e2m1_x4(w.x >> 4); dw[i][k][5] = (int)e2m1_x4(w.y >> 4);
                    dw[i][k][6] = (int)e2m1_x4(w.z >> 4); dw[i][k][7] = (int)e2m1_x4(w.w >> 4);
                    ws[i][k] = mxfp4_scale(sc[i][k]);
                }
#pragma unroll 1
            for (int jj = 0; jj < nc; jj++) {
                float acc[RW];
#pragma unroll
                for (int i = 0; i < RW; i++) acc[i] = 0.0f;
#pragma unroll
                for (int k = 0; k < KB; k++) {
                    const int b = hl + 32 * k, bc = min(b, nb - 1);
                    const u32x4 x0 = *(const u32x4 *)(xq + jj * cpad + 32 * bc);
                    const u32x4 x1 = *(const u32x4 *)(xq + jj * cpad + 32 * bc + 16);
                    const float xs = xd[jj * nbp + bc];
#pragma unroll
                    for (int i = 0; i < RW; i++) {
                        int sd = 0;
                        sd = __builtin_amdgcn_sdot4(dw[i][k][0], (int)x0.x, sd, false);
                        sd = __builtin_amdgcn_sdot4(dw[i][k][1], (int)x0.y, sd, false);
                        sd = __builtin_amdgcn_sdot4(dw[i][k][2], (int)x0.z, sd, false);
                        sd = __builtin_amdgcn_sdot4(dw[i][k][3], (int)x0.w, sd, false);
                        sd = __builtin_amdgcn_sdot4(dw[i][k][4], (int)x1.x, sd, false);
                        sd = __builtin_amdgcn_sdot4(dw[i][k][5], (int)x1.y, sd, false);
                        sd = __builtin_amdgcn_sdot4(dw[i][k][6], (int)x1.z, sd, false);
                        sd = __builtin_amdgcn_sdot4(dw[i][k][7], (int)x1.w, sd, false);
                        const float term = __fmul_rn(__fmul_rn((float)sd, ws[i][k]), xs);
                        if (b < nb) acc[i] = __fadd_rn(acc[i], term);
                    }
                }
#pragma unroll
                for (int i = 0; i < RW; i++) {
                    const float v = xsum32(acc[i]);
                    if (hl == 0) res[(p * 8 * RW + hw * RW + i) * RS + jj] = v;
                }
            }
        };
        // two passes in flight: fetch 0 and 1, then compute one and fetch
        // the one two ahead
        u32x4 wa[RW][KB], wb[RW][KB];
        uint32_t sa[RW][KB], sb[RW][KB];
        fetch(wa, sa, 0);
        fetch(wb, sb, 1);
#pragma unroll
        for (int p = 0; p + 2 < PASSES; p += 2) {
            compute(wa, sa, p);
            fetch(wa, sa, p + 2);
            compute(wb, sb, p + 1);
            fetch(wb, sb, p + 3);
        }
        compute(wa, sa, PASSES - 2);
        compute(wb, sb, PASSES - 1);
        __syncthreads();

        if (EPI == CJ_EPI_GLU) {
            // output o (rows 2o, 2o+1) of member jj: thread t is (jj = t/32 + jb, o = t%32);
            // the 32 values of a member are one 32-block of its activation
            const int64_t ab = row0 / GRT;
#pragma unroll 1
            for (int jb = 0; jb < nc; jb += 8) {
                const int jj = jb + (t >> 5), o = t & 31;
                const bool on = jj < nc;
                const int64_t ai = row0 / 2 + o;
                float v = 0.0f;
                if (on && ai < a.act_n) v = glu_value(a.glu_form, ai, a.act_n, res[(2 * o) * RS + jj], res[(2 * o + 1) * RS + jj]);
                const float bm = xmax32(fabsf(v));
                const float inv = bm > 0.0f ? __fdiv_rn(127.0f, bm) : 0.0f;
                const int q = round_away(__fmul_rn(v, inv));
                const int sq = xsum32_i(q);
                if (on) {
                    uint8_t *ob = a.outp + (int64_t)mi[jj] * a.outp_stride + (ab >> 3) * 320;
                    ob[(ab & 7) * 32 + o] = (uint8_t)(int8_t)q;
                    if (o == 0) {
                        *(int32_t *)(ob + 256 + 4 * (ab & 7)) = sq;
                        *(float *)(ob + 288 + 4 * (ab & 7)) = __fdiv_rn(bm, 127.0f);
                    }
                }
            }
        } else {
            for (int idx = t; idx < nc * GRT; idx += 256) {
                const int jj = idx / GRT, rl = idx % GRT;
                const int64_t r = row0 + rl;
                if (r < a.rows) a.y[(int64_t)mi[jj] * a.y_stride + r] = res[rl * RS + jj];
            }
        }
    }
}

#define MOE_GRP_KERNEL(E, EPI, KB, GRT)                                                                      \
    extern "C" __global__ void __launch_bounds__(256) cj_moe_mxq8_##E##_k##KB##_t##GRT(cj_moe_grp_args a) {  \
        moe_grp_body<EPI, KB, GRT>(a);                                                                       \
    }
// one row a half-wave a pass and members in chunks of CC (fewer registers and
// less LDS: more workgroups a CU when each expert has few rows)
#define MOE_GRP_KERNEL_RC(E, EPI, KB, GRT, RW, CC)                                                             \
    extern "C" __global__ void __launch_bounds__(256)                                                          \
        cj_moe_mxq8_##E##_k##KB##_t##GRT##_r##RW##_c##CC(cj_moe_grp_args a) {                                  \
        moe_grp_body<EPI, KB, GRT, RW, CC>(a);                                                                 \
    }
MOE_GRP_KERNEL_RC(g, CJ_EPI_GLU, 3, 64, 1, 4)
MOE_GRP_KERNEL_RC(g, CJ_EPI_GLU, 3, 64, 2, 4)
MOE_GRP_KERNEL_RC(s, CJ_EPI_STORE, 3, 32, 1, 4)
MOE_GRP_KERNEL_RC(s, CJ_EPI_STORE, 3, 32, 2, 4)
#define MOE_GRP_KBS(E, EPI, GRT) \
    MOE_GRP_KERNEL(E, EPI, 1, GRT) MOE_GRP_KERNEL(E, EPI, 2, GRT) MOE_GRP_KERNEL(E, EPI, 3, GRT) MOE_GRP_KERNEL(E, EPI, 4, GRT)
MOE_GRP_KBS(g, CJ_EPI_GLU, 64)
MOE_GRP_KBS(s, CJ_EPI_STORE, 32)
MOE_GRP_KBS(s, CJ_EPI_STORE, 64)

GEMV_FAMILY(cj_gemv_q6k, CJ_Q6_K, 2)
GEMV_FAMILY(cj_gemv_q80, CJ_Q8_0, 4)
GEMV_FAMILY_N2(cj_gemv_q80, CJ_Q8_0)
GEMV_KERNEL_S(cj_gemv_q6k_l64_s, CJ_Q6_K, 2)
// cj_gemv_q40b_r<RW>: Q4_0 block-parallel, RW rows a wave (4·RW a workgroup)
extern "C" __global__ void __launch_bounds__(256) cj_gemv_q40b_r2(cj_gemv_args a) { q40_gemv<2>(a); }
extern "C" __global__ void __launch_bounds__(256) cj_gemv_q40b_r4(cj_gemv_args a) { q40_gemv<4>(a); }
GEMV_KERNEL(cj_gemv_mxfp4, CJ_MXFP4, 64, 1)
GEMV_KERNEL(cj_gemv_f32, CJ_F32, 64, 1)
GEMV_KERNEL(cj_gemv_mxfp4_r32, CJ_MXFP4, 32, 1)
GEMV_KERNEL(cj_gemv_f32_r32, CJ_F32, 32, 1)
GEMV_KERNEL(cj_gemv_mxfp4_r1, CJ_MXFP4, 1, 1)
GEMV_KERNEL(cj_gemv_f32_r1, CJ_F32, 1, 1)
