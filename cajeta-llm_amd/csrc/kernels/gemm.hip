// gemm.hip — the batched ("Cols") quantised mat-mat for gfx950: Y[c] = W·x_c
// for many activation columns at once (batched decode over sequences, a
// prefill chunk over tokens), on the int8 matrix cores.
//
// Every column is computed exactly as the one-column GEMV computes it (the
// reference's many-row CPU kernels equal the one-row kernel column by
// column, selftest/CpuInt8MatVecTest.cajeta:225-300): the integer dot of each
// 32-element sub-block comes from one v_mfma_i32_16x16x32_i8 with a zeroed
// accumulator (an exact int32 sum, in any order), and the f32 arithmetic that
// follows — block scales, mins and the fold over blocks — runs per (row,
// column) in the reference's order:
//   Q8_0 : fs = Σ_j (d_j·xs_j)·isum_j over the 8 blocks of each 256, acc += fs
//          (Quant.q80MatVecIntoQ8Sub, io/Quant.cajeta:3079-3110)
//   Q4_K : sumi = Σ_s sc_s·dot_s, dmins = Σ_s mn_s·bsum_s (ints);
//          acc = (acc + (d·xs)·sumi) − (dmin·xs)·dmins per block
//          (Quant.q4kMatVecIntoQ8, io/Quant.cajeta:3374-3445)
// Those per-output f32 steps (four VALU operations per output and 32-block
// for Q8_0) bound the kernel at large column counts, not the matrix cores.
//
// MFMA 16x16x32 int8 lane layout (checked on the part): lane l supplies A row
// l % 16 and B column l % 16, elements k = 8·(l / 16) .. +7, and receives
// D[4·(l / 16) + i][l % 16], i < 4.
//
// Tiling: a workgroup of 4 waves owns 64 weight rows (16 a wave) × 16·NT
// columns. The K dimension runs in groups of 256 elements (8 Q8_0 blocks, one
// Q4_K block). Each group's activation packs (the 320-byte block of every
// column of the tile, verbatim) are staged in LDS once for the 4 waves; the
// weights are staged in LDS too for Q8_0 and stream straight into registers
// for Q4_K. Both are requested one group ahead, so the loads of group g+1 are
// in flight while group g computes. Column tiles of one row block are
// adjacent in dispatch order and share the rows' weights in cache.
#include "common.h"

typedef int v4i __attribute__((ext_vector_type(4)));

DEV v4i mfma_i8(long a, long b) {
    const v4i z = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, z, 0, 0, 0);
}

DEV long ld8(const uint8_t *p) { return *(const long *)p; }

// K loops run every group but the last with an unconditional prefetch of the
// next, then the last without one: a load under a branch would make the
// compiler wait at the join for every load in flight (the prefetch
// included), and a prefetch in the last group would only re-read data and
// delay the end. PF<true> / PF<false> pick the form at compile time.
template <bool B>
struct PF {
    static constexpr bool on = B;
};

#define GEMM_CS 336   // LDS bytes a staged column (the 320-byte block, padded against bank conflicts)

// The group's activation blocks of the tile's columns into registers (NV
// 16-byte words a thread), then into LDS: word w of column c at c·GEMM_CS + 16w.
template <int NT>
struct BStage {
    static constexpr int CT = 16 * NT, WORDS = CT * 20, NV = (WORDS + 255) / 256;
    u32x4 v[NV];
};

template <int NT>
DEV void b_fetch(BStage<NT> &s, const cj_gemv_args &a, int64_t c0, int64_t g) {
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < BStage<NT>::NV; i++) {
        const int w = min(t + 256 * i, BStage<NT>::WORDS - 1);
        const int64_t c = min(c0 + w / 20, (int64_t)a.batch - 1);
        s.v[i] = *(const u32x4 *)(a.xp + c * a.xp_stride + g * 320 + 16 * (w % 20));
    }
}

template <int NT>
DEV void b_store(const BStage<NT> &s, uint8_t *lds) {
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < BStage<NT>::NV; i++) {
        const int w = t + 256 * i;
        if (w < BStage<NT>::WORDS) *(u32x4 *)(lds + (w / 20) * GEMM_CS + 16 * (w % 20)) = s.v[i];
    }
}

// ------------------------------------------------------------------- Q8_0

// Prepared row: [qs nb32·32][d nb32·2 → padded to 16]. A group of 8 blocks
// is 256 code bytes and one 16-byte scale word a row (the scale array is
// padded to 16 bytes, so a short last group stays inside it).

// Q8_0, tiled: a group's 64 weight rows × (256 code bytes + 16 scale bytes)
// are staged in LDS beside the columns' pack blocks, as 1088 16-byte words
// loaded coalesced one group ahead (per-lane 8-byte row loads straight into
// registers queued on the address unit: 32 columns 55.6 → 42.5 µs at
// 28672×4096, a 512-row prefill chunk 30.4 → 27.6 ms), and read back as the
// MFMA operands. Row stride 264 bytes: 16 consecutive lanes' 8-byte reads
// of 16 rows fall on distinct banks. Per 32-element block and output the f32
// steps are the reference's, fs = Σ_j (d_j·xs_j)·isum_j over the group's 8
// blocks (the first nj of a short last group), then acc += fs.
#define GEMM_AS 264
#define GEMM_AW 1088     // staged words a group: 64 rows × 16 code words + 64 scale words

template <int NT, bool FULL>
DEV void q80_tile_group(const uint8_t *aq, const uint8_t *ad, const uint8_t *lds, int q, int m, int nj,
                          float (&acc)[NT][4]) {
    float dr[4][8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint4 dw = *(const uint4 *)(ad + (4 * q + i) * 16);
        const uint32_t hw[4] = {dw.x, dw.y, dw.z, dw.w};
#pragma unroll
        for (int j = 0; j < 8; j++) dr[i][j] = h2f(hw[j >> 1] >> (16 * (j & 1)));
    }
    long aw[8];
#pragma unroll
    for (int j = 0; j < 8; j++) aw[j] = *(const long *)(aq + m * GEMM_AS + 32 * j + 8 * q);
#pragma unroll
    for (int n = 0; n < NT; n++) {
        const uint8_t *col = lds + (16 * n + m) * GEMM_CS;
        const float4 x0 = *(const float4 *)(col + 288), x1 = *(const float4 *)(col + 304);
        const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        long bq[8];
#pragma unroll
        for (int j = 0; j < 8; j++) bq[j] = *(const long *)(col + 32 * j + 8 * q);
        v4i d[8];
#pragma unroll
        for (int j = 0; j < 8; j++) d[j] = mfma_i8(aw[j], bq[j]);
        float fs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            if (FULL || j < nj) {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    fs[i] = __fadd_rn(fs[i], __fmul_rn(__fmul_rn(dr[i][j], xs[j]), (float)d[j][i]));
            }
        }
#pragma unroll
        for (int i = 0; i < 4; i++) acc[n][i] = __fadd_rn(acc[n][i], fs[i]);
    }
}

template <int NT>
DEV void gemm_q80(const cj_gemv_args &a, uint8_t *lds) {
    constexpr int NV = BStage<NT>::NV, AV = (GEMM_AW + 255) / 256;
    __shared__ __align__(16) uint8_t aq[64 * GEMM_AS];
    __shared__ __align__(16) uint8_t ad[64 * 16];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, q = lane >> 4, m = lane & 15;
    const int64_t c0 = (int64_t)blockIdx.x * 16 * NT;
    const int64_t rw0 = (int64_t)blockIdx.y * 64, r0 = rw0 + 16 * wave;
    const int64_t nb32 = a.cols / 32, ngrp = (a.cols + 255) / 256;
    const uint8_t *bsrc[NV];
    int bdst[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) {
        const int w = min(t + 256 * i, BStage<NT>::WORDS - 1);
        bsrc[i] = a.xp + min(c0 + w / 20, (int64_t)a.batch - 1) * a.xp_stride + 16 * (w % 20);
        bdst[i] = t + 256 * i < BStage<NT>::WORDS ? (w / 20) * GEMM_CS + 16 * (w % 20) : -1;
    }
    // this thread's weight words: row base and word of the group
    const uint8_t *arow[AV];
    int aword[AV];
#pragma unroll
    for (int i = 0; i < AV; i++) {
        const int idx = min(t + 256 * i, GEMM_AW - 1);
        const int row = idx < 1024 ? idx >> 4 : idx - 1024;
        arow[i] = a.w + min(rw0 + row, a.rows - 1) * a.row_bytes;
        aword[i] = idx;
    }
    float acc[NT][4];
#pragma unroll
    for (int n = 0; n < NT; n++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[n][i] = 0.0f;
    u32x4 bv[NV], av[AV];
    auto fetch = [&](int64_t g) {
#pragma unroll
        for (int i = 0; i < NV; i++) bv[i] = *(const u32x4 *)(bsrc[i] + g * 320);
#pragma unroll
        for (int i = 0; i < AV; i++) {
            const int idx = aword[i];
            if (idx < 1024) {   // code word: block 8g + w/2 (the last block repeats past the row)
                const int w16 = idx & 15;
                const int64_t blk = min(8 * g + (w16 >> 1), nb32 - 1);
                av[i] = *(const u32x4 *)(arow[i] + blk * 32 + 16 * (w16 & 1));
            } else {            // the row's 8 block scales of the group (the scale array is padded to 16)
                av[i] = *(const u32x4 *)(arow[i] + nb32 * 32 + 16 * g);
            }
        }
    };
    auto stage = [&]() {
#pragma unroll
        for (int i = 0; i < NV; i++)
            if (bdst[i] >= 0) *(u32x4 *)(lds + bdst[i]) = bv[i];
#pragma unroll
        for (int i = 0; i < AV; i++) {
            const int idx = t + 256 * i;
            if (idx < 1024) {
                uint8_t *dst = aq + (idx >> 4) * GEMM_AS + 16 * (idx & 15);
                *(uint2 *)dst = make_uint2(av[i].x, av[i].y);
                *(uint2 *)(dst + 8) = make_uint2(av[i].z, av[i].w);
            } else if (idx < GEMM_AW) {
                *(u32x4 *)(ad + (idx - 1024) * 16) = av[i];
            }
        }
    };
    fetch(0);
    auto group = [&](int64_t g, auto pf) {
        __syncthreads();   // the previous group's LDS reads are done
        stage();
        __syncthreads();
        if constexpr (decltype(pf)::on) fetch(g + 1);
        const int nj = (int)min((int64_t)8, nb32 - 8 * g);
        const uint8_t *aqw = aq + 16 * wave * GEMM_AS, *adw = ad + 16 * wave * 16;
        if (nj == 8) q80_tile_group<NT, true>(aqw, adw, lds, q, m, 8, acc);
        else q80_tile_group<NT, false>(aqw, adw, lds, q, m, nj, acc);
    };
    for (int64_t g = 0; g + 1 < ngrp; g++) group(g, PF<true>{});
    group(ngrp - 1, PF<false>{});
#pragma unroll
    for (int n = 0; n < NT; n++) {
        const int64_t c = c0 + 16 * n + m;
        if (c >= a.batch) continue;
        float *y = a.y + c * a.y_stride + a.y_off;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int64_t r = r0 + 4 * q + i;
            if (r < a.rows) y[r] = a.epi == CJ_EPI_ACCUM ? __fadd_rn(y[r], acc[n][i]) : acc[n][i];
        }
    }
}

// ------------------------------------------------------------------- Q4_K

// The GEMV's chunk-major prepared row: qs piece c (16 bytes) of block b at
// (c·nb + b)·16, the 16-byte header {d, dmin, scales[12]} at 128·nb + 16·b.
// Group g4 (elements 64·g4 .. +63) of a block is qs bytes 32·g4 .. +31: low
// nibbles are sub-block 2·g4, high nibbles 2·g4 + 1, so one 8-byte load
// (bytes 32·g4 + 8q ..) feeds both sub-blocks' MFMAs.
struct Q4kA {
    long q[4];
    uint4 h[4];
};

DEV void q4k_fetch_a(Q4kA &A, const uint8_t *wa, const uint8_t *const (&wh)[4], int64_t nb, int64_t b, int q) {
#pragma unroll
    for (int g4 = 0; g4 < 4; g4++) {
        const int byte = 32 * g4 + 8 * q;
        A.q[g4] = ld8(wa + ((int64_t)(byte >> 4) * nb + b) * 16 + (byte & 15));
    }
#pragma unroll
    for (int i = 0; i < 4; i++) A.h[i] = *(const uint4 *)(wh[i] + b * 16);
}

template <int NT>
DEV void gemm_q4k(const cj_gemv_args &a, uint8_t *lds) {
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, q = lane >> 4, m = lane & 15;
    const int64_t c0 = (int64_t)blockIdx.x * 16 * NT;
    const int64_t r0 = (int64_t)blockIdx.y * 64 + 16 * wave;
    const int64_t nb = a.cols / 256;
    const uint8_t *wa = a.w + min(r0 + m, a.rows - 1) * a.row_bytes;
    const uint8_t *wh[4];
#pragma unroll
    for (int i = 0; i < 4; i++) wh[i] = a.w + min(r0 + 4 * q + i, a.rows - 1) * a.row_bytes + nb * 128;
    const uint8_t *bsrc[BStage<NT>::NV];
    int bdst[BStage<NT>::NV];
#pragma unroll
    for (int i = 0; i < BStage<NT>::NV; i++) {
        const int w = min(t + 256 * i, BStage<NT>::WORDS - 1);
        bsrc[i] = a.xp + min(c0 + w / 20, (int64_t)a.batch - 1) * a.xp_stride + 16 * (w % 20);
        bdst[i] = t + 256 * i < BStage<NT>::WORDS ? (w / 20) * GEMM_CS + 16 * (w % 20) : -1;
    }
    const uint64_t M = 0x0F0F0F0F0F0F0F0Full;
    float acc[NT][4];
#pragma unroll
    for (int n = 0; n < NT; n++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[n][i] = 0.0f;
    u32x4 bv[BStage<NT>::NV];
    Q4kA A, An;
#pragma unroll
    for (int i = 0; i < BStage<NT>::NV; i++) bv[i] = *(const u32x4 *)bsrc[i];
    q4k_fetch_a(A, wa, wh, nb, 0, q);
    auto block = [&](int64_t b, auto pf) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < BStage<NT>::NV; i++)
            if (bdst[i] >= 0) *(u32x4 *)(lds + bdst[i]) = bv[i];
        __syncthreads();
        if constexpr (decltype(pf)::on) {
#pragma unroll
            for (int i = 0; i < BStage<NT>::NV; i++) bv[i] = *(const u32x4 *)(bsrc[i] + (b + 1) * 320);
            q4k_fetch_a(An, wa, wh, nb, b + 1, q);
        }
        // the 4 rows' 6-bit scales and mins, and their block scales
        int sc[4][8], mn[4][8];
        float dd[4], dm[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t X = A.h[i].y, Y = A.h[i].z, Z = A.h[i].w;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t a8 = (X >> (8 * j)) & 255, b8 = (Y >> (8 * j)) & 255, c8 = (Z >> (8 * j)) & 255;
                sc[i][j] = (int)(a8 & 63);
                mn[i][j] = (int)(b8 & 63);
                sc[i][j + 4] = (int)((c8 & 15) | ((a8 >> 2) & 48));
                mn[i][j + 4] = (int)((c8 >> 4) | ((b8 >> 2) & 48));
            }
            dd[i] = h2f(A.h[i].x);
            dm[i] = h2f(A.h[i].x >> 16);
        }
        long lo[4], hi[4];
#pragma unroll
        for (int g4 = 0; g4 < 4; g4++) {
            const uint64_t w = (uint64_t)A.q[g4];
            lo[g4] = (long)(w & M);
            hi[g4] = (long)((w >> 4) & M);
        }
#pragma unroll
        for (int n = 0; n < NT; n++) {
            const uint8_t *col = lds + (16 * n + m) * GEMM_CS;
            // the tile's 8 operand reads and 8 products back to back, then the
            // exact integer sums (any order) and the f32 steps
            long bl[4], bh[4];
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                bl[g4] = *(const long *)(col + 64 * g4 + 8 * q);
                bh[g4] = *(const long *)(col + 64 * g4 + 32 + 8 * q);
            }
            v4i dl[4], dh[4];
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                dl[g4] = mfma_i8(lo[g4], bl[g4]);
                dh[g4] = mfma_i8(hi[g4], bh[g4]);
            }
            const int4 s0 = *(const int4 *)(col + 256), s1 = *(const int4 *)(col + 272);
            const float xs = *(const float *)(col + 288);
            const int bsum[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                int sumi = 0, dmins = 0;
#pragma unroll
                for (int g4 = 0; g4 < 4; g4++)
                    sumi += __mul24(dl[g4][i], sc[i][2 * g4]) + __mul24(dh[g4][i], sc[i][2 * g4 + 1]);
#pragma unroll
                for (int s2 = 0; s2 < 8; s2++) dmins += __mul24(bsum[s2], mn[i][s2]);
                acc[n][i] = __fsub_rn(__fadd_rn(acc[n][i], __fmul_rn(__fmul_rn(dd[i], xs), (float)sumi)),
                                      __fmul_rn(__fmul_rn(dm[i], xs), (float)dmins));
            }
        }
        if constexpr (decltype(pf)::on) A = An;
    };
    for (int64_t b = 0; b + 1 < nb; b++) block(b, PF<true>{});
    block(nb - 1, PF<false>{});
#pragma unroll
    for (int n = 0; n < NT; n++) {
        const int64_t c = c0 + 16 * n + m;
        if (c >= a.batch) continue;
        float *y = a.y + c * a.y_stride + a.y_off;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int64_t r = r0 + 4 * q + i;
            if (r < a.rows) y[r] = a.epi == CJ_EPI_ACCUM ? __fadd_rn(y[r], acc[n][i]) : acc[n][i];
        }
    }
}

// ----------------------------------------------- few columns: split K

// For a handful of columns (batched decode) the weights dominate and the
// output tile is small, so the K dimension is shared out: a workgroup of W
// waves owns 16 rows × 16·NT columns, wave w takes the groups g ≡ w (mod W),
// streaming its weights straight into registers one group ahead, and hands
// each group's per-output terms to wave 0, which folds them into the
// accumulators in group order (the reference's order, exactly) through LDS,
// W groups a round. The columns' pack blocks reach the waves through LDS: a
// round's blocks are staged by coalesced 16-byte loads a round ahead (the
// per-lane 8-byte loads they replace kept the address unit 63% busy).
//   Q8_0: the group's fs (one value an output);
//   Q4_K: the block's (d·xs)·sumi and (dmin·xs)·dmins (two values an output).

// One K-group of the split-K Q8_0 kernel: the f32 terms of the 8 blocks
// (FULL: all 8 exist), from the wave's staged weights (codes of row r at
// r·GEMM_AS, the rows' scale words after them) and the round's column blocks.
template <int NT, bool FULL>
DEV void q80_sk_group(const uint8_t *aq, const uint8_t *slot, int q, int m, int nj, float (&fs)[NT][4]) {
    const uint8_t *ad = aq + 16 * GEMM_AS;
    uint32_t hw[4][4];   // the f16 scales of rows 4q + i, two a word
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint4 dw = *(const uint4 *)(ad + (4 * q + i) * 16);
        hw[i][0] = dw.x; hw[i][1] = dw.y; hw[i][2] = dw.z; hw[i][3] = dw.w;
    }
    long aw[8];
#pragma unroll
    for (int j = 0; j < 8; j++) aw[j] = *(const long *)(aq + m * GEMM_AS + 32 * j + 8 * q);
#pragma unroll
    for (int n = 0; n < NT; n++) {
        // the tile's column blocks from the round's LDS stage (column c's
        // 320-byte block at c·GEMM_CS of the wave's slot)
        const uint8_t *col = slot + (16 * n + m) * GEMM_CS;
        const float4 x0 = *(const float4 *)(col + 288), x1 = *(const float4 *)(col + 304);
        const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        long bq[8];
#pragma unroll
        for (int j = 0; j < 8; j++) bq[j] = *(const long *)(col + 32 * j + 8 * q);
        v4i d[8];
#pragma unroll
        for (int j = 0; j < 8; j++) d[j] = mfma_i8(aw[j], bq[j]);
#pragma unroll
        for (int i = 0; i < 4; i++) fs[n][i] = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            if (FULL || j < nj) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    // d_j·xs_j: the f16 scale times xs in one rounding (v_fma_mix with a −0 addend)
                    const float dx = (j & 1) ? mul_h16hi(hw[i][j >> 1], xs[j]) : mul_h16lo(hw[i][j >> 1], xs[j]);
                    fs[n][i] = __fadd_rn(fs[n][i], __fmul_rn(dx, (float)d[j][i]));
                }
            }
        }
    }
}

// A wave's weights of one group — 16 rows × 16 code words + 16 scale words —
// as 5 coalesced 16-byte words a lane: code word i (< 4) is word lane % 16 of
// row 4i + lane / 16 (block 8g + word/2; a short last group repeats the
// row's last block), word 4 is row lane % 16's scale word (lanes 16.. repeat
// lanes 0..15). Staged in the wave's own LDS slot (GEMM_AS-byte rows).
#define SK_AS (16 * GEMM_AS + 256)   // LDS bytes a wave's staged group

DEV void sk_a_load(u32x4 (&v)[5], const uint8_t *const (&arow)[4], const uint8_t *srow, int64_t g, int64_t nb32,
                   int lane) {
    const int w16 = lane & 15;
    const int64_t blk = min(8 * g + (w16 >> 1), nb32 - 1);
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = *(const u32x4 *)(arow[i] + blk * 32 + 16 * (w16 & 1));
    v[4] = *(const u32x4 *)(srow + 16 * g);
}

DEV void sk_a_store(const u32x4 (&v)[5], uint8_t *al, int lane) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint8_t *dst = al + (4 * i + (lane >> 4)) * GEMM_AS + 16 * (lane & 15);
        *(uint2 *)dst = make_uint2(v[i].x, v[i].y);
        *(uint2 *)(dst + 8) = make_uint2(v[i].z, v[i].w);
    }
    if (lane < 16) *(u32x4 *)(al + 16 * GEMM_AS + 16 * lane) = v[4];
}

// A wave's share of the pack blocks: the 16·NT columns' 320-byte blocks of
// its own group, 20·16·NT words, as 5·NT coalesced 16-byte words a lane —
// word i = 5n + k is word (lane + 64k) of column tile n: column
// (lane + 64k) / 20, word (lane + 64k) % 20 — staged in the wave's own LDS
// slot (column c at c·GEMM_CS). The offsets are worked out once.
template <int NT>
struct SkB {
    uint32_t off[5 * NT];   // bytes from the group's block of column c0
    uint32_t dst[5];        // slot offsets in column tile 0
    DEV void init(const cj_gemv_args &a, int64_t c0, int lane) {
#pragma unroll
        for (int k = 0; k < 5; k++) {
            const int idx = lane + 64 * k, col = idx / 20, word = idx % 20;
            dst[k] = col * GEMM_CS + 16 * word;
#pragma unroll
            for (int n = 0; n < NT; n++) {
                const int64_t c = min(c0 + col + 16 * n, (int64_t)a.batch - 1);
                off[5 * n + k] = (uint32_t)((c - c0) * a.xp_stride + 16 * word);
            }
        }
    }
    DEV void load(u32x4 (&v)[5 * NT], const uint8_t *base) const {
#pragma unroll
        for (int i = 0; i < 5 * NT; i++) v[i] = *(const u32x4 *)(base + off[i]);
    }
    DEV void store(const u32x4 (&v)[5 * NT], uint8_t *slot) const {
#pragma unroll
        for (int n = 0; n < NT; n++)
#pragma unroll
            for (int k = 0; k < 5; k++) *(u32x4 *)(slot + 16 * n * GEMM_CS + dst[k]) = v[5 * n + k];
    }
};

// Split-K Q8_0: every wave stages its own group's weights and column blocks
// (no workgroup barrier between the staging and the reads: a wave's LDS
// operations complete in order), so a round needs one barrier, for the
// hand-off of the terms. The fold is shared out: output slot v = 4n + i of
// every lane (column 16n + m, row 4q + i) belongs to wave v, which adds the
// round's terms of the waves in group order; the hand-off buffer alternates
// by round (buffer rd & 1 is rewritten two rounds on, after the next
// barrier, which a wave reaches only once it has folded round rd).
template <int NT, int W>
DEV void gemm_sk_q80(const cj_gemv_args &a) {
    static_assert(NT * 4 <= W, "an output slot a wave");
    constexpr int BS = 16 * NT * GEMM_CS;   // a wave's column-block slot
    __shared__ __align__(16) float hand[2][W][NT * 4][64];
    __shared__ __align__(16) uint8_t bl[W * BS];
    __shared__ __align__(16) uint8_t al[W * SK_AS];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, q = lane >> 4, m = lane & 15;
    const int64_t c0 = (int64_t)blockIdx.x * 16 * NT, r0 = (int64_t)blockIdx.y * 16;
    const int64_t nb32 = a.cols / 32, ngrp = (a.cols + 255) / 256;
    const uint8_t *arow[4];
#pragma unroll
    for (int i = 0; i < 4; i++) arow[i] = a.w + min(r0 + 4 * i + q, a.rows - 1) * a.row_bytes;
    const uint8_t *srow = a.w + min(r0 + m, a.rows - 1) * a.row_bytes + nb32 * 32;
    const uint8_t *xb = a.xp + c0 * a.xp_stride;
    uint8_t *bw = bl + wave * BS, *aw = al + wave * SK_AS;
    float acc = 0.0f;   // output slot `wave` of this lane (waves past NT·4 hold none)
    SkB<NT> B;
    B.init(a, c0, lane);
    u32x4 bv[5 * NT], av[5];
    {
        const int64_t g0 = min((int64_t)wave, ngrp - 1);
        B.load(bv, xb + g0 * 320);
        sk_a_load(av, arow, srow, g0, nb32, lane);
        B.store(bv, bw);
        sk_a_store(av, aw, lane);
    }
    const int64_t rounds = (ngrp + W - 1) / W;
    auto round = [&](int64_t rd, auto pf) {
        const int64_t g = rd * W + wave;
        if constexpr (decltype(pf)::on) {
            // the wave's next group (clamped: past the end it re-reads the
            // last), before the branch below
            const int64_t gn = min(g + W, ngrp - 1);
            B.load(bv, xb + gn * 320);
            sk_a_load(av, arow, srow, gn, nb32, lane);
        }
        if (g < ngrp) {
            float fs[NT][4];
            const int nj = (int)min((int64_t)8, nb32 - 8 * g);
            if (nj == 8) q80_sk_group<NT, true>(aw, bw, q, m, 8, fs);
            else q80_sk_group<NT, false>(aw, bw, q, m, nj, fs);
#pragma unroll
            for (int n = 0; n < NT; n++)
#pragma unroll
                for (int i = 0; i < 4; i++) hand[rd & 1][wave][4 * n + i][lane] = fs[n][i];
        }
        if constexpr (decltype(pf)::on) {   // the wave's own slots: its reads above come first
            B.store(bv, bw);
            sk_a_store(av, aw, lane);
        }
        __syncthreads();   // round rd's terms are handed
        if (wave < NT * 4) {
            const int live = (int)min((int64_t)W, ngrp - rd * W);
            for (int w = 0; w < live; w++) acc = __fadd_rn(acc, hand[rd & 1][w][wave][lane]);
        }
    };
    for (int64_t rd = 0; rd + 1 < rounds; rd++) round(rd, PF<true>{});
    round(rounds - 1, PF<false>{});
    if (wave >= NT * 4) return;
    const int n = wave >> 2, i = wave & 3;
    const int64_t c = c0 + 16 * n + m, r = r0 + 4 * q + i;
    if (c < a.batch && r < a.rows) {
        float *y = a.y + c * a.y_stride + a.y_off + r;
        *y = a.epi == CJ_EPI_ACCUM ? __fadd_rn(*y, acc) : acc;
    }
}

// Split-K Q4_K, staged and folded as the Q8_0 form. A wave's weights of one
// block: 16 rows × (8 code chunks + the header), 144 16-byte words, as 3
// words a lane — word idx = lane + 64k: code chunk idx % 8 of row idx / 8
// (idx < 128), the header of row idx − 128 (idx < 144) — staged as rows of
// Q4S bytes (the row's 128 code bytes in order) and the 16 headers after.
#define Q4S 136
#define SK4_AS (16 * Q4S + 256)

DEV void q4k_sk_group(const uint8_t *aq, const uint8_t *col, int q, int m, float (&t1)[4], float (&t2)[4]) {
    const uint64_t M = 0x0F0F0F0F0F0F0F0Full;
    int sc[4][8], mn[4][8];
    float dd[4], dm[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint4 h = *(const uint4 *)(aq + 16 * Q4S + (4 * q + i) * 16);
        const uint32_t X = h.y, Y = h.z, Z = h.w;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t a8 = (X >> (8 * j)) & 255, b8 = (Y >> (8 * j)) & 255, c8 = (Z >> (8 * j)) & 255;
            sc[i][j] = (int)(a8 & 63);
            mn[i][j] = (int)(b8 & 63);
            sc[i][j + 4] = (int)((c8 & 15) | ((a8 >> 2) & 48));
            mn[i][j + 4] = (int)((c8 >> 4) | ((b8 >> 2) & 48));
        }
        dd[i] = h2f(h.x);
        dm[i] = h2f(h.x >> 16);
    }
    long lo[4], hi[4], bl8[4], bh8[4];
#pragma unroll
    for (int g4 = 0; g4 < 4; g4++) {
        const uint64_t w = *(const uint64_t *)(aq + m * Q4S + 32 * g4 + 8 * q);
        lo[g4] = (long)(w & M);
        hi[g4] = (long)((w >> 4) & M);
        bl8[g4] = *(const long *)(col + 64 * g4 + 8 * q);
        bh8[g4] = *(const long *)(col + 64 * g4 + 32 + 8 * q);
    }
    const int4 s0 = *(const int4 *)(col + 256), s1 = *(const int4 *)(col + 272);
    const float xs = *(const float *)(col + 288);
    // Σ_s sc_s·dot_s and Σ_s mn_s·bsum_s are exact int32 sums: any order
    v4i dl[4], dh[4];
#pragma unroll
    for (int g4 = 0; g4 < 4; g4++) {
        dl[g4] = mfma_i8(lo[g4], bl8[g4]);
        dh[g4] = mfma_i8(hi[g4], bh8[g4]);
    }
    int sumi[4] = {0, 0, 0, 0};
#pragma unroll
    for (int g4 = 0; g4 < 4; g4++)
#pragma unroll
        for (int i = 0; i < 4; i++)
            sumi[i] += __mul24(dl[g4][i], sc[i][2 * g4]) + __mul24(dh[g4][i], sc[i][2 * g4 + 1]);
    const int bsum[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        int dmins = 0;
#pragma unroll
        for (int s2 = 0; s2 < 8; s2++) dmins += __mul24(bsum[s2], mn[i][s2]);
        t1[i] = __fmul_rn(__fmul_rn(dd[i], xs), (float)sumi[i]);
        t2[i] = __fmul_rn(__fmul_rn(dm[i], xs), (float)dmins);
    }
}

template <int NT, int W>
DEV void gemm_sk_q4k(const cj_gemv_args &a) {
    static_assert(NT * 4 <= W, "an output slot a wave");
    constexpr int BS = 16 * NT * GEMM_CS;
    __shared__ __align__(16) float hand[2][W][NT * 4][2][64];
    __shared__ __align__(16) uint8_t bl[W * BS];
    __shared__ __align__(16) uint8_t al[W * SK4_AS];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, q = lane >> 4, m = lane & 15;
    const int64_t c0 = (int64_t)blockIdx.x * 16 * NT, r0 = (int64_t)blockIdx.y * 16;
    const int64_t nb = a.cols / 256;
    // this lane's three weight words: code chunks of rows lane/8 and 8 + lane/8,
    // the header of row lane % 16 (lanes 16.. repeat it)
    const uint8_t *ap[3];
    int adst[2];
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int row = 8 * k + (lane >> 3), chunk = lane & 7;
        ap[k] = a.w + min(r0 + row, a.rows - 1) * a.row_bytes + (int64_t)chunk * nb * 16;
        adst[k] = row * Q4S + 16 * chunk;
    }
    ap[2] = a.w + min(r0 + m, a.rows - 1) * a.row_bytes + nb * 128;
    const uint8_t *xb = a.xp + c0 * a.xp_stride;
    uint8_t *bw = bl + wave * BS, *aw = al + wave * SK4_AS;
    auto aload = [&](u32x4 (&v)[3], int64_t b) {
#pragma unroll
        for (int k = 0; k < 3; k++) v[k] = *(const u32x4 *)(ap[k] + b * 16);
    };
    auto astore = [&](const u32x4 (&v)[3]) {
#pragma unroll
        for (int k = 0; k < 2; k++) {
            *(uint2 *)(aw + adst[k]) = make_uint2(v[k].x, v[k].y);
            *(uint2 *)(aw + adst[k] + 8) = make_uint2(v[k].z, v[k].w);
        }
        if (lane < 16) *(u32x4 *)(aw + 16 * Q4S + 16 * lane) = v[2];
    };
    float acc = 0.0f;   // output slot `wave` of this lane (waves past NT·4 hold none)
    SkB<NT> B;
    B.init(a, c0, lane);
    u32x4 bv[5 * NT], av[3];
    {
        const int64_t b0 = min((int64_t)wave, nb - 1);
        B.load(bv, xb + b0 * 320);
        aload(av, b0);
        B.store(bv, bw);
        astore(av);
    }
    const int64_t rounds = (nb + W - 1) / W;
    auto round = [&](int64_t rd, auto pf) {
        const int64_t b = rd * W + wave;
        if constexpr (decltype(pf)::on) {   // the wave's next block (clamped past the end)
            const int64_t bn = min(b + W, nb - 1);
            B.load(bv, xb + bn * 320);
            aload(av, bn);
        }
        if (b < nb) {
#pragma unroll
            for (int n = 0; n < NT; n++) {
                float t1[4], t2[4];
                q4k_sk_group(aw, bw + (16 * n + m) * GEMM_CS, q, m, t1, t2);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    hand[rd & 1][wave][4 * n + i][0][lane] = t1[i];
                    hand[rd & 1][wave][4 * n + i][1][lane] = t2[i];
                }
            }
        }
        if constexpr (decltype(pf)::on) {   // the wave's own slots: its reads above come first
            B.store(bv, bw);
            astore(av);
        }
        __syncthreads();   // round rd's terms are handed
        if (wave < NT * 4) {
            const int live = (int)min((int64_t)W, nb - rd * W);
            for (int w = 0; w < live; w++)
                acc = __fsub_rn(__fadd_rn(acc, hand[rd & 1][w][wave][0][lane]), hand[rd & 1][w][wave][1][lane]);
        }
    };
    for (int64_t rd = 0; rd + 1 < rounds; rd++) round(rd, PF<true>{});
    round(rounds - 1, PF<false>{});
    if (wave >= NT * 4) return;
    const int n = wave >> 2, i = wave & 3;
    const int64_t c = c0 + 16 * n + m, r = r0 + 4 * q + i;
    if (c < a.batch && r < a.rows) {
        float *y = a.y + c * a.y_stride + a.y_off + r;
        *y = a.epi == CJ_EPI_ACCUM ? __fadd_rn(*y, acc) : acc;
    }
}

// Kernels by column-tile width: 16·NT columns a workgroup.
#define GEMM_KERNELS(NT)                                                                   \
    extern "C" __global__ void __launch_bounds__(256) cj_gemm_q80_n##NT(cj_gemv_args a) { \
        __shared__ __align__(16) uint8_t lds[16 * NT * GEMM_CS];                           \
        gemm_q80<NT>(a, lds);                                                             \
    }                                                                                      \
    extern "C" __global__ void __launch_bounds__(256) cj_gemm_q4k_n##NT(cj_gemv_args a) { \
        __shared__ __align__(16) uint8_t lds[16 * NT * GEMM_CS];                           \
        gemm_q4k<NT>(a, lds);                                                              \
    }
GEMM_KERNELS(2)
extern "C" __global__ void __launch_bounds__(256) cj_gemm_q80_n4(cj_gemv_args a) {
    __shared__ __align__(16) uint8_t lds[16 * 4 * GEMM_CS];
    gemm_q80<4>(a, lds);
}

// Split-K kernels: 16 rows × 16·NT columns a workgroup of 8 waves (the
// widths whose registers fit two waves a SIMD without spilling).
extern "C" __global__ void __launch_bounds__(512) cj_gemm_sk_q80_n1(cj_gemv_args a) { gemm_sk_q80<1, 8>(a); }
extern "C" __global__ void __launch_bounds__(512) cj_gemm_sk_q80_n2(cj_gemv_args a) { gemm_sk_q80<2, 8>(a); }
extern "C" __global__ void __launch_bounds__(512) cj_gemm_sk_q4k_n1(cj_gemv_args a) { gemm_sk_q4k<1, 8>(a); }

// ------------------------------------------------------------------- Q6_K

// Many columns of Q6_K × q8_K (no matrix-core form: the 16-element
// sub-block scales sit inside the 32-element dot an MFMA forms). A
// workgroup takes 16 rows (4 a wave) and NC columns, and walks the rows in
// sweeps of 16 blocks: a sweep's activation blocks of the NC columns are
// staged in LDS once for the four waves (16-byte pieces swizzled so that
// every 8 lanes of a read touch 8 distinct bank groups), and each lane — a
// unit (block, quarter: 64 elements) of the sweep — decodes its unit of the
// wave's 4 rows once to signed q − 32, then reads each column's 64 values
// once for the 4 rows. The next sweep's activation and weights are requested
// before the current sweep's arithmetic. Per (row, column) the block terms
// are the one-column GEMV's — sumi = Σ_sb sc_sb·dot_sb over q − 32, an exact
// integer, then (d·xs)·sumi — and lane (row, column) of the wave folds them
// in block order, sweep after sweep (Quant.q6kMatVecIntoQ8,
// io/Quant.cajeta:3448-3486): each column is bit for bit what cj_matvec
// gives it.
// Four 6-bit codes q (0..63, one a byte) as the int8 values q − 32: bit 5
// set, clearing it subtracts 32; clear, q − 32 = q + 224 is q + 32 with bits
// 6 and 7 set: bit 5 of the clear set shifted up by one and by two, the
// last shift in its own instruction (written as C, the two shifts become a
// multiply by 6, which issues at a quarter of the rate).
DEV uint32_t q6_signed(uint32_t q) {
    const uint32_t m = ~q & 0x20202020u;
    uint32_t r;
    asm("v_lshl_or_b32 %0, %1, 1, %2" : "=v"(r) : "v"(m), "v"((q ^ 0x20202020u) | (m << 2)));
    return r;
}

// One unit of a Q6_K row as loaded: low and high code nibbles, the high bit
// pairs, the unit's eight sub-block scales and the block's f16 scale.
struct Q6Unit {
    uint4 qa, qb, qh;
    uint2 sc;
    uint32_t dh;
};

DEV Q6Unit q6_load(const uint8_t *w, int64_t nb, int b, int g, int hl) {
    Q6Unit u;
    u.qa = ld_stream16(w + (int64_t)b * 128 + 64 * g + 16 * hl);
    u.qb = ld_stream16(w + (int64_t)b * 128 + 64 * g + 32 + 16 * hl);
    u.qh = ld_stream16(w + nb * 128 + (int64_t)b * 64 + 32 * g + 16 * hl);
    u.sc = *(const uint2 *)(w + nb * 192 + (int64_t)b * 16 + 8 * g);
    u.dh = *(const uint16_t *)(w + nb * 208 + 2 * b);
    return u;
}

template <int NC>
DEV void gemm_q6k_cols(const cj_gemv_args &a) {
    constexpr int SB = 16;                             // blocks a sweep
    __shared__ __align__(16) uint8_t xq[NC * SB * 256];
    __shared__ float xsl[NC * SB];
    __shared__ float terms[4][4][NC][SB + 1];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int nb = (int)(a.cols / 256);
    const int64_t c0 = (int64_t)blockIdx.y * NC, rbase = (int64_t)blockIdx.x * 16 + 4 * wave;
    const uint8_t *xcol[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) xcol[c] = a.xp + min(c0 + c, (int64_t)a.batch - 1) * a.xp_stride;
    const uint8_t *wrow[4];
#pragma unroll
    for (int rr = 0; rr < 4; rr++) wrow[rr] = a.w + min(rbase + rr, a.rows - 1) * a.row_bytes;
    // this lane's unit of a sweep: block bl, quarter j (g: 128-element half)
    const int bl = lane >> 2, j = lane & 3, g = j >> 1, hl = j & 1;
    const int sw = ((bl & 1) << 2) | (g << 1);
    // staging: thread t carries 16-byte piece ci of sweep block sbl, every column
    const int sbl = t >> 4, ci = t & 15;
    const int sp = (ci & 8) | ((ci & 7) ^ (((sbl & 1) << 2) | ((ci >> 3) << 1)));
    const uint8_t *xsp = a.xp + min(c0 + (t >> 4), (int64_t)a.batch - 1) * a.xp_stride + 288;
    u32x4 xv[NC];                                      // a native vector: a uint4 array copies through memory
    float xsv = 0.0f;
    Q6Unit wu[4];
    auto fetch = [&](int s0) __attribute__((always_inline)) {
        const int sb = min(SB, nb - s0);
        const int64_t xo = (int64_t)(s0 + min(sbl, sb - 1)) * 320 + 16 * ci;   // past the row: its last block again
#pragma unroll
        for (int c = 0; c < NC; c++) xv[c] = *(const u32x4 *)(xcol[c] + xo);
        xsv = *(const float *)(xsp + (int64_t)(s0 + min(ci, sb - 1)) * 320);
        const int b = s0 + min(bl, sb - 1);
#pragma unroll
        for (int rr = 0; rr < 4; rr++) wu[rr] = q6_load(wrow[rr], nb, b, g, hl);
    };
    const int frr = lane / NC, fc = lane % NC;         // the folding lane's (row, column)
    float acc = 0.0f;
    fetch(0);
    for (int s0 = 0; s0 < nb; s0 += SB) {
        const int sb = min(SB, nb - s0);
        if (sbl < sb) {
#pragma unroll
            for (int c = 0; c < NC; c++) *(u32x4 *)(xq + (c * SB + sbl) * 256 + 16 * sp) = xv[c];
        }
        if (t < NC * SB) xsl[t] = xsv;
        lds_barrier();                                 // the sweep's activation is staged
        uint32_t v[4][4][4];
        int scv[4][4];
        float d[4];
#pragma unroll
        for (int rr = 0; rr < 4; rr++) {
            const Q6Unit &u = wu[rr];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint4 ql = (k & 1) ? u.qb : u.qa;
                const int sh = (k >> 1) * 4;
                const uint32_t M = 0x0F0F0F0Fu, H = 0x03030303u;
                v[rr][k][0] = q6_signed(((ql.x >> sh) & M) | (((u.qh.x >> (2 * k)) & H) << 4));
                v[rr][k][1] = q6_signed(((ql.y >> sh) & M) | (((u.qh.y >> (2 * k)) & H) << 4));
                v[rr][k][2] = q6_signed(((ql.z >> sh) & M) | (((u.qh.z >> (2 * k)) & H) << 4));
                v[rr][k][3] = q6_signed(((ql.w >> sh) & M) | (((u.qh.w >> (2 * k)) & H) << 4));
                const int byte_i = 2 * k + hl;
                const uint32_t word = byte_i < 4 ? u.sc.x : u.sc.y;
                scv[rr][k] = (int)(int8_t)((word >> (8 * (byte_i & 3))) & 255);
            }
            d[rr] = h2f(u.dh);
        }
        if (s0 + SB < nb) fetch(s0 + SB);              // the next sweep's operands, in flight meanwhile
        __builtin_amdgcn_sched_barrier(0);
        const bool own = j == 0 && bl < sb;
        const uint8_t *xb = xq + bl * 256 + 128 * g;
        // at 8 columns a column's 64 values and scale are read a column ahead
        // (one wave a SIMD there: nothing else hides the LDS latency); at 4
        // the registers that takes would halve the waves a SIMD
        constexpr bool AHEAD = NC >= 8;
        constexpr int CU = AHEAD ? NC : 2;            // the column loop's unroll
        u32x4 an[4];
        float xn;
        auto xread = [&](int c) __attribute__((always_inline)) {
#pragma unroll
            for (int k = 0; k < 4; k++) an[k] = *(const u32x4 *)(xb + c * SB * 256 + 16 * ((hl + 2 * k) ^ sw));
            xn = xsl[c * SB + bl];
        };
        if (AHEAD) xread(0);
#pragma unroll CU
        for (int c = 0; c < NC; c++) {
            if (!AHEAD) xread(c);
            u32x4 av[4];
#pragma unroll
            for (int k = 0; k < 4; k++) av[k] = an[k];
            const float xs = xn;
            if (AHEAD && c + 1 < NC) xread(c + 1);
#pragma unroll
            for (int rr = 0; rr < 4; rr++) {
                int sumi = 0;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    int dt = 0;
                    dt = sdot4(v[rr][k][0], av[k].x, dt); dt = sdot4(v[rr][k][1], av[k].y, dt);
                    dt = sdot4(v[rr][k][2], av[k].z, dt); dt = sdot4(v[rr][k][3], av[k].w, dt);
                    // |dt| <= 16·32·128 and |sc| <= 128: a 24-bit multiply is exact
                    sumi += __mul24(scv[rr][k], dt);
                }
                sumi += dpp_i<DPP_XOR1>(sumi);
                sumi += dpp_i<DPP_XOR2>(sumi);
                const float term = __fmul_rn(__fmul_rn(d[rr], xs), (float)sumi);
                if (own) terms[wave][rr][c][bl] = term;
            }
        }
        lds_barrier();                                 // the sweep's terms are written
        if (lane < 4 * NC)
            for (int q = 0; q < sb; q++) acc = __fadd_rn(acc, terms[wave][frr][fc][q]);
        lds_barrier();                                 // and read, with the activation, before the next sweep
    }
    const int64_t row = rbase + frr, col = c0 + fc;
    if (lane < 4 * NC && row < a.rows && col < a.batch) {
        float *y = a.y + col * a.y_stride + a.y_off + row;
        *y = a.epi == CJ_EPI_ACCUM ? __fadd_rn(*y, acc) : acc;
    }
}
extern "C" __global__ void __launch_bounds__(256) cj_gemm_q6k_c4(cj_gemv_args a) { gemm_q6k_cols<4>(a); }
extern "C" __global__ void __launch_bounds__(256) cj_gemm_q6k_c8(cj_gemv_args a) { gemm_q6k_cols<8>(a); }

// Q6_K × 16 columns on the int8 matrix cores. A 32-element run of a block
// holds two 16-element sub-blocks with scales of their own, so each run takes
// two v_mfma_i32_16x16x32_i8 over the same activation operand: one with the
// weights of lanes 32-63 (elements 16-31 of the run) zeroed, one with lanes
// 0-31 zeroed — each product an exact int32 dot of one sub-block. The
// activation is the A operand (its rows the 16 columns) and the weights the
// B operand (its columns the 16 rows), so lane l receives columns
// 4·(l / 16) + i of weight row l % 16 and applies that row's sub-block scales
// to them: sumi = Σ_sb sc_sb·dot_sb, an exact integer, then (d·xs)·sumi per
// (row, column) and block, as the one-column GEMV forms it. A workgroup owns
// 16 rows × 16 columns; its four waves take a round's 16 blocks four apiece
// (wave w blocks w, w + 4, …), hand the terms through LDS, and thread
// (row, column) folds them in block order, round after round
// (Quant.q6kMatVecIntoQ8, io/Quant.cajeta:3448-3486): each column is bit for
// bit what cj_matvec gives it.
// One block's operands for cj_gemm_q6k_m16, as one lane loads them.
struct Q6M {
    long q[2][2], h[2], xv[2][4];
    u32x4 sc;
    uint32_t dh;
    float xs[4];
};

extern "C" __global__ void __launch_bounds__(256) cj_gemm_q6k_m16(cj_gemv_args a) {
    constexpr int RB = 16;                             // blocks a round
    __shared__ __align__(16) float terms[RB][16][20];  // [block][row][column], rows padded against bank conflicts
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int n = lane & 15, kg = lane >> 4;
    const int nb = (int)(a.cols / 256);
    const int64_t r0 = (int64_t)blockIdx.x * 16, c0 = (int64_t)blockIdx.y * 16;
    const int64_t last = (int64_t)a.batch - 1;
    const uint8_t *w = a.w + min(r0 + n, a.rows - 1) * a.row_bytes;               // B: weight row r0 + n
    const uint8_t *xa = a.xp + min(c0 + n, last) * a.xp_stride + 8 * kg;          // A: column c0 + n
    const uint8_t *xsp[4];                                                        // the received columns' scales
#pragma unroll
    for (int i = 0; i < 4; i++) xsp[i] = a.xp + min(c0 + 4 * kg + i, last) * a.xp_stride + 288;
    const bool lo = kg < 2;
    // the wave's blocks: j-th is block 16·(j / 4) + wave + 4·(j % 4) of the row;
    // past the row the last block is read again and its terms left unfolded
    const int rounds = (nb + RB - 1) / RB, J = 4 * rounds;
    auto load = [&](Q6M &o, int jj) __attribute__((always_inline)) {
        const int b = min(RB * (jj >> 2) + wave + 4 * (jj & 3), nb - 1);
#pragma unroll
        for (int g = 0; g < 2; g++) {
#pragma unroll
            for (int kk = 0; kk < 4; kk++) o.xv[g][kk] = ld8(xa + (int64_t)b * 320 + 128 * g + 32 * kk);
#pragma unroll
            for (int p = 0; p < 2; p++) o.q[g][p] = ld8(w + (int64_t)b * 128 + 64 * g + 32 * p + 8 * kg);
            o.h[g] = ld8(w + (int64_t)nb * 128 + (int64_t)b * 64 + 32 * g + 8 * kg);
        }
        o.sc = *(const u32x4 *)(w + (int64_t)nb * 192 + (int64_t)b * 16);
        o.dh = *(const uint16_t *)(w + (int64_t)nb * 208 + 2 * b);
#pragma unroll
        for (int c = 0; c < 4; c++) o.xs[c] = *(const float *)(xsp[c] + (int64_t)b * 320);
    };
    const int frow = t >> 4, fcol = t & 15;
    float acc = 0.0f;
    Q6M cur, nxt;
    load(cur, 0);
    for (int jj = 0; jj < J; jj++) {
        load(nxt, min(jj + 1, J - 1));                 // the next block in flight meanwhile
        int sumi[4] = {0, 0, 0, 0};
#pragma unroll
        for (int g = 0; g < 2; g++) {
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                // the run's 8 codes of this lane as int8 q − 32
                const long ql = cur.q[g][kk & 1], qh = cur.h[g];
                const int sh = 4 * (kk >> 1);
                const uint32_t M = 0x0F0F0F0Fu, H = 0x03030303u;
                const uint32_t lo32 = q6_signed((((uint32_t)ql >> sh) & M) | ((((uint32_t)qh >> (2 * kk)) & H) << 4));
                const uint32_t hi32 = q6_signed((((uint32_t)(ql >> 32) >> sh) & M) |
                                                ((((uint32_t)(qh >> 32) >> (2 * kk)) & H) << 4));
                const long wv = (long)(((uint64_t)hi32 << 32) | lo32);
                const v4i d0 = mfma_i8(cur.xv[g][kk], lo ? wv : 0);   // sub-block 8g + 2kk
                const v4i d1 = mfma_i8(cur.xv[g][kk], lo ? 0 : wv);   // sub-block 8g + 2kk + 1
                const int sb = 8 * g + 2 * kk;
                const uint32_t word = cur.sc[sb >> 2];
                const int s0 = (int)(int8_t)(word >> (8 * (sb & 3))), s1 = (int)(int8_t)(word >> (8 * ((sb & 3) + 1)));
                // |dot| <= 16·32·127 and |sc| <= 128: 24-bit multiplies are exact
#pragma unroll
                for (int c = 0; c < 4; c++) sumi[c] += __mul24(s0, d0[c]) + __mul24(s1, d1[c]);
            }
        }
        const float d = h2f(cur.dh);
        f32x4 tv;
#pragma unroll
        for (int c = 0; c < 4; c++) tv[c] = __fmul_rn(__fmul_rn(d, cur.xs[c]), (float)sumi[c]);
        *(f32x4 *)&terms[wave + 4 * (jj & 3)][n][4 * kg] = tv;
        cur = nxt;
        if ((jj & 3) == 3) {
            lds_barrier();                             // the round's terms are written
            const int nbr = min(RB, nb - RB * (jj >> 2));
            for (int k = 0; k < nbr; k++) acc = __fadd_rn(acc, terms[k][frow][fcol]);
            lds_barrier();                             // and read before the next round writes them
        }
    }
    const int64_t row = r0 + frow, col = c0 + fcol;
    if (row < a.rows && col < a.batch) {
        float *y = a.y + col * a.y_stride + a.y_off + row;
        *y = a.epi == CJ_EPI_ACCUM ? __fadd_rn(*y, acc) : acc;
    }
}

// Q4_0 many-column GEMV (cj_matmul over f32 activation columns): the
// one-column kernel's sweeps for NC columns a workgroup, RW rows a wave
// (4·RW a workgroup). A sweep's 64 blocks of every column are staged in LDS
// (swizzled) once for the four waves. A lane runs its block's RW·NC dot
// chains side by side, four code bytes at a time: the rows' 8 codes of those
// bytes decoded once, then each column's 8 x values read once for all RW
// rows; each chain still adds its products in the block's element order.
// Lane l < RW·NC folds chain l (row l / NC, column l % NC) a sweep behind,
// as the one-column kernel does. The next sweep's x is requested before its
// codes, so staging it (at the end of a sweep) never waits for the weight
// stream, and forming a sweep waits only for codes requested a sweep earlier.
// A sweep's x for NC columns: float4 f = threadIdx.x + 256·m of its NC·512
// (column f / 512, block (f % 512) / 8, float4 f % 8), into registers, then
// swizzled into LDS. Unrolled by template recursion, so every index is a
// constant from the start and the array lives in registers.
template <int M, int NC>
struct Q40X {
    static DEV void load(f32x4 (&xr)[2 * NC], const cj_gemv_args &a, int64_t c0, int nb, int j) {
        const int f = threadIdx.x + 256 * M, c = f >> 9, bb = (f & 511) >> 3, i = f & 7;
        const int blk = min(64 * j + bb, nb - 1);
        const float *col = (const float *)(a.xp + min(c0 + c, (int64_t)a.batch - 1) * a.xp_stride);
        xr[M] = *(const f32x4 *)(col + 32 * (int64_t)blk + 4 * i);
        if constexpr (M + 1 < 2 * NC) Q40X<M + 1, NC>::load(xr, a, c0, nb, j);
    }
    static DEV void store(const f32x4 (&xr)[2 * NC], float *xsm) {
        const int f = threadIdx.x + 256 * M, c = f >> 9, bb = (f & 511) >> 3, i = f & 7;
        *(f32x4 *)(xsm + c * 2048 + 32 * bb + 4 * (i ^ (bb & 7))) = xr[M];
        if constexpr (M + 1 < 2 * NC) Q40X<M + 1, NC>::store(xr, xsm);
    }
};
// A sweep's codes and scales for the wave's rows (blocks past the row re-read the last one).
template <int RW>
DEV void q40_fetch(uint4 (&q)[RW], uint32_t (&d)[RW], const uint8_t *const (&wr)[RW], int nb, int j, int lane) {
    const int b = min(64 * j + lane, nb - 1);
#pragma unroll
    for (int k = 0; k < RW; k++) {
        q[k] = ld_stream16(wr[k] + 16 * (int64_t)b);
        d[k] = *(const uint16_t *)(wr[k] + 16 * (int64_t)nb + 2 * b);
    }
}

template <int RW, int NC>
DEV void gemm_q40_cols(const cj_gemv_args &a) {
    constexpr int CH = RW * NC;
    __shared__ __align__(16) float xsm[NC * 2048];
    __shared__ __align__(16) float tb[4][2][CH][Q40_TS];
    const int t = threadIdx.x, w = t >> 6, lane = t & 63;
    const int nb = (int)(a.cols / 32), sweeps = (nb + 63) >> 6;
    const int fr = min(lane, CH - 1);
#pragma unroll
    for (int k = 0; k < CH; k++) tb[w][1][k][lane] = 0.0f;
    const int64_t c0 = (int64_t)blockIdx.y * NC;
    const int64_t rbase = (int64_t)blockIdx.x * (4 * RW) + w * RW;
    const uint8_t *wr[RW];
#pragma unroll
    for (int k = 0; k < RW; k++) wr[k] = a.w + min(rbase + k, a.rows - 1) * a.row_bytes;
    f32x4 xr[2 * NC];
    uint4 qn[RW];
    uint32_t dn[RW];
    Q40X<0, NC>::load(xr, a, c0, nb, 0);
    q40_fetch<RW>(qn, dn, wr, nb, 0, lane);
    Q40X<0, NC>::store(xr, xsm);
    __syncthreads();
    float acc = 0.0f;
    const float *xb = xsm + 32 * lane;     // this lane's block of column 0
    const int sw = lane & 7;               // its swizzle
    for (int j = 0; j < sweeps; j++) {
        uint4 q[RW];
        uint32_t d[RW];
#pragma unroll
        for (int k = 0; k < RW; k++) { q[k] = qn[k]; d[k] = dn[k]; }
        Q40X<0, NC>::load(xr, a, c0, nb, j + 1);    // past the last sweep: re-reads of the last block, never used
        q40_fetch<RW>(qn, dn, wr, nb, j + 1, lane);
        float dot[RW][NC];
#pragma unroll
        for (int k = 0; k < RW; k++)
#pragma unroll
            for (int c = 0; c < NC; c++) dot[k][c] = 0.0f;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            // code bytes 4g..4g+3 of each row: elements 4g+jj (low nibble) and 16+4g+jj (high)
            float wl[RW][4], wh[RW][4];
#pragma unroll
            for (int k = 0; k < RW; k++) {
                const uint32_t word = (g == 0 ? q[k].x : g == 1 ? q[k].y : g == 2 ? q[k].z : q[k].w) ^ 0x88888888u;
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    wl[k][jj] = (float)((int)(word << (28 - 8 * jj)) >> 28);
                    wh[k][jj] = (float)((int)(word << (24 - 8 * jj)) >> 28);
                }
            }
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const f32x4 xl = *(const f32x4 *)(xb + c * 2048 + 4 * (g ^ sw));
                const f32x4 xh = *(const f32x4 *)(xb + c * 2048 + 4 * ((4 + g) ^ sw));
#pragma unroll
                for (int jj = 0; jj < 4; jj++)
#pragma unroll
                    for (int k = 0; k < RW; k++) {
                        dot[k][c] = __fadd_rn(dot[k][c], __fmul_rn(wl[k][jj], xl[jj]));
                        dot[k][c] = __fadd_rn(dot[k][c], __fmul_rn(wh[k][jj], xh[jj]));
                    }
            }
        }
#pragma unroll
        for (int k = 0; k < RW; k++) {
            const float dk = h2f(d[k]);
#pragma unroll
            for (int c = 0; c < NC; c++) tb[w][j & 1][k * NC + c][lane] = __fmul_rn(dk, dot[k][c]);
        }
        acc = q40_fold64(tb[w][(j + 1) & 1][fr], acc);   // sweep j − 1 (a zeroed row before the first)
        __syncthreads();               // every wave has read this sweep's x
        Q40X<0, NC>::store(xr, xsm);
        __syncthreads();
    }
    acc = q40_fold(tb[w][(sweeps - 1) & 1][fr], nb - 64 * (sweeps - 1), acc);
    if (lane < CH) {
        const int64_t row = rbase + lane / NC, col = c0 + lane % NC;
        if (row < a.rows && col < a.batch) {
            float *y = a.y + col * a.y_stride + a.y_off + row;
            *y = a.epi == CJ_EPI_ACCUM ? __fadd_rn(*y, acc) : acc;
        }
    }
}
extern "C" __global__ void __launch_bounds__(256) cj_gemm_q40_r2_c4(cj_gemv_args a) { gemm_q40_cols<2, 4>(a); }
extern "C" __global__ void __launch_bounds__(256) cj_gemm_q40_r4_c4(cj_gemv_args a) { gemm_q40_cols<4, 4>(a); }
