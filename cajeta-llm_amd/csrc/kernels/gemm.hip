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
//
// MFMA 16x16x32 int8 lane layout (checked on the part): lane l supplies A row
// l % 16 and B column l % 16, elements k = 8·(l / 16) .. +7, and receives
// D[4·(l / 16) + i][l % 16], i < 4. A wave owns 16 weight rows × 16 columns;
// a workgroup puts up to 4 waves side by side over the columns.
//
// Activations are the per-column packs (320-byte blocks, per-256 scale for
// Q4_K, per-32 scales for Q8_0) `xp_stride` bytes apart; outputs `y_stride`
// floats apart. The weights are the GEMV's prepared rows.
#include "common.h"

typedef int v4i __attribute__((ext_vector_type(4)));

DEV v4i mfma_i8(long a, long b) {
    const v4i z = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, z, 0, 0, 0);
}

DEV long ld8(const uint8_t *p) { return *(const long *)p; }

// Q8_0: prepared row [qs nb32·32][d nb32·2 → pad 16].
DEV void gemm_q80_tile(const cj_gemv_args &a, int64_t r0, int64_t c0, float (&acc)[4]) {
    const int lane = threadIdx.x & 63, q = lane >> 4, m = lane & 15;
    const int64_t nb32 = a.cols / 32, ngrp = (a.cols + 255) / 256;
    const int64_t ra = min(r0 + m, a.rows - 1);                  // the A row this lane supplies
    const int64_t cb = min(c0 + m, (int64_t)a.batch - 1);        // the B column this lane supplies
    const uint8_t *wa = a.w + ra * a.row_bytes + 8 * q;
    const uint8_t *xb = a.xp + cb * a.xp_stride + 8 * q;
    // the lane's output rows (4q .. 4q+3) and column m
    const uint8_t *wd[4];
#pragma unroll
    for (int i = 0; i < 4; i++) wd[i] = a.w + min(r0 + 4 * q + i, a.rows - 1) * a.row_bytes + nb32 * 32;
    const uint8_t *xs_base = a.xp + min(c0 + m, (int64_t)a.batch - 1) * a.xp_stride;
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = 0.0f;
    for (int64_t g = 0; g < ngrp; g++) {
        const int nj = (int)min((int64_t)8, nb32 - 8 * g);
        long af[8], bf[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int64_t blk = 8 * g + min(j, nj - 1);
            af[j] = ld8(wa + blk * 32);
            bf[j] = ld8(xb + g * 320 + 32 * min(j, nj - 1));
        }
        const float4 x0 = *(const float4 *)(xs_base + g * 320 + 288);
        const float4 x1 = *(const float4 *)(xs_base + g * 320 + 304);
        const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        // the group's 8 f16 scales of each output row in one 16-byte load (the
        // scale array is padded to 16 bytes, so a short last group stays in it)
        uint16_t dh[4][8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint4 h = *(const uint4 *)(wd[i] + 16 * g);
            const uint32_t hw[4] = {h.x, h.y, h.z, h.w};
#pragma unroll
            for (int j = 0; j < 8; j++) dh[i][j] = (uint16_t)(hw[j >> 1] >> (16 * (j & 1)));
        }
        float fs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            if (j < nj) {
                const v4i d = mfma_i8(af[j], bf[j]);
#pragma unroll
                for (int i = 0; i < 4; i++) fs[i] = __fadd_rn(fs[i], __fmul_rn(__fmul_rn(h2f(dh[i][j]), xs[j]), (float)d[i]));
            }
        }
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] = __fadd_rn(acc[i], fs[i]);
    }
}

// Q4_K: the GEMV's chunk-major prepared row — qs piece c (16 bytes) of block
// b at (c·nb + b)·16, the 16-byte header {d, dmin, scales[12]} at 128·nb + 16·b.
// Group g (elements 64g .. 64g+63) of a block is qs bytes 32g .. 32g+31:
// low nibbles are sub-block 2g, high nibbles sub-block 2g+1, so one 8-byte
// load (bytes 32g + 8q ..) feeds both sub-blocks' MFMAs.
DEV void gemm_q4k_tile(const cj_gemv_args &a, int64_t r0, int64_t c0, float (&acc)[4]) {
    const int lane = threadIdx.x & 63, q = lane >> 4, m = lane & 15;
    const int64_t nb = a.cols / 256;
    const int64_t ra = min(r0 + m, a.rows - 1);
    const int64_t cb = min(c0 + m, (int64_t)a.batch - 1);
    const uint8_t *wa = a.w + ra * a.row_bytes;
    const uint8_t *xb = a.xp + cb * a.xp_stride;
    const uint8_t *wh[4];
#pragma unroll
    for (int i = 0; i < 4; i++) wh[i] = a.w + min(r0 + 4 * q + i, a.rows - 1) * a.row_bytes + nb * 128;
    const uint8_t *xo = a.xp + min(c0 + m, (int64_t)a.batch - 1) * a.xp_stride;   // the lane's output column
    const uint32_t M = 0x0F0F0F0Fu;
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = 0.0f;
    for (int64_t b = 0; b < nb; b++) {
        long wq[4], alo[4], ahi[4];
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int byte = 32 * g + 8 * q;                           // qs byte of this lane's 8
            wq[g] = ld8(wa + ((int64_t)(byte >> 4) * nb + b) * 16 + (byte & 15));
            alo[g] = ld8(xb + b * 320 + 64 * g + 8 * q);
            ahi[g] = ld8(xb + b * 320 + 64 * g + 32 + 8 * q);
        }
        const int4 s0 = *(const int4 *)(xo + b * 320 + 256), s1 = *(const int4 *)(xo + b * 320 + 272);
        const float xs = *(const float *)(xo + b * 320 + 288);
        uint4 hd[4];
#pragma unroll
        for (int i = 0; i < 4; i++) hd[i] = *(const uint4 *)(wh[i] + b * 16);
        int dot[4][8];
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const uint64_t w = (uint64_t)wq[g];
            const long lo = (long)(w & (((uint64_t)M << 32) | M));
            const long hi = (long)((w >> 4) & (((uint64_t)M << 32) | M));
            const v4i dl = mfma_i8(lo, alo[g]);
            const v4i dh = mfma_i8(hi, ahi[g]);
#pragma unroll
            for (int i = 0; i < 4; i++) { dot[i][2 * g] = dl[i]; dot[i][2 * g + 1] = dh[i]; }
        }
        const int bs[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t A = hd[i].y, B = hd[i].z, C = hd[i].w;
            int sumi = 0, dmins = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t a8 = (A >> (8 * j)) & 255, b8 = (B >> (8 * j)) & 255, c8 = (C >> (8 * j)) & 255;
                const int sc_lo = (int)(a8 & 63), mn_lo = (int)(b8 & 63);
                const int sc_hi = (int)((c8 & 15) | ((a8 >> 2) & 48)), mn_hi = (int)((c8 >> 4) | ((b8 >> 2) & 48));
                sumi += __mul24(dot[i][j], sc_lo) + __mul24(dot[i][j + 4], sc_hi);
                dmins += __mul24(bs[j], mn_lo) + __mul24(bs[j + 4], mn_hi);
            }
            const float d = h2f(hd[i].x), dmin = h2f(hd[i].x >> 16);
            acc[i] = __fsub_rn(__fadd_rn(acc[i], __fmul_rn(__fmul_rn(d, xs), (float)sumi)),
                               __fmul_rn(__fmul_rn(dmin, xs), (float)dmins));
        }
    }
}

// Workgroup (column tile, row tile): 16 rows, and 16 columns a wave over the
// workgroup's 1..4 waves. The column tiles of one row tile are adjacent in
// dispatch order, so they run together and share the rows' weights in cache.
template <int FMT>
DEV void gemm_body(const cj_gemv_args &a) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, waves = blockDim.x >> 6;
    const int64_t r0 = (int64_t)blockIdx.y * 16;
    const int64_t c0 = ((int64_t)blockIdx.x * waves + wave) * 16;
    if (c0 >= a.batch) return;                     // uniform per wave; no barrier follows
    float acc[4];
    if (FMT == CJ_Q8_0) gemm_q80_tile(a, r0, c0, acc);
    else gemm_q4k_tile(a, r0, c0, acc);
    const int64_t c = c0 + (lane & 15);
    if (c >= a.batch) return;
    float *y = a.y + c * a.y_stride + a.y_off;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int64_t r = r0 + 4 * (lane >> 4) + i;
        if (r < a.rows) y[r] = a.epi == CJ_EPI_ACCUM ? __fadd_rn(y[r], acc[i]) : acc[i];
    }
}

extern "C" __global__ void __launch_bounds__(256) cj_gemm_q80(cj_gemv_args a) { gemm_body<CJ_Q8_0>(a); }
extern "C" __global__ void __launch_bounds__(256) cj_gemm_q4k(cj_gemv_args a) { gemm_body<CJ_Q4_K>(a); }
