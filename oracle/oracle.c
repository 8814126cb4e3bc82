/*
 * oracle.c — CPU restatement of cajeta-llm's CPU-backend decode arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h). Built with -ffp-contract=off so
 * every `a + b * c` below rounds twice, as written. Each function names the
 * reference file:line it restates; `L/` = src/main/cajeta/dev/cajeta/llm/.
 *
 * OR_PLANT (normally undefined) compiles one deliberate mistake into a
 * throw-away build, so the CPU tests can show that the check pinning that
 * function fails on it (tests/test_oracle.py, test_planted_mistakes_are_caught).
 */
#ifndef OR_PLANT
#define OR_PLANT 0
#endif
#include "oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <stdio.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float bits_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline int32_t rd_i32(const uint8_t *p) { int32_t v; memcpy(&v, p, 4); return v; }
static inline uint16_t rd_u16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline void wr_i32(uint8_t *p, int32_t v) { memcpy(p, &v, 4); }

int or_model_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ---------------------------------------------------------------- formats */

int or_block_bytes(int t) {
    switch (t) {
    case OR_F32: return 4; case OR_F16: return 2; case OR_Q4_0: return 18; case OR_Q8_0: return 34;
    case OR_Q4_K: return 144; case OR_Q6_K: return 210; case OR_MXFP4: return 17; default: return -1;
    }
}
int or_block_elems(int t) {
    switch (t) {
    case OR_F32: case OR_F16: return 1; case OR_Q4_0: case OR_Q8_0: case OR_MXFP4: return 32;
    case OR_Q4_K: case OR_Q6_K: return 256; default: return -1;
    }
}

/* IEEE half -> float, exact (GgufFile.halfBitsToF32, L/io/GgufFile.cajeta:1055). */
float or_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    uint32_t e = (h >> 10) & 31, m = h & 1023;
    if (e == 31) return bits_f(sign | 0x7f800000u | (m << 13));
    if (e == 0) {
        if (m == 0) return bits_f(sign);
        float v = (float)m * (1.0f / 16777216.0f); /* m * 2^-24, exact */
        return sign ? -v : v;
    }
    return bits_f(sign | ((e + 112) << 23) | (m << 13));
}

/* float -> half, round to nearest even (Quant.f32ToHalfBits, L/io/Quant.cajeta:838-859,
 * which is ggml's fp32_to_fp16; restated here as plain mantissa rounding). */
uint16_t or_f32_to_f16(float f) {
    uint32_t x = f_bits(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return sign | 0x7e00;          /* NaN */
    if (ax >= 0x477ff000u) return sign | 0x7c00;         /* rounds past 65504 -> inf */
    if (ax < 0x38800000u) {                              /* below 2^-14: half subnormal */
        uint32_t e = ax >> 23;
        if (e < 102) return sign;                        /* < 2^-25: rounds to zero */
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t sh = 126 - e;                           /* value*2^24 = m >> sh */
        uint32_t q = m >> sh, rem = m & ((1u << sh) - 1), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return sign | (uint16_t)q;
    }
    uint32_t r = ax + 0xfffu + ((ax >> 13) & 1u);
    return sign | (uint16_t)((r >> 13) - (112u << 10));
}

/* Q4_K / Q5_K header scales (Quant.headK4, L/io/Quant.cajeta:2044-2080). */
static void head_k4(const uint8_t *b, float *d, float *dmin, int sc[8], int mn[8]) {
    *d = or_f16_to_f32(rd_u16(b));
    *dmin = or_f16_to_f32(rd_u16(b + 2));
    const uint8_t *s = b + 4;
    for (int j = 0; j < 4; j++) { sc[j] = s[j] & 63; mn[j] = s[4 + j] & 63; }
    for (int j = 0; j < 4; j++) {
#if OR_PLANT == 4
        sc[4 + j] = (s[8 + j] & 15) | ((s[4 + j] >> 2) & 48);   /* planted: a transposed index */
#else
        sc[4 + j] = (s[8 + j] & 15) | ((s[j] >> 2) & 48);
#endif
        mn[4 + j] = (s[8 + j] >> 4) | ((s[4 + j] >> 2) & 48);
    }
}

/* E2M1 code value (Quant.mxfp4Code, L/io/Quant.cajeta:1106-1120). */
static int mxfp4_code(int nib) {
    static const int mag[8] = {0, 1, 2, 3, 4, 6, 8, 12};
    int v = mag[nib & 7];
    return (nib & 8) ? -v : v;
}
/* E8M0 half-scale 2^(e-128) incl. the e<2 denormals (Quant.mxfp4Scale, :1124-1131). */
static float mxfp4_scale(int e) {
    uint32_t b = e < 2 ? (0x00200000u << e) : ((uint32_t)(e - 1) << 23);
    return bits_f(b);
}

/* Quant.dequantize (L/io/Quant.cajeta:693-734) and the block bodies it calls:
 * q80Block :752, q40Block :1186-1196, q4kBlock :2084-2104, q6kBlock :2135-2154,
 * mxfp4Block :1133-1144. */
int or_dequant(int type, const uint8_t *raw, int64_t nb, float *out) {
    int bb = or_block_bytes(type), be = or_block_elems(type);
    if (bb < 0) return -1;
    for (int64_t b = 0; b < nb; b++) {
        const uint8_t *r = raw + b * bb;
        float *o = out + b * be;
        switch (type) {
        case OR_F32: memcpy(o, r, 4); break;
        case OR_F16: o[0] = or_f16_to_f32(rd_u16(r)); break;
        case OR_Q8_0: {
            float d = or_f16_to_f32(rd_u16(r));
            for (int j = 0; j < 32; j++) o[j] = d * (float)(int8_t)r[2 + j];
        } break;
        case OR_Q4_0: {
            float d = or_f16_to_f32(rd_u16(r));
            for (int j = 0; j < 16; j++) {
                int q = r[2 + j];
                o[j] = d * (float)((q & 15) - 8);
                o[j + 16] = d * (float)((q >> 4) - 8);
            }
        } break;
        case OR_Q4_K: {
            float d, dmin; int sc[8], mn[8];
            head_k4(r, &d, &dmin, sc, mn);
            for (int e = 0; e < 256; e++) {
                int g = e / 64, rr = e % 64, s = rr / 32, l = rr % 32;
                int q = (r[16 + 32 * g + l] >> (4 * s)) & 15;
                int sb = e / 32;
                o[e] = d * (float)sc[sb] * (float)q - dmin * (float)mn[sb];
            }
        } break;
        case OR_Q6_K: {
            float d = or_f16_to_f32(rd_u16(r + 208));
            for (int e = 0; e < 256; e++) {
                int g = e / 128, rr = e % 128, sl = rr / 64, l64 = rr % 64;
                int ql = (r[64 * g + l64] >> (4 * sl)) & 15;
                int sh = rr / 32, l32 = rr % 32;
                int qh = (r[128 + 32 * g + l32] >> (2 * sh)) & 3;
                int q = (ql | (qh << 4)) - 32;
                int scb = (int8_t)r[192 + e / 16];
                o[e] = d * (float)scb * (float)q;
            }
        } break;
        case OR_MXFP4: {
            float d = mxfp4_scale(r[0]);
            for (int j = 0; j < 16; j++) {
                int b8 = r[1 + j];
                o[j] = (float)mxfp4_code(b8 & 15) * d;
                o[j + 16] = (float)mxfp4_code((b8 >> 4) & 15) * d;
            }
        } break;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------ packs */

/* Math.round as the pack kernels use it: half away from zero (the CPU row
 * form's trunc + 2·frac trick, L/model/Prim.cajeta:1190-1240, is the same map). */
static inline int round_away(float v) { return (int)roundf(v); }

/* Quant.q8kPackPad (L/io/Quant.cajeta:3232-3276): per 256 values one scale
 * amax/127, q = round(v·127/amax), eight int32 sums of 32, scale bits at 288. */
void or_q8k_pack(const float *x, int64_t n, int64_t npad, uint8_t *out) {
    int64_t blocks = npad / 256;
    for (int64_t b = 0; b < blocks; b++) {
        uint8_t *ob = out + b * 320;
        int64_t e0 = b * 256;
        float amax = 0.0f;
        for (int i = 0; i < 256; i++) {
            float v = e0 + i < n ? x[e0 + i] : 0.0f;
            float av = v < 0.0f ? 0.0f - v : v;
            if (av > amax) amax = av;
        }
        float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
        memset(ob, 0, 320);
        for (int sb = 0; sb < 8; sb++) {
            int s = 0;
            for (int k = 0; k < 32; k++) {
                int64_t e = e0 + sb * 32 + k;
                float v = e < n ? x[e] : 0.0f;
                int q = round_away(v * inv);
                ob[sb * 32 + k] = (uint8_t)(int8_t)q;
                s += q;
            }
            wr_i32(ob + 256 + sb * 4, s);
        }
        wr_i32(ob + 288, (int32_t)f_bits(amax / 127.0f));
    }
}

/* Quant.q8kPack32Pad (L/io/Quant.cajeta:3285-3321) in the form the device
 * pack uses (QuantKernel.q8kPack32BlockSerial, L/io/QuantKernel.cajeta:42841-42872):
 * each 32 values quantize against their own amax; scale j at 288+4j. */
void or_q8k_pack32(const float *x, int64_t n, int64_t npad, uint8_t *out) {
    int64_t blocks = npad / 256;
    for (int64_t b = 0; b < blocks; b++) {
        uint8_t *ob = out + b * 320;
        memset(ob, 0, 320);
        for (int sb = 0; sb < 8; sb++) {
            int64_t e0 = b * 256 + sb * 32;
            float amax = 0.0f;
            for (int i = 0; i < 32; i++) {
                float v = e0 + i < n ? x[e0 + i] : 0.0f;
                float av = v < 0.0f ? 0.0f - v : v;
                if (av > amax) amax = av;
            }
            float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
            int s = 0;
            for (int k = 0; k < 32; k++) {
                float v = e0 + k < n ? x[e0 + k] * inv : 0.0f;
                int q = round_away(v);
                ob[sb * 32 + k] = (uint8_t)(int8_t)q;
                s += q;
            }
            wr_i32(ob + 256 + sb * 4, s);
            wr_i32(ob + 288 + sb * 4, (int32_t)f_bits(amax / 127.0f));
        }
    }
}

/* ---------------------------------------------------------------- GEMVs */

/* Quant.q4kMatVecIntoQ8 (L/io/Quant.cajeta:3374-3445) on the packed form:
 * per block an exact integer sumi and dmins, then
 * acc = (acc + d·xs·sumi) − dmin·xs·dmins in block order. */
static void mv_q4k(const uint8_t *w, int64_t rows, int64_t cols, const uint8_t *xp, float *y) {
    int64_t bpr = cols / 256;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < rows; i++) {
        float acc = 0.0f;
        for (int64_t b = 0; b < bpr; b++) {
            const uint8_t *r = w + (i * bpr + b) * 144;
            const uint8_t *xb = xp + b * 320;
            float d, dmin; int sc[8], mn[8];
            head_k4(r, &d, &dmin, sc, mn);
            int32_t sumi = 0;
            for (int g = 0; g < 4; g++) {
                int32_t lo = 0, hi = 0;
                for (int l = 0; l < 32; l++) {
                    int q = r[16 + 32 * g + l];
                    lo += (q & 15) * (int8_t)xb[64 * g + l];
                    hi += ((q >> 4) & 15) * (int8_t)xb[64 * g + 32 + l];
                }
                sumi += lo * sc[2 * g] + hi * sc[2 * g + 1];
            }
            int32_t dmins = 0;
            for (int sb = 0; sb < 8; sb++) dmins += mn[sb] * rd_i32(xb + 256 + 4 * sb);
            float xs = bits_f((uint32_t)rd_i32(xb + 288));
#if OR_PLANT == 1
            acc = acc + d * xs * (float)sumi;             /* planted: the min term dropped */
#else
            acc = acc + d * xs * (float)sumi - dmin * xs * (float)dmins;
#endif
        }
        y[i] = acc;
    }
}

/* Quant.q6kMatVecIntoQ8 (L/io/Quant.cajeta:3448-3486): per block
 * sumi = Σ_sb scale_sb·dot_sb (int), acc = acc + d·xs·sumi. */
static void mv_q6k(const uint8_t *w, int64_t rows, int64_t cols, const uint8_t *xp, float *y) {
    int64_t bpr = cols / 256;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < rows; i++) {
        float acc = 0.0f;
        for (int64_t b = 0; b < bpr; b++) {
            const uint8_t *r = w + (i * bpr + b) * 210;
            const uint8_t *xb = xp + b * 320;
            float d = or_f16_to_f32(rd_u16(r + 208));
            int32_t sumi = 0;
            for (int sb = 0; sb < 16; sb++) {
                int n = sb / 8, k = (sb % 8) / 2, h = sb % 2;
                int32_t dot = 0;
                for (int t = 0; t < 16; t++) {
                    int l = 16 * h + t;
                    int qlb = r[64 * n + 32 * (k % 2) + l];
                    int lo4 = k < 2 ? (qlb & 15) : (qlb >> 4);
                    int qhb = r[128 + 32 * n + l];
                    int q = (lo4 | (((qhb >> (2 * k)) & 3) << 4)) - 32;
                    dot += q * (int8_t)xb[128 * n + 32 * k + l];
                }
                sumi += (int8_t)r[192 + sb] * dot;
            }
            float xs = bits_f((uint32_t)rd_i32(xb + 288));
            acc = acc + d * xs * (float)sumi;
        }
        y[i] = acc;
    }
}

/* Quant.q80MatVecIntoQ8Sub with spb = 8 (L/io/Quant.cajeta:3079-3110): per 32
 * columns an exact integer dot times (d_j · xs_j), summed per 256 into fs,
 * then acc += fs. Blocks past `cols` (a row padded to whole 256s by
 * Quant.q80Interleave8Pad) hold zeros and are skipped. */
static void mv_q80(const uint8_t *w, int64_t rows, int64_t cols, const uint8_t *xp, float *y) {
    int64_t nbk = cols / 32, sbpr = (cols + 255) / 256;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < rows; i++) {
        float acc = 0.0f;
        for (int64_t b = 0; b < sbpr; b++) {
            const uint8_t *xb = xp + b * 320;
            float fs = 0.0f;
            for (int j = 0; j < 8; j++) {
                int64_t blk = b * 8 + j;
                if (blk >= nbk) break;
                const uint8_t *r = w + (i * nbk + blk) * 34;
                int32_t isum = 0;
                for (int k = 0; k < 32; k++) isum += (int8_t)r[2 + k] * (int8_t)xb[32 * j + k];
                float xs = bits_f((uint32_t)rd_i32(xb + 288 + 4 * j));
                fs = fs + (or_f16_to_f32(rd_u16(r)) * xs) * (float)isum;
            }
            acc = acc + fs;
        }
        y[i] = acc;
    }
}

/* Quant.q40MatVecIntoAt (L/io/Quant.cajeta:1516-1545): f32 activations. */
static void mv_q40(const uint8_t *w, int64_t rows, int64_t cols, const float *x, float *y) {
    int64_t bpr = cols / 32;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < rows; i++) {
        float acc = 0.0f;
        for (int64_t b = 0; b < bpr; b++) {
            const uint8_t *r = w + (i * bpr + b) * 18;
            float dv = or_f16_to_f32(rd_u16(r));
            float dot = 0.0f;
            const float *xb = x + b * 32;
            for (int j = 0; j < 16; j++) {
                int q = r[2 + j];
                dot = dot + (float)((q & 15) - 8) * xb[j];
                dot = dot + (float)((q >> 4) - 8) * xb[j + 16];
            }
            acc = acc + dv * dot;
        }
        y[i] = acc;
    }
}

/* Quant.mxfp4MatVecIntoScalar (L/io/Quant.cajeta:1146-1182): f32 activations,
 * elements in natural order, acc = acc + code·d·x. */
static void mv_mxfp4(const uint8_t *w, int64_t rows, int64_t cols, const float *x, float *y) {
    int64_t bpr = cols / 32;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < rows; i++) {
        float acc = 0.0f;
        for (int64_t b = 0; b < bpr; b++) {
            const uint8_t *r = w + (i * bpr + b) * 17;
            float d = mxfp4_scale(r[0]);
            const float *xb = x + b * 32;
            for (int k = 0; k < 32; k++) {
                int byv = r[1 + (k & 15)];
                int nib = k < 16 ? (byv & 15) : ((byv >> 4) & 15);
                acc = acc + (float)mxfp4_code(nib) * d * xb[k];
            }
        }
        y[i] = acc;
    }
}

/* MXFP4 in the reference's device Q8 form, the two kernels of
 * QuantKernel.mxfp4MatVecCoopQ8Launch (L/io/QuantKernel.cajeta:43699-43713).
 *
 * mxfp4QuantActKernel (:43614-43636): per 32-element block the largest
 * |x| (order free: max is exact), inv = 127 / bmax (0 for an all-zero
 * block), q = Math.round(x·inv) (half away from zero, as the packs),
 * d = bmax / 127. */
void or_mxfp4_quant_act(const float *x, int64_t cols, int8_t *xq, float *xd) {
    for (int64_t b = 0; b < cols / 32; b++) {
        float bmax = 0.0f;
        for (int k = 0; k < 32; k++) {
            float v = fabsf(x[32 * b + k]);
            if (v > bmax) bmax = v;
        }
        float inv = bmax > 0.0f ? 127.0f / bmax : 0.0f;
        for (int k = 0; k < 32; k++) {
#if OR_PLANT == 15
            xq[32 * b + k] = (int8_t)round_away(x[32 * b + k] * inv * 0.5f);   /* planted: half the codes */
#else
            xq[32 * b + k] = (int8_t)round_away(x[32 * b + k] * inv);
#endif
        }
        xd[b] = bmax / 127.0f;
    }
}

/* mxfp4MatVecKernelCoopQ8 (:43660-43697): a row is a wave of 32 lanes; lane
 * L takes blocks L, L+32, ... in turn: s = the exact integer dot of the
 * block's 32 codes (Quant.mxfp4Kv's int8 table, :43273-43276; low nibbles
 * are elements 0..15, high 16..31) with the q8 codes, then
 * acc = acc + (float)s·d_w·d_x (left to right). The lanes' sums are folded
 * by Wave.reduceSumF32 over the 32 lanes, the xor butterfly (strides 16, 8,
 * 4, 2, 1: lane L adds lane L^k; specs/archive/wave-agnostic-coop-kernels-
 * spec.md:22-25 describes the wave reduces as that butterfly). */
static void mv_mxfp4_q8(const uint8_t *w, int64_t rows, int64_t cols, const int8_t *xq, const float *xd, float *y) {
    static const int8_t kv[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};
    int64_t bpr = cols / 32;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < rows; i++) {
        float acc[32];
        for (int l = 0; l < 32; l++) {
            acc[l] = 0.0f;
            for (int64_t b = l; b < bpr; b += 32) {
                const uint8_t *r = w + (i * bpr + b) * 17;
                float dw = mxfp4_scale(r[0]);
                const int8_t *xb = xq + b * 32;
                int32_t sdot = 0;
                for (int j = 0; j < 16; j++) {
                    sdot += kv[r[1 + j] & 15] * xb[j];
#if OR_PLANT == 16
                    sdot += kv[(r[1 + j] >> 4) & 15] * xb[j];          /* planted: high nibbles on the low half */
#else
                    sdot += kv[(r[1 + j] >> 4) & 15] * xb[16 + j];
#endif
                }
                acc[l] = acc[l] + (float)sdot * dw * xd[b];
            }
        }
        for (int k = 16; k > 0; k >>= 1)
            for (int l = 0; l < 32; l++)
                if (l < k) acc[l] = acc[l] + acc[l + k];
        y[i] = acc[0];
    }
}

/* Both kernels over an f32 activation: the MXFP4 mat-vec the engine's MoE
 * experts use. */
int or_matvec_mxfp4_q8(const uint8_t *w, int64_t rows, int64_t cols, const float *x, float *y) {
    if (cols % 32) return -1;
    int8_t *xq = (int8_t *)malloc((size_t)cols);
    float *xd = (float *)malloc(sizeof(float) * (size_t)(cols / 32));
    or_mxfp4_quant_act(x, cols, xq, xd);
    mv_mxfp4_q8(w, rows, cols, xq, xd, y);
    free(xq); free(xd);
    return 0;
}

/* F32 weights (the MoE router): HostOps.matvecRow (L/model/HostOps.cajeta:52-89),
 * the CPU backend's unpacked f32 Linear (Linear.matvecInto, L/model/Linear.cajeta:1996):
 * each output starts at 0 and adds x_i·w_i for i ascending. */
static void mv_f32(const float *w, int64_t rows, int64_t cols, const float *x, float *y) {
    for (int64_t i = 0; i < rows; i++) {
        float acc = 0.0f;
        for (int64_t c = 0; c < cols; c++) acc = acc + w[i * cols + c] * x[c];
        y[i] = acc;
    }
}

int or_matvec(int type, const uint8_t *w, int64_t rows, int64_t cols,
              const uint8_t *xp, const float *xf, float *y) {
    switch (type) {
    case OR_Q4_K: mv_q4k(w, rows, cols, xp, y); return 0;
    case OR_Q6_K: mv_q6k(w, rows, cols, xp, y); return 0;
    case OR_Q8_0: mv_q80(w, rows, cols, xp, y); return 0;
    case OR_Q4_0: mv_q40(w, rows, cols, xf, y); return 0;
    case OR_MXFP4: mv_mxfp4(w, rows, cols, xf, y); return 0;
    case OR_F32: mv_f32((const float *)w, rows, cols, xf, y); return 0;
    default: return -1;
    }
}

/* ------------------------------------------------------------ primitives */

/* RMSNorm in the order of the reference's device-decode norms: 256 lane
 * partials, lane j summing x[j + 256k]^2 in k order (ragged past n), folded
 * 128, 64, ..., 1. For whole 256s that is the CPU row form
 * (Prim.rmsnormPackRowCpuKernel, L/model/Prim.cajeta:977-1071); other widths
 * go to rmsnormRowF32 (:742-775) through Prim.rmsnormDevice (:1440-1450), the
 * resident layer's fallback when the fused norm + pack declines a width
 * (CausalLM.cajeta:3643, :3819; the final norm at :1635). The host floor's
 * element-order sum (Prim.rmsnormRowHost, :120-151) belongs to the
 * non-resident path and is not taken here. form 1 = (1 + w). */
void or_rmsnorm(const float *x, const float *w, int64_t n, float eps, int form, float *out) {
    float ss = 0.0f;
    float p[256];
    for (int j = 0; j < 256; j++) p[j] = 0.0f;
    for (int64_t k = 0; k * 256 < n; k++)
        for (int j = 0; j < 256 && k * 256 + j < n; j++) { float a = x[k * 256 + j]; p[j] = p[j] + a * a; }
    for (int s = 128; s > 0; s >>= 1)
        for (int j = 0; j < s; j++) p[j] = p[j] + p[j + s];
    ss = p[0];
#if OR_PLANT == 5
    float scale = 1.0f / sqrtf(ss / (float)n);     /* planted: eps dropped */
#else
    float scale = 1.0f / sqrtf(ss / (float)n + eps);
#endif
    for (int64_t i = 0; i < n; i++) {
        float wi = form == 1 ? 1.0f + w[i] : w[i];
        out[i] = x[i] * scale * wi;
    }
}

/* exp(x) in f32 as the reference CPU backend computes it. Its Math.exp is
 * glibc's expf: the reference's recorded CPU softmax outputs
 * (attnScoreKernel h32kv4d128c256, tests/golden/wave) are glibc expf's bits in
 * all 8192 values. glibc's expf is ARM optimized-routines' algorithm
 * (math/expf.c, EXP2F_TABLE_BITS 5): with z = x·32/ln2 in f64, k = round(z) by
 * adding 1.5·2^52 and r = z − k, both as fused multiply-adds of x (as the
 * FMA build of glibc computes them); 2^(k/32) from a table of 2^(i/32)
 * rounded to f64 with k's integer part added to the exponent bits; 2^(r/32)
 * as C0·r³ + C1·r² + C2·r + 1 in f64 by fused multiply-adds; rounded once to
 * f32. The table holds 2^(i/32) correctly rounded to f64 less i·2^47 in the
 * bit pattern. tests/test_oracle.py checks the table against 2^(i/32) and the
 * function against the C library's expf. */
static const uint64_t OR_EXP2_TAB[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
    0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
    0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
    0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
    0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
    0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL,
};
float or_expf(float x) {
    if (x != x) return x + x;
    if (x > 0x1.62e42ep6f) return INFINITY;
    if (x < -0x1.9fe368p6f) return 0.0f;
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / (32.0 * 32 * 32), c1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32),
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)x;
    double kd = fma(inv_ln2_n, xd, shift);
    uint64_t ki;
    memcpy(&ki, &kd, 8);
    kd = kd - shift;
    const double r = fma(inv_ln2_n, xd, -kd);
    const uint64_t sb = OR_EXP2_TAB[ki & 31] + (ki << 47);
    double s;
    memcpy(&s, &sb, 8);
#if OR_PLANT == 21
    const double z = c1, r2 = r * r;   /* planted: the cubic term dropped */
#else
    const double z = fma(c0, r, c1), r2 = r * r;
#endif
    double y = fma(c2, r, 1.0);
    y = fma(z, r2, y);
    return (float)(y * s);
}

/* The 2^(i/32) table of or_expf, for the check against its definition. */
void or_exp2_table(uint64_t *out) { memcpy(out, OR_EXP2_TAB, sizeof OR_EXP2_TAB); }

/* SwiGLU, exp form (Prim.gluF32/gluOne, L/model/Prim.cajeta:160-196):
 * silu(g) = g / (1 + exp(-g)). */
void or_glu_exp(const float *g, const float *u, int64_t n, float *out) {
    for (int64_t i = 0; i < n; i++) {
        float x = g[i];
        float a = x / (1.0f + or_expf(0.0f - x));
        out[i] = a * u[i];
    }
}

/* SwiGLU, the CPU backend's vector form (Prim.gluCpuKernel,
 * L/model/Prim.cajeta:214-273): silu = 0.5·x·(1 + tanh(x/2)) with tanh as
 * Eigen's published 13/6 rational approximation on an argument clamped to
 * ±7.90531110763549805; 16-wide chunks inside work blocks of 4096, the
 * remainder of a block in the exp form. */
static float glu_tanh_one(float x, float u) {
    const float tlo = -7.90531110763549805f;
    float xa = x > -16.0f ? x : -16.0f;
    float xb = -16.0f - xa;
    float xc = -16.0f - (xb > -32.0f ? xb : -32.0f);
    float t0 = 0.5f * fmaf(0.0f * xc, xc * xc, xc);
    float ta = t0 > tlo ? t0 : tlo;
    float tb = tlo - ta;
    float t = tlo - (tb > -15.8106222152709961f ? tb : -15.8106222152709961f);
    float t2 = t * t;
    float p = fmaf(-2.76076847742355e-16f, t2, 2.00018790482477e-13f);
    p = fmaf(p, t2, -8.60467152213735e-11f);
    p = fmaf(p, t2, 5.12229709037114e-08f);
    p = fmaf(p, t2, 1.48572235717979e-05f);
    p = fmaf(p, t2, 6.37261928875436e-04f);
    p = fmaf(p, t2, 4.89352455891786e-03f) * t;
    float q = fmaf(1.19825839466702e-06f, t2, 1.18534705686654e-04f);
    q = fmaf(q, t2, 2.26843463243900e-03f);
    q = fmaf(q, t2, 4.89352518554385e-03f);
    return 0.5f * xa * (1.0f + p / q) * u;
}
void or_glu_tanh(const float *g, const float *u, int64_t n, float *out) {
    for (int64_t b0 = 0; b0 < n; b0 += 4096) {
        int64_t hi = b0 + 4096 < n ? b0 + 4096 : n, i = b0;
#if OR_PLANT == 6
        for (; i + 16 <= hi; i++) out[i] = glu_tanh_one(g[i], u[i]);   /* planted: 16-wide chunks stepped by one */
#else
        for (; i + 16 <= hi; i += 16)
            for (int j = 0; j < 16; j++) out[i + j] = glu_tanh_one(g[i + j], u[i + j]);
#endif
        for (; i < hi; i++) { float x = g[i]; out[i] = x / (1.0f + or_expf(0.0f - x)) * u[i]; }
    }
}

/* Prim.invFreq, plain rope (L/model/Prim.cajeta:1866-1909): θ^(−2d/hd). */
void or_inv_freq(int hd, float theta, float *inv) {
    for (int d = 0; d < hd / 2; d++) inv[d] = powf(theta, (0.0f - (float)(2 * d)) / (float)hd);
}

/* Split-half RoPE (Prim.ropeRowHost, L/model/Prim.cajeta:1917-1940 and
 * qkPrepKernel, L/model/AttnKernel.cajeta:175-196): pair (d, d+hd/2). */
void or_rope(float *t, int nheads, int hd, int pos, const float *inv) {
    int half = hd / 2;
    for (int h = 0; h < nheads; h++) {
        float *b = t + (int64_t)h * hd;
        for (int d = 0; d < half; d++) {
            float ang = (float)pos * inv[d];
            float c = cosf(ang), s = sinf(ang);
            float a = b[d], bb = b[d + half];
            b[d] = a * c - bb * s;
#if OR_PLANT == 2
            b[d + half] = a * s - bb * c;                 /* planted: a sign */
#else
            b[d + half] = a * s + bb * c;
#endif
        }
    }
}

/* First-occurrence argmax (HostOps.argmaxRow, L/model/HostOps.cajeta:106-121). */
int or_argmax(const float *v, int64_t n) {
    int best = 0; float bv = v[0];
#if OR_PLANT == 3
    for (int64_t i = 1; i < n; i++) if (v[i] >= bv) { bv = v[i]; best = (int)i; }   /* planted: last occurrence */
#else
    for (int64_t i = 1; i < n; i++) if (v[i] > bv) { bv = v[i]; best = (int)i; }
#endif
    return best;
}

/* MoeFfn.routeFromLogits (L/model/MoeFfn.cajeta:908-986): full softmax over
 * the experts, top-k by probability (strict >, ties keep the lower index),
 * optional renormalisation by the clamped sum, then the expert_weights_scale
 * factor when it is neither 0 nor 1. Returns -1 on NaN logits. */
int or_moe_route(const float *lb, int ne, int k, int norm, float w_scale, int32_t *sel, float *w) {
    float probs[512];
    if (ne > 512) return -2;
    float mx = lb[0];
    for (int e = 1; e < ne; e++) if (lb[e] > mx) mx = lb[e];
    float sum = 0.0f;
    for (int e = 0; e < ne; e++) { float p = or_expf(lb[e] - mx); probs[e] = p; sum = sum + p; }
    for (int e = 0; e < ne; e++) probs[e] = probs[e] / sum;
    for (int j = 0; j < k; j++) {
        int best = -1; float bp = 0.0f;
        for (int e = 0; e < ne; e++)
#if OR_PLANT == 11
            if (probs[e] >= 0.0f && (best < 0 || probs[e] >= bp)) { best = e; bp = probs[e]; }   /* planted: ties keep the higher index */
#else
            if (probs[e] >= 0.0f && (best < 0 || probs[e] > bp)) { best = e; bp = probs[e]; }
#endif
        if (best < 0) return -1;
        sel[j] = best; w[j] = bp; probs[best] = -1.0f;
    }
#if OR_PLANT == 12
    norm = 0;                                   /* planted: the renormalisation dropped */
#endif
    if (norm) {
        float ws = 0.0f;
        for (int j = 0; j < k; j++) ws = ws + w[j];
        if (ws < 0.00006103515625f) ws = 0.00006103515625f;
        for (int j = 0; j < k; j++) w[j] = w[j] / ws;
    }
    if (w_scale != 0.0f && w_scale != 1.0f)
        for (int j = 0; j < k; j++) w[j] = w[j] * w_scale;
    return 0;
}

/* Checkpoint.unpermuteRows (L/io/Checkpoint.cajeta:236-274): GGUF row
 * (h·hd + 2b + a) holds HF row (h·hd + a·half + b). */
void or_unpermute_rows(const uint8_t *src, uint8_t *dst, int64_t rows, int64_t rb, int nh) {
    int64_t hd = rows / nh, half = hd / 2;
    for (int h = 0; h < nh; h++)
        for (int a = 0; a < 2; a++)
            for (int64_t b = 0; b < half; b++)
#if OR_PLANT == 8
                memcpy(dst + (h * hd + a * half + b) * rb, src + (h * hd + 2 * b + (1 - a)) * rb, (size_t)rb);
#else
                memcpy(dst + (h * hd + a * half + b) * rb, src + (h * hd + 2 * b + a) * rb, (size_t)rb);
#endif
}

/* ------------------------------------------------------------- attention */

static inline float kv_at(const void *plane, int f32, int64_t i) {
    return f32 ? ((const float *)plane)[i] : or_f16_to_f32(((const uint16_t *)plane)[i]);
}

/* AttnKernel.cpuSq16 / cpuHeadNorm (L/model/AttnKernel.cajeta:233-268): one
 * head's QK-norm at head size 128 — squares summed in pairs, the pairs
 * folded as a tree within each 16, two 16s a 32, the four 32s added in
 * order; scale = 1/sqrt(tot/128 + eps); x·scale·w (form 1: w + 1). */
static float sq16(const float *x) {
    float a[8];
    for (int j = 0; j < 8; j++) a[j] = x[2 * j] * x[2 * j] + x[2 * j + 1] * x[2 * j + 1];
    float c0 = a[0] + a[1], c1 = a[2] + a[3], c2 = a[4] + a[5], c3 = a[6] + a[7];
    return (c0 + c1) + (c2 + c3);
}

void or_head_norm128(float *x, const float *w, float eps, int form) {
    float w0 = sq16(x) + sq16(x + 16), w1 = sq16(x + 32) + sq16(x + 48);
    float w2 = sq16(x + 64) + sq16(x + 80), w3 = sq16(x + 96) + sq16(x + 112);
#if OR_PLANT == 10
    float tot = w0 + (w1 + (w2 + w3));                  /* planted: the 32s folded from the end */
#else
    float tot = ((w0 + w1) + w2) + w3;
#endif
    float scale = 1.0f / sqrtf(tot / 128.0f + eps);
    for (int j = 0; j < 128; j++) {
        float wi = form == 1 ? 1.0f + w[j] : w[j];
        x[j] = x[j] * scale * wi;
    }
}

/* AttnKernel.qkPrepCpuKernel (:272-354) at head size 128: every q and k head
 * normed (norm != 0), then RoPE with cos/sin of pos·inv[d] (or_rope). */
int or_qk_prep128(float *q, float *k, const float *qw, const float *kw, const float *inv, int nh, int nkv,
                  int norm, float eps, int form, int pos) {
    if (norm) {
        for (int h = 0; h < nh; h++) or_head_norm128(q + (int64_t)h * 128, qw, eps, form);
        for (int h = 0; h < nkv; h++) or_head_norm128(k + (int64_t)h * 128, kw, eps, form);
    }
    or_rope(q, nh, 128, pos, inv);
    or_rope(k, nkv, 128, pos, inv);
    return 0;
}

/* The generic qkPrepKernel (L/model/AttnKernel.cajeta:127-206), the CPU
 * backend's prep where qkPrepCpuKernel (head size 128 only) does not serve:
 * a workgroup of 128 lanes a head, lane l summing x[l]², x[l+128]², ... in
 * order; Workgroup.reduce folds each 32-lane wave by the butterfly from the
 * adjacent lane up (lane distance 1, 2, 4, 8, 16) and adds the four wave
 * sums in wave order — the order cpuHeadNorm writes out for head size 128
 * (:233-268) and the one the reference's recorded h6kv2d64 rows fix (the
 * stride-halving tree gives other bits for k head 0); scale =
 * 1/sqrt(tot/hd + eps); x·scale·w (form 1: w + 1); then RoPE. At head size
 * 128 the CPU kernel's order applies (or_qk_prep128). */
int or_qk_prep(float *q, float *k, const float *qw, const float *kw, const float *inv, int nh, int nkv, int hd,
               int norm, float eps, int form, int pos) {
    if (hd == 128) return or_qk_prep128(q, k, qw, kw, inv, nh, nkv, norm, eps, form, pos);
    if (hd > 256 || hd % 2) return -1;
    if (norm) {
        for (int h = 0; h < nh + nkv; h++) {
            float *x = h < nh ? q + (int64_t)h * hd : k + (int64_t)(h - nh) * hd;
            const float *w = h < nh ? qw : kw;
            float red[128];
            for (int l = 0; l < 128; l++) {
                float ss = 0.0f;
                for (int i = l; i < hd; i += 128) ss = ss + x[i] * x[i];
                red[l] = ss;
            }
            float tot = 0.0f;
            for (int wv = 0; wv < 4; wv++) {
                float *v = red + 32 * wv;
#if OR_PLANT == 19
                for (int l = 1; l < 32; l++) v[0] = v[0] + v[l];   /* planted: a wave's lanes summed in order */
#else
                for (int d = 1; d < 32; d <<= 1)
                    for (int l = 0; l < 32; l += 2 * d) v[l] = v[l] + v[l + d];
#endif
                tot = tot + v[0];
            }
            float scale = 1.0f / sqrtf(tot / (float)hd + eps);
            for (int j = 0; j < hd; j++) {
                float wi = form == 1 ? 1.0f + w[j] : w[j];
                x[j] = x[j] * scale * wi;
            }
        }
    }
    or_rope(q, nh, hd, pos, inv);
    or_rope(k, nkv, hd, pos, inv);
    return 0;
}

/* routerTopKKernel (L/io/QuantKernel.cajeta:39850-39960; launch :40701-40709)
 * on the CPU backend: block e's 256 lanes each sum w[e][j]·x[j] for j = lane,
 * lane+256, ... (each product rounded, then added), the lanes folded by the
 * stride-halving tree (128, ..., 1) — the order the reference's recorded
 * e128h2048k8 logits fix; then the last block's first wave of 32 lanes: the
 * max, each lane's sum of exp(logit − max) over its experts lane, lane+32,
 * ... in order, the 32 sums by the butterfly; `used` picks, each the largest
 * probability below the previous pick (equal probability: the next index
 * up), w = p/sum; the renormalisation by the ordered sum of w clamped at
 * 2^-14 (normTopk), then ×wScale unless it is 0 or 1. */
void or_router_topk(const float *w_router, const float *x, int experts, int cols, int used, int norm_topk,
                    float w_scale, float *logits, int32_t *sel, float *w) {
    for (int e = 0; e < experts; e++) {
        float red[256];
        for (int l = 0; l < 256; l++) {
            float acc = 0.0f;
            for (int j = l; j < cols; j += 256) acc = acc + w_router[(int64_t)e * cols + j] * x[j];
            red[l] = acc;
        }
#if OR_PLANT == 20
        for (int l = 1; l < 256; l++) red[0] = red[0] + red[l];   /* planted: the lanes summed in order */
#else
        for (int r = 128; r > 0; r >>= 1)
            for (int l = 0; l < r; l++) red[l] = red[l] + red[l + r];
#endif
        logits[e] = red[0];
    }
    float mx = -3.4028234663852886e38f;
    for (int e = 0; e < experts; e++) if (logits[e] > mx) mx = logits[e];
    float ls[32];
    for (int l = 0; l < 32; l++) {
        float s = 0.0f;
        for (int e = l; e < experts; e += 32) s = s + or_expf(logits[e] - mx);
        ls[l] = s;
    }
    for (int m = 16; m > 0; m >>= 1) {
        float nx[32];
        for (int i = 0; i < 32; i++) nx[i] = ls[i] + ls[i ^ m];
        memcpy(ls, nx, sizeof nx);
    }
    const float sum = ls[0];
    float vlast = 3.4028234663852886e38f;
    int ilast = experts;
    for (int k = 0; k < used; k++) {
        float vk = -1.0f;
        int ik = experts;
        for (int e = 0; e < experts; e++) {
            const float p = or_expf(logits[e] - mx);
            const int ok = p < vlast || (p == vlast && e > ilast);
#if OR_PLANT == 18
            if (ok && (p > vk || (p == vk && e > ik))) { vk = p; ik = e; }   /* planted: ties to the higher index */
#else
            if (ok && (p > vk || (p == vk && e < ik))) { vk = p; ik = e; }
#endif
        }
        sel[k] = ik;
        w[k] = vk / sum;
        vlast = vk;
        ilast = ik;
    }
    if (norm_topk) {
        float ws = 0.0f;
        for (int k = 0; k < used; k++) ws = ws + w[k];
        if (ws < 0.00006103515625f) ws = 0.00006103515625f;
        for (int k = 0; k < used; k++) w[k] = w[k] / ws;
    }
    if (w_scale != 0.0f && w_scale != 1.0f)
        for (int k = 0; k < used; k++) w[k] = w[k] * w_scale;
}

/* AttnKernel.cpuDecodeSplits (L/model/AttnKernel.cajeta:4879-4889). */
int or_cpu_decode_splits(int count, int rows, int nkv, int workers) {
    int w = workers < 1 ? 1 : workers, rk = rows * nkv < 1 ? 1 : rows * nkv;
    int s = (2 * w + rk - 1) / rk;
    if (s > 64) s = 64;
    if (s > count) s = count;
    if (s < 1) s = 1;
    return s;
}

/* AttnKernel.cpuDecodeHead (L/model/AttnKernel.cajeta:4216-4285): one query
 * head's online softmax over positions [t0, t1); 16-lane score partials,
 * folded pairwise; one exp per key. Writes acc[hd], m, l. */
static void decode_head(const float *q, const void *kp, const void *vp, int f32, int64_t kvdim,
                        int64_t koff, int hd, int t0, int t1, float scale, float *part) {
    float acc[256];
    for (int d = 0; d < hd; d++) acc[d] = 0.0f;
    float m = -3.0e38f, l = 0.0f;
    for (int t = t0; t < t1; t++) {
        int64_t ko = (int64_t)t * kvdim + koff;
        float dl[16];
        for (int j = 0; j < 16; j++) dl[j] = 0.0f;
        for (int v = 0; v < hd / 16; v++)
            for (int j = 0; j < 16; j++) {
                float pr = q[16 * v + j] * kv_at(kp, f32, ko + 16 * v + j);
                dl[j] = v == 0 ? pr : dl[j] + pr;
            }
        float sc = ((((dl[0] + dl[1]) + (dl[2] + dl[3])) + ((dl[4] + dl[5]) + (dl[6] + dl[7])))
                    + (((dl[8] + dl[9]) + (dl[10] + dl[11])) + ((dl[12] + dl[13]) + (dl[14] + dl[15])))) * scale;
        if (sc > m) {
            float c = or_expf(m - sc);
#if OR_PLANT != 7
            for (int d = 0; d < hd; d++) acc[d] = acc[d] * c;   /* (7 plants: the rescale dropped) */
#endif
            l = l * c;
            m = sc;
        }
        float p = or_expf(sc - m);
        l = l + p;
        for (int d = 0; d < hd; d++) acc[d] = acc[d] + kv_at(vp, f32, ko + d) * p;
    }
    for (int d = 0; d < hd; d++) part[d] = acc[d];
    part[hd] = m;
    part[hd + 1] = l;
}

/* reducePackBlockCpu's merge (L/model/AttnKernel.cajeta:5268-5400): per
 * head, the splits' (acc[hd], m, l) partials [nh][splits][hd+2] merge as
 * four interleaved sub-sums (splits s ≡ sub mod 4, ascending) of w·l and
 * w·acc with w = exp(m − max), added in sub order, then ·(1/Σ). */
void or_attn_merge(const float *part, int nh, int splits, int hd, float *out) {
    int stride = hd + 2;
    for (int h = 0; h < nh; h++) {
        const float *pb0 = part + (int64_t)h * splits * stride;
        float gm = -3.0e38f;
        for (int s = 0; s < splits; s++) if (pb0[s * stride + hd] > gm) gm = pb0[s * stride + hd];
        float tacc[256], gt = 0.0f;
        for (int sub = 0; sub < 4; sub++) {
            float a[256], gl = 0.0f;
            for (int d = 0; d < hd; d++) a[d] = 0.0f;
            for (int sp = sub; sp < splits; sp += 4) {
                const float *pb = pb0 + sp * stride;
                float ls = pb[hd + 1];
                if (ls > 0.0f) {
                    float wt = or_expf(pb[hd] - gm);
                    gl = gl + wt * ls;
                    for (int d = 0; d < hd; d++) a[d] = a[d] + pb[d] * wt;
                }
            }
            if (sub == 0) { for (int d = 0; d < hd; d++) tacc[d] = a[d]; gt = gl; }
            else { for (int d = 0; d < hd; d++) tacc[d] = tacc[d] + a[d]; gt = gt + gl; }
        }
        float rs = 1.0f / gt;
        for (int d = 0; d < hd; d++) out[(int64_t)h * hd + d] = tacc[d] * rs;
    }
}

/* attnScoreKernel's score (L/model/AttnKernel.cajeta:397-425): lane i of 32
 * sums q[d]·k[d] over d = i, i+32, ... in order; the 32 lane sums fold as the
 * butterfly (lane distance 16, 8, 4, 2, 1 — Wave.reduceSumF32; pinned by the
 * reference's recorded h32kv4d128c256 row); × scale. */
static float score32(const float *qh, const void *kp, int f32, int64_t ko, int hd, float scale) {
    float ls[32];
    for (int i = 0; i < 32; i++) {
        float s = 0.0f;
        for (int d = i; d < hd; d += 32) s = s + qh[d] * kv_at(kp, f32, ko + d);
        ls[i] = s;
    }
    for (int m = 16; m > 0; m >>= 1) {
        float nx[32];
        for (int i = 0; i < 32; i++) nx[i] = ls[i] + ls[i ^ m];
        memcpy(ls, nx, sizeof nx);
    }
    return ls[0] * scale;
}

void or_attn_scores(const float *q, const void *kp, int f32, int nh, int nkv, int hd, int count, float scale,
                    int softmax, float *scores) {
    const int group = nh / nkv;
    const int64_t kvdim = (int64_t)nkv * hd;
    for (int h = 0; h < nh; h++) {
        float *sc = scores + (int64_t)h * count;
        for (int t = 0; t < count; t++) sc[t] = score32(q + (int64_t)h * hd, kp, f32, (int64_t)t * kvdim + (h / group) * hd, hd, scale);
        if (!softmax) continue;
        /* attnCombineKernel passes 1-2 (:441-486): the max (exact in any
         * order), then exp(s − max) in place */
        float mx = -3.0e38f;
        for (int t = 0; t < count; t++) if (sc[t] > mx) mx = sc[t];
        for (int t = 0; t < count; t++) sc[t] = or_expf(sc[t] - mx);
    }
}

void or_attend(const float *q, const void *kp, const void *vp, int f32, int nh, int nkv, int hd,
               int count, int splits, float scale, int mode, float *out) {
    int64_t kvdim = (int64_t)nkv * hd;
    int group = nh / nkv;
    if (mode == 0) {
        /* attnDecodeCpuGqaKernel (:4289-4314) + reducePackBlockCpu (:5268-5400):
         * splits of ceil(count/splits) positions; merge in four interleaved
         * sub-sums (sp ≡ sub mod 4) added in sub order, then ·(1/Σ w·l). */
        int stride = hd + 2;
        float *part = (float *)malloc(sizeof(float) * (size_t)nh * splits * stride);
        int chunk = (count + splits - 1) / splits;
#pragma omp parallel for collapse(2) schedule(static)
        for (int kvh = 0; kvh < nkv; kvh++)
            for (int sp = 0; sp < splits; sp++) {
                int t0 = sp * chunk, t1 = t0 + chunk;
                if (t1 > count) t1 = count;
                if (t0 > count) t0 = count;
                for (int h = 0; h < group; h++) {
                    int hh = kvh * group + h;
                    decode_head(q + (int64_t)hh * hd, kp, vp, f32, kvdim, (int64_t)kvh * hd, hd, t0, t1,
                                scale, part + ((int64_t)hh * splits + sp) * stride);
                }
            }
        or_attn_merge(part, nh, splits, hd, out);
        free(part);
    } else {
        /* attnScoreKernel (:397-425): lane i of 32 sums q[d]·k[d] over
         * d = i, i+32, ... in order; the 32 lane sums fold as a butterfly
         * (lane distance 16, 8, 4, 2, 1 — the wave reduction, whose order the
         * reference's stdlib leaves open); × scale.
         * attnCombineKernel (:441-515): 128 lanes, lane l over t = l, l+128, ...:
         * max (exact in any order), exp(s − max) and its lane sums, the lane
         * sums folded with strides 64, ..., 1; then Σ_t p_t·v_t in ascending t,
         * scaled once by 1/Σp. */
        float *sc = (float *)malloc(sizeof(float) * (size_t)count);
        for (int h = 0; h < nh; h++) {
            int kvh = h / group;
            for (int t = 0; t < count; t++) sc[t] = score32(q + (int64_t)h * hd, kp, f32, (int64_t)t * kvdim + kvh * hd, hd, scale);
            float mx = -3.0e38f;
            for (int t = 0; t < count; t++) if (sc[t] > mx) mx = sc[t];
            float red[128];
            for (int l = 0; l < 128; l++) {
                float s = 0.0f;
                for (int t = l; t < count; t += 128) { float e = or_expf(sc[t] - mx); sc[t] = e; s = s + e; }
                red[l] = s;
            }
            for (int r = 64; r > 0; r >>= 1)
                for (int l = 0; l < r; l++) red[l] = red[l] + red[l + r];
            float sum = red[0];
            float rs = 1.0f / sum;
            for (int d = 0; d < hd; d++) {
                float acc = 0.0f;
                for (int t = 0; t < count; t++)
                    acc = acc + sc[t] * kv_at(vp, f32, (int64_t)t * kvdim + kvh * hd + d);
                out[(int64_t)h * hd + d] = acc * rs;
            }
        }
        free(sc);
    }
}

/* AttnKernel.attnPrefillCpuGqaKernel (L/model/AttnKernel.cajeta:3916-4004),
 * the CPU backend's prefill attend at head size 128: one pass per (row,
 * query head) over positions [t0, count) with an online softmax. Unlike the
 * decode form, q is scaled first (q·scale, rounded, then the dot), the
 * running max starts at -1e30, and the output is acc·(1/l). The score of a
 * key: 16 lane partials d_j = Σ_v qs[16v+j]·k[16v+j] (v ascending, each
 * product rounded then added) folded by the fixed pairwise tree. */
void or_prefill_attend(const float *q, const void *kp, const void *vp, int f32, int nh, int nkv, int hd,
                       int start, int rows, int window, float scale, float *out) {
    int64_t kvdim = (int64_t)nkv * hd;
    int group = nh / nkv;
    /* fp16 planes are widened to f32 once (exact), then read as f32 */
    float *kw = NULL, *vw = NULL;
    if (!f32) {
        int64_t n = (int64_t)(start + rows) * kvdim;
        kw = (float *)malloc(sizeof(float) * (size_t)n);
        vw = (float *)malloc(sizeof(float) * (size_t)n);
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < n; i++) {
            kw[i] = or_f16_to_f32(((const uint16_t *)kp)[i]);
            vw[i] = or_f16_to_f32(((const uint16_t *)vp)[i]);
        }
        kp = kw; vp = vw; f32 = 1;
    }
#pragma omp parallel for collapse(2) schedule(dynamic, 4)
    for (int kvh = 0; kvh < nkv; kvh++)
        for (int r = 0; r < rows; r++) {
            int count = start + r + 1, t0 = 0;
            if (window > 0 && count > window) t0 = count - window;
            for (int h = 0; h < group; h++) {
                int hh = kvh * group + h;
                const float *qr = q + (int64_t)r * nh * hd + (int64_t)hh * hd;
                float qs[128], acc[128];
                for (int d = 0; d < hd; d++) { qs[d] = qr[d] * scale; acc[d] = 0.0f; }
                float m = -1.0e30f, l = 0.0f;
                for (int t = t0; t < count; t++) {
                    int64_t ko = (int64_t)t * kvdim + (int64_t)kvh * hd;
                    float dl[16];
                    for (int j = 0; j < 16; j++) dl[j] = qs[j] * kv_at(kp, f32, ko + j);
                    for (int v = 1; v < hd / 16; v++)
                        for (int j = 0; j < 16; j++) dl[j] = dl[j] + qs[16 * v + j] * kv_at(kp, f32, ko + 16 * v + j);
#if OR_PLANT == 9
                    float sc = dl[0];                                  /* planted: lane 0's partial only */
#else
                    float sc = ((((dl[0] + dl[1]) + (dl[2] + dl[3])) + ((dl[4] + dl[5]) + (dl[6] + dl[7])))
                                + (((dl[8] + dl[9]) + (dl[10] + dl[11])) + ((dl[12] + dl[13]) + (dl[14] + dl[15]))));
#endif
                    if (sc > m) {
                        float c = or_expf(m - sc);
                        for (int d = 0; d < hd; d++) acc[d] = acc[d] * c;
                        l = l * c;
                        m = sc;
                    }
                    float p = or_expf(sc - m);
                    l = l + p;
                    for (int d = 0; d < hd; d++) acc[d] = acc[d] + kv_at(vp, f32, ko + d) * p;
                }
                float inv = 1.0f / l;
                float *o = out + (int64_t)r * nh * hd + (int64_t)hh * hd;
                for (int d = 0; d < hd; d++) o[d] = acc[d] * inv;
            }
        }
    free(kw); free(vw);
}

/* ------------------------------------------------------------------ model */

typedef struct { int type; const uint8_t *data; int64_t rows, cols; } or_tensor;
typedef struct {
    or_tensor attn_norm, q, k, v, o, ffn_norm, gate, up, down;
    or_tensor router, gate_exps, up_exps, down_exps;
} or_layer;

struct or_model {
    or_config c;
    or_tensor embd, out_norm, head;
    or_layer *L;
    void **kc, **vc;             /* per-layer K/V planes [ctx][n_kv*hd] */
    float *inv;
    /* scratch */
    float *hs, *xn, *q, *k, *v, *ao, *y, *g, *u, *logits, *eo, *acc;
    uint8_t *pk;
};

or_model *or_model_new(const or_config *cfg) {
    or_model *m = (or_model *)calloc(1, sizeof(or_model));
    m->c = *cfg;
    int nl = cfg->n_layers;
    m->L = (or_layer *)calloc((size_t)nl, sizeof(or_layer));
    m->kc = (void **)calloc((size_t)nl, sizeof(void *));
    m->vc = (void **)calloc((size_t)nl, sizeof(void *));
    size_t es = cfg->kv_f32 ? 4 : 2;
    size_t plane = (size_t)cfg->ctx * cfg->n_kv * cfg->head_dim * es;
    for (int l = 0; l < nl; l++) { m->kc[l] = calloc(1, plane); m->vc[l] = calloc(1, plane); }
    m->inv = (float *)malloc(sizeof(float) * (size_t)cfg->head_dim / 2);
    or_inv_freq(cfg->head_dim, cfg->theta, m->inv);
    int64_t h = cfg->hidden, qd = (int64_t)cfg->n_heads * cfg->head_dim, kvd = (int64_t)cfg->n_kv * cfg->head_dim;
    int64_t f = cfg->ffn > cfg->expert_ffn ? cfg->ffn : cfg->expert_ffn;
    int64_t wmax = h > qd ? h : qd; if (f > wmax) wmax = f;
    m->hs = calloc((size_t)h, 4); m->xn = calloc((size_t)wmax, 4); m->q = calloc((size_t)qd, 4);
    m->k = calloc((size_t)kvd, 4); m->v = calloc((size_t)kvd, 4); m->ao = calloc((size_t)qd, 4);
    m->y = calloc((size_t)wmax, 4); m->g = calloc((size_t)f + 256, 4); m->u = calloc((size_t)f + 256, 4);
    m->logits = calloc((size_t)cfg->vocab, 4); m->eo = calloc((size_t)h, 4); m->acc = calloc((size_t)h, 4);
    m->pk = calloc((size_t)((wmax + 255) / 256) * 320, 1);
    return m;
}

void or_model_free(or_model *m) {
    if (!m) return;
    for (int l = 0; l < m->c.n_layers; l++) { free(m->kc[l]); free(m->vc[l]); }
    free(m->kc); free(m->vc); free(m->L); free(m->inv);
    free(m->hs); free(m->xn); free(m->q); free(m->k); free(m->v); free(m->ao); free(m->y);
    free(m->g); free(m->u); free(m->logits); free(m->eo); free(m->acc); free(m->pk);
    free(m);
}

void or_model_reset(or_model *m) {
    size_t es = m->c.kv_f32 ? 4 : 2;
    size_t plane = (size_t)m->c.ctx * m->c.n_kv * m->c.head_dim * es;
    for (int l = 0; l < m->c.n_layers; l++) { memset(m->kc[l], 0, plane); memset(m->vc[l], 0, plane); }
}

/* A model's precomputed RoPE factors (GGUF rope_freqs.weight, hd/2 of
 * them): inv[d] = inv[d] / f[d] where f[d] != 0 (Attention's constructor,
 * L/model/Attention.cajeta:80-100; read by ModelConfig,
 * L/model/ModelConfig.cajeta:307-316). Refused (-1) unless n = hd/2. */
int or_model_set_rope_freqs(or_model *m, const float *f, int n) {
    int half = m->c.head_dim / 2;
    if (n != half) return -1;
    for (int d = 0; d < half; d++)
#if OR_PLANT == 17
        if (f[d] != 0.0f) m->inv[d] = m->inv[d] * f[d];      /* planted: multiplied, not divided */
#else
        if (f[d] != 0.0f) m->inv[d] = m->inv[d] / f[d];
#endif
    return 0;
}

/* The CPU worker count the decode split rule divides (the reference's
 * EngineOptions.cpuThreads, AttnKernel.cpuDecodeSplits :4879-4889); the
 * KV planes are kept, so decode steps can be replayed at another count. */
void or_model_set_workers(or_model *m, int workers) { m->c.workers = workers; }

int64_t or_model_trace(or_model *m, int what, float *out, int64_t n) {
    const or_config *c = &m->c;
    const float *src; int64_t cap;
    switch (what) {
    case 0: src = m->hs; cap = c->hidden; break;
    case 1: src = m->q; cap = (int64_t)c->n_heads * c->head_dim; break;
    case 2: src = m->ao; cap = (int64_t)c->n_heads * c->head_dim; break;
    case 3: src = m->g; cap = c->ffn; break;
    case 4: src = m->logits; cap = c->vocab; break;
    case 5: src = m->inv; cap = c->head_dim / 2; break;
    default: return -1;
    }
    if (n > cap) n = cap;
    memcpy(out, src, sizeof(float) * (size_t)n);
    return n;
}

int or_model_bind(or_model *m, const char *name, int type, const void *data, int64_t rows, int64_t cols) {
    or_tensor t = {type, (const uint8_t *)data, rows, cols};
    if (!strcmp(name, "token_embd.weight")) { m->embd = t; return 0; }
    if (!strcmp(name, "output_norm.weight")) { m->out_norm = t; return 0; }
    if (!strcmp(name, "output.weight")) { m->head = t; return 0; }
    int l; char rest[96];
    if (sscanf(name, "blk.%d.%95s", &l, rest) != 2 || l < 0 || l >= m->c.n_layers) return -1;
    or_layer *L = &m->L[l];
    if (!strcmp(rest, "attn_norm.weight")) L->attn_norm = t;
    else if (!strcmp(rest, "attn_q.weight")) L->q = t;
    else if (!strcmp(rest, "attn_k.weight")) L->k = t;
    else if (!strcmp(rest, "attn_v.weight")) L->v = t;
    else if (!strcmp(rest, "attn_output.weight")) L->o = t;
    else if (!strcmp(rest, "ffn_norm.weight")) L->ffn_norm = t;
    else if (!strcmp(rest, "ffn_gate.weight")) L->gate = t;
    else if (!strcmp(rest, "ffn_up.weight")) L->up = t;
    else if (!strcmp(rest, "ffn_down.weight")) L->down = t;
    else if (!strcmp(rest, "ffn_gate_inp.weight")) L->router = t;
    else if (!strcmp(rest, "ffn_gate_exps.weight")) L->gate_exps = t;
    else if (!strcmp(rest, "ffn_up_exps.weight")) L->up_exps = t;
    else if (!strcmp(rest, "ffn_down_exps.weight")) L->down_exps = t;
    else return -1;
    return 0;
}

/* Which pack a weight reads on the CPU backend (Linear.act32Here,
 * L/model/Linear.cajeta:1189-1192): Q8_0 per 32, K-quants per 256. */
static int act32(int type) { return type == OR_Q8_0; }

/* Stage x (n values) as the activation `type` reads, then y = W·x. */
static void linear(or_model *m, const or_tensor *w, const float *x, float *y) {
    int64_t npad = (w->cols + 255) / 256 * 256;
    if (w->type == OR_MXFP4) {   /* the device Q8 form (mxfp4MatVecCoopQ8Launch) */
        or_matvec_mxfp4_q8(w->data, w->rows, w->cols, x, y);
        return;
    }
    if (w->type == OR_Q4_0 || w->type == OR_F32) {
        or_matvec(w->type, w->data, w->rows, w->cols, NULL, x, y);
        return;
    }
    if (act32(w->type)) or_q8k_pack32(x, w->cols, npad, m->pk);
    else or_q8k_pack(x, w->cols, npad, m->pk);
    or_matvec(w->type, w->data, w->rows, w->cols, m->pk, NULL, y);
}

static void embed_row(or_model *m, int token, float *out) {
    const or_tensor *e = &m->embd;
    int64_t h = m->c.hidden;
    int be = or_block_elems(e->type), bb = or_block_bytes(e->type);
    int64_t row_bytes = h / be * bb;
    or_dequant(e->type, e->data + (int64_t)token * row_bytes, h / be, out);
}

/* One MoE FFN row (MoeFfn.forwardRow, L/model/MoeFfn.cajeta:1849-1913):
 * router logits, route, Σ_k w_k · down(silu(gate x) · up x). Expert tensors
 * are stacked [E][rows][cols] in one buffer each. */
static void moe_ffn(or_model *m, or_layer *L, const float *xn, float *out) {
    int ne = m->c.n_experts, nu = m->c.n_used;
    int64_t h = m->c.hidden, ef = m->c.expert_ffn;
    float lg[512]; int32_t sel[64]; float w[64];
    or_matvec(L->router.type, L->router.data, ne, h, NULL, xn, lg);
    or_moe_route(lg, ne, nu, m->c.norm_topk, m->c.w_scale, sel, w);
    for (int64_t j = 0; j < h; j++) m->acc[j] = 0.0f;
    for (int k = 0; k < nu; k++) {
        int e = sel[k];
        int64_t gb = ef * h / or_block_elems(L->gate_exps.type) * or_block_bytes(L->gate_exps.type);
        int64_t db = h * ef / or_block_elems(L->down_exps.type) * or_block_bytes(L->down_exps.type);
        or_tensor gt = {L->gate_exps.type, L->gate_exps.data + e * gb, ef, h};
        or_tensor ut = {L->up_exps.type, L->up_exps.data + e * gb, ef, h};
        or_tensor dt = {L->down_exps.type, L->down_exps.data + e * db, h, ef};
        linear(m, &gt, xn, m->g);
        linear(m, &ut, xn, m->u);
        or_glu_exp(m->g, m->u, ef, m->g);
        linear(m, &dt, m->g, m->eo);
        for (int64_t j = 0; j < h; j++) m->acc[j] = m->acc[j] + w[k] * m->eo[j];
    }
    memcpy(out, m->acc, sizeof(float) * (size_t)h);
}

/* The attention window of layer l: the configured window on windowed layers,
 * 0 (every position) on the global ones. A pattern P makes every P-th layer
 * global, (l + 1) % P == 0 (ModelConfig.gemma3Gguf,
 * L/model/ModelConfig.cajeta:570-576); gpt-oss alternates, P = 2. */
static int layer_window(const or_config *c, int l) {
    int p = c->swa_pattern > 0 ? c->swa_pattern : 2;
    return c->swa_window > 0 && ((l + 1) % p) != 0 ? c->swa_window : 0;
}

/* One decode token through every layer and the tail, in the order
 * CausalLM.residentLayer takes (L/model/CausalLM.cajeta:3625-3935) and the
 * fused tail (:1614-1661). */
int or_model_step(or_model *m, int token, int pos, float *logits) {
    or_config *c = &m->c;
    int64_t h = c->hidden, hd = c->head_dim, nh = c->n_heads, nkv = c->n_kv;
    int64_t kvd = nkv * hd;
    float scale = 1.0f / sqrtf((float)hd);
    embed_row(m, token, m->hs);
    for (int l = 0; l < c->n_layers; l++) {
        or_layer *L = &m->L[l];
        /* attention sublayer */
        or_rmsnorm(m->hs, (const float *)L->attn_norm.data, h, c->eps, 0, m->xn);
        linear(m, &L->q, m->xn, m->q);
        linear(m, &L->k, m->xn, m->k);
        linear(m, &L->v, m->xn, m->v);
        or_rope(m->q, (int)nh, (int)hd, pos, m->inv);
        or_rope(m->k, (int)nkv, (int)hd, pos, m->inv);
        for (int64_t i = 0; i < kvd; i++) {
            int64_t at = (int64_t)pos * kvd + i;
            if (c->kv_f32) { ((float *)m->kc[l])[at] = m->k[i]; ((float *)m->vc[l])[at] = m->v[i]; }
            else { ((uint16_t *)m->kc[l])[at] = or_f32_to_f16(m->k[i]); ((uint16_t *)m->vc[l])[at] = or_f32_to_f16(m->v[i]); }
        }
        /* the window clamps the range: PagedKvCache.attendRow
         * (L/model/PagedKvCache.cajeta:380-388), from = p + 1 - w */
        int count = pos + 1, from = 0;
        const int win = layer_window(c, l);
#if OR_PLANT == 13
        if (win > 0 && count > win) { from = count - win + 1; count = win - 1; }   /* planted: one position short */
#else
        if (win > 0 && count > win) { from = count - win; count = win; }
#endif
        size_t es = c->kv_f32 ? 4 : 2;
        const uint8_t *kb = (const uint8_t *)m->kc[l] + (size_t)from * kvd * es;
        const uint8_t *vb = (const uint8_t *)m->vc[l] + (size_t)from * kvd * es;
        int flash = hd == 128 && (nh == 4 * nkv || nh == 8 * nkv);
        int splits = flash ? or_cpu_decode_splits(count, c->attn_rows > 0 ? c->attn_rows : 1, (int)nkv, c->workers) : 1;
        or_attend(m->q, kb, vb, c->kv_f32, (int)nh, (int)nkv, (int)hd, count, splits, scale, flash ? 0 : 1, m->ao);
        linear(m, &L->o, m->ao, m->y);
        for (int64_t i = 0; i < h; i++) m->hs[i] = m->hs[i] + m->y[i];
        /* FFN sublayer */
        or_rmsnorm(m->hs, (const float *)L->ffn_norm.data, h, c->eps, 0, m->xn);
        if (c->n_experts > 0) {
            moe_ffn(m, L, m->xn, m->y);
        } else {
            int64_t f = c->ffn;
            linear(m, &L->gate, m->xn, m->g);
            linear(m, &L->up, m->xn, m->u);
            /* Prim.gluPackDevice fuses the exp form where the width is whole
             * 256s; otherwise Prim.gluDevice takes the CPU vector form. */
            if (f % 256 == 0) or_glu_exp(m->g, m->u, f, m->g);
            else or_glu_tanh(m->g, m->u, f, m->g);
            linear(m, &L->down, m->g, m->y);
        }
        for (int64_t i = 0; i < h; i++) m->hs[i] = m->hs[i] + m->y[i];
    }
    or_rmsnorm(m->hs, (const float *)m->out_norm.data, h, c->eps, 0, m->xn);
    linear(m, &m->head, m->xn, m->logits);
    if (logits) memcpy(logits, m->logits, sizeof(float) * (size_t)c->vocab);
    return or_argmax(m->logits, c->vocab);
}

/* The FFN sublayer of one row in place on hs (CausalLM.residentLayer steps
 * 7-10; the same per row in the many-row forward). */
static void ffn_row(or_model *m, or_layer *L, float *hs) {
    or_config *c = &m->c;
    int64_t h = c->hidden;
    or_rmsnorm(hs, (const float *)L->ffn_norm.data, h, c->eps, 0, m->xn);
    if (c->n_experts > 0) {
        moe_ffn(m, L, m->xn, m->y);
    } else {
        int64_t f = c->ffn;
        linear(m, &L->gate, m->xn, m->g);
        linear(m, &L->up, m->xn, m->u);
        if (f % 256 == 0) or_glu_exp(m->g, m->u, f, m->g);
        else or_glu_tanh(m->g, m->u, f, m->g);
        linear(m, &L->down, m->g, m->y);
    }
    for (int64_t i = 0; i < h; i++) hs[i] = hs[i] + m->y[i];
}

/* CausalLM.stepSeq with n > 1 (L/model/CausalLM.cajeta:801-883) →
 * forwardRowsBatched (:2873): every row through a layer before the next
 * layer; each row's norms, projections (the many-row kernels equal the
 * one-row kernel column by column, T/selftest/CpuInt8MatVecTest.cajeta:225-300),
 * RoPE and K/V append as in a decode step; the attention of all rows once
 * their K/V are appended (the prefill attend above, served at head size 128,
 * AttnKernel.cpuAttnServes :4439-4447); the tail on the last row only
 * (interior argmaxes are discarded, :793-799). Served like the MI355X
 * engine serves it: dense models at head size 128 whose projections read
 * int8 packs; anything else prefills one decode step a position. */
int or_model_prefill(or_model *m, const int32_t *tokens, int n, int start, float *logits) {
    or_config *c = &m->c;
    int64_t h = c->hidden, hd = c->head_dim, nh = c->n_heads, nkv = c->n_kv;
    int64_t kvd = nkv * hd, qd = nh * hd;
    if (n <= 0) return -1;
    int rows_form = n > 1 && hd == 128 && c->n_experts == 0;
    for (int l = 0; rows_form && l < c->n_layers; l++) {
        const or_tensor *ws[4] = {&m->L[l].q, &m->L[l].o, &m->L[l].gate, &m->L[l].down};
        for (int i = 0; i < 4; i++)
            if (ws[i]->type == OR_Q4_0 || ws[i]->type == OR_MXFP4 || ws[i]->type == OR_F32) rows_form = 0;
    }
    if (!rows_form) {
        int t = -1;
        for (int r = 0; r < n; r++) t = or_model_step(m, tokens[r], start + r, r == n - 1 ? logits : NULL);
        return t;
    }
    float scale = 1.0f / sqrtf((float)hd);
    float *HS = (float *)malloc(sizeof(float) * (size_t)(n * h));
    float *Q = (float *)malloc(sizeof(float) * (size_t)(n * qd));
    float *AO = (float *)malloc(sizeof(float) * (size_t)(n * qd));
    for (int r = 0; r < n; r++) embed_row(m, tokens[r], HS + (int64_t)r * h);
    for (int l = 0; l < c->n_layers; l++) {
        or_layer *L = &m->L[l];
        for (int r = 0; r < n; r++) {
            int pos = start + r;
            or_rmsnorm(HS + (int64_t)r * h, (const float *)L->attn_norm.data, h, c->eps, 0, m->xn);
            linear(m, &L->q, m->xn, Q + (int64_t)r * qd);
            linear(m, &L->k, m->xn, m->k);
            linear(m, &L->v, m->xn, m->v);
            or_rope(Q + (int64_t)r * qd, (int)nh, (int)hd, pos, m->inv);
            or_rope(m->k, (int)nkv, (int)hd, pos, m->inv);
            for (int64_t i = 0; i < kvd; i++) {
                int64_t at = (int64_t)pos * kvd + i;
                if (c->kv_f32) { ((float *)m->kc[l])[at] = m->k[i]; ((float *)m->vc[l])[at] = m->v[i]; }
                else { ((uint16_t *)m->kc[l])[at] = or_f32_to_f16(m->k[i]); ((uint16_t *)m->vc[l])[at] = or_f32_to_f16(m->v[i]); }
            }
        }
        int window = layer_window(c, l);
        or_prefill_attend(Q, m->kc[l], m->vc[l], c->kv_f32, (int)nh, (int)nkv, (int)hd, start, n, window, scale, AO);
        for (int r = 0; r < n; r++) {
            float *hs = HS + (int64_t)r * h;
            linear(m, &L->o, AO + (int64_t)r * qd, m->y);
            for (int64_t i = 0; i < h; i++) hs[i] = hs[i] + m->y[i];
            ffn_row(m, L, hs);
        }
    }
    memcpy(m->hs, HS + (int64_t)(n - 1) * h, sizeof(float) * (size_t)h);
    memcpy(m->q, Q + (int64_t)(n - 1) * qd, sizeof(float) * (size_t)qd);
    memcpy(m->ao, AO + (int64_t)(n - 1) * qd, sizeof(float) * (size_t)qd);
    free(HS); free(Q); free(AO);
    or_rmsnorm(m->hs, (const float *)m->out_norm.data, h, c->eps, 0, m->xn);
    linear(m, &m->head, m->xn, m->logits);
    if (logits) memcpy(logits, m->logits, sizeof(float) * (size_t)c->vocab);
    return or_argmax(m->logits, c->vocab);
}
