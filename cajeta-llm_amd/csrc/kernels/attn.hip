// attn.hip — decode attention for gfx950 over the paged fp16 K/V planes.
//
// K/V layout (MI355X-native): pages of 64 positions, head-major inside a
// page, so one kv head's 64 positions are one contiguous 64·hd·2-byte run:
//   element (pos, kvh, d) at ((pgtab[base + pos/64]·n_kv + kvh)·64 + pos%64)·hd + d
//
// cj_attn_decode: split-K over the context. One workgroup of 4 waves per
// (kv head, split); hd/16 lanes share a position (16 dims, two 128-bit loads
// of K and of V each), 64/(hd/16) positions per step, every lane an
// independent online softmax for its positions and all the group's query
// heads. Lanes fold per wave, the 4 waves fold through LDS into one partial
// (acc, m, l) per query head; the last split of a kv head to finish merges
// every split (the reference's reduce) into f32.
#include "common.h"

DEV int64_t kv_at(const int32_t *pgtab, int pg_base, int pos, int nkv, int kvh, int hd) {
    const int page = pgtab[pg_base + (pos >> 6)];
    return (((int64_t)page * nkv + kvh) * 64 + (pos & 63)) * hd;
}

DEV void h8_to_f(const uint4 v, float *f) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; i++) { f[2 * i] = h2f(w[i]); f[2 * i + 1] = h2f(w[i] >> 16); }
}

template <int HD, int G>
DEV void attn_body(const cj_attn_args &a) {
    constexpr int LP = HD / 16;       // lanes per position
    constexpr int P = 64 / LP;        // positions per wave step
    constexpr int U = 2;              // steps in flight
    constexpr int PIECE = P * U;      // positions a wave takes at a time
    __shared__ float wm[4][G], wl[4][G];
    __shared__ float wacc[4][G][HD];
    __shared__ int ticket;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int kvh = blockIdx.x / a.splits, sp = blockIdx.x % a.splits;
    const int p = lane / LP, j = lane % LP;
    int count, from;
    if (a.state) { count = a.state->pos + 1; from = 0; } else { count = a.count; from = a.from; }
    if (a.window > 0 && count > a.window) { from += count - a.window; count = a.window; }
    int chunk = (count + a.splits - 1) / a.splits;
    chunk = (chunk + PIECE - 1) / PIECE * PIECE;
    const int t0 = sp * chunk;
    const int t1 = t0 + chunk < count ? t0 + chunk : count;

    float qv[G][16];
#pragma unroll
    for (int h = 0; h < G; h++)
#pragma unroll
        for (int d = 0; d < 16; d++) qv[h][d] = a.q[(int64_t)(kvh * G + h) * HD + 16 * j + d];
    float m[G], l[G], acc[G][16];
#pragma unroll
    for (int h = 0; h < G; h++) {
        m[h] = -3.0e38f; l[h] = 0.0f;
#pragma unroll
        for (int d = 0; d < 16; d++) acc[h][d] = 0.0f;
    }

    for (int tb = t0 + wave * PIECE; tb < t1; tb += 4 * PIECE) {
        uint4 kr[U][2], vr[U][2];
        bool ok[U];
#pragma unroll
        for (int uu = 0; uu < U; uu++) {
            const int t = tb + uu * P + p;
            ok[uu] = t < t1;
            const int tt = from + (ok[uu] ? t : t0);
            const int64_t base = kv_at(a.pgtab, a.pg_base, tt, a.n_kv, kvh, HD) + 16 * j;
            kr[uu][0] = *(const uint4 *)(a.kc + base);
            kr[uu][1] = *(const uint4 *)(a.kc + base + 8);
            vr[uu][0] = *(const uint4 *)(a.vc + base);
            vr[uu][1] = *(const uint4 *)(a.vc + base + 8);
        }
#pragma unroll
        for (int uu = 0; uu < U; uu++) {
            float kf[16], vf[16];
            h8_to_f(kr[uu][0], kf); h8_to_f(kr[uu][1], kf + 8);
            h8_to_f(vr[uu][0], vf); h8_to_f(vr[uu][1], vf + 8);
            float s[G];
#pragma unroll
            for (int h = 0; h < G; h++) {
                float x = 0.0f;
#pragma unroll
                for (int d = 0; d < 16; d++) x = __fadd_rn(x, __fmul_rn(qv[h][d], kf[d]));
                s[h] = group_sum<LP>(x);
            }
            if (ok[uu]) {
#pragma unroll
                for (int h = 0; h < G; h++) {
                    const float sc = __fmul_rn(s[h], a.scale);
                    if (sc > m[h]) {
                        const float c = __expf(m[h] - sc);
#pragma unroll
                        for (int d = 0; d < 16; d++) acc[h][d] = __fmul_rn(acc[h][d], c);
                        l[h] = __fmul_rn(l[h], c);
                        m[h] = sc;
                    }
                    const float pr = __expf(sc - m[h]);
                    l[h] = __fadd_rn(l[h], pr);
#pragma unroll
                    for (int d = 0; d < 16; d++) acc[h][d] = __fadd_rn(acc[h][d], __fmul_rn(vf[d], pr));
                }
            }
        }
    }

    // fold the wave's position slots (lanes with equal j), then the 4 waves
#pragma unroll
    for (int h = 0; h < G; h++) {
        float M = m[h];
#pragma unroll
        for (int s = LP; s < 64; s <<= 1) M = fmaxf(M, __shfl_xor(M, s));
        const float c = l[h] > 0.0f ? __expf(m[h] - M) : 0.0f;
        float lt = __fmul_rn(l[h], c);
#pragma unroll
        for (int s = LP; s < 64; s <<= 1) lt = __fadd_rn(lt, __shfl_xor(lt, s));
#pragma unroll
        for (int d = 0; d < 16; d++) {
            float v = __fmul_rn(acc[h][d], c);
#pragma unroll
            for (int s = LP; s < 64; s <<= 1) v = __fadd_rn(v, __shfl_xor(v, s));
            acc[h][d] = v;
        }
        if (p == 0) {
#pragma unroll
            for (int d = 0; d < 16; d++) wacc[wave][h][16 * j + d] = acc[h][d];
        }
        if (lane == 0) { wm[wave][h] = lt > 0.0f ? M : -3.0e38f; wl[wave][h] = lt; }
    }
    __syncthreads();
    for (int e = tid; e < G * HD; e += 256) {
        const int h = e / HD, d = e % HD;
        float M = -3.0e38f;
#pragma unroll
        for (int w = 0; w < 4; w++) M = fmaxf(M, wm[w][h]);
        float lt = 0.0f, v = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            if (wl[w][h] > 0.0f) {
                const float c = __expf(wm[w][h] - M);
                lt = __fadd_rn(lt, __fmul_rn(wl[w][h], c));
                v = __fadd_rn(v, __fmul_rn(wacc[w][h][d], c));
            }
        }
        float *pb = a.part + ((int64_t)(kvh * G + h) * a.splits + sp) * (HD + 2);
        pb[d] = v;
        if (d == 0) { pb[HD] = lt > 0.0f ? M : -3.0e38f; pb[HD + 1] = lt; }
    }
    if (!a.out) return;

    // the last split of this kv head merges all of them
    __threadfence();
    __syncthreads();
    if (tid == 0) ticket = atomicAdd(&a.counters[kvh], 1);
    __syncthreads();
    if (ticket != a.splits - 1) return;
    __threadfence();
    for (int e = tid; e < G * HD; e += 256) {
        const int h = e / HD, d = e % HD;
        const int qh = kvh * G + h;
        const float *pb0 = a.part + (int64_t)qh * a.splits * (HD + 2);
        float gm = -3.0e38f;
        for (int s = 0; s < a.splits; s++) gm = fmaxf(gm, pb0[s * (HD + 2) + HD]);
        float gl = 0.0f, ac = 0.0f;
        for (int s = 0; s < a.splits; s++) {
            const float *pb = pb0 + s * (HD + 2);
            const float ls = pb[HD + 1];
            if (ls > 0.0f) {
                const float w = __expf(pb[HD] - gm);
                gl = __fadd_rn(gl, __fmul_rn(w, ls));
                ac = __fadd_rn(ac, __fmul_rn(pb[d], w));
            }
        }
        a.out[(int64_t)qh * HD + d] = __fmul_rn(ac, __fdiv_rn(1.0f, gl));
    }
    if (tid == 0) a.counters[kvh] = 0;
}

#define ATTN_KERNEL(HD, G) \
    extern "C" __global__ void __launch_bounds__(256) cj_attn_decode_h##HD##_g##G(cj_attn_args a) { attn_body<HD, G>(a); }
ATTN_KERNEL(128, 1)
ATTN_KERNEL(128, 2)
ATTN_KERNEL(128, 4)
ATTN_KERNEL(128, 8)
ATTN_KERNEL(64, 1)
ATTN_KERNEL(64, 2)
ATTN_KERNEL(64, 4)
ATTN_KERNEL(64, 8)

// Merge split partials into f32 (+ the pack of the result): one workgroup of
// 256 per 256 output values (the reference's attnReducePackQ8Kernel contract).
extern "C" __global__ void __launch_bounds__(256) cj_attn_merge(cj_merge_args a) {
    __shared__ float bmax[8];
    const int t = threadIdx.x, lane = t & 63;
    const int64_t e = (int64_t)blockIdx.x * 256 + t;
    const int64_t n = (int64_t)a.n_q * a.head_dim;
    float x = 0.0f;
    if (e < n) {
        const int h = (int)(e / a.head_dim), d = (int)(e % a.head_dim);
        const float *pb0 = a.part + (int64_t)h * a.splits * (a.head_dim + 2);
        float gm = -3.0e38f;
        for (int s = 0; s < a.splits; s++) gm = fmaxf(gm, pb0[s * (a.head_dim + 2) + a.head_dim]);
        float gl = 0.0f, ac = 0.0f;
        for (int s = 0; s < a.splits; s++) {
            const float *pb = pb0 + s * (a.head_dim + 2);
            const float ls = pb[a.head_dim + 1];
            if (ls > 0.0f) {
                const float w = __expf(pb[a.head_dim] - gm);
                gl = __fadd_rn(gl, __fmul_rn(w, ls));
                ac = __fadd_rn(ac, __fmul_rn(pb[d], w));
            }
        }
        x = __fmul_rn(ac, __fdiv_rn(1.0f, gl));
        if (a.out) a.out[e] = x;
    }
    if (!a.packed) return;
    const float av = fabsf(x);
    float am;
    if (a.per32) {
        float mm = group_max<32>(av);
        if ((lane & 31) == 0) bmax[t >> 5] = mm;
        __syncthreads();
        am = bmax[t >> 5];
    } else {
        float mm = group_max<64>(av);
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
    __shared__ float red[64];
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
        const float scale = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)hd), a.eps)));
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
