// common.h — device helpers for the gfx950 kernels (wave64, CDNA4).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include "args.h"

#define DEV __device__ __forceinline__

// fp16 bits <-> f32 through the hardware converts (exact / round-to-nearest-even).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));   // a native 16-byte vector
typedef float f32x4 __attribute__((ext_vector_type(4)));          // the same for f32 (HIP's float4 is a struct, copied by memcpy)

// A 16-byte load of weights a decode step reads once: nontemporal, so the
// stream does not displace what the caches hold for reuse (measured on
// MI355X: a 66 MB row stream 12.5 -> 11.4 us).
DEV uint4 ld_stream16(const uint8_t *p) {
    const u32x4 v = __builtin_nontemporal_load((const u32x4 *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

DEV float h2f(uint32_t bits16) { return __half2float(__ushort_as_half((unsigned short)(bits16 & 0xffffu))); }

// f16 × f32 products without the widening instruction: v_fma_mix_f32 reads
// the f16 half of w (low: op_sel 0, high: op_sel 1) and adds −0, so its one
// rounding is the product's own: x + (−0) = x for every x, −0 included,
// which makes it bit for bit __fmul_rn(h2f(half), b) (checked on gfx950 over
// 8.4M operand pairs with zeros, denormals and infinities). The compiler
// would fold an fma with −0 to a multiply and keep the widening, so the
// instruction is written out.
DEV float mul_h16lo(uint32_t w, float b) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(b), "v"(-0.0f));
    return r;
}
DEV float mul_h16hi(uint32_t w, float b) {
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(b), "v"(-0.0f));
    return r;
}
DEV uint16_t f2h(float f) { return __half_as_ushort(__float2half_rn(f)); }

// Two values into a K/V plane: fp16 (rounded to nearest even), or f32 as
// they are where the plane holds f32 (the reference's PagedKvCache keeps
// f32 K/V, model/PagedKvCache.cajeta).
DEV void kv_store2(uint16_t *plane, int f32, int64_t i0, float x0, int64_t i1, float x1) {
    if (f32) {
        ((float *)plane)[i0] = x0;
        ((float *)plane)[i1] = x1;
    } else {
        plane[i0] = f2h(x0);
        plane[i1] = f2h(x1);
    }
}

// Correctly rounded f32 square root. (HIP's __fsqrt_rn is the hardware's
// approximate v_sqrt_f32 unless OCML's rounded operations are enabled; the
// llvm.sqrt expansion for gfx950 rounds to nearest even.)
DEV float sqrt_rn(float x) { return __builtin_sqrtf(x); }

DEV int sdot4(uint32_t a, uint32_t b, int c) { return __builtin_amdgcn_sdot4((int)a, (int)b, c, false); }

// Exact integer exchange inside a quad of lanes (DPP quad_perm).
DEV int quad_xor1(int v) { return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false); }
DEV int quad_xor2(int v) { return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false); }

// A workgroup barrier for exchanges through LDS only: global loads in flight
// stay in flight across it (__syncthreads waits for them too, the vector
// memory counter covering loads as well as stores), so a prefetch issued
// before it keeps its distance. Global stores before it are not made visible.
DEV void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Lane exchanges in the VALU, without an LDS round trip: DPP (quad
// permutes and rotations inside each 16-lane row) and v_permlane16_swap /
// v_permlane32_swap across rows. Every lane of the wave must be active.
template <int CTRL>
DEV float dpp_f(float v) { return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false)); }
template <int CTRL>
DEV int dpp_i(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false); }
enum : int { DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HMIRROR = 0x141, DPP_ROR4 = 0x124, DPP_ROR8 = 0x128 };
// row_shl:K — lane i reads lane i + K of its 16-lane row
template <int K>
DEV float dpp_shl(float v) { return dpp_f<0x100 + K>(v); }
// The two halves of a xor-16 exchange: a holds rows 0,0,2,2 of the wave and b
// rows 1,1,3,3, so a + b (or max) is each lane's value with lane ^ 16's.
// (The results are copied out as scalars: a bit cast of the builtin's vector
// element reads element 0.)
DEV void swap16(int v, int &a, int &b) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    a = r[0];
    b = r[1];
}
DEV void swap32(int v, int &a, int &b) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    a = r[0];
    b = r[1];
}

// The 32-lane xor butterfly v + v(lane ^ m) for m = 16, 8, 4, 2, 1 in that
// order, every lane ending with its 32-lane group's sum — bit for bit the
// __shfl_xor loop. ^8 is a rotation by 8 inside the 16-lane row; after it the
// values repeat every 8 lanes, so a rotation by 4 brings lane ^ 4's value.
DEV float xsum32(float v) {
    int a, b;
    swap16(__float_as_int(v), a, b);
    v = __fadd_rn(__int_as_float(a), __int_as_float(b));
    v = __fadd_rn(v, dpp_f<DPP_ROR8>(v));
    v = __fadd_rn(v, dpp_f<DPP_ROR4>(v));
    v = __fadd_rn(v, dpp_f<DPP_XOR2>(v));
    return __fadd_rn(v, dpp_f<DPP_XOR1>(v));
}
DEV int xsum32_i(int v) {
    int a, b;
    swap16(v, a, b);
    v = a + b;
    v += dpp_i<DPP_ROR8>(v);
    v += dpp_i<DPP_ROR4>(v);
    v += dpp_i<DPP_XOR2>(v);
    return v + dpp_i<DPP_XOR1>(v);
}
DEV float xmax32(float v) {
    int a, b;
    swap16(__float_as_int(v), a, b);
    v = fmaxf(__int_as_float(a), __int_as_float(b));
    v = fmaxf(v, dpp_f<DPP_ROR8>(v));
    v = fmaxf(v, dpp_f<DPP_ROR4>(v));
    v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    return fmaxf(v, dpp_f<DPP_XOR1>(v));
}
// The maximum over aligned groups of 8 and of 16 lanes. After the two quad
// steps the four lanes of a quad agree, so lane 7 − i of the eight (the half
// mirror) stands for lane i ^ 4.
DEV float xmax8(float v) {
    v = fmaxf(v, dpp_f<DPP_XOR1>(v));
    v = fmaxf(v, dpp_f<DPP_XOR2>(v));
    return fmaxf(v, dpp_f<DPP_HMIRROR>(v));
}
DEV float xmax16(float v) {
    v = xmax8(v);
    return fmaxf(v, dpp_f<DPP_ROR8>(v));
}
// Lane 0's value of the fold v + v(lane + m), m = 32, 16, ..., 1 (the
// __shfl_down loop): lane 0 of the xor butterfly in the same order adds the
// same two values at every step.
DEV float fold64_lane0(float v) {
    int a, b;
    swap32(__float_as_int(v), a, b);
    v = __fadd_rn(__int_as_float(a), __int_as_float(b));
    swap16(__float_as_int(v), a, b);
    v = __fadd_rn(__int_as_float(a), __int_as_float(b));
    v = __fadd_rn(v, dpp_f<DPP_ROR8>(v));
    v = __fadd_rn(v, dpp_f<DPP_ROR4>(v));
    v = __fadd_rn(v, dpp_f<DPP_XOR2>(v));
    return __fadd_rn(v, dpp_f<DPP_XOR1>(v));
}
DEV float xmax64(float v) {
    int a, b;
    swap32(__float_as_int(xmax32(v)), a, b);
    return fmaxf(__int_as_float(a), __int_as_float(b));
}

template <int W>
DEV float group_sum(float v) {
#pragma unroll
    for (int m = W / 2; m > 0; m >>= 1) v += __shfl_xor(v, m);
    return v;
}
// The integer sum and the maximum do not depend on the order.
template <int W>
DEV int group_sum_i(int v) {
    static_assert(W == 32, "32-lane groups");
    return xsum32_i(v);
}
template <int W>
DEV float group_max(float v) {
    static_assert(W == 32 || W == 64, "32- or 64-lane groups");
    return W == 32 ? xmax32(v) : xmax64(v);
}

// Round half away from zero, the reference's Math.round on pack values.
DEV int round_away(float v) { return (int)roundf(v); }

// E8M0 half-scale 2^(e-128) with the e<2 denormal patterns (Quant.mxfp4Scale).
DEV float mxfp4_scale(uint32_t e) { return __uint_as_float(e < 2 ? (0x00200000u << e) : ((e - 1) << 23)); }
// E2M1 code as the reference's integer table {0,1,2,3,4,6,8,12} with the sign
// bit: an integer first, so code 8 is +0, not -0 (Quant.mxfp4Code).
DEV float mxfp4_val(uint32_t nib) {
    const int m = (int)(nib & 7);
    int v = m < 5 ? m : (m == 5 ? 6 : (m == 6 ? 8 : 12));
    if (nib & 8) v = -v;
    return (float)v;
}

// exp(x) in f32 as the reference CPU backend computes it: its Math.exp is
// glibc's expf (the reference's recorded CPU softmax outputs,
// attnScoreKernel h32kv4d128c256, are reproduced by glibc expf in all 8192
// values and not by a correctly rounded exp), whose algorithm is ARM
// optimized-routines' expf: k = round(x·32/ln2) and r = x·32/ln2 − k, each
// from one fused multiply-add of the f64 x (the round by adding 1.5·2^52);
// 2^(k/32) from a 32-entry table of 2^(i/32) rounded to f64, the integer
// part added to its exponent bits; 2^(r/32) by the degree-3 polynomial
// C0·r³ + C1·r² + C2·r + 1 in f64 with fused multiply-adds; one rounding to
// f32 at the end. The table entries are 2^(i/32) correctly rounded to f64,
// stored less i·2^47 in their bit patterns so that adding k·2^47 lands the
// exponent. Over every f32 input this gives glibc 2.35's expf bit for bit.
__device__ __constant__ uint64_t CJ_EXP2_TAB[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
    0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
    0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
    0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
    0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
    0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL,
};
// Branch-free: the main path runs on x clamped into its range (the same x
// wherever the result is used) and the special cases are selected after, so
// a caller's independent exps issue their table loads together. `tab` is the
// table: CJ_EXP2_TAB itself, or a kernel's LDS copy of it (cj_exp_table),
// which keeps a global round trip off each exp where the exps sit on a
// kernel's critical path.
DEV float cj_expf(float x, const uint64_t *tab) {
    const float hi = 0x1.62e42ep6f, lo = -0x1.9fe368p6f;
    const float xc = fminf(fmaxf(x, lo), hi);
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / (32.0 * 32 * 32), c1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32),
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double xd = (double)xc;
    double kd = __fma_rn(inv_ln2_n, xd, shift);
    const uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd = kd - shift;
    const double r = __fma_rn(inv_ln2_n, xd, -kd);
    const double s = __longlong_as_double((long long)(tab[ki & 31] + (ki << 47)));
    const double z = __fma_rn(c0, r, c1), r2 = r * r;
    double y = __fma_rn(c2, r, 1.0);
    y = __fma_rn(z, r2, y);
    float e = __double2float_rn(y * s);
    e = x > hi ? __uint_as_float(0x7f800000u) : e;
    e = x < lo ? 0.0f : e;
    return x != x ? x + x : e;
}
DEV float cj_expf(float x) { return cj_expf(x, CJ_EXP2_TAB); }
// A workgroup's LDS copy of the exp table (threads 0..31 write it; the
// caller's next barrier makes it visible).
DEV void cj_exp_table(uint64_t *tab) {
    if (threadIdx.x < 32) tab[threadIdx.x] = CJ_EXP2_TAB[threadIdx.x];
}

// SiLU(x)·u, exp form: x / (1 + exp(−x)) · u (Prim.gluF32 / gluOne).
DEV float silu_exp_mul(float x, float u) {
    return __fmul_rn(__fdiv_rn(x, __fadd_rn(1.0f, cj_expf(0.0f - x))), u);
}

// SiLU(x)·u, the CPU backend's vector form (Prim.gluCpuKernel): 0.5·x·(1 +
// tanh(x/2)) with tanh as Eigen's float rational approximation on a clamped
// argument; every step a correctly rounded op or an fma.
DEV float silu_tanh_mul(float x, float u) {
    const float tlo = -7.90531110763549805f;
    float xa = fmaxf(x, -16.0f);
    float xb = __fsub_rn(-16.0f, xa);
    float xc = __fsub_rn(-16.0f, fmaxf(xb, -32.0f));
    float t0 = __fmul_rn(0.5f, __fmaf_rn(__fmul_rn(0.0f, xc), __fmul_rn(xc, xc), xc));
    float ta = fmaxf(t0, tlo);
    float tb = __fsub_rn(tlo, ta);
    float t = __fsub_rn(tlo, fmaxf(tb, -15.8106222152709961f));
    float t2 = __fmul_rn(t, t);
    float p = __fmaf_rn(-2.76076847742355e-16f, t2, 2.00018790482477e-13f);
    p = __fmaf_rn(p, t2, -8.60467152213735e-11f);
    p = __fmaf_rn(p, t2, 5.12229709037114e-08f);
    p = __fmaf_rn(p, t2, 1.48572235717979e-05f);
    p = __fmaf_rn(p, t2, 6.37261928875436e-04f);
    p = __fmul_rn(__fmaf_rn(p, t2, 4.89352455891786e-03f), t);
    float q = __fmaf_rn(1.19825839466702e-06f, t2, 1.18534705686654e-04f);
    q = __fmaf_rn(q, t2, 2.26843463243900e-03f);
    q = __fmaf_rn(q, t2, 4.89352518554385e-03f);
    return __fmul_rn(__fmul_rn(__fmul_rn(0.5f, xa), __fadd_rn(1.0f, __fdiv_rn(p, q))), u);
}

// Element e of silu(g)·u over a row of n in the given form. The vector form
// (form 1) covers each 4096-wide work block in 16-wide chunks and leaves the
// block's tail to the exp form, as gluCpuKernel does.
DEV float glu_value(int form, int64_t e, int64_t n, float g, float u) {
    if (!form) return silu_exp_mul(g, u);
    const int64_t b0 = e & ~(int64_t)4095;
    const int64_t hi = b0 + 4096 < n ? b0 + 4096 : n;
    const int64_t vec_end = b0 + ((hi - b0) & ~(int64_t)15);
    return e < vec_end ? silu_tanh_mul(g, u) : silu_exp_mul(g, u);
}

// Zero the pad bytes [292, 320) of a per-256 pack block, so a pack's bytes
// are fully determined (thread t < 7 writes one word).
DEV void pack_zero_pad(uint8_t *blk, int t) {
    if (t < 7) *(uint32_t *)(blk + 292 + 4 * t) = 0u;
}

// One 256-wide pack block written by a whole workgroup of 256, thread t
// holding element t: the block (or 32-group) maximum, q = round-half-away(
// v·(127/amax)), the int32 sums of 32 and the f32 scale(s) — the layout of
// Quant.q8kPackPad / q8kPack32Pad (io/Quant.cajeta:3232-3321). `bmax` is 8
// floats of LDS; the function ends on a barrier, so it can be called in a
// loop over blocks.
DEV void pack256(float v, int per32, uint8_t *ob, float *bmax) {
    const int t = threadIdx.x, lane = t & 63;
    const float av = fabsf(v);
    float am;
    if (per32) {
        const float m = xmax32(av);
        if ((lane & 31) == 0) bmax[t >> 5] = m;
        lds_barrier();
        am = bmax[t >> 5];
    } else {
        const float m = xmax64(av);
        if (lane == 0) bmax[t >> 6] = m;
        lds_barrier();
        am = fmaxf(fmaxf(bmax[0], bmax[1]), fmaxf(bmax[2], bmax[3]));
    }
    const float inv = am > 0.0f ? __fdiv_rn(127.0f, am) : 0.0f;
    const int q = round_away(__fmul_rn(v, inv));
    ob[t] = (uint8_t)(int8_t)q;
    const int s = xsum32_i(q);
    if ((lane & 31) == 0) *(int32_t *)(ob + 256 + 4 * (t >> 5)) = s;
    if (per32) {
        if ((lane & 31) == 0) *(float *)(ob + 288 + 4 * (t >> 5)) = __fdiv_rn(am, 127.0f);
    } else {
        if (t == 0) *(float *)(ob + 288) = __fdiv_rn(am, 127.0f);
        pack_zero_pad(ob, t);
    }
    lds_barrier();
}

// Lane-uniform reads of another lane's value (the lane index must be the
// same on every lane of the wave).
DEV float lane_f(float v, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); }

// max(v, the value DPP control CTRL brings from another lane); lanes the
// control gives no source keep `v` (the source falls back to `v` itself).
template <int CTRL, int ROWS>
DEV float dpp_max(float v) {
    const int s = __builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROWS, 0xF, false);
    return fmaxf(v, __int_as_float(s));
}

// Inclusive prefix maximum over the 64 lanes by DPP: row_shr 1, 2, 4, 8
// within each row of 16, then row_bcast 15 and 31 across rows (max is exact
// in any order, so this equals the running maximum).
DEV float wave_prefix_max(float v) {
    v = dpp_max<0x111, 0xF>(v);   // row_shr:1
    v = dpp_max<0x112, 0xF>(v);   // row_shr:2
    v = dpp_max<0x114, 0xF>(v);   // row_shr:4
    v = dpp_max<0x118, 0xF>(v);   // row_shr:8
    v = dpp_max<0x142, 0xA>(v);   // row_bcast:15 into rows 1 and 3
    v = dpp_max<0x143, 0xC>(v);   // row_bcast:31 into rows 2 and 3
    return v;
}

// The value of lane − 1 (wave_shr:1); lane 0 gets `first`.
DEV float wave_shr1(float v, float first) {
    const int s = __builtin_amdgcn_update_dpp(__float_as_int(first), __float_as_int(v), 0x138, 0xF, 0xF, false);
    return __int_as_float(s);
}

// ---------------------------------------------------------------------------
// Activation staging into LDS: the 320-byte block layout of the reference's
// Quant.q8kPackPad / q8kPack32Pad ([0,256) q, [256,288) 8 int32 sums of 32,
// [288,320) the f32 scale(s)). 256 threads; thread t owns element t of every
// 256-wide block, so a block's amax is one workgroup reduction.
//
// The RMSNorm follows the reference's device-decode order exactly: thread t
// accumulates x[t + 256k]^2 in k order, then the 256 partials fold with
// strides 128, 64, ..., 1 — the same adds, so the same bits.
// ---------------------------------------------------------------------------

#define STAGE_CHUNK 16     // 256-wide blocks held in registers at a time

// RMSNorm scale of x[0..n) in the order of the reference's device-decode
// norms: thread t sums x[t + 256k]^2 in k order (t + 256k < n, so a width
// that is not whole 256s leaves the last round ragged) and the 256 partials
// fold 128, 64, ..., 1 (lanes of wave 0 for the last six). For whole 256s
// that is the CPU row form (Prim.rmsnormPackRowCpuKernel, model/Prim.cajeta:
// 977-1071); other widths take rmsnormRowF32 (:742-775) through
// Prim.rmsnormDevice (:1440-1450), as the resident layer does for them
// (CausalLM.cajeta:3643, :3819). Then 1/sqrt(ss/n + eps). `red` is 256 floats
// of LDS.
// A callable run where a prologue's loads are in flight and not yet used.
struct NoMid {
    DEV void operator()() const {}
};

// mid() runs after the row's loads are requested and before any is used:
// loads it requests stay in flight while the sum is formed (loads complete
// in the order requested, so waiting for the row's values does not wait
// for them).
// Thread t's values t + 256·k, k < K, of a row of n (past the row: its last
// value again, never summed), every load unconditional.
template <int K>
DEV void norm_load(const float *x, int64_t n, float (&xv)[64]) {
#pragma unroll
    for (int k = 0; k < 64; k++) xv[k] = k < K ? x[min((int64_t)threadIdx.x + 256 * k, n - 1)] : 0.0f;
}

template <class Mid = NoMid>
DEV float stage_norm_scale(const float *x, int64_t n, float eps, float *red, Mid &&mid = Mid{}) {
    const int t = threadIdx.x;
    // the row's values loaded at once (up to 64 a thread: 16, 32 or 64 loads,
    // each form with no load under a branch of its own — one branch a load
    // made the compiler wait at the joins, a memory round trip every few
    // loads), then summed in order: thread t's values t, t + 256, … < n
    float xv[64];
    const int64_t rounds = (n + 255) >> 8;
    if (rounds <= 16) norm_load<16>(x, n, xv);
    else if (rounds <= 32) norm_load<32>(x, n, xv);
    else norm_load<64>(x, n, xv);
    mid();
    float p = 0.0f;
#pragma unroll
    for (int k = 0; k < 64; k++) p = t + 256 * (int64_t)k < n ? __fadd_rn(p, __fmul_rn(xv[k], xv[k])) : p;
    for (int64_t e = t + 256 * 64; e < n; e += 256) p = __fadd_rn(p, __fmul_rn(x[e], x[e]));
    red[t] = p;
    lds_barrier();
    if (t < 128) red[t] = __fadd_rn(red[t], red[t + 128]);
    lds_barrier();
    if (t < 64) {
        const float s = fold64_lane0(__fadd_rn(red[t], red[t + 64]));
        if (t == 0) red[0] = s;
    }
    lds_barrier();
    const float ss = red[0];
    lds_barrier();
    return __fdiv_rn(1.0f, sqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)n), eps)));
}

// The staged value of element e: x[e], or x[e]·scale·w[e] under the norm.
DEV float stage_value(const float *x, int64_t n, int64_t e, bool norm, float scale, const float *w, int form) {
    if (e >= n) return 0.0f;
    const float xv = x[e];
    if (!norm) return xv;
    const float wi = form == 1 ? __fadd_rn(1.0f, w[e]) : w[e];
    return __fmul_rn(__fmul_rn(xv, scale), wi);
}

// Quantize the staged values of nblk blocks into LDS 320-byte blocks at sx.
// Thread t owns 16 consecutive values of each 4096-wide round (block t/16,
// values 16·(t%16)..+15), so a 32-group is two neighbouring lanes and a
// 256-block sixteen: the block maximum, the int8 codes and the 32-sums are
// lane-local plus xor shuffles, with no barrier until the end. The codes
// are the reference's q8kPack ones: q = round-half-away(v · (127/amax)).
DEV void stage_pack(const float *x, int64_t n, int nblk, bool norm, float scale, const float *w, int form,
                    int per32, uint8_t *sx, float *xout, int bstride = 320) {
    const int t = threadIdx.x;
    const int64_t total = (int64_t)nblk * 256;
    // 16-byte reads where the row (and the norm weights) are 16-byte aligned
    // (the per-value form below loads each value under a branch of its own,
    // and the compiler waits at every join)
    const bool al = ((reinterpret_cast<uintptr_t>(x) | (norm ? reinterpret_cast<uintptr_t>(w) : 0)) & 15) == 0;
    for (int64_t e0 = 16 * t; e0 < total; e0 += 4096) {
        float v[16];
        if (e0 + 16 <= n && al) {
            f32x4 xv[4];
#pragma unroll
            for (int k = 0; k < 4; k++) xv[k] = *(const f32x4 *)(x + e0 + 4 * k);
            if (norm) {
                f32x4 wv[4];
#pragma unroll
                for (int k = 0; k < 4; k++) wv[k] = *(const f32x4 *)(w + e0 + 4 * k);
#pragma unroll
                for (int k = 0; k < 16; k++) {
                    const float wk = wv[k >> 2][k & 3];
                    const float wi = form == 1 ? __fadd_rn(1.0f, wk) : wk;
                    v[k] = __fmul_rn(__fmul_rn(xv[k >> 2][k & 3], scale), wi);
                }
            } else {
#pragma unroll
                for (int k = 0; k < 16; k++) v[k] = xv[k >> 2][k & 3];
            }
        } else {
#pragma unroll
            for (int k = 0; k < 16; k++) v[k] = stage_value(x, n, e0 + k, norm, scale, w, form);
        }
        if (xout) {
#pragma unroll
            for (int k = 0; k < 16; k++) if (e0 + k < n) xout[e0 + k] = v[k];
        }
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
        const int in = (int)(e0 & 255);           // offset inside the block
        uint8_t *b = sx + blk * bstride;
        *(uint4 *)(b + in) = make_uint4(wd[0], wd[1], wd[2], wd[3]);
        const int g = in >> 5, j = (in >> 4) & 15;   // 32-group, lane of the block
        if (!(j & 1)) *(int32_t *)(b + 256 + 4 * g) = sum;
        if (per32) {
            if (!(j & 1)) *(float *)(b + 288 + 4 * g) = __fdiv_rn(am, 127.0f);
        } else {
            if (j == 0) *(float *)(b + 288) = __fdiv_rn(am, 127.0f);
            else if (j < 8) *(uint32_t *)(b + 288 + 4 * j) = 0u;   // pad bytes 292..319
        }
    }
    lds_barrier();
}

// An f32 activation in LDS by 32-element blocks, swizzled: float4 i of block
// b at float4 slot 8b + (i ^ (b & 7)). Lanes that read float4 i of eight
// consecutive blocks then touch every bank once (unswizzled, a lane a block
// puts all 64 lanes on the same four banks).
DEV int64_t swz32(int64_t idx) {
    const int64_t b = idx >> 5;
    const int i = (int)(idx >> 2) & 7;
    return (b << 5) + ((i ^ (int)(b & 7)) << 2) + (idx & 3);
}

// The staged values as f32 into LDS (formats that read f32 activations);
// swz: in the block-swizzled order above.
DEV void stage_f32(const float *x, int64_t n, int nblk, bool norm, float scale, const float *w, int form, float *xf,
                   bool swz = false) {
    // 16 values a thread a round, all loads issued before the first use
    const int64_t total = (int64_t)nblk * 256;
    for (int64_t e0 = 16 * threadIdx.x; e0 < total; e0 += 4096) {
        float v[16];
        if (e0 + 16 <= n) {
            float4 xv[4], wv[4];
#pragma unroll
            for (int k = 0; k < 4; k++) xv[k] = *(const float4 *)(x + e0 + 4 * k);
            if (norm) {
#pragma unroll
                for (int k = 0; k < 4; k++) wv[k] = *(const float4 *)(w + e0 + 4 * k);
            }
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float xs[4] = {xv[k].x, xv[k].y, xv[k].z, xv[k].w};
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    if (norm) {
                        const float wc = c == 0 ? wv[k].x : c == 1 ? wv[k].y : c == 2 ? wv[k].z : wv[k].w;
                        const float wi = form == 1 ? __fadd_rn(1.0f, wc) : wc;
                        v[4 * k + c] = __fmul_rn(__fmul_rn(xs[c], scale), wi);
                    } else {
                        v[4 * k + c] = xs[c];
                    }
                }
            }
        } else {
#pragma unroll
            for (int k = 0; k < 16; k++) v[k] = stage_value(x, n, e0 + k, norm, scale, w, form);
        }
#pragma unroll
        for (int k = 0; k < 4; k++)
            *(float4 *)(xf + (swz ? swz32(e0 + 4 * k) : e0 + 4 * k)) =
                make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
    }
    lds_barrier();
}

// ---- Q4_0, block by block (Quant.q40MatVecIntoAt, L/io/Quant.cajeta:1516-1545)
// A block's dot starts at 0 and adds its 32 rounded products in the order
// (lo_j − 8)·x[j], (hi_j − 8)·x[j + 16], j ascending; the row then adds the
// rounded d·dot block after block. Blocks are independent until that fold.

// Block b's 32 x values from the swizzled LDS row.
DEV void q40_xblock(const float *xs, int b, float4 (&x)[8]) {
#pragma unroll
    for (int i = 0; i < 8; i++) x[i] = *(const float4 *)(xs + 32 * b + 4 * (i ^ (b & 7)));
}

// The block's 16 code bytes as the exact floats q − 8 (element order: the
// low nibbles are elements 0..15, the high ones 16..31). q ^ 8 read as a
// signed 4-bit field is q − 8.
DEV void q40_decode(const uint4 &q, float (&v)[32]) {
    const uint32_t ws[4] = {q.x ^ 0x88888888u, q.y ^ 0x88888888u, q.z ^ 0x88888888u, q.w ^ 0x88888888u};
#pragma unroll
    for (int g = 0; g < 4; g++) {
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
            v[4 * g + jj] = (float)((int)(ws[g] << (28 - 8 * jj)) >> 28);
            v[16 + 4 * g + jj] = (float)((int)(ws[g] << (24 - 8 * jj)) >> 28);
        }
    }
}

// The block's dot, from 0, in the reference's order.
DEV float q40_dot(const float (&v)[32], const float4 (&x)[8]) {
    float xf[32];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        xf[4 * i] = x[i].x; xf[4 * i + 1] = x[i].y; xf[4 * i + 2] = x[i].z; xf[4 * i + 3] = x[i].w;
    }
    float dot = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; j++) {
        dot = __fadd_rn(dot, __fmul_rn(v[j], xf[j]));
        dot = __fadd_rn(dot, __fmul_rn(v[16 + j], xf[16 + j]));
    }
    return dot;
}

#define Q40_TS 68   // a wave's term row stride (floats): 16-byte reads, rows on distinct banks

// A chain's n new terms (its LDS row) folded onto acc in block order.
DEV float q40_fold(const float *row, int n, float acc) {
    int i = 0;
    for (; i + 4 <= n; i += 4) {
        const float4 p = *(const float4 *)(row + i);
        acc = __fadd_rn(acc, p.x);
        acc = __fadd_rn(acc, p.y);
        acc = __fadd_rn(acc, p.z);
        acc = __fadd_rn(acc, p.w);
    }
    for (; i < n; i++) acc = __fadd_rn(acc, row[i]);
    return acc;
}

// A whole sweep's 64 terms, unrolled: the reads all issued before the adds,
// which the compiler can then interleave with other work.
DEV float q40_fold64(const float *row, float acc) {
    f32x4 p[16];
#pragma unroll
    for (int i = 0; i < 16; i++) p[i] = *(const f32x4 *)(row + 4 * i);
#pragma unroll
    for (int i = 0; i < 16; i++) {
        acc = __fadd_rn(acc, p[i].x);
        acc = __fadd_rn(acc, p[i].y);
        acc = __fadd_rn(acc, p[i].z);
        acc = __fadd_rn(acc, p[i].w);
    }
    return acc;
}

// Copy an already-packed activation (nblk blocks of 320 bytes) into LDS,
// block b at sx + b·bstride.
DEV void stage_copy(const uint8_t *xp, int nblk, uint8_t *sx, int bstride = 320) {
    const int t = threadIdx.x;
    const int n16 = nblk * 20;
    // four 16-byte words a thread a round, loaded before any is stored
    for (int i0 = t; i0 < n16; i0 += 1024) {
        u32x4 v[4];
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = ((const u32x4 *)xp)[min(i0 + 256 * k, n16 - 1)];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int i = i0 + 256 * k;
            if (i < n16) *(u32x4 *)(sx + (i / 20) * bstride + (i % 20) * 16) = v[k];
        }
    }
    lds_barrier();
}

DEV int32_t step_pos(const cj_step_state *st, int32_t pos) { return st ? st->pos : pos; }

// MoeFfn.routeFromLogits (model/MoeFfn.cajeta:908-986) for one row of
// logits: softmax over the experts, top-k by probability with strict >
// (ties keep the lower index), the optional renormalisation by the sum
// clamped at 2^-14, then ×w_scale when it is neither 0 nor 1. The first wave
// of the workgroup computes (up to 256 experts); every thread passes the
// barriers. The logits and probabilities live in LDS; the max and the sum
// run on one lane in expert order as the reference forms them, the exps and
// the divides a lane an expert. Each top-k pick of the reference is the first
// strict maximum of its scan over the experts not yet picked — the largest
// valid probability, the lowest index among equals — so pick k is the expert
// with exactly k experts ahead of it in that order, counted a lane an expert.
// Result in s.sel / s.w (n_used entries). Logits that are not finite leave
// no valid probability: the reference refuses the row by name; here
// `status` (may be null) is set to 1 (the host raises after the step) and
// expert 0 keeps every later index in bounds.
struct RouteLds {
    float lgs[256], pr[256];
    float bc[2];
    int sel[64];
    float w[64];
};
DEV void route_row(const float *lg, int ne, int n_used, int norm_topk, float w_scale, int32_t *status, RouteLds &s) {
    const int t = threadIdx.x;
    if (t < 64)
        for (int e = t; e < ne; e += 64) s.lgs[e] = lg[e];
    lds_barrier();
    if (t == 0) {
        float mx = s.lgs[0];
        for (int e = 1; e < ne; e++) if (s.lgs[e] > mx) mx = s.lgs[e];
        s.bc[0] = mx;
    }
    lds_barrier();
    if (t < 64) {
        const float mx = s.bc[0];
        for (int e = t; e < ne; e += 64) s.pr[e] = cj_expf(s.lgs[e] - mx);
    }
    lds_barrier();
    if (t == 0) {
        float sum = 0.0f;
        for (int e = 0; e < ne; e++) sum = __fadd_rn(sum, s.pr[e]);
        s.bc[1] = sum;
    }
    lds_barrier();
    if (t < 64) {
        const float sum = s.bc[1];
        for (int e = t; e < ne; e += 64) s.pr[e] = __fdiv_rn(s.pr[e], sum);   // the probabilities
    }
    lds_barrier();
    if (t < 64) {
        // The picks in order: the larger probability first, on a tie the
        // lower index, an entry that is not a number never (the repeated
        // arg-max of routeFromLogits). That is a total order, so expert e is
        // pick number (experts ahead of e) when that is below n_used: one
        // pass of comparisons instead of n_used rounds of a wave reduction.
        int nvalid = 0;
        for (int j = 0; 64 * j < ne; j++) {
            const int e = t + 64 * j;
            const float v = e < ne ? s.pr[e] : -1.0f;
            const bool ok = v >= 0.0f;
            nvalid += __popcll(__ballot(ok));
            if (ok) {
                int ahead = 0;
                for (int x = 0; x < ne; x++) {
                    const float o = s.pr[x];
                    ahead += (o >= 0.0f && (o > v || (o == v && x < e))) ? 1 : 0;
                }
                if (ahead < n_used) {
                    s.sel[ahead] = e;
                    s.w[ahead] = v;
                }
            }
        }
        // fewer valid experts than picks: expert 0 with weight 0, flagged
        if (t == 0)
            for (int k = nvalid; k < n_used; k++) {
                s.sel[k] = 0;
                s.w[k] = 0.0f;
                if (status) status[0] = 1;
            }
    }
    lds_barrier();
    if (t == 0) {
        if (norm_topk) {
            float ws = 0.0f;
            for (int k = 0; k < n_used; k++) ws = __fadd_rn(ws, s.w[k]);
            if (ws < 0.00006103515625f) ws = 0.00006103515625f;
            for (int k = 0; k < n_used; k++) s.w[k] = __fdiv_rn(s.w[k], ws);
        }
        if (w_scale != 0.0f && w_scale != 1.0f)
            for (int k = 0; k < n_used; k++) s.w[k] = __fmul_rn(s.w[k], w_scale);
    }
    lds_barrier();
}
