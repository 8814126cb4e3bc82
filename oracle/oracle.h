/*
 * oracle.h — CPU restatement of cajeta-llm's CPU-backend decode arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the MI355X
 * backend: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it. The product path never links, loads or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative
 * to src/main/cajeta/dev/cajeta/llm/ of jklappenbach/cajeta-llm). Pinning
 * (tests/test_oracle.py; each check is also shown to fail on a build with a
 * deliberate mistake, OR_PLANT):
 *   - dequant (Q8_0, Q4_0, Q4_K, Q6_K, MXFP4): bit-exact against the
 *     reference's committed golden pairs (tests/golden/kquant, mxfp4).
 *   - fp16 conversions: every half pattern and RNE ties against IEEE.
 *   - q8_K / per-32 packs: closed form + round-half-away special cases.
 *   - GEMVs (all formats): float64 product of the dequantised weights with
 *     the values the pack stands for, to fp32 accumulation rounding.
 *   - rmsnorm, rope, silu (both forms), attention (split-K and two-pass),
 *     argmax, MoE route, split count, q/k row permutation: closed forms,
 *     invariants and float64 brute force on small inputs; the whole decode
 *     step against a float64 forward of the reference's toy GGUF.
 *   - or_expf: the reference CPU backend's Math.exp is glibc's expf (its
 *     recorded softmax outputs are glibc expf's bits); or_expf restates that
 *     algorithm and equals the C library's expf (checked on a sample here and
 *     over every f32 input when it was written), and the kernels compute the
 *     same steps.
 *   - the reference's recorded CPU-backend outputs (tests/golden/wave):
 *     two-pass scores + softmax exps, QK-norm + RoPE at head sizes 128 and 64,
 *     the split merge + pack, the router mat-vec + top-k, bit for bit (the
 *     router's last pick weights to the ulp that exp's rounding leaves).
 *   - parity unpinned: the stdlib's reduction trees beyond what the
 *     reference's own code and recorded rows fix, FMA contraction by the
 *     Cajeta compiler elsewhere, and end-to-end logits of the real reference
 *     binary (the cajeta toolchain is absent, so end-to-end is the
 *     restatement).
 */
#ifndef CJ_ORACLE_H
#define CJ_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (GgufFile / Quant.GG_*) */
enum { OR_F32 = 0, OR_F16 = 1, OR_Q4_0 = 2, OR_Q8_0 = 8, OR_Q4_K = 12, OR_Q6_K = 14, OR_MXFP4 = 39 };

int   or_block_bytes(int type);
int   or_block_elems(int type);
float or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);

/* block decode of `nblocks` blocks (Quant.dequantize, io/Quant.cajeta:693-734) */
int or_dequant(int type, const uint8_t *raw, int64_t nblocks, float *out);

/* activation packs: 320-byte blocks (io/Quant.cajeta:3232-3321) */
void or_q8k_pack(const float *x, int64_t n, int64_t npad, uint8_t *out);
void or_q8k_pack32(const float *x, int64_t n, int64_t npad, uint8_t *out);

/* one weight × one activation. Q4_K/Q6_K read a per-256 pack, Q8_0 a
 * per-32 pack (xp); Q4_0 and MXFP4 read f32 activations (xf). */
int or_matvec(int type, const uint8_t *w, int64_t rows, int64_t cols,
              const uint8_t *xp, const float *xf, float *y);
/* MXFP4 in the reference's device Q8 form: the per-32 activation quant
 * (xq: cols int8, xd: cols/32 scales) and the mat-vec over it. */
void or_mxfp4_quant_act(const float *x, int64_t cols, int8_t *xq, float *xd);
int or_matvec_mxfp4_q8(const uint8_t *w, int64_t rows, int64_t cols, const float *x, float *y);

/* primitives */
void  or_rmsnorm(const float *x, const float *w, int64_t n, float eps, int form, float *out);
/* exp(x) in f32 from correctly rounded steps (shared with the kernels). */
float or_expf(float x);
void or_exp2_table(uint64_t *out);
/* routerTopKKernel (io/QuantKernel.cajeta:39850-39960): logits[e] = W[e]·x by
 * 256 lane partials and the stride-halving tree; softmax by 32 lanes; top-k
 * picks, renormalised and scaled. Writes logits[experts], sel[used], w[used]. */
void or_router_topk(const float *w_router, const float *x, int experts, int cols, int used, int norm_topk,
                    float w_scale, float *logits, int32_t *sel, float *w);
/* attnScoreKernel (model/AttnKernel.cajeta:397-425) over a position-major
 * K plane [t][n_kv·hd]: scores[h][t] = the 32-lane score × scale; with
 * softmax != 0, attnCombineKernel's in-place pass 1-2 follows (each row's
 * max, then exp(s − max)). */
void or_attn_scores(const float *q, const void *kp, int f32, int nh, int nkv, int hd, int count, float scale,
                    int softmax, float *scores);
/* The generic qkPrepKernel (model/AttnKernel.cajeta:127-206) at any head size:
 * QK-norm by 128 lane partials and the stride-halving tree, then RoPE. */
int or_qk_prep(float *q, float *k, const float *qw, const float *kw, const float *inv, int nh, int nkv, int hd,
               int norm, float eps, int form, int pos);
void  or_glu_exp(const float *g, const float *u, int64_t n, float *out);
void  or_glu_tanh(const float *g, const float *u, int64_t n, float *out);
void  or_inv_freq(int hd, float theta, float *inv);
void  or_rope(float *t, int nheads, int hd, int pos, const float *inv);
int   or_argmax(const float *v, int64_t n);
int   or_moe_route(const float *logits, int n_experts, int n_used, int norm_topk,
                   float w_scale, int32_t *sel, float *w);
void  or_unpermute_rows(const uint8_t *src, uint8_t *dst, int64_t rows, int64_t row_bytes, int n_head);

/* decode attention over an fp16 (or f32) KV plane for ONE layer.
 * k/v planes are position-major: [ctx][n_kv*hd]. `count` positions from 0.
 * mode 0: split-K online softmax (AttnKernel.cpuDecodeHead + reduce),
 * mode 1: two-pass score/softmax/combine (attnScoreKernel + attnCombineKernel). */
void or_attend(const float *q, const void *kplane, const void *vplane, int kv_f32,
               int n_h, int n_kv, int hd, int count, int splits, float scale,
               int mode, float *out);
int  or_cpu_decode_splits(int count, int rows, int n_kv, int workers);
/* the split-K merge alone: partials [n_h][splits][hd+2] → out [n_h·hd] */
void or_attn_merge(const float *part, int n_h, int splits, int hd, float *out);
/* QK-norm of one 128-wide head in place, and the CPU decode prep at hd 128
 * (norm != 0: every head normed; then RoPE at `pos` with the given inv). */
void or_head_norm128(float *x, const float *w, float eps, int form);
int  or_qk_prep128(float *q, float *k, const float *qw, const float *kw, const float *inv, int n_h, int n_kv,
                   int norm, float eps, int form, int pos);

/* prefill attention for `rows` consecutive query rows at positions
 * start .. start+rows-1 of one sequence (hd 128): q rows [rows][n_h*hd], the
 * planes position-major as above and already holding every row's K/V;
 * window > 0 cuts each row to its last `window` positions. */
void or_prefill_attend(const float *q, const void *kplane, const void *vplane, int kv_f32,
                       int n_h, int n_kv, int hd, int start, int rows, int window, float scale,
                       float *out);

/* ---- whole-model decode (CausalLM.residentLayer order) ---- */
typedef struct or_model or_model;

typedef struct {
    int32_t n_layers, hidden, n_heads, n_kv, head_dim, ffn, vocab, ctx;
    float   eps, theta;
    int32_t kv_f32;        /* 1: f32 KV (config-literal), 0: fp16 (resident path) */
    int32_t workers;       /* CPU worker count the attention split choice uses */
    int32_t n_experts, n_used, norm_topk, expert_ffn;
    int32_t swa_window;    /* >0: windowed layers (swa_pattern) attend the last swa_window positions */
    int32_t attn_rows;     /* rows of the decode batch the split rule divides the workers over (0: 1) */
    float   w_scale;       /* expert_weights_scale (0: none) */
    int32_t swa_pattern;   /* layer l attends every position when (l + 1) % swa_pattern == 0 (<= 0: 2) */
} or_config;

or_model *or_model_new(const or_config *cfg);
void      or_model_free(or_model *m);
/* Bind a tensor by its GGUF name; the data stays owned by the caller. */
int       or_model_bind(or_model *m, const char *name, int type, const void *data,
                        int64_t rows, int64_t cols);
/* One decode step: token at position pos. Writes logits (vocab) if non-null
 * and returns the greedy argmax. */
int       or_model_step(or_model *m, int token, int pos, float *logits);
void      or_model_reset(or_model *m);
void      or_model_set_workers(or_model *m, int workers);
int       or_model_set_rope_freqs(or_model *m, const float *f, int n);
/* A prefill chunk: tokens[0..n) at positions start .. start+n-1 through
 * every layer as rows (head size 128: the prefill attention; otherwise one
 * decode step a row), then the tail on the last row. Writes its logits if
 * non-null and returns their greedy argmax. */
int       or_model_prefill(or_model *m, const int32_t *tokens, int n, int start, float *logits);
/* The last step's buffers as the last layer left them: 0 hs, 1 rotated q,
 * 2 attention output, 3 SiLU·up activation, 4 logits. Returns the length. */
int64_t   or_model_trace(or_model *m, int what, float *out, int64_t n);
int       or_model_threads(void);

#ifdef __cplusplus
}
#endif
#endif
