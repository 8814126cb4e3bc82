// args.h — kernel argument blocks shared by the gfx950 code object and the
// host runtime. Every kernel in kernels.hsaco takes exactly one of these by
// value, so hipModuleLaunchKernel passes one pointer and the layout is
// fixed in one place. Plain C types only.
#pragma once
#include <stdint.h>

// Weight formats (ggml type ids, the reference's Quant.GG_*).
#define CJ_F32 0
#define CJ_F16 1
#define CJ_Q4_0 2
#define CJ_Q8_0 8
#define CJ_Q4_K 12
#define CJ_Q6_K 14
#define CJ_MXFP4 39

// GEMV prologue: where the activation comes from.
#define CJ_PRO_PACKED 0     // an int8 pack already in HBM (320-byte blocks)
#define CJ_PRO_PACK 1       // f32 x in HBM, packed into LDS here
#define CJ_PRO_NORM_PACK 2  // f32 x in HBM, RMSNorm'd then packed into LDS
#define CJ_PRO_F32 3        // f32 x in HBM, used as f32 (Q4_0, MXFP4)
#define CJ_PRO_NORM_F32 4   // f32 x in HBM, RMSNorm'd, used as f32
#define CJ_PRO_MXQ8 5       // f32 x in HBM, per-32 int8 codes + scales in LDS (MXFP4 device Q8 form)

// GEMV epilogue: what happens to each output row.
#define CJ_EPI_STORE 0      // y[row] = v
#define CJ_EPI_ACCUM 1      // y[row] += v (residual rides the store)
#define CJ_EPI_QKV_ROPE 2   // q|k rows in GGUF pair order: RoPE, q out, K/V fp16 append
#define CJ_EPI_GLU 3        // gate/up rows interleaved: silu(g)·u, then the pack of the result
#define CJ_EPI_ARGMAX 4     // logits out + first-occurrence argmax into the token history

// Device-resident decode state the per-token graph reads and advances.
typedef struct {
    int32_t pos;          // position of the token being decoded
    int32_t fixed_until;  // tokens[p] for p < fixed_until are given (prompt), not predicted
    int32_t pad[2];
} cj_step_state;

typedef struct {
    // tensors
    const uint8_t *w;       // prepared weight rows
    const float *x;         // f32 activation (PRO_PACK / NORM_PACK / F32)
    const uint8_t *xp;      // packed activation (PRO_PACKED)
    const float *nw;        // norm weight (NORM_*)
    float *y;               // output rows (STORE / ACCUM / ARGMAX logits)
    // epilogue extras
    float *q_out;           // QKV: rotated q (HF order)
    uint16_t *kc, *vc;      // QKV: K/V planes (page-blocked, head-major), fp16 (or f32: kv_f32)
    const int32_t *pgtab;   // QKV: KV page table
    const float *rope_cs;   // QKV: [ctx][half] (cos, sin) pairs
    float *act;             // GLU: silu(g)·u out (f32)
    uint8_t *act_pack;      // GLU: packed result for the down projection
    int32_t *counters;      // GLU: per-256-block arrival counters; ARGMAX: one counter
    float *part_v;          // ARGMAX: per-workgroup best value
    int32_t *part_i;        // ARGMAX: per-workgroup best index
    int32_t *tokens;        // ARGMAX: token history, tokens[pos+1] written past the prompt
    int32_t *preds;         // ARGMAX: preds[pos+1] = the argmax at every step
    cj_step_state *state;   // device step state (pos); null: use `pos`
    // shapes
    int64_t rows, cols;     // weight rows (outputs) and columns (inputs)
    int64_t row_bytes;      // prepared bytes per row
    int64_t y_off;          // output row offset (reference yOff)
    int32_t type;           // CJ_Q4_K ...
    int32_t pro, epi;
    int32_t per32;          // activation pack at one scale per 32 (Q8_0 consumers)
    int32_t rows_per_wg;    // output rows per workgroup
    float eps;
    int32_t norm_form;      // 0: w, 1: (1 + w)
    int32_t n_q, n_kv, head_dim;   // QKV layout (rows: q heads, k heads, v heads)
    int32_t pg_base;        // QKV: page-table base of the sequence
    int32_t pos;            // host position when state is null
    int32_t act_n;          // GLU: real width of the activation (ffn)
    int32_t act_per32;      // GLU: the down projection reads a per-32 pack
    int32_t glu_form;       // GLU: 0 exp form, 1 rational-tanh form
    int32_t batch;          // columns of activation (Cols variants), 1 at decode
    int64_t x_stride;       // floats between activation vectors (batch / expert k)
    int64_t xp_stride;      // bytes between packed activation vectors
    int64_t y_stride;       // floats between output vectors (y, act) per batch / expert k
    // MoE indirection: workgroups cover n_sel copies of the rows; copy k reads
    // weight w + sel[k]·expert_bytes, activation x + (k / sel_per_x)·x_stride
    // (the pack likewise), writes at k·y_stride
    const int32_t *sel;
    int64_t expert_bytes;
    int32_t n_sel;
    int32_t sel_per_x;      // copies sharing one activation (many rows: n_used); ≤ 1: activation k
    // the MoE route inside the expert gate|up launch (route_logits non-null):
    // copy c = r·n_sel_row + k routes row r from its logits, takes expert
    // sel_r[k] itself, and the row's first workgroup writes the row's
    // selections and weights for the down and combine launches
    const float *route_logits;
    int32_t *route_sel;
    float *route_w;
    int32_t *route_status;
    int32_t route_experts, route_used, route_norm_topk;
    float route_scale;
    // NORM_F32 prologue: workgroup 0 also writes the normed f32 activation
    // here (for the launches after it; may be null)
    float *xout;
    int32_t kv_f32;         // QKV: the K/V planes hold f32 (kc, vc point at floats)
    int32_t pad_kv;
} cj_gemv_args;

typedef struct {
    float *hs; const float *y; const float *w; int64_t n; int32_t n_used; int32_t pad;
} cj_combine_args;

typedef struct {
    uint8_t *out;           // packed blocks
    const float *x;         // input rows
    const float *w;         // norm weight (norm variants)
    float *xout;            // normed f32 out (may be null)
    int64_t n, npad;        // real and padded widths
    int64_t rows;           // rows (each n wide in x, npad/256*320 bytes in out)
    float eps;
    int32_t form, per32, do_norm;
} cj_pack_args;

// The MoE combine with the next RMSNorm + pack: hs_out = hs_in + Σ_k w_k·y_k
// (k order), then `p`'s norm and pack of hs_out (p.x unused).
typedef struct {
    float *hs_out; const float *hs_in; const float *y; const float *w;
    int64_t n; int32_t n_used; int32_t pad;
    cj_pack_args p;
} cj_combine_norm_args;

typedef struct {
    float *out; const float *g, *u;
    uint8_t *packed;        // optional pack of the result
    int64_t n, npad;
    int32_t form;           // 0 exp, 1 rational tanh
    int32_t per32;
} cj_glu_args;

typedef struct { float *a; const float *b; int64_t n; } cj_add_args;

typedef struct { void *dst; const void *src; int64_t n16; } cj_copy_args;

typedef struct {
    float *q, *k; const float *v;
    uint16_t *kc, *vc;
    const float *qw, *kw;    // optional per-head norm weights (norm != 0)
    const float *rope_cs;    // [ctx][half] (cos, sin)
    const int32_t *pgtab;
    const cj_step_state *state;
    int32_t n_q, n_kv, head_dim, norm, form, pg_base, pos;
    float eps;
    int32_t kv_f32;          // the K/V planes hold f32
} cj_qkprep_args;

// Output dimensions a workgroup of the fp16-K/V two-pass combine (HD/CJ_COMBINE_DH
// workgroups a query head): the kernels' tiling and the launches' grids.
#define CJ_COMBINE_DH 16

typedef struct {
    float *part;             // split-K: [n_q][64][hd + 2] partials; two-pass: scores [n_q][splits]
    float *out;              // merged f32 output (null: partials only)
    const float *q;
    const uint16_t *kc, *vc;
    const int32_t *pgtab;
    const cj_step_state *state;
    int32_t *counters;       // per kv head arrival counters (merge in the last)
    int32_t n_q, n_kv, head_dim;
    int32_t splits;          // two-pass: the scores row stride (≥ count)
    int32_t pg_base;
    int32_t count, from;     // host values when state is null
    int32_t window;          // >0: attend the last `window` positions only
    int32_t workers;         // split-K: the CPU worker count the split rule uses
    float scale;
    int32_t pg_n;            // pages the sequence owns from pg_base (bounds the table prefetch)
    int32_t per32;           // split-K with an output: pack `packed` at one scale per 32
    uint8_t *packed;         // split-K with an output: the q8 pack of the merged output (may be null)
    // many-row forms (rowtab non-null): row r is sequence slot rowtab[2r] at
    // position states[slot].pos + rowtab[2r+1]; its pages from slot·pg_n
    const int32_t *rowtab;
    const cj_step_state *states;
    int32_t nrows;           // rows in the batch (the split rule divides the workers over rows·n_kv)
    int32_t spl;             // split slots a row (grid: rows · n_kv · spl)
    int64_t q_stride;        // floats between rows of q (and of out)
    int64_t part_stride;     // floats between rows of the partials
} cj_attn_args;

typedef struct {
    float *out; uint8_t *packed; const float *part;
    const cj_step_state *state;  // non-null: splits follow the device position
    int32_t n_q, head_dim, splits, per32;
    int32_t n_kv, workers, window, nrows;
    // many-row form (rowtab non-null): as cj_attn_args
    const int32_t *rowtab;
    const cj_step_state *states;
    int64_t part_stride, out_stride, pack_stride;
} cj_merge_args;

// The many-row step kernels (batched decode: a row a sequence; prefill: a
// row a position of one sequence). Row r is slot rowtab[2r] at position
// states[slot].pos + rowtab[2r+1].
typedef struct {
    const int32_t *rowtab;
    cj_step_state *states;
    int32_t *tokens, *preds;    // per-slot histories, hist ints apart
    int64_t hist;
    // embedding
    const uint8_t *table; int64_t row_bytes; int32_t type; int32_t nrows;
    // row buffers
    const float *in; float *out; uint8_t *packed;
    int64_t in_stride, out_stride, pack_stride;
    // q|k|v: RoPE, q rows out, fp16 K/V append
    float *q_out; uint16_t *kc, *vc; const int32_t *pgtab; const float *rope_cs;
    int32_t pg_n, n_q, n_kv, head_dim;
    // widths: embedding / GLU width n (padded npad); GLU form and pack
    int64_t n, npad;
    int32_t form, per32;
    // argmax partials: [rows][nchunks] of 1024-wide chunks
    float *pv; int32_t *pi; int32_t nchunks;
    int32_t kv_f32;          // q|k|v: the K/V planes hold f32
} cj_rows_args;

typedef struct {
    // the step's greedy pick from per-workgroup (value, index) partials
    const float *pv; const int32_t *pi; int32_t n, pos;
    int32_t *tokens, *preds; cj_step_state *state;
    int32_t *host_tok;      // pinned host mirror of `tokens` (null: none): the host reads a step's token without a copy
} cj_pick_args;

typedef struct {
    float *out; const uint8_t *table; const int32_t *tokens; const cj_step_state *state;
    int32_t type; int64_t hidden; int64_t row_bytes; int32_t token;
    int32_t vocab;           // > 0: a device-read token id outside [0, vocab) writes zeros and sets *status
    int32_t *status;
} cj_embed_args;

typedef struct {
    int32_t *tok; const float *v; float *pv; int32_t *pi; int32_t *counter;
    int64_t n; int32_t row;
} cj_argmax_args;

typedef struct {
    float *out; const uint8_t *raw;
    int64_t elems;           // rows · cols elements decoded
    int64_t row_bytes, cols;
    int32_t type;
    int32_t prepared;        // 1: the gemv row layout, 0: GGUF file blocks
} cj_dequant_args;

typedef struct {
    uint8_t *dst; const uint8_t *src; int64_t rows, cols, src_row_bytes, dst_row_bytes; int32_t type; int32_t pad;
} cj_prepare_args;

typedef struct {
    const float *logits; int32_t *sel; float *w; int32_t n_experts, n_used, norm_topk, rows;
    float w_scale;           // expert_weights_scale: applied when neither 0 nor 1
    int32_t pad;
    int32_t *status;         // set to 1 when a row's logits are not finite (may be null)
} cj_route_args;

// The rows' expert selections grouped by expert (MoeFfn.forwardRowsZeroSync
// reads each selected expert once for all the rows that chose it).
typedef struct {
    const int32_t *sel;      // [n_sel] expert of selection i (= r·n_used + k)
    int32_t *cnt;            // [n_experts] selections of each expert
    int32_t *mem;            // [n_experts][cap] expert e's selections (any order)
    int32_t n_sel, n_experts, cap, pad;
} cj_moe_group_args;

// A grouped MXFP4 expert product (the device Q8 form) over the selections of
// each expert: workgroup (row tile, expert) streams its 64 weight rows once
// and dots them with every member selection's per-32 activation codes.
typedef struct {
    const uint8_t *w;        // expert bank of prepared MXFP4 rows: expert e at w + e·expert_bytes
    const uint8_t *xp;       // input per-32 packs (320-byte blocks), xp_stride bytes a row
    uint8_t *outp;           // SiLU·up form: each selection's activation as per-32 packs, outp_stride bytes apart
    float *y;                // store form: each selection's outputs, y_stride floats apart
    const int32_t *cnt, *mem;   // from cj_moe_group
    int64_t expert_bytes, row_bytes, rows, cols;
    int64_t xp_stride, outp_stride, y_stride;
    int32_t cap, x_per;      // selection i reads input row i / x_per
    int32_t glu_form, act_n;
} cj_moe_grp_args;

// routerTopKKernel's arguments (io/QuantKernel.cajeta:39850-39960): the
// router mat-vec of one f32 row and its top-k in one launch.
typedef struct {
    int32_t *sel; float *w; float *logits; const float *w_router; const float *x;
    int32_t *counter;        // zero before the launch; the selecting workgroup leaves it zero
    int32_t experts, cols, used, norm_topk;
    float w_scale;
} cj_router_topk_args;

typedef struct {
    // one MoE expert stage: rows of expert sel[k] for each k < n_used
    const uint8_t *w;        // stacked experts [E][rows][row_bytes]
    const float *x;          // f32 input (gate/up: the normed hidden; down: per-k activations)
    float *y;                // gate/up: act out [n_used][rows]; down: accumulate into y[rows]
    const int32_t *sel; const float *wts;
    int64_t rows, cols, row_bytes, expert_bytes;
    int32_t n_used, stage;   // stage 0: gate|up + silu·u, 1: down + weighted combine
    int32_t type;
    int32_t pad;
} cj_moe_args;
