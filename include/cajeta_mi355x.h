/*
 * cajeta_mi355x.h — the C-ABI of the MI355X (gfx950) decode backend for
 * cajeta-llm.
 *
 * Every entry point takes only int32/int64/float scalars, opaque int64
 * handles and pointers to primitive arrays, so Cajeta's @Native (which
 * marshals no structs or callbacks, README.md:8-10) can bind each one
 * directly. Every call returns an int32 status (CJ_OK = 0, negative on
 * error) or a handle (> 0, or 0 on error); cj_last_error copies the message.
 * A refused launch enqueues nothing and returns an error: nothing is ever
 * skipped silently.
 *
 * Launches are "NoSync": they enqueue on the library's single in-order HIP
 * stream (the reference's QuantKernel.stream(), io/QuantKernel.cajeta:60-80)
 * and return. Device buffers are handles from cj_buf_alloc; every launch
 * checks that the extents it will touch fit inside the buffers it is given.
 *
 * Citations (file:line) are into jklappenbach/cajeta-llm,
 * src/main/cajeta/dev/cajeta/llm/ unless stated otherwise.
 */
#ifndef CAJETA_MI355X_H
#define CAJETA_MI355X_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CJ_OK 0
#define CJ_ERR_ARG (-1)       /* an argument or extent check failed */
#define CJ_ERR_HIP (-2)       /* the HIP runtime reported an error */
#define CJ_ERR_NOKERNEL (-3)  /* the kernel is not in the loaded code object */
#define CJ_ERR_STATE (-4)     /* not initialised, or a stale handle */
#define CJ_ERR_CAPACITY (-5)  /* KV pages or context exhausted (DeviceKv.prep, model/DeviceKv.cajeta:409-412) */
#define CJ_ERR_IO (-6)        /* a model file could not be read or parsed */

/* Weight formats: ggml type ids (io/Quant.cajeta GG_*). */
#define CJ_TYPE_F32 0
#define CJ_TYPE_F16 1
#define CJ_TYPE_Q4_0 2
#define CJ_TYPE_Q8_0 8
#define CJ_TYPE_Q4_K 12
#define CJ_TYPE_Q6_K 14
#define CJ_TYPE_MXFP4 39

/* ------------------------------------------------------------- runtime */

/* Select the device, create the stream, load kernels.hsaco with
 * hipModuleLoad. Replaces Device.force(backend) (LlmEngine.cajeta:168-170). */
int32_t cj_init(int32_t device);
int32_t cj_shutdown(void);
/* Copy the last error message (NUL-terminated, truncated to cap). */
int32_t cj_last_error(int8_t *buf, int32_t cap);
/* 1 when `name` (NUL-terminated) is a kernel this backend registered, else 0:
 * the registry behind KernelCap.usable (model/KernelCap.cajeta:228-300),
 * answered under the reference's kernel names (q4kQ8WaveMatVecKernel, ...). */
int32_t cj_kernel_available(const int8_t *name);
/* out[0] = compute units, out[1] = HBM bytes, out[2] = LDS bytes per CU. */
int32_t cj_device_info(int64_t *out, int32_t n);

/* ------------------------------------------------------------- buffers */

/* KernelBuffer<T> (the cajeta.xpu runtime): device memory by handle. */
int64_t cj_buf_alloc(int64_t bytes);
int32_t cj_buf_free(int64_t buf);
int64_t cj_buf_size(int64_t buf);
int32_t cj_buf_upload(int64_t buf, int64_t off, const int8_t *src, int64_t bytes);
int32_t cj_buf_download(int64_t buf, int64_t off, int8_t *dst, int64_t bytes);
/* Device-to-device copy of `bytes` (a multiple of 16) with a plain
 * streaming kernel: the device leg of a KernelBuffer copy, and the
 * known-size kernel the HBM counter summaries are calibrated against. */
int32_t cj_buf_copy(int64_t dst, int64_t src, int64_t bytes);
/* Zero a buffer with a fill kernel (safe inside a captured graph). */
int32_t cj_buf_zero(int64_t buf);

/* ------------------------------------------------------ stream / graph */

int32_t cj_stream_sync(void);
/* Capture the launches enqueued between begin and end into a hipGraph: the
 * deferred per-token replay of KernelStream (io/QuantKernel.cajeta:69-77). */
int32_t cj_graph_begin(void);
int64_t cj_graph_end(void);
int32_t cj_graph_launch(int64_t graph);
int32_t cj_graph_free(int64_t graph);
/* Event.recordOn / Event.waitHost (model/CausalLM.cajeta:1245-1256). */
int64_t cj_event_record(void);
int32_t cj_event_wait(int64_t ev);
int32_t cj_event_free(int64_t ev);

/* ------------------------------------------------------- launch seam */

/* q8_K activation pack of `rows` rows of n floats into 320-byte blocks, the
 * rows padded to npad (a multiple of 256); per32 = one scale per 32 values.
 * Replaces QuantKernel.q8kPackLaunchNoSync / q8kPackRowsLaunchNoSync
 * (io/QuantKernel.cajeta:42783-42800) and the q8kPack32 form (:42876-42888). */
int32_t cj_q8k_pack(int64_t out, int64_t x, int64_t rows, int64_t n, int64_t npad, int32_t per32);

/* RMSNorm (+ the pack of the result when packed != 0). out may be 0 when
 * only the pack is wanted. Replaces Prim.rmsnormPackDevice
 * (model/Prim.cajeta:1392-1406), rmsnormPack32RowsDevice (:1428-1438) and
 * rmsnormDevice (:1440). form 0: x·s·w, 1: x·s·(1+w). */
int32_t cj_rmsnorm_pack(int64_t out, int64_t packed, int64_t x, int64_t w, int64_t dim,
                        float eps, int32_t form, int32_t per32);

/* Byte size of one prepared row of `type` with `cols` columns, and the
 * load-time re-layout of GGUF rows into it (Quant.splitInto,
 * io/Quant.cajeta:184-251, re-designed for 128-bit loads). */
int64_t cj_prepared_row_bytes(int32_t type, int64_t cols);
int32_t cj_prepare_weight(int64_t dst, int64_t src, int32_t type, int64_t rows, int64_t cols);

/* y[y_off + r] (+)= Σ_c W[r][c]·x[c] over a PREPARED weight. For Q4_K/Q6_K
 * `act` is a per-256 q8_K pack, for Q8_0 a per-32 pack, for Q4_0/MXFP4 f32.
 * Replaces the route dispatch Linear.launchOne (model/Linear.cajeta:6569-6761)
 * over q4kQ8WaveMatVecLaunchNoSync (io/QuantKernel.cajeta:33558),
 * q6kQ8WaveMatVecKernel (:36273), q80Q8WaveMatVecKernel (:42509),
 * q40F32WaveMatVecKernel and mxfp4MatVecKernel (:43202); accum = 1 is
 * matvecStagedAccum's residual store (model/Linear.cajeta:5776). */
int32_t cj_matvec(int32_t type, int64_t y, int64_t w, int64_t act, int64_t rows, int64_t cols,
                  int64_t y_off, int32_t accum);

/* y[y_off + r] (+)= the MXFP4 mat-vec in the reference's device Q8 form over
 * a PREPARED MXFP4 weight and f32 x (16-byte aligned, cols a multiple of
 * 32): x quantized per 32 elements (q = round-half-away(x·127/max|x|),
 * scale max|x|/127), each row an exact integer dot a block folded by 32
 * lanes and their xor-butterfly sum — the arithmetic the engine's MoE
 * experts use. Replaces QuantKernel.mxfp4MatVecCoopQ8Launch
 * (io/QuantKernel.cajeta:43699-43713: mxfp4QuantActKernel :43614 and
 * mxfp4MatVecKernelCoopQ8 :43660). */
int32_t cj_matvec_mxfp4_q8(int64_t y, int64_t w, int64_t x, int64_t rows, int64_t cols, int64_t y_off,
                           int32_t accum);

/* Y[c][y_off + r] (+)= Σ_k W[r][k]·x_c[k] for ncols activation columns at once,
 * each column bit-for-bit what cj_matvec gives it: on the int8 matrix cores
 * for Q8_0 and Q4_K, as a many-column GEMV (each weight read once for up to
 * 16 columns, 4 for Q4_0) for Q6_K and Q4_0. `xp` holds the columns' packs
 * (per-256 for Q4_K and Q6_K, per-32 for Q8_0; for Q4_0 the f32 columns
 * themselves, at least cols·4 bytes a column) xp_stride bytes apart; y holds
 * the outputs y_stride floats apart. Replaces the many-column kernels the reference routes
 * batched decode and prefill rows through: Linear.matmulBatchKeep
 * (model/Linear.cajeta:3576) over q4kQ8WaveMatVecColsKernel
 * (io/QuantKernel.cajeta:33646), q4kQ8X8RowsKernel (:1479) and
 * q80Q8X8RowsKernel (:10236). */
int32_t cj_matmul(int32_t type, int64_t y, int64_t w, int64_t xp, int64_t rows, int64_t cols, int32_t ncols,
                  int64_t xp_stride, int64_t y_stride, int64_t y_off, int32_t accum);

/* out = act(g)·u (act 0: SiLU exp form, 1: the CPU backend's rational-tanh
 * form), plus its pack when packed != 0. Replaces Prim.gluPackDevice
 * (model/Prim.cajeta:1775-1785), gluPack32Device (:1789-1800), gluDevice. */
int32_t cj_glu(int64_t out, int64_t packed, int64_t g, int64_t u, int64_t n, int32_t form, int32_t per32);

/* a += b (Prim.addDevice, model/Prim.cajeta:1629). */
int32_t cj_add(int64_t a, int64_t b, int64_t n);

/* Per-position (cos, sin) table for split-half RoPE: rope[p][d] =
 * (cos(p·inv[d]), sin(p·inv[d])) with inv[d] = theta^(-2d/hd)
 * (Prim.invFreq, model/Prim.cajeta:1866-1909). Writes ctx·hd floats. */
int32_t cj_rope_table(int64_t out, int32_t head_dim, float theta, int32_t ctx);
/* The same with a model's precomputed per-dimension factors (GGUF
 * `rope_freqs.weight`, n_freqs = head_dim/2 host floats): each dimension's
 * inverse frequency is divided by its factor where the factor is not 0
 * (Attention's constructor, model/Attention.cajeta:80-100; ModelConfig's
 * load of the tensor, model/ModelConfig.cajeta:307-316). A count other
 * than head_dim/2 is refused with the reference's message. */
int32_t cj_rope_table_freqs(int64_t out, int32_t head_dim, float theta, int32_t ctx, const float *freqs,
                            int32_t n_freqs);

/* QK-norm (norm != 0) + RoPE + fp16 K/V append at position pos through the
 * page table. q [n_q·hd], k/v [n_kv·hd] f32 in HF (split-half) order.
 * Replaces AttnKernel.qkPrepLaunchNoSync (model/AttnKernel.cajeta:208-231). */
int32_t cj_qk_prep(int64_t q, int64_t k, int64_t v, int64_t kcache, int64_t vcache, int64_t qw, int64_t kw,
                   int64_t rope, int64_t pgtab, int32_t pg_base, int32_t n_q, int32_t n_kv, int32_t head_dim,
                   int32_t norm, float eps, int32_t form, int32_t pos);

/* Decode attention of n_q query heads over positions [from, from+count) of
 * the paged fp16 K/V, in the form the reference picks by shape:
 *  - head_dim 128 with 4 or 8 query heads per kv head: split-K into
 *    cj_decode_splits(count, n_kv, workers) splits, partials
 *    [n_q][64][hd+2] (acc, max, sum) into `part`; when out != 0 the last
 *    split of each kv head merges into out [n_q·hd] (counters: n_kv int32
 *    words, zero before the call and left zero after). Replaces
 *    AttnKernel.attnDecodeCpuGqaKernel / cpuDecodeHead
 *    (model/AttnKernel.cajeta:4216-4314) behind
 *    attendDecodePartialsLaunchNoSync (:5090-5135) and, with out,
 *    attendDecodeLaunchNoSync (:6900-6970).
 *  - otherwise: scores [n_q][count] into `part`, then softmax and the
 *    weighted sum into out (required). Replaces attnScoreKernel +
 *    attnCombineKernel (:397-515).
 * `workers` is the CPU backend's worker count the split rule uses. */
int32_t cj_attend(int64_t part, int64_t out, int64_t q, int64_t kcache, int64_t vcache, int64_t pgtab,
                  int32_t pg_base, int64_t counters, int32_t n_q, int32_t n_kv, int32_t head_dim,
                  int32_t count, int32_t from, int32_t workers, float scale);

/* Splits of a split-K decode attend: two work items a worker over the kv
 * heads, within [1, min(64, count)]. Replaces AttnKernel.cpuDecodeSplits
 * (model/AttnKernel.cajeta:4879-4889). */
int32_t cj_decode_splits(int32_t count, int32_t n_kv, int32_t workers);

/* Merge the first `splits` split partials ([n_q][64][hd+2] as cj_attend
 * writes them) into f32 out and/or their pack. Replaces
 * attnReducePackQ8Kernel (model/AttnKernel.cajeta:5165-5259). */
int32_t cj_attn_merge(int64_t out, int64_t packed, int64_t part, int32_t n_q, int32_t head_dim,
                      int32_t splits, int32_t per32);

/* out[0..hidden) = decoded row `token` of a GGUF-layout table. Replaces
 * EmbedKernel.embedRowLaunchNoSync (model/EmbedKernel.cajeta:69-265). */
int32_t cj_embed_row(int64_t out, int64_t table, int32_t type, int64_t hidden, int32_t token);

/* The same with the token id read on the device from the int32 `tokens[slot]`
 * — the slot the previous step's argmax wrote — so a per-launch route needs
 * no host round trip: EmbedKernel.embedRowLaunchNoSync(ty, hs, packed, tok,
 * blocksPerRow) (model/EmbedKernel.cajeta:306-311). The table holds `vocab`
 * rows; an id outside [0, vocab) writes zeros and sets the int32 at `status`
 * (a buffer handle, or 0 for none) to 1 instead of reading past the table. */
int32_t cj_embed_row_slot(int64_t out, int64_t table, int32_t type, int64_t hidden, int32_t vocab, int64_t tokens,
                          int32_t slot, int64_t status);

/* tok[row] = first-occurrence argmax of v[0..n) (argmaxRowLaunchNoSync,
 * io/QuantKernel.cajeta:41520-41527). */
int32_t cj_argmax_row(int64_t tok, int32_t row, int64_t v, int64_t n);

/* cj_argmax_row without any allocation: no counterpart in the reference. It
 * is for callers that cannot allocate device memory (code under hipGraph
 * capture, tight serving loops, harnesses that forbid hipMalloc). The
 * argmax's per-workgroup partials and ticket counter live in a static
 * 33 KB device array the library holds on each GPU until the process ends,
 * so n is limited to 4,194,304 values (CJ_ERR_ARG beyond). Every call on a
 * GPU shares that GPU's array: calls that overlap on one GPU race. The
 * result equals cj_argmax_row's (the same kernel). */
int32_t cj_argmax_row_noalloc(int64_t tok, int32_t row, int64_t v, int64_t n);

/* Dequantize rows·cols elements of a weight, GGUF layout (prepared = 0) or
 * the prepared layout (1). Quant.dequantize (io/Quant.cajeta:693-734). */
int32_t cj_dequant(int64_t out, int64_t raw, int32_t type, int64_t rows, int64_t cols, int32_t prepared);

/* MoE router selection over `rows` rows of n_experts logits: softmax,
 * top-k by probability (ties to the lower index), optional renormalisation,
 * then ×w_scale when w_scale is neither 0 nor 1 (expert_weights_scale).
 * A row whose logits are not finite sets the int32 at `status` (a buffer
 * handle, or 0 for none) to 1, where the reference throws
 * "moe router: the logits of this row are not finite".
 * MoeFfn.routeFromLogits (model/MoeFfn.cajeta:908-986). */
int32_t cj_moe_route(int64_t sel, int64_t weights, int64_t logits, int32_t rows, int32_t n_experts,
                     int32_t n_used, int32_t norm_topk, float w_scale, int64_t status);

/* The router mat-vec and its top-k in one launch: logits[e] = w_router[e]·x
 * (experts rows of cols f32), then sel[used] and w[used] as the reference's
 * device router selects them (softmax over the experts, top-k by
 * probability, ties to the lower index, renormalised when norm_topk, then
 * ×w_scale unless it is 0 or 1). counter: one int32, zero before the call
 * and left zero. Replaces QuantKernel.routerTopKLaunchNoSync(sel, w, logits,
 * wRouter, x, counter, experts, cols, used, normTopk, wScale)
 * (io/QuantKernel.cajeta:40701-40709; routerTopKKernel :39850-39960). */
int32_t cj_router_topk(int64_t sel, int64_t w, int64_t logits, int64_t w_router, int64_t x, int64_t counter,
                       int32_t experts, int32_t cols, int32_t used, int32_t norm_topk, float w_scale);

/* The two-pass decode attention's score pass alone: scores[h][t] =
 * (q_h · K_t)·scale for t < count over positions [from, from + count) of the
 * paged fp16 K plane, kv head h / (n_q/n_kv). Replaces attnScoreKernel's
 * launch (model/AttnKernel.cajeta:397-425, the first half of
 * attendDecodeLaunchNoSync's two-pass form). */
int32_t cj_attn_scores(int64_t scores, int64_t q, int64_t kcache, int64_t pgtab, int32_t pg_base, int32_t n_q,
                       int32_t n_kv, int32_t head_dim, int32_t count, int32_t from, float scale);

/* ------------------------------------------------------------ engine */

/* The LlmEngine surface (LlmEngine.cajeta:165-546) over a GGUF model:
 * path "mem:<name>" loads an image made by cj_synth_gguf. ctx is the KV
 * capacity per sequence, max_seqs the sequence slots. */
int64_t cj_engine_load(const int8_t *path, int32_t ctx, int32_t max_seqs);
/* cj_engine_load with the K/V cache's options. kv_pages: the pool's size in
 * pages of 64 positions shared by every slot (0: every slot at its full
 * context, what cj_engine_load gives) — the CausalLM(cfg, maxSeq, maxSeqs,
 * numBlocks) constructor's numBlocks (model/CausalLM.cajeta:64-94). A
 * smaller pool holds more slots than it could at full context; the
 * scheduler preempts the youngest running request when a request's next
 * rows do not fit, and resumes it later by recomputing its stream.
 * kv_f32 != 0: the K/V planes hold f32, the reference's PagedKvCache mode
 * (model/PagedKvCache.cajeta), read by the two-pass attention (head size
 * 64, or GQA other than 4 and 8 at 128; up to 6144 positions); other models
 * are refused with the reason. */
int64_t cj_engine_load_kv(const int8_t *path, int32_t ctx, int32_t max_seqs, int32_t kv_pages, int32_t kv_f32);
int32_t cj_engine_close(int64_t eng);
/* Up to 14 values: n_layers, hidden, n_heads, n_kv, head_dim, ffn, vocab,
 * ctx, n_experts, n_used, weight type, head type, expert ffn, and the CPU
 * worker count the split-K attention rule is evaluated for (512). */
int32_t cj_engine_config(int64_t eng, int64_t *out, int32_t n);
/* LlmEngine.submitTokens (:477) → Scheduler.submitSampled (sched/Scheduler.cajeta:267):
 * a greedy request whose stop tokens are the model's end-of-generation set
 * (LlmEngine.defaultStops, :458-474); returns its id (0, 1, ... in
 * submission order). A prompt that cannot fit a sequence slot with one
 * decode position is refused (CJ_ERR_CAPACITY). */
int32_t cj_engine_submit(int64_t eng, const int32_t *prompt, int32_t n, int32_t max_new);
/* The same with the caller's SampleParams.stopTokens (n_stops >= 0; an empty
 * list means no stop token). */
int32_t cj_engine_submit_stops(int64_t eng, const int32_t *prompt, int32_t n, int32_t max_new, const int32_t *stops,
                               int32_t n_stops);
/* LlmEngine.stepOnce (:504) → Scheduler.stepOnce (sched/Scheduler.cajeta:414-605):
 * ONE scheduler step — admit waiting requests into free sequence slots
 * (FIFO), feed each running request's pending rows (a prompt chunk of up to
 * the prefill chunk size, or one decode position; every decoding request
 * together as one batched step; a sole running greedy request through the
 * pipelined step, Scheduler.pipeFor/stepPipelined :613-702: its next step
 * is queued before the previous one's token is read, so the first such call
 * emits no token and a finish drains one queued step), append each produced
 * greedy token, check its stops (stop token → FINISH_EOS, then the budget →
 * FINISH_BUDGET), retire finished requests and admit again (preempted ones
 * first). A request whose next rows do not fit the K/V pool preempts the
 * youngest running request (itself, if youngest). Returns 1 while a request
 * is unfinished, 0 when all are done, < 0 on error. */
int32_t cj_engine_step_once(int64_t eng);
/* LlmEngine.runAll (:500) → Scheduler.runAll (:1005): stepOnce until every
 * request is done; CJ_ERR_STATE ("not done after N steps") past max_steps. */
int32_t cj_engine_run_all(int64_t eng, int32_t max_steps);
/* LlmEngine.request (:508): writes up to cap generated ids, *state
 * (0 waiting, 1 running, 2 preempted, 3 done: sched/Request.cajeta:9-13)
 * and *finish (Request.FINISH_*: 0 none,
 * 1 budget, 2 end-of-generation token, 4 cancelled; sched/Request.cajeta:18-23).
 * Returns the generated count. */
int32_t cj_engine_request(int64_t eng, int32_t id, int32_t *tokens, int32_t cap, int32_t *state, int32_t *finish);
/* LlmEngine.cancel (:512) → Scheduler.cancel (:288-315), between steps:
 * 1 when cancelled (DONE with FINISH_CANCEL, its slot freed), 0 when the id
 * was never issued or is already done. */
int32_t cj_engine_cancel(int64_t eng, int32_t id);
/* The model's end-of-generation set (LlmEngine.eogTokens), which requests
 * submitted afterwards take as their stop tokens. */
int32_t cj_engine_set_eog(int64_t eng, const int32_t *ids, int32_t n);

/* CausalLM seam: prefill and free greedy decode of one sequence slot.
 * prefill feeds tokens[0..n) at positions pos0..: with n > 1 as prefill
 * chunks of up to the chunk size (CausalLM.stepSeq, model/CausalLM.cajeta:
 * 801-883: every row through a layer, the tail on the last row only) — the
 * prefill attend on dense head-size-128 models, each row's decode attention
 * on the others (head size 64, MoE), which the reference prefills a decode
 * step a position — and one graph-captured decode step a position where
 * the many-row path does not serve the model; decode runs `steps` greedy
 * steps from the state prefill left and writes the generated ids. logits:
 * the last step's (or the prompt's last row's) logits. */
int32_t cj_engine_reset(int64_t eng, int32_t seq);
int32_t cj_engine_prefill(int64_t eng, int32_t seq, const int32_t *tokens, int32_t n);
int32_t cj_engine_decode(int64_t eng, int32_t seq, int32_t steps, int32_t *out_tokens);
/* Batched greedy decode: `steps` tokens for each of n prefilled slots at once,
 * one row a slot sharing every weight read (CausalLM.decodeBatchRows,
 * model/CausalLM.cajeta:4133-4360; the reference's batched Cols kernels,
 * io/QuantKernel.cajeta:33646, and batch attention, model/AttnKernel.cajeta:5761,
 * :6599). out_tokens[i·n + r] is slot r's token i. */
int32_t cj_engine_decode_batch(int64_t eng, const int32_t *slots, int32_t n, int32_t steps, int32_t *out_tokens);
/* The CPU worker count the attention's split rule divides by
 * (EngineOptions.cpuThreads → Device.multiprocessorCount on the CPU backend,
 * AttnKernel.cpuDecodeSplits, model/AttnKernel.cajeta:4879-4889): the split
 * count, and with it the rounding of the merged attention, follow it exactly
 * as the reference's CPU backend with that many workers would. Default 512. */
int32_t cj_engine_set_cpu_threads(int64_t eng, int32_t threads);
/* Rows a prefill chunk (CausalLM.CHUNK_MAX, model/CausalLM.cajeta:52; at most
 * the row buffers' capacity); 0 or 1: prefill as one decode step a position. */
int32_t cj_engine_set_prefill_chunk(int64_t eng, int32_t rows);
int32_t cj_engine_logits(int64_t eng, int32_t seq, float *out, int64_t n);
/* Predicted (argmax) ids at positions 1..n of the slot's history. */
int32_t cj_engine_preds(int64_t eng, int32_t seq, int32_t *out, int32_t n);
/* Average device time per decode step over the last cj_engine_decode call (µs). */
float cj_engine_last_step_us(int64_t eng);
/* Debug taps of the last step (CausalLM.sniffBuf, model/CausalLM.cajeta:2260-2360):
 * what 0 = residual hs [hidden], 1 = rotated q [n_heads·hd], 2 = attention
 * output [n_heads·hd], 3 = SiLU·up activation [ffn], 4 = logits [vocab] —
 * each as the last layer left it; 5 = the down projection's activation pack
 * (as f32 words); 6 = the last batched decode step's logits [rows][vocab]. */
int32_t cj_engine_trace(int64_t eng, int32_t what, float *out, int64_t n);
/* Measurement seam, no counterpart in the reference's decode API (its
 * benches time whole steps from the host): `reps` back-to-back
 * launches of one launch kind of the slot's step, layer 0, at its current
 * position, timed between HIP events on the engine's stream; the step state
 * is left unchanged. kind: 0 embed, 1 q|k|v, 2 attention, 3 o, 4 gate|up,
 * 5 down, 6 router, 7 top-k, 8 expert gate|up, 9 expert down, 10 combine,
 * 11 head + argmax. Writes the mean µs, the launch's algorithmic HBM bytes
 * and the kernel's name (the last one for a two-launch kind). */
int32_t cj_engine_time_kernel(int64_t eng, int32_t seq, int32_t kind, int32_t reps, float *avg_us, int64_t *bytes,
                              int8_t *name, int32_t name_cap);
/* Measurement seam, no counterpart in the reference: the same launch kind
 * timed inside the step — `steps` whole decode steps of the slot enqueued as
 * the step runs them (after one warm-up step), an event before and after each
 * of the kind's launches (every layer); writes the mean interval in µs (each
 * includes the launch's share of the kernel boundary). kind: 1 q|k|v,
 * 2 attention, 3 o, 4 gate|up, 5 down. The step state is left unchanged. */
int32_t cj_engine_time_kernel_in_step(int64_t eng, int32_t seq, int32_t kind, int32_t steps, float *avg_us);
/* Replay the captured step graph (on != 0, the default) or enqueue the
 * step's launches each token. The kernels and their arguments are the same;
 * the eager form is for tools that cannot follow graph launches. No
 * counterpart in the reference (its host loop launches each kernel). */
int32_t cj_engine_set_graphs(int64_t eng, int32_t on);
/* Algorithmic HBM bytes of one whole decode step attending `count`
 * positions: weights at their GGUF size, K/V read and appended, activation
 * vectors once. */
int64_t cj_engine_step_bytes(int64_t eng, int32_t count);

/* -------------------------------------------------- synthetic models */

/* Write a seeded random-init GGUF (v3, llama metadata, q/k rows in GGUF's
 * rope order) for `spec` — "c1" ... "c5" or "key=value;..." — to `path`, or
 * to an in-process image when path is "mem:<name>". */
int32_t cj_synth_gguf(const int8_t *spec, const int8_t *path, int64_t seed);
/* Host address and size of an in-process image (for checkers). */
int32_t cj_image_info(const int8_t *name, int64_t *addr, int64_t *size);
int32_t cj_image_free(const int8_t *name);
/* Open a GGUF as the engine's loader does — one file, or a split model
 * (<base>-%05d-of-%05d.gguf) from any of its shards — and report its tensor
 * and shard counts; no GPU needed (GgufFile's directory,
 * io/GgufFile.cajeta:45-55, :467-560). Missing or mismatched shards fail
 * with the reason. */
int32_t cj_gguf_info(const int8_t *path, int64_t *n_tensors, int64_t *n_shards);

#ifdef __cplusplus
}
#endif
#endif
