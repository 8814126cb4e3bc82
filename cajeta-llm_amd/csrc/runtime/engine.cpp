// engine.cpp — the decode engine behind the LlmEngine surface: a GGUF model
// loaded into prepared, fused device weights, paged fp16 K/V drawn from a
// shared page pool, and the whole per-token decode step (embedding → layers
// → norm → head → argmax) captured once per sequence slot into a hipGraph
// and replayed per token. Position and token history live on the device, so
// step N+1 is enqueued without waiting for step N (the reference's
// queueStep/awaitStep pipelining, model/CausalLM.cajeta:1208-1256): the
// scheduler's pipelined greedy decode queues it before reading step N's
// token, which the head's pick also writes to pinned host memory.
//
// Per dense layer the step is six launches:
//   1. q|k|v GEMV, RMSNorm + pack in the prologue, RoPE + fp16 K/V append
//      in the epilogue (residentLayer steps 1-3, CausalLM.cajeta:3636-3694)
//   2. split-K flash decode partials (step 4; or the two-pass scores, then
//      the softmax + p·V combine, where the reference takes that form)
//   3. the split merge, f32 out (step 5)
//   4. o GEMV, pack prologue, residual-accumulate epilogue (step 6)
//   5. gate|up GEMV, RMSNorm + pack prologue, SiLU·up epilogue (7-9)
//   6. down GEMV, pack prologue, residual-accumulate epilogue (step 10)
// MoE layers (gpt-oss shape) replace 5-6 with router GEMV, top-k, indirected
// expert gate|up, indirected expert down and the weighted combine.
#include "gguf.h"
#include "rt.h"
#include <chrono>
#include <cmath>
#include <cstring>
#include <algorithm>
#include <deque>
#include <memory>
#include <set>
#include <vector>

namespace cj {

namespace {

struct DevW {            // a prepared device weight
    void *p = nullptr;
    int type = 0;
    int64_t rows = 0, cols = 0, row_bytes = 0;
};

struct Layer {
    DevW qkv, o, gu, down;           // dense
    DevW router, gu_exps, down_exps; // MoE
    float *attn_norm = nullptr, *ffn_norm = nullptr;
    int window = 0;
    uint16_t *kc = nullptr, *vc = nullptr;
};

struct Seq {
    int32_t *tokens = nullptr;   // device token history (inputs)
    int32_t *preds = nullptr;    // device argmax per position
    cj_step_state *state = nullptr;
    int pg_base = 0;
    hipGraphExec_t graph = nullptr;
    int pos = 0;                 // host mirror
    int fixed_until = 0;
};

// A request of the scheduler (sched/Request.cajeta): its ids (prompt, then
// generated), how many positions the model has consumed, and its state.
struct Request {
    // Request.WAITING/RUNNING/PREEMPTED/DONE (sched/Request.cajeta:9-13)
    enum { WAITING = 0, RUNNING = 1, PREEMPTED = 2, DONE = 3 };
    // Request.FINISH_* (sched/Request.cajeta:18-23)
    enum { FINISH_NONE = 0, FINISH_BUDGET = 1, FINISH_EOS = 2, FINISH_CANCEL = 4 };
    std::vector<int32_t> all;     // prompt then generated ids (Request.all)
    std::vector<int32_t> stops;   // stop tokens: the model's EOG set unless the caller gave its own
    int prompt_len = 0, max_new = 0, gen = 0;
    int cached = 0;               // positions the model has consumed (Request.cachedLen)
    // ids all[0, feed) go to the model from the host (the prompt, or after a
    // preemption the whole stream, recomputed); past that the device holds
    // each id: the pick that produced it wrote it into the slot's history
    int feed = 0;
    int stamp = 0, pre_stamp = 0; // admission order (the preemption age), preemption order (the resume FIFO)
    int state = WAITING, slot = -1, finish = FINISH_NONE;
};

// The launches of one decode step, by kind (the timing seam addresses one).
enum Kind {
    K_EMBED = 0, K_QKV = 1, K_ATTN = 2, K_O = 3, K_GATE_UP = 4, K_DOWN = 5,
    K_ROUTER = 6, K_ROUTE = 7, K_EXP_GATE_UP = 8, K_EXP_DOWN = 9, K_COMBINE = 10, K_HEAD = 11,
    K_NORM = 12,  // RMSNorm + pack of the residual (before q|k|v; the FFN and head ones alike)
    K_MERGE = 13  // the split-K attention's merge + pack alone (part of K_ATTN in the step)
};

}  // namespace

struct Engine {
    Gguf file;
    int n_layers = 0, hidden = 0, n_heads = 0, n_kv = 0, head_dim = 0, ffn = 0, vocab = 0, ctx = 0, max_seqs = 1;
    int n_experts = 0, n_used = 0, expert_ffn = 0, norm_topk = 1;
    float w_scale = 0.0f;      // expert_weights_scale (0: none)
    int32_t *route_status = nullptr;   // set by the router when a row's logits are not finite
    float eps = 1e-5f, theta = 10000.0f, scale = 1.0f;
    int wtype = 0, head_type = 0, embd_type = 0;
    int64_t embd_row_bytes = 0;
    void *embd = nullptr;
    float *out_norm = nullptr;
    DevW head;
    std::vector<Layer> layers;
    int pages_per_seq = 0, workers = 512;
    int32_t *pgtab = nullptr;
    float *rope = nullptr;
    // scratch
    float *hs = nullptr, *q = nullptr, *attn = nullptr, *act = nullptr, *logits = nullptr, *part = nullptr;
    float *hs2 = nullptr;      // MoE models: the combine writes the residual here and back, alternately
    float *hs_last = nullptr;  // the buffer the last enqueued step's residual ended in
    uint8_t *act_pack = nullptr, *attn_pack = nullptr, *xpack = nullptr;
    float *xn = nullptr;       // the normed residual as f32 (f32-activation consumers)
    int32_t *glu_counters = nullptr, *argmax_counter = nullptr, *attn_counters = nullptr;
    float *part_v = nullptr;
    int32_t *part_i = nullptr;
    float *moe_logits = nullptr, *moe_w = nullptr, *moe_y = nullptr;
    int32_t *moe_sel = nullptr;
    std::vector<Seq> seqs;
    std::set<int> eog;
    std::vector<Request> reqs;
    std::vector<int> slot_req;   // the request in each sequence slot, or -1 (Scheduler.slotReq)
    int64_t sched_steps = 0;
    float last_step_us = 0.0f;
    std::vector<void *> owned;
    int only = -1;             // enqueue only this kind, of layer only_layer (-1: the whole step)
    int only_layer = 0;
    bool graphs = true;        // replay the captured step (false: enqueue its launches each token)
    // the split-K merge as a wave per 64 dimensions, f32 out packed by the o
    // projection (CJ_MERGE_W=0: the 256-wide merge + pack, for comparisons)
    bool merge_w = [] { const char *e = getenv("CJ_MERGE_W"); return !e || strcmp(e, "0") != 0; }();
    // the one-row step's MoE route inside the MXFP4 experts' gate|up launch
    // (each workgroup routes the row, then streams its expert): one launch
    // fewer a layer, C5 2.372 -> 2.337 ms a token (CJ_ROUTE_FUSED=0: the
    // route as its own launch, for comparisons)
    bool fuse_route = [] { const char *e = getenv("CJ_ROUTE_FUSED"); return !e || strcmp(e, "0") != 0; }();
    // the MoE combine with the next RMSNorm + pack in one launch
    // (CJ_COMBINE_NORM=0: two launches, for comparisons)
    bool combine_norm = [] { const char *e = getenv("CJ_COMBINE_NORM"); return !e || strcmp(e, "0") != 0; }();
    bool route_fused(const Layer &L) const { return fuse_route && L.gu_exps.type == CJ_MXFP4; }
    void route_into(cj_gemv_args &a, const float *logits, int32_t *sel, float *w) const {
        a.sel = nullptr; a.route_logits = logits; a.route_sel = sel; a.route_w = w; a.route_status = route_status;
        a.route_experts = n_experts; a.route_used = n_used; a.route_norm_topk = norm_topk; a.route_scale = w_scale;
    }
    int32_t *pinned = nullptr; // pinned host staging: [ctx + 2] token ids, then a cj_step_state
    // the K/V page pool (PagedKvCache's blocks, model/CausalLM.cajeta:64-94):
    // a slot draws 64-position pages as its sequence grows and returns them
    // when it is reset or its request leaves; the default pool holds every
    // slot at its full context
    int kv_pages = 0;
    // the K/V planes hold f32 (the reference's PagedKvCache mode), where the
    // attention takes the two-pass form
    bool kv_f32 = false;
    std::vector<int32_t> free_pages;
    std::vector<std::vector<int32_t>> slot_pages;
    int32_t *pinned_pg = nullptr;   // host mirror of the page table (pinned: the source of its uploads)
    // the pipelined greedy decode (Scheduler.pipeFor/stepPipelined,
    // sched/Scheduler.cajeta:613-702): the step in flight and the one before
    bool pipe_in = false;
    int pipe_req = -1, pipe_out = 0;
    int pipe_pos[2] = {0, 0};       // the position each in-flight step consumes
    hipEvent_t pipe_ev[2] = {nullptr, nullptr};
    int32_t *host_tok = nullptr;    // pinned [max_seqs][ctx + 2]: the head's pick writes every token here too
    int stamp_n = 0;
    int64_t preempted_n = 0, resumed_n = 0;
    int64_t embd_row_file_bytes = 0;
    // the many-row path: batched decode (a row a sequence) and prefill
    // chunks (a row a position)
    cj_step_state *states = nullptr;           // [max_seqs]; seqs[s].state = states + s
    int32_t *tokens_all = nullptr, *preds_all = nullptr;   // [max_seqs][ctx + 2]
    bool rows_ok = false;      // the many-row path serves the model (int8-pack projections; MoE experts indirected)
    bool rows_split = false;   // decode attention rows take the split-K rows kernel (else the two-pass rows)
    bool rows_prefill = false; // prompts go through prefill chunks of rows
    bool rows_pf_attend = false;   // a chunk's attention is the prefill attend (else each row's decode attention)
    int chunk = 512;           // prefill rows a chunk (CausalLM.CHUNK_MAX)
    int rows_cap = 0;          // rows the row buffers hold
    float *r_hs = nullptr, *r_qkv = nullptr, *r_q = nullptr, *r_attn = nullptr, *r_gu = nullptr;
    // MoE rows: the normed rows (f32), router logits, selections, weights,
    // the selections' SiLU·up activations and down outputs, and an all-zero
    // selection list (the router's indirection: every row reads one weight)
    float *r_xn = nullptr, *r_moe_logits = nullptr, *r_moe_w = nullptr, *r_act = nullptr, *r_moe_y = nullptr;
    int32_t *r_moe_sel = nullptr, *r_zero_sel = nullptr;
    int32_t *r_grp_cnt = nullptr, *r_grp_mem = nullptr;   // the rows' selections grouped by expert
    uint8_t *r_exp_pack = nullptr;                         // each selection's SiLU·up as per-32 packs
    float *r_logits = nullptr, *r_part = nullptr, *r_pv = nullptr;
    int32_t *r_pi = nullptr, *r_tab_pf = nullptr, *r_tab_b = nullptr;
    uint8_t *r_xp = nullptr, *r_ap = nullptr, *r_actp = nullptr;
    int32_t *pinned_tab = nullptr;             // pinned staging of a row table
    int batch_rows = 0;                        // rows of the last batched decode step
    std::vector<hipGraphExec_t> batch_graphs;  // [n]: the batched step of n rows (the row table is read at replay)

    // in-step timing: an event before and after each launch of probe_kind
    int probe_kind = -1, probe_n = 0;
    std::vector<hipEvent_t> probe_ev;
    void probe(int kind) {
        if (kind == probe_kind && probe_n < (int)probe_ev.size()) (void)hipEventRecord(probe_ev[probe_n++], stream());
    }
    int time_in_step(int s, int kind, int steps, float *avg_us);

    bool want(int kind, int l) const {
        return only < 0 || (only == kind && l == (kind == K_EMBED || kind == K_HEAD ? 0 : only_layer));
    }

    void *alloc(size_t n) {
        void *p = dev_alloc(n);
        if (p) owned.push_back(p);
        return p;
    }
    ~Engine() {
        for (auto &s : seqs)
            if (s.graph) (void)hipGraphExecDestroy(s.graph);
        for (auto &g : batch_graphs)
            if (g) (void)hipGraphExecDestroy(g);
        (void)hipStreamSynchronize(stream());
        for (void *p : owned) dev_free(p);
        if (pinned) (void)hipHostFree(pinned);
        if (pinned_tab) (void)hipHostFree(pinned_tab);
        if (pinned_pg) (void)hipHostFree(pinned_pg);
        if (host_tok) (void)hipHostFree(host_tok);
        for (auto &e : pipe_ev)
            if (e) (void)hipEventDestroy(e);
    }
    int load(const std::string &path, int ctx_, int max_seqs_, int kv_pages_, bool kv_f32_);
    // the page pool
    int ensure_pages(int s, int64_t upto);
    bool pages_fit(int s, int64_t upto) const;
    void release_pages(int s);
    int upload_weight(const std::string &name, DevW &w, int expect_rows, int64_t expect_cols);
    int fuse_rows(const std::vector<std::string> &names, DevW &w, bool interleave, int64_t rows_each, int64_t experts);
    int capture(int s);
    int enqueue_step(int s);
    int run_step(int s);
    int norm_pack(const float *w, int per32, bool f32_out, const float *x = nullptr);
    // rows a workgroup the head's GEMV aims at: 64 where 128 would leave a
    // workgroup a CU or fewer
    // the head's rows a workgroup, by its format: Q8_0 32, others 64 (128
    // for large vocabularies measured slower: C5's 201,088-row Q8_0 head
    // 115.6 -> 108.6 us at 64 -> 106.0 at 32; C3's 128,256-row Q6_K head
    // 75.2 -> 74.1 at 64, 75.5 at 32)
    int head_target(int type) const { return type == CJ_Q8_0 ? 32 : 64; }
    // the many-row path
    int rows_alloc(int cap);
    int rows_linear(const DevW &W, const uint8_t *xp, int64_t xp_stride, float *y, int64_t y_stride, bool accum, int n);
    int rows_norm_pack(const float *w, int per32, int n);
    int launch_norm_pack_rows(cj_pack_args &a, int n);
    int rows_forward(const int32_t *tab, int n, bool prefill);
    int rows_pack(const float *x, int64_t n, int per32, int rows);
    int rows_moe(const Layer &L, int n);
    int enqueue_batch(int n);
    int prefill_rows(int s, const int32_t *toks, int n);
    int decode_batch(const int32_t *slots, int n, int steps, int32_t *out);
    int prefill(int s, const int32_t *toks, int n);
    int decode(int s, int steps, int32_t *out);
    int reset(int s);
    int check_route();
    // the scheduler (sched/Scheduler.cajeta)
    int submit(const int32_t *prompt, int n, int max_new, const int32_t *stops, int n_stops);
    int admit();
    void retire(Request &r, int finish);
    void consume(Request &r, int32_t tok);
    int step_once();
    int sole_running() const;
    int youngest_running() const;
    bool pipe_for(int i, const Request &r, int n);
    int step_pipelined(int i, Request &r);
    int queue_pipe_step(int s, int slot_ev);
    int await_pipe(int32_t *tok);
    int finish_pipe();
    int drain_pipe();
    int preempt(int i);
    int cancel(int i);
    int64_t kind_bytes(int kind, int count) const;
    int64_t step_bytes(int count) const;
    int time_kind(int s, int kind, int reps, float *avg_us, std::string &kernel);
};

namespace {

std::string lname(int l, const char *t) { return "blk." + std::to_string(l) + "." + t; }

}  // namespace

int Engine::upload_weight(const std::string &name, DevW &w, int expect_rows, int64_t expect_cols) {
    const GgufTensor *t = file.tensor(name);
    if (!t) return fail(CJ_ERR_IO, "model: tensor %s is missing", name.c_str());
    if (t->cols() != expect_cols || (expect_rows > 0 && t->rows() != expect_rows))
        return fail(CJ_ERR_IO, "model: tensor %s is %lldx%lld, expected %lldx%lld", name.c_str(), (long long)t->rows(),
                    (long long)t->cols(), (long long)expect_rows, (long long)expect_cols);
    w.type = t->type; w.rows = t->rows(); w.cols = t->cols();
    if (t->type == CJ_F32) {
        w.row_bytes = w.cols * 4;
        w.p = alloc((size_t)t->bytes);
        if (!w.p) return fail(CJ_ERR_HIP, "model: out of device memory at %s", name.c_str());
        CJ_HIP(hipMemcpy(w.p, t->data, (size_t)t->bytes, hipMemcpyHostToDevice));
        return CJ_OK;
    }
    w.row_bytes = prepared_row_bytes(t->type, t->cols());
    if (w.row_bytes <= 0 || !gemv_supported(t->type, t->cols()))
        return fail(CJ_ERR_IO, "model: %s has type %d x %lld columns, not served", name.c_str(), t->type, (long long)t->cols());
    w.p = alloc((size_t)(w.row_bytes * w.rows));
    void *stage = dev_alloc((size_t)t->bytes);
    if (!w.p || !stage) { dev_free(stage); return fail(CJ_ERR_HIP, "model: out of device memory at %s", name.c_str()); }
    hipError_t e = hipMemcpy(stage, t->data, (size_t)t->bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) { dev_free(stage); return fail(CJ_ERR_HIP, "upload %s: %s", name.c_str(), hipGetErrorString(e)); }
    int rc = cj_prepare_weight((int64_t)(uintptr_t)w.p, (int64_t)(uintptr_t)stage, t->type, w.rows, w.cols);
    (void)hipStreamSynchronize(stream());
    dev_free(stage);
    return rc;
}

// Concatenate (or row-interleave) prepared weights into one fused weight.
// With `experts` > 0 each tensor is [experts][rows_each] and the fusion is
// per expert.
int Engine::fuse_rows(const std::vector<std::string> &names, DevW &w, bool interleave, int64_t rows_each, int64_t experts) {
    std::vector<DevW> parts(names.size());
    for (size_t i = 0; i < names.size(); i++) {
        int rc = upload_weight(names[i], parts[i], -1, hidden);
        if (rc) return rc;
        if (i && (parts[i].type != parts[0].type))
            return fail(CJ_ERR_IO, "model: %s and %s differ in type; the fused route needs one", names[0].c_str(), names[i].c_str());
    }
    const int64_t rb = parts[0].row_bytes;
    const int64_t E = experts > 0 ? experts : 1;
    if (interleave)
        for (size_t i = 0; i < parts.size(); i++)
            if (rows_each <= 0 || parts[i].rows != E * rows_each)   // the row copies below read E·rows_each rows of each part
                return fail(CJ_ERR_IO, "model: %s has %lld rows, expected %lld (%lld experts x %lld)", names[i].c_str(),
                            (long long)parts[i].rows, (long long)(E * rows_each), (long long)E, (long long)rows_each);
    int64_t total = 0;
    for (auto &p : parts) total += p.rows;
    w.type = parts[0].type; w.cols = parts[0].cols; w.row_bytes = rb; w.rows = total;
    w.p = alloc((size_t)(total * rb));
    if (!w.p) return fail(CJ_ERR_HIP, "model: out of device memory fusing %s", names[0].c_str());
    if (!interleave) {
        int64_t off = 0;
        for (auto &p : parts) {
            CJ_HIP(hipMemcpyAsync((char *)w.p + off * rb, p.p, (size_t)(p.rows * rb), hipMemcpyDeviceToDevice, stream()));
            off += p.rows;
        }
    } else {
        // row 2i = part0 row i, row 2i+1 = part1 row i (per expert)
        const int64_t per = rows_each;
        for (int64_t e = 0; e < E; e++)
            for (size_t k = 0; k < parts.size(); k++) {
                char *dst = (char *)w.p + (e * per * parts.size() + k) * rb;
                const char *src = (const char *)parts[k].p + e * per * rb;
                CJ_HIP(hipMemcpy2DAsync(dst, (size_t)(parts.size() * rb), src, (size_t)rb, (size_t)rb, (size_t)per,
                                        hipMemcpyDeviceToDevice, stream()));
            }
    }
    CJ_HIP(hipStreamSynchronize(stream()));
    for (auto &p : parts) {
        auto it = std::find(owned.begin(), owned.end(), p.p);
        if (it != owned.end()) owned.erase(it);
        dev_free(p.p);
    }
    return CJ_OK;
}

int Engine::load(const std::string &path, int ctx_, int max_seqs_, int kv_pages_, bool kv_f32_) {
    std::string err;
    if (!file.open(path, err)) return fail(CJ_ERR_IO, "model: %s", err.c_str());
    const std::string arch = file.get_str("general.architecture", "");
    if (arch != "llama") return fail(CJ_ERR_IO, "model: architecture '%s' is not served (llama)", arch.c_str());
    const std::string kp = arch + ".";
    hidden = (int)file.get_int(kp + "embedding_length", -1);
    ffn = (int)file.get_int(kp + "feed_forward_length", -1);
    n_layers = (int)file.get_int(kp + "block_count", -1);
    n_heads = (int)file.get_int(kp + "attention.head_count", -1);
    if (hidden <= 0 || ffn <= 0 || n_layers <= 0 || n_heads <= 0)
        return fail(CJ_ERR_IO, "gguf config: missing a required %s* hyperparameter", kp.c_str());
    n_kv = (int)file.get_int(kp + "attention.head_count_kv", n_heads);
    head_dim = (int)file.get_int(kp + "attention.key_length", file.get_int(kp + "rope.dimension_count", hidden / n_heads));
    eps = (float)file.get_float(kp + "attention.layer_norm_rms_epsilon", 1e-5);
    theta = (float)file.get_float(kp + "rope.freq_base", 10000.0);
    n_experts = (int)file.get_int(kp + "expert_count", 0);
    n_used = (int)file.get_int(kp + "expert_used_count", 0);
    expert_ffn = (int)file.get_int(kp + "expert_feed_forward_length", ffn);
    norm_topk = (int)file.get_int(kp + "expert_weights_norm", 1);
    w_scale = (float)file.get_float(kp + "expert_weights_scale", 0.0);
    if (n_experts > 0) {
        // only softmax gating has a witness in the reference (MoeFfn ctor,
        // model/MoeFfn.cajeta:417-432): anything else is refused by name
        const int64_t gating = file.get_int(kp + "expert_gating_func", 1);
        if (gating != 1)
            return fail(CJ_ERR_IO, "moe: expert_gating_func %lld%s is not served; only softmax (1) is", (long long)gating,
                        gating == 2 ? " (sigmoid)" : "");
    }
    if (n_experts < 0 || n_experts > 256 || (n_experts > 0 && (n_used <= 0 || n_used > 16 || n_used > n_experts)))
        return fail(CJ_ERR_IO, "model: %d experts, %d used (served: up to 256, 1..16 used)", n_experts, n_used);
    const int swa = (int)file.get_int(kp + "attention.sliding_window", 0);
    // every swa_pattern-th layer attends every position, (l + 1) % P == 0
    // (ModelConfig.gemma3Gguf, model/ModelConfig.cajeta:570-576); gpt-oss
    // alternates, so 2 where the key is absent
    const int swa_pattern = (int)file.get_int(kp + "attention.sliding_window_pattern", 2);
    if (swa > 0 && swa_pattern <= 0) return fail(CJ_ERR_IO, "model: sliding_window_pattern %d", swa_pattern);
    const GgufTensor *te = file.tensor("token_embd.weight");
    if (!te) return fail(CJ_ERR_IO, "model: token_embd.weight is missing");
    vocab = (int)file.get_int(kp + "vocab_size", te->rows());
    if (file.has("tokenizer.ggml.eos_token_id")) eog.insert((int)file.get_int("tokenizer.ggml.eos_token_id", -1));
    scale = 1.0f / sqrtf((float)head_dim);
    ctx = ctx_ > 0 ? ctx_ : (int)file.get_int(kp + "context_length", 4096);
    max_seqs = max_seqs_ > 0 ? max_seqs_ : 1;
    if (head_dim != 64 && head_dim != 128) return fail(CJ_ERR_IO, "model: head_dim %d is not served (64, 128)", head_dim);
    const int grp = n_heads / n_kv;
    if (n_heads % n_kv || (grp != 1 && grp != 2 && grp != 4 && grp != 8))
        return fail(CJ_ERR_IO, "model: GQA %d/%d is not served", n_heads, n_kv);

    // embedding: GGUF layout, decoded per row on device
    embd_type = te->type;
    embd_row_bytes = ggml_row_bytes(te->type, te->cols());
    embd_row_file_bytes = embd_row_bytes;
    if (embd_row_bytes <= 0 || te->cols() != hidden || te->rows() != vocab)
        return fail(CJ_ERR_IO, "model: token_embd.weight shape/type not served");
    embd = alloc((size_t)te->bytes);
    if (!embd) return fail(CJ_ERR_HIP, "model: out of device memory (embedding)");
    CJ_HIP(hipMemcpy(embd, te->data, (size_t)te->bytes, hipMemcpyHostToDevice));

    auto upload_f32 = [&](const std::string &name, int64_t n, float **dst) -> int {
        const GgufTensor *t = file.tensor(name);
        if (!t || t->type != CJ_F32 || t->cols() * t->rows() != n) return fail(CJ_ERR_IO, "model: %s missing or not f32[%lld]", name.c_str(), (long long)n);
        *dst = (float *)alloc((size_t)n * 4);
        if (!*dst) return fail(CJ_ERR_HIP, "model: out of device memory at %s", name.c_str());
        CJ_HIP(hipMemcpy(*dst, t->data, (size_t)n * 4, hipMemcpyHostToDevice));
        return CJ_OK;
    };

    layers.resize(n_layers);
    const int64_t qd = (int64_t)n_heads * head_dim, kvd = (int64_t)n_kv * head_dim;
    pages_per_seq = (ctx + 63) / 64;
    if (!(head_dim == 128 && (grp == 4 || grp == 8)) && pages_per_seq > 2048)
        return fail(CJ_ERR_ARG, "model: context %d exceeds the two-pass attention's 2048 pages", ctx);
    // the pool: numBlocks 0 holds every slot at its full context (CausalLM's
    // constructor, model/CausalLM.cajeta:83-88); fewer pages share the pool
    // and the scheduler preempts when it runs dry
    if (kv_pages_ < 0) return fail(CJ_ERR_ARG, "model: %d K/V pages", kv_pages_);
    kv_pages = kv_pages_ > 0 ? kv_pages_ : pages_per_seq * max_seqs;
    // f32 K/V (PagedKvCache's mode): the two-pass attention reads it; the
    // split-K and prefill-attend forms (head size 128 with 4 or 8 query
    // heads a kv head) keep fp16, as the reference's resident decode does
    kv_f32 = kv_f32_;
    if (kv_f32 && ((head_dim == 128 && (grp == 4 || grp == 8)) || ctx > 6144))
        return fail(CJ_ERR_ARG, "model: f32 K/V is served by the two-pass attention (head size 64, or GQA other than 4 "
                                "and 8 at 128) up to 6144 positions; this model takes the fp16 split-K form");
    const int64_t plane = (int64_t)kv_pages * n_kv * 64 * head_dim * (kv_f32 ? 4 : 2);
    int rc;
    for (int l = 0; l < n_layers; l++) {
        Layer &L = layers[l];
        if ((rc = upload_f32(lname(l, "attn_norm.weight"), hidden, &L.attn_norm))) return rc;
        if ((rc = upload_f32(lname(l, "ffn_norm.weight"), hidden, &L.ffn_norm))) return rc;
        if ((rc = fuse_rows({lname(l, "attn_q.weight"), lname(l, "attn_k.weight"), lname(l, "attn_v.weight")}, L.qkv, false, 0, 0))) return rc;
        if (L.qkv.rows != qd + 2 * kvd) return fail(CJ_ERR_IO, "model: layer %d q|k|v rows %lld", l, (long long)L.qkv.rows);
        if ((rc = upload_weight(lname(l, "attn_output.weight"), L.o, hidden, qd))) return rc;
        if (n_experts > 0) {
            if ((rc = upload_weight(lname(l, "ffn_gate_inp.weight"), L.router, n_experts, hidden))) return rc;
            if ((rc = fuse_rows({lname(l, "ffn_gate_exps.weight"), lname(l, "ffn_up_exps.weight")}, L.gu_exps, true, expert_ffn, n_experts))) return rc;
            if ((rc = upload_weight(lname(l, "ffn_down_exps.weight"), L.down_exps, (int)((int64_t)n_experts * hidden), expert_ffn))) return rc;
            // every GEMV format serves an expert bank through the indirected
            // launch (the K-quants need whole 256-element rows)
            for (const DevW *e : {&L.gu_exps, &L.down_exps})
                if (!gemv_supported(e->type, e->cols) || e->type == CJ_F32)
                    return fail(CJ_ERR_IO, "model: expert type %d x %lld columns not served", e->type, (long long)e->cols);
        } else {
            if ((rc = fuse_rows({lname(l, "ffn_gate.weight"), lname(l, "ffn_up.weight")}, L.gu, true, ffn, 0))) return rc;
            if ((rc = upload_weight(lname(l, "ffn_down.weight"), L.down, hidden, ffn))) return rc;
        }
        L.window = (swa > 0 && ((l + 1) % swa_pattern) != 0) ? swa : 0;
        L.kc = (uint16_t *)alloc((size_t)plane);
        L.vc = (uint16_t *)alloc((size_t)plane);
        if (!L.kc || !L.vc) return fail(CJ_ERR_HIP, "model: out of device memory for the K/V planes");
    }
    if ((rc = upload_f32("output_norm.weight", hidden, &out_norm))) return rc;
    const std::string head_name = file.tensor("output.weight") ? "output.weight" : "token_embd.weight";
    if ((rc = upload_weight(head_name, head, vocab, hidden))) return rc;
    wtype = layers[0].qkv.type;
    head_type = head.type;
    if (is_f32_act(wtype)) return fail(CJ_ERR_IO, "model: attention weights of type %d are not served", wtype);

    // K/V page table: entry s·pages_per_seq + j is the pool page holding
    // slot s's positions [64j, 64j + 64), drawn as the slot grows (entries
    // not drawn yet read page 0 and are never dereferenced)
    const size_t tab_n = (size_t)pages_per_seq * max_seqs;
    pgtab = (int32_t *)alloc(tab_n * 4);
    rope = (float *)alloc((size_t)ctx * head_dim * 4);
    if (!pgtab || !rope) return fail(CJ_ERR_HIP, "model: out of device memory");
    if (hipHostMalloc((void **)&pinned_pg, tab_n * 4, 0) != hipSuccess) return fail(CJ_ERR_HIP, "model: pinned page table");
    memset(pinned_pg, 0, tab_n * 4);
    CJ_HIP(hipMemcpy(pgtab, pinned_pg, tab_n * 4, hipMemcpyHostToDevice));
    free_pages.resize((size_t)kv_pages);
    for (int i = 0; i < kv_pages; i++) free_pages[(size_t)i] = kv_pages - 1 - i;   // drawn from the back: 0, 1, 2, ...
    slot_pages.assign((size_t)max_seqs, {});
    // Llama-3.1-style precomputed RoPE factors (ModelConfig, model/ModelConfig.cajeta:307-316)
    const GgufTensor *rf = file.tensor("rope_freqs.weight");
    if (rf && rf->type != CJ_F32) return fail(CJ_ERR_IO, "model: rope_freqs.weight is type %d, not f32", rf->type);
    if (rf && rf->bytes < rf->cols() * rf->rows() * 4) return fail(CJ_ERR_IO, "model: rope_freqs.weight is truncated");
    std::vector<float> factors;
    if (rf) {
        factors.resize((size_t)(rf->cols() * rf->rows()));
        memcpy(factors.data(), rf->data, factors.size() * 4);
    }
    if ((rc = cj_rope_table_freqs((int64_t)(uintptr_t)rope, head_dim, theta, ctx, rf ? factors.data() : nullptr,
                                  (int32_t)factors.size())))
        return rc;

    const int64_t fmax = std::max<int64_t>(ffn, (int64_t)expert_ffn * std::max(1, n_used));
    const int64_t fpad = (std::max<int64_t>(ffn, expert_ffn) + 255) / 256 * 256;
    hs = (float *)alloc((size_t)hidden * 4);
    hs2 = (float *)alloc((size_t)hidden * 4);
    hs_last = hs;
    q = (float *)alloc((size_t)qd * 4);
    attn = (float *)alloc((size_t)qd * 4);
    act = (float *)alloc((size_t)fmax * 4 + 1024);
    act_pack = (uint8_t *)alloc((size_t)fpad / 256 * 320);
    attn_pack = (uint8_t *)alloc((size_t)(qd + 255) / 256 * 320);
    xpack = (uint8_t *)alloc((size_t)(hidden + 255) / 256 * 320);
    xn = (float *)alloc((size_t)hidden * 4);
    logits = (float *)alloc((size_t)vocab * 4);
    // split-K partials [n_heads][64][hd + 2], or two-pass scores [n_heads][ctx]
    part = (float *)alloc((size_t)n_heads * std::max<int64_t>(64 * (head_dim + 2), ctx) * 4);
    glu_counters = (int32_t *)alloc((size_t)fpad / 256 * 4 + 64);
    argmax_counter = (int32_t *)alloc(64);
    attn_counters = (int32_t *)alloc((size_t)n_kv * 4 + 64);
    const int64_t max_wg = (vocab + 3) / 4 + 64;
    part_v = (float *)alloc((size_t)max_wg * 4);
    part_i = (int32_t *)alloc((size_t)max_wg * 4);
    moe_logits = (float *)alloc((size_t)std::max(1, n_experts) * 4 + 64);
    moe_w = (float *)alloc(64 * 4);
    moe_sel = (int32_t *)alloc(64 * 4);
    route_status = (int32_t *)alloc(64);
    moe_y = (float *)alloc((size_t)hidden * std::max(1, n_used) * 4);
    if (!hs || !hs2 || !q || !attn || !act || !act_pack || !attn_pack || !xpack || !xn || !logits || !part || !glu_counters || !argmax_counter ||
        !attn_counters || !part_v || !part_i || !moe_logits || !moe_w || !moe_sel || !moe_y || !route_status)
        return fail(CJ_ERR_HIP, "model: out of device memory (scratch)");
    CJ_HIP(hipMemset(glu_counters, 0, (size_t)fpad / 256 * 4 + 64));
    CJ_HIP(hipMemset(argmax_counter, 0, 64));
    CJ_HIP(hipMemset(attn_counters, 0, (size_t)n_kv * 4 + 64));
    CJ_HIP(hipMemset(route_status, 0, 64));

    if (hipHostMalloc((void **)&pinned, (size_t)(ctx + 2) * 4 + sizeof(cj_step_state) + 64, 0) != hipSuccess)
        return fail(CJ_ERR_HIP, "model: pinned staging buffer");
    if (hipHostMalloc((void **)&host_tok, (size_t)(ctx + 2) * max_seqs * 4, 0) != hipSuccess)
        return fail(CJ_ERR_HIP, "model: pinned token mirror");
    memset(host_tok, 0xff, (size_t)(ctx + 2) * max_seqs * 4);
    for (auto &e : pipe_ev) CJ_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    // sequence slots: histories and step states side by side, so the
    // many-row kernels reach every slot's from one base
    const size_t hist = (size_t)(ctx + 2);
    tokens_all = (int32_t *)alloc(hist * max_seqs * 4);
    preds_all = (int32_t *)alloc(hist * max_seqs * 4);
    states = (cj_step_state *)alloc(sizeof(cj_step_state) * (size_t)max_seqs);
    if (!tokens_all || !preds_all || !states) return fail(CJ_ERR_HIP, "model: out of device memory (sequence slots)");
    CJ_HIP(hipMemset(tokens_all, 0, hist * max_seqs * 4));
    CJ_HIP(hipMemset(preds_all, 0, hist * max_seqs * 4));
    CJ_HIP(hipMemset(states, 0, sizeof(cj_step_state) * (size_t)max_seqs));
    seqs.resize(max_seqs);
    slot_req.assign((size_t)max_seqs, -1);
    batch_graphs.assign((size_t)max_seqs + 1, nullptr);
    for (int s = 0; s < max_seqs; s++) {
        Seq &S = seqs[s];
        S.tokens = tokens_all + hist * s;
        S.preds = preds_all + hist * s;
        S.state = states + s;
        S.pg_base = s * pages_per_seq;
    }

    // the many-row path (batched decode: a row a sequence; prefill chunks: a
    // row a position) where the projections read int8 packs; MoE experts go
    // through the indirected GEMV over every row's selections
    rows_ok = !is_f32_act(head.type);
    for (auto &L : layers) {
        for (const DevW *w : {&L.qkv, &L.o})
            if (is_f32_act(w->type)) rows_ok = false;
        if (n_experts == 0)
            for (const DevW *w : {&L.gu, &L.down})
                if (is_f32_act(w->type)) rows_ok = false;
    }
    rows_split = head_dim == 128 && (grp == 4 || grp == 8);
    // prompts: the prefill attend where the reference's CPU prefill serves
    // the shape (dense, head size 128: AttnKernel.cpuAttnServes,
    // model/AttnKernel.cajeta:4439-4447); the other models prefill a decode
    // step a position, which rows of the two-pass decode attention repeat
    // row for row (a split-K row's split count follows the rows, so MoE
    // models at head size 128 keep the step a position)
    rows_pf_attend = n_experts == 0 && head_dim == 128 && !kv_f32;
    rows_prefill = rows_ok && (rows_pf_attend || !rows_split);
    if (rows_ok && (rc = rows_alloc(std::max(chunk, max_seqs)))) return rc;
    CJ_HIP(hipDeviceSynchronize());
    return CJ_OK;
}

// Row buffers for up to `cap` rows (prefill chunk or decode batch).
int Engine::rows_alloc(int cap) {
    const int64_t qd = (int64_t)n_heads * head_dim, kvd = (int64_t)n_kv * head_dim;
    const int64_t hb = ((int64_t)hidden + 255) / 256 * 320, qb = (qd + 255) / 256 * 320;
    const int64_t fb = ((int64_t)ffn + 255) / 256 * 320;
    const int64_t nch = ((int64_t)vocab + 1023) / 1024;
    const int64_t b = std::max(1, max_seqs);
    r_hs = (float *)alloc((size_t)(cap * (int64_t)hidden * 4));
    r_qkv = (float *)alloc((size_t)(cap * (qd + 2 * kvd) * 4));
    r_q = (float *)alloc((size_t)(cap * qd * 4));
    r_attn = (float *)alloc((size_t)(cap * qd * 4));
    r_gu = (float *)alloc((size_t)(cap * 2 * (int64_t)ffn * 4));
    r_xp = (uint8_t *)alloc((size_t)(cap * hb));
    r_ap = (uint8_t *)alloc((size_t)(cap * qb));
    r_actp = (uint8_t *)alloc((size_t)(cap * fb));
    r_logits = (float *)alloc((size_t)(b * vocab * 4));
    // split-K partials [b][n_heads][64][hd + 2], or the two-pass score rows [cap][n_heads][ctx]
    r_part = (float *)alloc((size_t)std::max<int64_t>(b * n_heads * 64 * (head_dim + 2),
                                                      rows_split ? 0 : (int64_t)cap * n_heads * ctx) * 4);
    if (n_experts > 0) {
        const int64_t sels = (int64_t)cap * n_used;
        r_xn = (float *)alloc((size_t)((int64_t)cap * hidden * 4));
        r_moe_logits = (float *)alloc((size_t)((int64_t)cap * n_experts * 4));
        r_moe_sel = (int32_t *)alloc((size_t)(sels * 4));
        r_moe_w = (float *)alloc((size_t)(sels * 4));
        r_act = (float *)alloc((size_t)(sels * expert_ffn * 4 + 1024));
        r_moe_y = (float *)alloc((size_t)(sels * hidden * 4));
        r_zero_sel = (int32_t *)alloc((size_t)(cap * 4));
        r_grp_cnt = (int32_t *)alloc((size_t)std::max(1, n_experts) * 4);
        r_grp_mem = (int32_t *)alloc((size_t)std::max(1, n_experts) * sels * 4);
        r_exp_pack = (uint8_t *)alloc((size_t)(sels * (((int64_t)expert_ffn + 255) / 256 * 320)));
        if (!r_xn || !r_moe_logits || !r_moe_sel || !r_moe_w || !r_act || !r_moe_y || !r_zero_sel || !r_grp_cnt ||
            !r_grp_mem || !r_exp_pack)
            return fail(CJ_ERR_HIP, "model: out of device memory (MoE row buffers for %d rows)", cap);
        CJ_HIP(hipMemset(r_zero_sel, 0, (size_t)(cap * 4)));
    }
    r_pv = (float *)alloc((size_t)(b * nch * 4));
    r_pi = (int32_t *)alloc((size_t)(b * nch * 4));
    r_tab_pf = (int32_t *)alloc((size_t)cap * 8);
    r_tab_b = (int32_t *)alloc((size_t)b * 8);
    if (!r_hs || !r_qkv || !r_q || !r_attn || !r_gu || !r_xp || !r_ap || !r_actp || !r_logits || !r_part || !r_pv ||
        !r_pi || !r_tab_pf || !r_tab_b)
        return fail(CJ_ERR_HIP, "model: out of device memory (row buffers for %d rows)", cap);
    if (hipHostMalloc((void **)&pinned_tab, (size_t)cap * 8, 0) != hipSuccess)
        return fail(CJ_ERR_HIP, "model: pinned row-table staging");
    rows_cap = cap;
    return CJ_OK;
}

// The prologue of an expert product: MXFP4 experts read their f32 input
// through the device Q8 form (per-32 codes in LDS, mxfp4MatVecCoopQ8Launch,
// io/QuantKernel.cajeta:43699); other f32-activation formats read it as
// f32; int8 formats read `pack_pro`.
static int expert_pro(int type, int pack_pro) {
    return type == CJ_MXFP4 ? CJ_PRO_MXQ8 : is_f32_act(type) ? CJ_PRO_F32 : pack_pro;
}

// One decode step of sequence s on the stream (captured once into a graph).
int Engine::enqueue_step(int s) {
    Seq &S = seqs[s];
    int rc;
    if (want(K_EMBED, 0)) {
        cj_embed_args a{};
        a.out = hs; a.table = (const uint8_t *)embd; a.tokens = S.tokens; a.state = S.state;
        a.type = embd_type; a.hidden = hidden; a.row_bytes = embd_row_bytes;
        if ((rc = launch("cj_embed", (uint32_t)((hidden + 255) / 256), 256, 0, a))) return rc;
    }
    const int grp = n_heads / n_kv;
    const bool per32 = wtype == CJ_Q8_0;
    // the reference's choice of form: split-K for hd 128 with 4 or 8 query
    // heads a kv head, else the two-pass score/combine
    const bool split = head_dim == 128 && (grp == 4 || grp == 8);
    char attn_kernel[64], combine_kernel[64], fused_kernel[64];
    const char *kvs = kv_f32 ? "f32_" : "";
    if (split) snprintf(attn_kernel, sizeof attn_kernel, "cj_attn_split_h128_g%d", grp);
    else snprintf(attn_kernel, sizeof attn_kernel, "cj_attn_scores_%sh%d", kvs, head_dim);
    snprintf(combine_kernel, sizeof combine_kernel, "cj_attn_combine_%sh%d", kvs, head_dim);
    snprintf(fused_kernel, sizeof fused_kernel, "cj_attn_fused_h%d", head_dim);
    // the residual: hs, or on MoE models the buffer the last combine wrote
    // (it alternates between hs and hs2, see K_COMBINE below)
    float *cur = hs;
    bool normed = false;   // the previous combine already formed this norm's pack
    for (int l = 0; l < n_layers; l++) {
        Layer &L = layers[l];
        // Q4_K projections fold the RMSNorm + pack into their prologue (the
        // weight stream is in flight while it runs); others read a pack
        const bool qkv_norm = L.qkv.type == CJ_Q4_K && hidden <= 4096;
        if (!qkv_norm && !normed && want(K_NORM, l) && (rc = norm_pack(L.attn_norm, L.qkv.type == CJ_Q8_0, false, cur)))
            return rc;
        normed = false;
        if (want(K_QKV, l)) {   // 1. q|k|v over the normed residual, RoPE + K/V append epilogue
            cj_gemv_args a{};
            a.w = (const uint8_t *)L.qkv.p; a.xp = xpack; a.q_out = q; a.kc = L.kc; a.vc = L.vc;
            a.pgtab = pgtab; a.rope_cs = rope; a.state = S.state; a.rows = L.qkv.rows; a.cols = hidden;
            a.row_bytes = L.qkv.row_bytes; a.type = L.qkv.type; a.pro = CJ_PRO_PACKED; a.epi = CJ_EPI_QKV_ROPE;
            if (qkv_norm) { a.pro = CJ_PRO_NORM_PACK; a.x = cur; a.nw = L.attn_norm; a.norm_form = 0; }
            a.per32 = per32; a.eps = eps; a.n_q = n_heads; a.n_kv = n_kv; a.head_dim = head_dim; a.pg_base = S.pg_base;
            a.batch = 1; a.kv_f32 = kv_f32;
            probe(K_QKV);
            if ((rc = run_gemv(a, plan_gemv(a.type, a.rows, a.cols, 8, a.pro, a.epi)))) return rc;
            probe(K_QKV);
        }
        if (want(K_ATTN, l) || want(K_MERGE, l)) {   // 2. attention
            probe(K_ATTN);
            cj_attn_args a{};
            a.part = part; a.out = attn; a.q = q; a.kc = L.kc; a.vc = L.vc; a.pgtab = pgtab; a.state = S.state;
            a.counters = attn_counters; a.n_q = n_heads; a.n_kv = n_kv; a.head_dim = head_dim; a.workers = workers;
            a.pg_base = S.pg_base; a.pg_n = pages_per_seq; a.window = L.window; a.scale = scale;
            if (split) {
                // partials, then the merge (a launch boundary orders them: a
                // merge by the last workgroup of each kv head would need
                // device-scope fences, which cost far more than the launch on
                // this part): a lane per (output dimension, sub-sum) writing
                // f32, which the o projection packs, or the 256-wide merge + pack
                a.out = nullptr;
                if (want(K_ATTN, l) && (rc = launch(attn_kernel, (uint32_t)(n_kv * 64), 256, 0, a))) return rc;
                cj_merge_args m{};
                m.out = attn; m.packed = attn_pack; m.part = part; m.state = S.state; m.n_q = n_heads;
                m.head_dim = head_dim; m.per32 = L.o.type == CJ_Q8_0; m.n_kv = n_kv; m.workers = workers;
                m.window = L.window;
                if (merge_w) {
                    m.packed = nullptr;
                    if ((rc = launch("cj_attn_merge_q", (uint32_t)(n_heads * (head_dim / 32)), 128, 0, m))) return rc;
                } else if ((rc = launch("cj_attn_merge", (uint32_t)(((int64_t)n_heads * head_dim + 255) / 256), 256, 0, m))) {
                    return rc;
                }
            } else if (want(K_ATTN, l)) {
                a.splits = ctx;
                const int64_t span = L.window > 0 ? std::min(L.window, ctx) : ctx;
                if (!kv_f32 && span <= (head_dim == 64 ? 256 : 128)) {
                    // every step's span fits one workgroup: the one-launch form
                    if ((rc = launch(fused_kernel, (uint32_t)n_heads, 256, 0, a))) return rc;
                } else {
                    // the grid covers the longest window; the kernel idles past count
                    if ((rc = launch2(attn_kernel, (uint32_t)((span + 255) / 256), (uint32_t)n_heads, 256, 0, a)))
                        return rc;
                    if ((rc = launch(combine_kernel, (uint32_t)(n_heads * (head_dim / (kv_f32 ? 32 : CJ_COMBINE_DH))), 256, 0, a))) return rc;
                }
            }
        }
        if (want(K_ATTN, l) || want(K_MERGE, l)) probe(K_ATTN);
        if (want(K_O, l)) {   // 3. o projection, residual into hs
            cj_gemv_args a{};
            a.w = (const uint8_t *)L.o.p; a.x = attn; a.xp = attn_pack; a.y = cur; a.rows = L.o.rows; a.cols = L.o.cols;
            a.row_bytes = L.o.row_bytes; a.type = L.o.type; a.pro = split && !merge_w ? CJ_PRO_PACKED : CJ_PRO_PACK;
            a.epi = CJ_EPI_ACCUM;
            a.per32 = L.o.type == CJ_Q8_0; a.batch = 1;
            probe(K_O);
            // 16 rows a workgroup here (q|k|v keeps 8): C5's o 7.17 -> 6.97 us,
            // q|k|v at 16 measured 7.0 -> 8.2
            if ((rc = run_gemv(a, plan_gemv(a.type, a.rows, a.cols, 16, a.pro, a.epi)))) return rc;
            probe(K_O);
        }
        const bool gu_norm = n_experts == 0 && L.gu.type == CJ_Q4_K && hidden <= 4096;
        // MoE with an f32 router and MXFP4 experts (both read the f32 norm,
        // neither the pack): the router's prologue forms the norm and writes
        // it for the experts
        const bool router_norm = n_experts > 0 && L.router.type == CJ_F32 && L.gu_exps.type == CJ_MXFP4 &&
                                 L.down_exps.type == CJ_MXFP4;
        if (!gu_norm && !router_norm && want(K_NORM, l)) {   // the FFN norm: pack (int8 consumers) and/or f32 (router, f32-activation experts)
            const int ct = n_experts ? L.gu_exps.type : L.gu.type;
            if ((rc = norm_pack(L.ffn_norm, ct == CJ_Q8_0, n_experts > 0, cur))) return rc;
        }
        if (n_experts == 0) {
            if (want(K_GATE_UP, l)) {   // 4. gate|up over the pack, SiLU·up epilogue
                cj_gemv_args a{};
                a.w = (const uint8_t *)L.gu.p; a.xp = xpack; a.act = act;
                a.rows = L.gu.rows; a.cols = hidden; a.row_bytes = L.gu.row_bytes;
                a.type = L.gu.type; a.pro = CJ_PRO_PACKED; a.epi = CJ_EPI_GLU; a.per32 = L.gu.type == CJ_Q8_0;
                a.eps = eps; a.act_n = ffn; a.act_per32 = L.down.type == CJ_Q8_0; a.glu_form = (ffn % 256) ? 1 : 0;
                a.batch = 1;
                if (gu_norm) { a.pro = CJ_PRO_NORM_PACK; a.x = cur; a.nw = L.ffn_norm; a.norm_form = 0; }
                probe(K_GATE_UP);
                if ((rc = run_gemv(a, plan_gemv(a.type, a.rows, a.cols, 16, a.pro, a.epi)))) return rc;
                probe(K_GATE_UP);
            }
            if (want(K_DOWN, l)) {   // 5. down, residual into hs
                cj_gemv_args a{};
                a.w = (const uint8_t *)L.down.p; a.x = act; a.y = cur; a.rows = L.down.rows; a.cols = L.down.cols;
                a.row_bytes = L.down.row_bytes; a.type = L.down.type; a.pro = CJ_PRO_PACK; a.epi = CJ_EPI_ACCUM;
                a.per32 = L.down.type == CJ_Q8_0; a.batch = 1;
                probe(K_DOWN);
                // 16 rows a workgroup, as the o projection (C1 141.3-142.9 -> 140.0-140.3 us)
                if ((rc = run_gemv(a, plan_gemv(a.type, a.rows, a.cols, 16, a.pro, a.epi)))) return rc;
                probe(K_DOWN);
            }
        } else {
            if (want(K_ROUTER, l)) {   // router logits from the normed hidden (f32 weights)
                cj_gemv_args a{};
                a.w = (const uint8_t *)L.router.p; a.x = xn; a.y = moe_logits; a.rows = n_experts;
                a.cols = hidden; a.row_bytes = L.router.row_bytes; a.type = CJ_F32; a.pro = CJ_PRO_F32;
                a.epi = CJ_EPI_STORE; a.eps = eps; a.batch = 1;
                if (router_norm) { a.pro = CJ_PRO_NORM_F32; a.x = cur; a.nw = L.ffn_norm; a.norm_form = 0; a.xout = xn; }
                if ((rc = run_gemv(a, plan_gemv(CJ_F32, a.rows, a.cols, 0, a.pro, a.epi)))) return rc;
            }
            const bool fused = route_fused(L);
            if (!fused && want(K_ROUTE, l)) {
                cj_route_args a{moe_logits, moe_sel, moe_w, n_experts, n_used, norm_topk, 1, w_scale, 0, route_status};
                if ((rc = launch("cj_moe_route", 1, 64, 0, a))) return rc;
            }
            if (want(K_EXP_GATE_UP, l)) {   // the selected experts' gate|up, SiLU·up into act[k]
                cj_gemv_args a{};
                a.w = (const uint8_t *)L.gu_exps.p; a.x = xn; a.xp = xpack; a.act = act; a.rows = 2 * (int64_t)expert_ffn;
                a.cols = hidden; a.row_bytes = L.gu_exps.row_bytes; a.type = L.gu_exps.type;
                a.pro = expert_pro(a.type, CJ_PRO_PACKED); a.epi = CJ_EPI_GLU; a.eps = eps;
                a.per32 = a.type == CJ_Q8_0; a.act_n = expert_ffn; a.glu_form = 0; a.batch = 1;
                a.sel = moe_sel; a.n_sel = n_used; a.expert_bytes = 2 * (int64_t)expert_ffn * L.gu_exps.row_bytes;
                a.y_stride = expert_ffn;
                if (fused) route_into(a, moe_logits, moe_sel, moe_w);
                if ((rc = run_gemv(a, plan_gemv(a.type, a.rows, a.cols, 32, a.pro, a.epi)))) return rc;
            }
            if (want(K_EXP_DOWN, l)) {   // the selected experts' down into moe_y[k]
                cj_gemv_args a{};
                a.w = (const uint8_t *)L.down_exps.p; a.x = act; a.y = moe_y; a.rows = hidden; a.cols = expert_ffn;
                a.row_bytes = L.down_exps.row_bytes; a.type = L.down_exps.type;
                a.pro = expert_pro(a.type, CJ_PRO_PACK); a.epi = CJ_EPI_STORE; a.per32 = a.type == CJ_Q8_0;
                a.batch = 1; a.sel = moe_sel; a.n_sel = n_used; a.expert_bytes = (int64_t)hidden * L.down_exps.row_bytes;
                a.x_stride = expert_ffn; a.y_stride = hidden;
                if ((rc = run_gemv(a, plan_gemv(a.type, a.rows, a.cols, 32, a.pro, a.epi)))) return rc;
            }
            if (want(K_COMBINE, l)) {   // hs += Σ_k w_k · y_k in k order
                // with the next RMSNorm + pack where that is a launch of its
                // own (the next layer's attention norm, or the final norm):
                // the combined residual goes to the other buffer
                const bool last = l + 1 == n_layers;
                const bool next_fused = !last && layers[l + 1].qkv.type == CJ_Q4_K && hidden <= 4096;
                if (combine_norm && only < 0 && !next_fused && hidden % 4 == 0 && hidden <= 4096 && n_used <= 8) {
                    float *nxt = cur == hs ? hs2 : hs;
                    cj_combine_norm_args a{};
                    a.hs_out = nxt; a.hs_in = cur; a.y = moe_y; a.w = moe_w; a.n = hidden; a.n_used = n_used;
                    a.p.out = xpack; a.p.w = last ? out_norm : layers[l + 1].attn_norm;
                    a.p.xout = last && is_f32_act(head.type) ? xn : nullptr; a.p.n = hidden;
                    a.p.npad = ((int64_t)hidden + 255) / 256 * 256; a.p.rows = 1; a.p.eps = eps; a.p.form = 0;
                    a.p.per32 = last ? head.type == CJ_Q8_0 : layers[l + 1].qkv.type == CJ_Q8_0; a.p.do_norm = 1;
                    if ((rc = launch("cj_moe_combine_norm", (uint32_t)(a.p.npad / 256), 256, (uint32_t)(hidden * 4), a)))
                        return rc;
                    cur = nxt;
                    normed = true;
                } else {
                    cj_combine_args a{cur, moe_y, moe_w, hidden, n_used};
                    if ((rc = launch("cj_moe_combine", (uint32_t)((hidden + 255) / 256), 256, 0, a))) return rc;
                }
            }
        }
    }
    hs_last = cur;
    if (only < 0 && !normed && (rc = norm_pack(out_norm, head.type == CJ_Q8_0, is_f32_act(head.type), cur))) return rc;
    if (want(K_HEAD, 0)) {   // head over the final norm's pack + greedy argmax; advances the step
        cj_gemv_args a{};
        a.w = (const uint8_t *)head.p; a.x = xn; a.xp = xpack; a.y = logits;
        a.part_v = part_v; a.part_i = part_i; a.tokens = S.tokens; a.preds = S.preds; a.state = S.state;
        if (only == K_HEAD) { a.state = nullptr; a.pos = S.pos; }   // timed alone: leave the step where it is
        a.rows = vocab; a.cols = hidden; a.row_bytes = head.row_bytes; a.type = head.type;
        a.pro = is_f32_act(head.type) ? CJ_PRO_F32 : CJ_PRO_PACKED; a.epi = CJ_EPI_ARGMAX;
        a.per32 = head.type == CJ_Q8_0; a.eps = eps; a.batch = 1;
        GemvPlan p = plan_gemv(a.type, a.rows, a.cols, head_target(a.type), a.pro, a.epi);
        if ((int64_t)p.grid > (vocab + 3) / 4 + 64) return fail(CJ_ERR_STATE, "head grid exceeds the partial buffers");
        if ((rc = run_gemv(a, p))) return rc;
        if (only < 0) {
            cj_pick_args k{};
            k.pv = part_v; k.pi = part_i; k.n = (int32_t)p.grid; k.tokens = S.tokens; k.preds = S.preds;
            k.state = S.state; k.host_tok = host_tok + (size_t)s * (ctx + 2);
            if ((rc = launch("cj_argmax_pick", 1, 256, 0, k))) return rc;
        }
    }
    return CJ_OK;
}

int Engine::capture(int s) {
    Seq &S = seqs[s];
    if (S.graph) return CJ_OK;
    CJ_HIP(hipStreamSynchronize(stream()));
    CJ_HIP(hipStreamBeginCapture(stream(), hipStreamCaptureModeThreadLocal));
    int rc = enqueue_step(s);
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(stream(), &g);
    if (rc) { if (g) (void)hipGraphDestroy(g); return rc; }
    if (e != hipSuccess) return fail(CJ_ERR_HIP, "capture: %s", hipGetErrorString(e));
    e = hipGraphInstantiate(&S.graph, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) { S.graph = nullptr; return fail(CJ_ERR_HIP, "graph instantiate: %s", hipGetErrorString(e)); }
    return CJ_OK;
}

// RMSNorm of the residual hs with weight w, once for all the workgroups of
// the next projection: its pack into xpack and, for f32-activation
// consumers, the normed values into xn (one workgroup; the norm is a
// reduction over the whole row).
int Engine::norm_pack(const float *w, int per32, bool f32_out, const float *x) {
    cj_pack_args a{};
    a.out = xpack; a.x = x ? x : hs; a.w = w; a.xout = f32_out ? xn : nullptr; a.n = hidden;
    a.npad = ((int64_t)hidden + 255) / 256 * 256; a.rows = 1; a.eps = eps; a.form = 0; a.per32 = per32; a.do_norm = 1;
    return launch("cj_norm_pack", (uint32_t)(a.npad / 256), 256, 0, a);
}

// ------------------------------------------------------------ many rows

// y rows = W · x rows for n packed activation rows: the int8 matrix-core
// product where the format has one, else the one-row GEMV a row (both
// compute each row exactly as the decode step does).
int Engine::rows_linear(const DevW &W, const uint8_t *xp, int64_t xp_stride, float *y, int64_t y_stride, bool accum, int n) {
    cj_gemv_args a{};
    a.w = (const uint8_t *)W.p; a.rows = W.rows; a.cols = W.cols; a.row_bytes = W.row_bytes; a.type = W.type;
    a.pro = CJ_PRO_PACKED; a.epi = accum ? CJ_EPI_ACCUM : CJ_EPI_STORE; a.per32 = W.type == CJ_Q8_0;
    if (gemm_supported(W.type)) {
        a.xp = xp; a.y = y; a.batch = n; a.xp_stride = xp_stride; a.y_stride = y_stride;
        return run_gemm(a);
    }
    const GemvPlan p = plan_gemv(a.type, a.rows, a.cols, 8, a.pro, a.epi);
    a.batch = 1;
    for (int r = 0; r < n; r++) {
        a.xp = xp + r * xp_stride;
        a.y = y + r * y_stride;
        int rc = run_gemv(a, p);
        if (rc) return rc;
    }
    return CJ_OK;
}

// RMSNorm + pack of n residual rows. A few rows (batched decode): a
// workgroup a 256-block and row, each forming its row's sum of squares (the
// one-row norm + pack's arithmetic), so the launch fills the chip; many rows
// (prefill chunks): a workgroup a row, which reads each row once (C4:
// batched step 9.14 → 8.93 ms with the first, a 512-row chunk 27.6 → 28.4
// ms with it, hence the split).
int Engine::launch_norm_pack_rows(cj_pack_args &a, int n) {
    if (n <= 64) return launch2("cj_norm_pack_rows", (uint32_t)(a.npad / 256), (uint32_t)n, 256, 0, a);
    return launch("cj_pack", (uint32_t)n, 256, (uint32_t)(a.npad / 256 * 320), a);
}

int Engine::rows_norm_pack(const float *w, int per32, int n) {
    cj_pack_args a{};
    const int64_t npad = ((int64_t)hidden + 255) / 256 * 256;
    a.out = r_xp; a.x = r_hs; a.w = w; a.n = hidden; a.npad = npad; a.rows = n; a.eps = eps; a.form = 0;
    a.per32 = per32; a.do_norm = 1;
    return launch_norm_pack_rows(a, n);
}

// The f32 rows x (n wide) packed into r_ap, a workgroup a row.
int Engine::rows_pack(const float *x, int64_t n, int per32, int rows) {
    cj_pack_args p{};
    p.out = r_ap; p.x = x; p.n = n; p.npad = (n + 255) / 256 * 256; p.rows = rows; p.per32 = per32;
    return launch("cj_pack", (uint32_t)rows, 256, (uint32_t)(p.npad / 256 * 320), p);
}

// The MoE FFN of n rows (MoeFfn.forwardRowsZeroSync, model/MoeFfn.cajeta:1559
// and its comment at :1510-1515: one router product and one top-k over the
// rows, one indirected product per expert bank over every row's
// selections, one combine), each row computed exactly as the one-row step
// computes it: the FFN norm (f32 rows for the router and f32-activation
// experts, the pack for int8 experts), the f32 router of every row, top-k,
// gate|up + SiLU·up of selection (r, k) from row r's activation, down of
// each selection, the weighted sum onto the residual rows in k order.
int Engine::rows_moe(const Layer &L, int n) {
    int rc;
    const int64_t npad = ((int64_t)hidden + 255) / 256 * 256, hb = npad / 256 * 320;
    const int sels = n * n_used;
    // MXFP4 banks read each selected expert once for all its rows: the rows'
    // per-32 packs are the codes the device Q8 form quantizes (the same
    // per-32 maximum, 127/max, round-half-away, max/127)
    const bool grouped = L.gu_exps.type == CJ_MXFP4 && L.down_exps.type == CJ_MXFP4 && n_experts <= 256 &&
                         n <= rows_cap && hidden % 32 == 0 && expert_ffn % 32 == 0 && hidden <= 4096 &&
                         expert_ffn <= 4096;
    {
        cj_pack_args p{};
        p.out = r_xp; p.x = r_hs; p.w = L.ffn_norm; p.xout = r_xn; p.n = hidden; p.npad = npad; p.rows = n;
        p.eps = eps; p.form = 0; p.per32 = L.gu_exps.type == CJ_Q8_0 || grouped; p.do_norm = 1;
        if ((rc = launch_norm_pack_rows(p, n))) return rc;
    }
    {   // router logits of every row: the indirection's copies all read the router (expert_bytes 0)
        cj_gemv_args a{};
        a.w = (const uint8_t *)L.router.p; a.x = r_xn; a.y = r_moe_logits; a.rows = n_experts; a.cols = hidden;
        a.row_bytes = L.router.row_bytes; a.type = CJ_F32; a.pro = CJ_PRO_F32; a.epi = CJ_EPI_STORE; a.eps = eps;
        a.batch = 1; a.sel = r_zero_sel; a.n_sel = n; a.sel_per_x = 1; a.expert_bytes = 0; a.x_stride = hidden;
        a.y_stride = n_experts;
        if ((rc = run_gemv(a, plan_gemv(CJ_F32, a.rows, a.cols, 0, a.pro, a.epi)))) return rc;
    }
    {   // the route as its own launch: inside the gate|up launch every one
        // of the rows' many workgroups would wait out its row's route
        cj_route_args a{r_moe_logits, r_moe_sel, r_moe_w, n_experts, n_used, norm_topk, n, w_scale, 0, route_status};
        if ((rc = launch("cj_moe_route", (uint32_t)n, 64, 0, a))) return rc;
    }
    if (grouped) {
        cj_moe_group_args g{r_moe_sel, r_grp_cnt, r_grp_mem, sels, n_experts, sels, 0};
        if ((rc = launch("cj_moe_group", 1, 256, 0, g))) return rc;
        const int64_t efb = ((int64_t)expert_ffn + 255) / 256 * 320;
        const char *rcv = getenv("CJ_GRP_RC");   // "<rw><cc>": 14, 24
        auto grp = [&](const char *form, int grt, cj_moe_grp_args &q) {
            const int nbq = (int)(q.cols / 32), kb = std::min(4, std::max(1, (nbq + 31) / 32));
            const int cc = rcv && kb == 3 ? 4 : 16;
            const uint32_t lds = (uint32_t)(cc * ((q.cols + 15) & ~15) + cc * ((nbq + 3) & ~3) * 4 + grt * (cc + 1) * 4);
            char kname[48];
            if (rcv && kb == 3) snprintf(kname, sizeof kname, "cj_moe_mxq8_%s_k%d_t%d_r%c_c4", form, kb, grt, rcv[0]);
            else snprintf(kname, sizeof kname, "cj_moe_mxq8_%s_k%d_t%d", form, kb, grt);
            return launch2(kname, (uint32_t)((q.rows + grt - 1) / grt), (uint32_t)n_experts, 256, lds, q);
        };
        const int grt_g = 64;
        const int grt_s = getenv("CJ_GRT_S") ? atoi(getenv("CJ_GRT_S")) : 32;
        {   // gate|up + SiLU·up of each selection (r, k) = r·n_used + k over row r, into its pack
            cj_moe_grp_args q{};
            q.w = (const uint8_t *)L.gu_exps.p; q.xp = r_xp; q.outp = r_exp_pack; q.cnt = r_grp_cnt; q.mem = r_grp_mem;
            q.expert_bytes = 2 * (int64_t)expert_ffn * L.gu_exps.row_bytes; q.row_bytes = L.gu_exps.row_bytes;
            q.rows = 2 * (int64_t)expert_ffn; q.cols = hidden; q.xp_stride = hb; q.outp_stride = efb; q.cap = sels;
            q.x_per = n_used; q.glu_form = 0; q.act_n = expert_ffn;
            if ((rc = grp("g", grt_g, q))) return rc;
        }
        {   // down of every selection
            cj_moe_grp_args q{};
            q.w = (const uint8_t *)L.down_exps.p; q.xp = r_exp_pack; q.y = r_moe_y; q.cnt = r_grp_cnt; q.mem = r_grp_mem;
            q.expert_bytes = (int64_t)hidden * L.down_exps.row_bytes; q.row_bytes = L.down_exps.row_bytes;
            q.rows = hidden; q.cols = expert_ffn; q.xp_stride = efb; q.y_stride = hidden; q.cap = sels; q.x_per = 1;
            if ((rc = grp("s", grt_s, q))) return rc;
        }
        cj_combine_args c{r_hs, r_moe_y, r_moe_w, hidden, n_used};
        return launch2("cj_moe_combine", (uint32_t)((hidden + 255) / 256), (uint32_t)n, 256, 0, c);
    }
    {   // gate|up + SiLU·up of selection (r, k) = r·n_used + k over row r
        cj_gemv_args a{};
        a.w = (const uint8_t *)L.gu_exps.p; a.x = r_xn; a.xp = r_xp; a.act = r_act; a.rows = 2 * (int64_t)expert_ffn;
        a.cols = hidden; a.row_bytes = L.gu_exps.row_bytes; a.type = L.gu_exps.type;
        a.pro = expert_pro(a.type, CJ_PRO_PACKED); a.epi = CJ_EPI_GLU; a.eps = eps;
        a.per32 = a.type == CJ_Q8_0; a.act_n = expert_ffn; a.glu_form = 0; a.batch = 1;
        a.sel = r_moe_sel; a.n_sel = sels; a.sel_per_x = n_used; a.x_stride = hidden; a.xp_stride = hb;
        a.expert_bytes = 2 * (int64_t)expert_ffn * L.gu_exps.row_bytes; a.y_stride = expert_ffn;
        if ((rc = run_gemv(a, plan_gemv(a.type, a.rows, a.cols, 32, a.pro, a.epi)))) return rc;
    }
    {   // down of every selection
        cj_gemv_args a{};
        a.w = (const uint8_t *)L.down_exps.p; a.x = r_act; a.y = r_moe_y; a.rows = hidden; a.cols = expert_ffn;
        a.row_bytes = L.down_exps.row_bytes; a.type = L.down_exps.type;
        a.pro = expert_pro(a.type, CJ_PRO_PACK); a.epi = CJ_EPI_STORE; a.per32 = a.type == CJ_Q8_0;
        a.batch = 1; a.sel = r_moe_sel; a.n_sel = sels; a.sel_per_x = 1;
        a.expert_bytes = (int64_t)hidden * L.down_exps.row_bytes; a.x_stride = expert_ffn; a.y_stride = hidden;
        if ((rc = run_gemv(a, plan_gemv(a.type, a.rows, a.cols, 32, a.pro, a.epi)))) return rc;
    }
    cj_combine_args c{r_hs, r_moe_y, r_moe_w, hidden, n_used};
    return launch2("cj_moe_combine", (uint32_t)((hidden + 255) / 256), (uint32_t)n, 256, 0, c);
}

// The layers over n rows (row table `tab` on the device): embedding, then per
// layer the norm + pack rows, q|k|v product, RoPE + K/V append rows, the
// attention (prefill: the prefill attend + pack; batched decode: split-K
// rows + merge/pack), o product into the residual rows, FFN norm + pack,
// gate|up product, SiLU·up + pack rows, down product into the residual rows
// (CausalLM.decodeBatchRows, model/CausalLM.cajeta:4133-4360, and
// forwardRowsBatched, :2873).
int Engine::rows_forward(const int32_t *tab, int n, bool prefill) {
    const int64_t qd = (int64_t)n_heads * head_dim;
    const int64_t hb = ((int64_t)hidden + 255) / 256 * 320, qb = (qd + 255) / 256 * 320;
    const int64_t fpad = ((int64_t)ffn + 255) / 256 * 256;
    const int grp = n_heads / n_kv;
    int rc;
    cj_rows_args ra{};
    ra.rowtab = tab; ra.states = states; ra.tokens = tokens_all; ra.preds = preds_all; ra.hist = ctx + 2;
    {
        cj_rows_args e = ra;
        e.table = (const uint8_t *)embd; e.row_bytes = embd_row_bytes; e.type = embd_type; e.nrows = n;
        e.out = r_hs; e.out_stride = hidden; e.n = hidden;
        if ((rc = launch2("cj_rows_embed", (uint32_t)((hidden + 255) / 256), (uint32_t)n, 256, 0, e))) return rc;
    }
    for (int l = 0; l < n_layers; l++) {
        Layer &L = layers[l];
        if ((rc = rows_norm_pack(L.attn_norm, L.qkv.type == CJ_Q8_0, n))) return rc;
        if ((rc = rows_linear(L.qkv, r_xp, hb, r_qkv, L.qkv.rows, false, n))) return rc;
        {
            cj_rows_args q = ra;
            q.in = r_qkv; q.in_stride = L.qkv.rows; q.q_out = r_q; q.out_stride = qd; q.kc = L.kc; q.vc = L.vc;
            q.pgtab = pgtab; q.rope_cs = rope; q.pg_n = pages_per_seq; q.n_q = n_heads; q.n_kv = n_kv;
            q.head_dim = head_dim; q.nrows = n; q.kv_f32 = kv_f32;
            const int64_t qkv_vals = (int64_t)(n_heads + 2 * n_kv) * head_dim;
            if ((rc = launch2("cj_rows_qkv", (uint32_t)((qkv_vals + 511) / 512), (uint32_t)n, 256, 0, q))) return rc;
        }
        cj_attn_args a{};
        a.q = r_q; a.kc = L.kc; a.vc = L.vc; a.pgtab = pgtab; a.n_q = n_heads; a.n_kv = n_kv; a.head_dim = head_dim;
        a.workers = workers; a.scale = scale; a.pg_n = pages_per_seq; a.window = L.window; a.rowtab = tab;
        a.states = states; a.nrows = n; a.q_stride = qd;
        if (prefill && rows_pf_attend) {
            a.out = r_attn;
            const int ns = grp >= 8 ? grp / 4 : 1, rb = 16 * ns / grp;
            char kname[48];
            snprintf(kname, sizeof kname, "cj_attn_prefill_h128_g%d", grp);
            if ((rc = launch(kname, (uint32_t)(n_kv * ((n + rb - 1) / rb)), 256, 0, a))) return rc;
            if ((rc = rows_pack(r_attn, qd, L.o.type == CJ_Q8_0, n))) return rc;
        } else if (!rows_split) {
            // each row's two-pass decode attention (the fused form where
            // every span fits one workgroup), then the pack of the rows
            a.out = r_attn; a.part = r_part; a.splits = ctx; a.part_stride = (int64_t)n_heads * ctx;
            const int64_t span = L.window > 0 ? std::min(L.window, ctx) : ctx;
            const char *kvs = kv_f32 ? "f32_" : "";
            char kname[48];
            if (!kv_f32 && span <= (head_dim == 64 ? 256 : 128)) {
                snprintf(kname, sizeof kname, "cj_attn_fused_rows_h%d", head_dim);
                if ((rc = launch2(kname, (uint32_t)n_heads, (uint32_t)n, 256, 0, a))) return rc;
            } else {
                if (!kv_f32 && n_heads / n_kv <= 16 && !getenv("CJ_SCORES_OLD")) {
                    // a lane a position, its K row read once for the kv head's query heads
                    snprintf(kname, sizeof kname, "cj_attn_scores_grp_rows_h%d", head_dim);
                    if ((rc = launch2(kname, (uint32_t)((span + 255) / 256), (uint32_t)(n * n_kv), 256, 0, a)))
                        return rc;
                } else {
                    snprintf(kname, sizeof kname, "cj_attn_scores_rows_%sh%d", kvs, head_dim);
                    if ((rc = launch2(kname, (uint32_t)((span + 255) / 256), (uint32_t)(n * n_heads), 256, 0, a)))
                        return rc;
                }
                const int hpw = 256 / head_dim;
                if (!kv_f32 && (n_heads / n_kv) % hpw == 0 && !getenv("CJ_COMBINE_OLD")) {
                    // a workgroup per kv head's group of 256/hd query heads: V staged once for them
                    snprintf(kname, sizeof kname, "cj_attn_combine_grp_rows_h%d", head_dim);
                    if ((rc = launch2(kname, (uint32_t)(n_heads / hpw), (uint32_t)n, 256, 0, a))) return rc;
                } else {
                    snprintf(kname, sizeof kname, "cj_attn_combine_rows_%sh%d", kvs, head_dim);
                    if ((rc = launch2(kname, (uint32_t)(n_heads * (head_dim / (kv_f32 ? 32 : CJ_COMBINE_DH))), (uint32_t)n, 256, 0, a))) return rc;
                }
            }
            if ((rc = rows_pack(r_attn, qd, L.o.type == CJ_Q8_0, n))) return rc;
        } else {
            // split slots a row: the rule's count over every row's kv heads
            const int rk = n * n_kv;
            const int spl = std::min(64, std::max(1, (2 * workers + rk - 1) / rk));
            a.part = r_part; a.spl = spl; a.part_stride = (int64_t)n_heads * 64 * (head_dim + 2);
            char kname[48];
            snprintf(kname, sizeof kname, "cj_attn_split_rows_h128_g%d", grp);
            if ((rc = launch(kname, (uint32_t)(n * n_kv * spl), 256, 0, a))) return rc;
            cj_merge_args m{};
            m.packed = r_ap; m.part = r_part; m.n_q = n_heads; m.head_dim = head_dim; m.per32 = L.o.type == CJ_Q8_0;
            m.n_kv = n_kv; m.workers = workers; m.window = L.window; m.nrows = n; m.rowtab = tab; m.states = states;
            m.part_stride = a.part_stride; m.pack_stride = qb;
            if ((rc = launch("cj_attn_merge_rows", (uint32_t)(n * (qd / 256)), 256, 0, m))) return rc;
        }
        if ((rc = rows_linear(L.o, r_ap, qb, r_hs, hidden, true, n))) return rc;
        if (n_experts > 0) {
            if ((rc = rows_moe(L, n))) return rc;
            continue;
        }
        if ((rc = rows_norm_pack(L.ffn_norm, L.gu.type == CJ_Q8_0, n))) return rc;
        if ((rc = rows_linear(L.gu, r_xp, hb, r_gu, L.gu.rows, false, n))) return rc;
        {
            cj_rows_args g = ra;
            g.in = r_gu; g.in_stride = L.gu.rows; g.packed = r_actp; g.pack_stride = fpad / 256 * 320;
            g.n = ffn; g.npad = fpad; g.form = (ffn % 256) ? 1 : 0; g.per32 = L.down.type == CJ_Q8_0; g.nrows = n;
            if ((rc = launch2("cj_rows_glu", (uint32_t)((fpad / 256 + 3) / 4), (uint32_t)n, 256, 0, g))) return rc;
        }
        if ((rc = rows_linear(L.down, r_actp, fpad / 256 * 320, r_hs, hidden, true, n))) return rc;
    }
    return CJ_OK;
}

// One batched decode step over the n slots of the batch row table: the
// layers, then every row's final norm, head and greedy pick (advancing each
// slot's position).
int Engine::enqueue_batch(int n) {
    int rc;
    if ((rc = rows_forward(r_tab_b, n, false))) return rc;
    const int64_t hb = ((int64_t)hidden + 255) / 256 * 320;
    if ((rc = rows_norm_pack(out_norm, head.type == CJ_Q8_0, n))) return rc;
    if ((rc = rows_linear(head, r_xp, hb, r_logits, vocab, false, n))) return rc;
    cj_rows_args k{};
    k.rowtab = r_tab_b; k.states = states; k.tokens = tokens_all; k.preds = preds_all; k.hist = ctx + 2;
    k.in = r_logits; k.in_stride = vocab; k.n = vocab; k.pv = r_pv; k.pi = r_pi; k.nchunks = (vocab + 1023) / 1024;
    k.nrows = n;
    if ((rc = launch2("cj_rows_argmax", (uint32_t)k.nchunks, (uint32_t)n, 256, 0, k))) return rc;
    return launch("cj_rows_pick", (uint32_t)n, 256, 0, k);
}

// A prompt of n > 1 tokens as prefill chunks of up to `chunk` rows
// (CausalLM.stepSeq, model/CausalLM.cajeta:801-883): every row of a chunk
// through each layer, the prefill attend over the positions so far; the
// final norm, head and greedy pick on the prompt's last row only.
int Engine::prefill_rows(int s, const int32_t *toks, int n) {
    Seq &S = seqs[s];
    int rc;
    memcpy(pinned, toks, (size_t)n * 4);
    cj_step_state *st = (cj_step_state *)(pinned + ctx + 2);
    *st = cj_step_state{};
    st->pos = S.pos;
    st->fixed_until = S.pos + n;
    CJ_HIP(hipMemcpyAsync(S.tokens + S.pos, pinned, (size_t)n * 4, hipMemcpyHostToDevice, stream()));
    CJ_HIP(hipMemcpyAsync(S.state, st, sizeof *st, hipMemcpyHostToDevice, stream()));
    for (int c0 = 0; c0 < n; c0 += chunk) {
        const int m = std::min(chunk, n - c0);
        CJ_HIP(hipStreamSynchronize(stream()));   // the staging is free again
        for (int r = 0; r < m; r++) { pinned_tab[2 * r] = s; pinned_tab[2 * r + 1] = c0 + r; }
        CJ_HIP(hipMemcpyAsync(r_tab_pf, pinned_tab, (size_t)m * 8, hipMemcpyHostToDevice, stream()));
        if ((rc = rows_forward(r_tab_pf, m, true))) return rc;
        if (c0 + m < n) continue;
        // the tail on the prompt's last row
        const int last = S.pos + n - 1;
        if ((rc = norm_pack(out_norm, head.type == CJ_Q8_0, is_f32_act(head.type), r_hs + (int64_t)(m - 1) * hidden)))
            return rc;
        cj_gemv_args a{};
        a.w = (const uint8_t *)head.p; a.x = xn; a.xp = xpack; a.y = logits;
        a.part_v = part_v; a.part_i = part_i; a.tokens = S.tokens; a.preds = S.preds; a.state = nullptr; a.pos = last;
        a.rows = vocab; a.cols = hidden; a.row_bytes = head.row_bytes; a.type = head.type;
        a.pro = is_f32_act(head.type) ? CJ_PRO_F32 : CJ_PRO_PACKED; a.epi = CJ_EPI_ARGMAX;
        a.per32 = head.type == CJ_Q8_0; a.eps = eps; a.batch = 1;
        GemvPlan p = plan_gemv(a.type, a.rows, a.cols, head_target(a.type), a.pro, a.epi);
        if ((int64_t)p.grid > (vocab + 3) / 4 + 64) return fail(CJ_ERR_STATE, "head grid exceeds the partial buffers");
        if ((rc = run_gemv(a, p))) return rc;
        cj_pick_args k{};
        k.pv = part_v; k.pi = part_i; k.n = (int32_t)p.grid; k.pos = last; k.tokens = S.tokens; k.preds = S.preds;
        k.state = nullptr;
        if ((rc = launch("cj_argmax_pick", 1, 256, 0, k))) return rc;
    }
    S.pos += n;
    st->pos = S.pos;
    st->fixed_until = S.pos;
    CJ_HIP(hipMemcpyAsync(S.state, st, sizeof *st, hipMemcpyHostToDevice, stream()));
    CJ_HIP(hipStreamSynchronize(stream()));
    S.fixed_until = S.pos;
    return check_route();
}

// `steps` greedy tokens for each of n prefilled slots at once (one row a
// slot): out[i·n + r] is slot r's token i. Models the many-row path does
// not serve (f32-activation projections) decode slot by slot (the same
// tokens: rows only share weights).
int Engine::decode_batch(const int32_t *slots, int n, int steps, int32_t *out) {
    if (n <= 0 || n > max_seqs) return fail(CJ_ERR_ARG, "decode batch of %d slots (1..%d)", n, max_seqs);
    for (int r = 0; r < n; r++) {
        const int s = slots[r];
        if (s < 0 || s >= max_seqs) return fail(CJ_ERR_ARG, "sequence slot %d out of range", s);
        for (int q2 = 0; q2 < r; q2++)
            if (slots[q2] == s) return fail(CJ_ERR_ARG, "slot %d twice in one batch", s);
        if (seqs[s].pos == 0) return fail(CJ_ERR_STATE, "decode of slot %d before prefill", s);
        if (seqs[s].pos + steps > ctx)
            return fail(CJ_ERR_CAPACITY, "kv pool exhausted: slot %d position %d of %d", s, seqs[s].pos + steps, ctx);
    }
    if (steps <= 0) return CJ_OK;
    int rc;
    for (int r = 0; r < n; r++)
        if ((rc = ensure_pages(slots[r], (int64_t)seqs[slots[r]].pos + steps))) return rc;
    if (!rows_ok || n > rows_cap) {
        std::vector<int32_t> tmp((size_t)steps);
        for (int r = 0; r < n; r++) {
            if ((rc = decode(slots[r], steps, tmp.data()))) return rc;
            if (out)
                for (int i = 0; i < steps; i++) out[(size_t)i * n + r] = tmp[i];
        }
        return CJ_OK;
    }
    // the row table names each row's slot; the graphs read it at replay, so
    // a new set of slots (admissions, retirements) reuses the graph of its
    // row count instead of capturing again
    CJ_HIP(hipStreamSynchronize(stream()));   // the staging and the table are free again
    for (int r = 0; r < n; r++) { pinned_tab[2 * r] = slots[r]; pinned_tab[2 * r + 1] = 0; }
    CJ_HIP(hipMemcpyAsync(r_tab_b, pinned_tab, (size_t)n * 8, hipMemcpyHostToDevice, stream()));
    batch_rows = n;
    hipGraphExec_t &batch_graph = batch_graphs[(size_t)n];
    if (graphs && !batch_graph) {
        CJ_HIP(hipStreamSynchronize(stream()));
        CJ_HIP(hipStreamBeginCapture(stream(), hipStreamCaptureModeThreadLocal));
        rc = enqueue_batch(n);
        hipGraph_t g = nullptr;
        hipError_t e = hipStreamEndCapture(stream(), &g);
        if (rc) { if (g) (void)hipGraphDestroy(g); return rc; }
        if (e != hipSuccess) return fail(CJ_ERR_HIP, "batch capture: %s", hipGetErrorString(e));
        e = hipGraphInstantiate(&batch_graph, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (e != hipSuccess) { batch_graph = nullptr; return fail(CJ_ERR_HIP, "batch graph instantiate: %s", hipGetErrorString(e)); }
    }
    hipEvent_t e0, e1;
    CJ_HIP(hipEventCreate(&e0));
    CJ_HIP(hipEventCreate(&e1));
    CJ_HIP(hipEventRecord(e0, stream()));
    for (int i = 0; i < steps; i++) {
        if (graphs) CJ_HIP(hipGraphLaunch(batch_graph, stream()));
        else if ((rc = enqueue_batch(n))) return rc;
        if ((i & 7) == 7 && i + 1 < steps) CJ_HIP(hipStreamSynchronize(stream()));
    }
    CJ_HIP(hipEventRecord(e1, stream()));
    CJ_HIP(hipEventSynchronize(e1));
    float ms = 0.0f;
    CJ_HIP(hipEventElapsedTime(&ms, e0, e1));
    last_step_us = ms * 1000.0f / (float)steps;
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    std::vector<int32_t> tmp((size_t)steps);
    for (int r = 0; r < n; r++) {
        Seq &S = seqs[slots[r]];
        if (out) {
            CJ_HIP(hipMemcpy(tmp.data(), S.tokens + S.pos + 1, (size_t)steps * 4, hipMemcpyDeviceToHost));
            for (int i = 0; i < steps; i++) out[(size_t)i * n + r] = tmp[i];
        }
        S.pos += steps;
    }
    return check_route();
}

// After the stream is drained: an error when the router met a row whose
// logits are not finite since the last check (the reference throws there,
// MoeFfn.routeFromLogits, model/MoeFfn.cajeta:945-952). The word is cleared.
int Engine::check_route() {
    if (n_experts == 0) return CJ_OK;
    int32_t st = 0;
    CJ_HIP(hipMemcpy(&st, route_status, 4, hipMemcpyDeviceToHost));
    if (!st) return CJ_OK;
    CJ_HIP(hipMemset(route_status, 0, 4));
    return fail(CJ_ERR_STATE, "moe router: the logits of a row are not finite (%d experts, top-%d)", n_experts, n_used);
}

// One decode step of slot s on the stream: the graph, or its launches.
int Engine::run_step(int s) {
    if (!graphs) return enqueue_step(s);
    CJ_HIP(hipGraphLaunch(seqs[s].graph, stream()));
    return CJ_OK;
}

// Slot s holds pages for positions [0, upto) once this returns: the pages
// it lacks are drawn from the pool and their table entries uploaded, on the
// stream ahead of the work that writes them (PagedKvCache / DeviceKv
// tryEnsureRows, model/DeviceKv.cajeta:193-200). A dry pool is an error
// that names the shortfall; the scheduler preempts before it gets here.
int Engine::ensure_pages(int s, int64_t upto) {
    if (upto > (int64_t)pages_per_seq * 64) return fail(CJ_ERR_CAPACITY, "kv pool exhausted: position %lld of %d", (long long)upto, ctx);
    std::vector<int32_t> &P = slot_pages[(size_t)s];
    const size_t need = (size_t)((upto + 63) / 64);
    if (need <= P.size()) return CJ_OK;
    if (need - P.size() > free_pages.size())
        return fail(CJ_ERR_CAPACITY, "kv pool exhausted: slot %d needs %zu more pages, %zu of %d free", s, need - P.size(),
                    free_pages.size(), kv_pages);
    const size_t j0 = P.size();
    int32_t *mirror = pinned_pg + (size_t)s * pages_per_seq;
    while (P.size() < need) {
        mirror[P.size()] = free_pages.back();
        P.push_back(free_pages.back());
        free_pages.pop_back();
    }
    // the mirror's entries are not written again before the slot is reset,
    // which drains the stream first: the copy may read them when it runs
    CJ_HIP(hipMemcpyAsync(pgtab + (size_t)s * pages_per_seq + j0, mirror + j0, (need - j0) * 4, hipMemcpyHostToDevice,
                          stream()));
    return CJ_OK;
}

bool Engine::pages_fit(int s, int64_t upto) const {
    if (upto > (int64_t)pages_per_seq * 64) return false;
    const size_t need = (size_t)((upto + 63) / 64), have = slot_pages[(size_t)s].size();
    return need <= have || need - have <= free_pages.size();
}

// The slot's pages back to the pool (the stream is drained first: work
// queued for the slot may still read them).
void Engine::release_pages(int s) {
    std::vector<int32_t> &P = slot_pages[(size_t)s];
    if (P.empty()) return;
    (void)hipStreamSynchronize(stream());
    for (size_t j = P.size(); j-- > 0;) free_pages.push_back(P[j]);
    P.clear();
}

int Engine::reset(int s) {
    if (s < 0 || s >= (int)seqs.size()) return fail(CJ_ERR_ARG, "sequence slot %d out of range", s);
    Seq &S = seqs[s];
    cj_step_state st{};
    CJ_HIP(hipStreamSynchronize(stream()));
    release_pages(s);
    CJ_HIP(hipMemcpy(S.state, &st, sizeof st, hipMemcpyHostToDevice));
    S.pos = 0;
    S.fixed_until = 0;
    return CJ_OK;
}

int Engine::prefill(int s, const int32_t *toks, int n) {
    if (s < 0 || s >= (int)seqs.size()) return fail(CJ_ERR_ARG, "sequence slot %d out of range", s);
    Seq &S = seqs[s];
    if (n <= 0) return fail(CJ_ERR_ARG, "prefill of %d tokens", n);
    if (S.pos + n > ctx) return fail(CJ_ERR_CAPACITY, "kv pool exhausted: position %d of %d", S.pos + n, ctx);
    for (int i = 0; i < n; i++)
        if (toks[i] < 0 || toks[i] >= vocab) return fail(CJ_ERR_ARG, "token %d outside the vocabulary", toks[i]);
    int rc;
    if ((rc = ensure_pages(s, (int64_t)S.pos + n))) return rc;
    if (n > 1 && rows_prefill && chunk > 1) return prefill_rows(s, toks, n);
    if (graphs && (rc = capture(s))) return rc;
    // through pinned staging: the copies are ordered on the stream and the
    // staging is not reused before the synchronize below
    memcpy(pinned, toks, (size_t)n * 4);
    cj_step_state *st = (cj_step_state *)(pinned + ctx + 2);
    *st = cj_step_state{};
    st->pos = S.pos;
    st->fixed_until = S.pos + n;
    CJ_HIP(hipMemcpyAsync(S.tokens + S.pos, pinned, (size_t)n * 4, hipMemcpyHostToDevice, stream()));
    CJ_HIP(hipMemcpyAsync(S.state, st, sizeof *st, hipMemcpyHostToDevice, stream()));
    for (int i = 0; i < n; i++) {
        if ((rc = run_step(s))) return rc;
        // bound the work in flight on long prompts (tools that track every
        // dispatch hold a record per queued kernel)
        if ((i & 15) == 15) CJ_HIP(hipStreamSynchronize(stream()));
    }
    CJ_HIP(hipStreamSynchronize(stream()));
    S.pos += n;
    S.fixed_until = S.pos;
    return check_route();
}

int Engine::decode(int s, int steps, int32_t *out) {
    if (s < 0 || s >= (int)seqs.size()) return fail(CJ_ERR_ARG, "sequence slot %d out of range", s);
    Seq &S = seqs[s];
    if (S.pos == 0) return fail(CJ_ERR_STATE, "decode before prefill");
    if (steps <= 0) return CJ_OK;
    if (S.pos + steps > ctx) return fail(CJ_ERR_CAPACITY, "kv pool exhausted: position %d of %d", S.pos + steps, ctx);
    int rc;
    if ((rc = ensure_pages(s, (int64_t)S.pos + steps))) return rc;
    if (graphs && (rc = capture(s))) return rc;
    hipEvent_t e0, e1;
    CJ_HIP(hipEventCreate(&e0));
    CJ_HIP(hipEventCreate(&e1));
    CJ_HIP(hipEventRecord(e0, stream()));
    for (int i = 0; i < steps; i++) {
        if ((rc = run_step(s))) return rc;
        // at most 32 steps in flight (a few thousand dispatches): profilers
        // that track every queued kernel fail beyond ~8k
        if ((i & 31) == 31 && i + 1 < steps) CJ_HIP(hipStreamSynchronize(stream()));
    }
    CJ_HIP(hipEventRecord(e1, stream()));
    CJ_HIP(hipEventSynchronize(e1));
    float ms = 0.0f;
    CJ_HIP(hipEventElapsedTime(&ms, e0, e1));
    last_step_us = ms * 1000.0f / (float)steps;
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (out) CJ_HIP(hipMemcpy(out, S.tokens + S.pos + 1, (size_t)steps * 4, hipMemcpyDeviceToHost));
    S.pos += steps;
    return check_route();
}

// Algorithmic HBM bytes of one launch of `kind` (layer 0 shapes) with
// `count` attended positions: weights at their GGUF file size, the K/V read
// and written, and the activation vectors read and written once.
int64_t Engine::kind_bytes(int kind, int count) const {
    const Layer &L = layers[0];
    const int64_t qd = (int64_t)n_heads * head_dim, kvd = (int64_t)n_kv * head_dim, h = hidden;
    const int64_t kvb = kv_f32 ? 4 : 2;   // bytes a K/V element
    auto wb = [](const DevW &w) { return w.rows * ggml_row_bytes(w.type, w.cols); };
    switch (kind) {
    case K_EMBED: return embd_row_file_bytes + h * 4;
    case K_QKV: return wb(L.qkv) + ((h + 255) / 256) * 320 + qd * 4 + 2 * kvd * kvb;
    case K_ATTN: return (int64_t)count * kvd * 2 * kvb + qd * 8 + ((qd + 255) / 256) * 320;
    case K_O: return wb(L.o) + (merge_w ? qd * 4 : ((qd + 255) / 256) * 320) + h * 8;
    case K_GATE_UP: return wb(L.gu) + ((h + 255) / 256) * 320 + (int64_t)ffn * 4;
    case K_DOWN: return wb(L.down) + (int64_t)ffn * 4 + h * 8;
    case K_ROUTER: return wb(L.router) + h * 8 + (int64_t)n_experts * 4;
    case K_ROUTE: return (int64_t)n_experts * 4 + (int64_t)n_used * 8;
    case K_EXP_GATE_UP:
        return n_used * (2 * (int64_t)expert_ffn * ggml_row_bytes(L.gu_exps.type, h)) + h * 8 + (int64_t)n_used * expert_ffn * 4;
    case K_EXP_DOWN:
        return n_used * (h * ggml_row_bytes(L.down_exps.type, expert_ffn)) + (int64_t)n_used * (expert_ffn + h) * 4;
    case K_COMBINE: return (int64_t)n_used * h * 4 + h * 8;
    case K_HEAD: return wb(head) + ((h + 255) / 256) * 320 + (int64_t)vocab * 4;
    case K_NORM: return h * 8 + ((h + 255) / 256) * 320;
    case K_MERGE: return (int64_t)n_heads * 64 * (head_dim + 2) * 4 + qd * 4 + (merge_w ? 0 : ((qd + 255) / 256) * 320);
    default: return 0;
    }
}

// Algorithmic HBM bytes of one whole decode step attending `count` positions.
int64_t Engine::step_bytes(int count) const {
    int64_t b = kind_bytes(K_EMBED, count) + kind_bytes(K_HEAD, count) + kind_bytes(K_NORM, count);
    for (int l = 0; l < n_layers; l++) {
        const int c = layers[l].window > 0 ? std::min(count, layers[l].window) : count;
        const int norms = (layers[l].qkv.type == CJ_Q4_K ? 0 : 1) + (n_experts == 0 && layers[l].gu.type == CJ_Q4_K ? 0 : 1);
        b += norms * kind_bytes(K_NORM, c) + kind_bytes(K_QKV, c) + kind_bytes(K_ATTN, c) + kind_bytes(K_O, c);
        if (n_experts == 0) b += kind_bytes(K_GATE_UP, c) + kind_bytes(K_DOWN, c);
        else
            for (int k : {K_ROUTER, K_ROUTE, K_EXP_GATE_UP, K_EXP_DOWN, K_COMBINE}) b += kind_bytes(k, c);
    }
    return b;
}

// The in-step duration of one launch kind: `steps` whole decode steps of
// sequence s enqueued eagerly (the step's own launch order and data), an
// event recorded on the stream before and after every launch of the kind;
// the mean interval over the layers and steps (each includes the launch's
// share of the kernel boundary, as in the step). The step state is left as
// it was.
int Engine::time_in_step(int s, int kind, int steps, float *avg_us) {
    if (s < 0 || s >= (int)seqs.size()) return fail(CJ_ERR_ARG, "sequence slot %d out of range", s);
    if (kind != K_QKV && kind != K_ATTN && kind != K_O && kind != K_GATE_UP && kind != K_DOWN)
        return fail(CJ_ERR_ARG, "time in step: kind %d is not probed", kind);
    if (n_experts > 0 && (kind == K_GATE_UP || kind == K_DOWN))
        return fail(CJ_ERR_ARG, "time in step: kind %d is not part of this model's step", kind);
    if (steps <= 0 || steps > 64) return fail(CJ_ERR_ARG, "time in step: %d steps", steps);
    Seq &S = seqs[s];
    if (S.pos == 0) return fail(CJ_ERR_STATE, "time: prefill first");
    cj_step_state saved{};
    CJ_HIP(hipStreamSynchronize(stream()));
    CJ_HIP(hipMemcpy(&saved, S.state, sizeof saved, hipMemcpyDeviceToHost));
    const int per = 2 * n_layers;
    probe_ev.assign((size_t)per, nullptr);
    int rc = CJ_OK;
    for (auto &e : probe_ev)
        if (hipEventCreate(&e) != hipSuccess) { e = nullptr; rc = fail(CJ_ERR_HIP, "time in step: event create"); }
    double sum = 0.0;
    int n = 0;
    for (int i = 0; i <= steps && !rc; i++) {   // step 0 warms up
        CJ_HIP(hipMemcpy(S.state, &saved, sizeof saved, hipMemcpyHostToDevice));
        probe_kind = kind;
        probe_n = 0;
        rc = enqueue_step(s);
        probe_kind = -1;
        if (rc) break;
        CJ_HIP(hipStreamSynchronize(stream()));
        if (probe_n != per) { rc = fail(CJ_ERR_STATE, "time in step: %d probes, %d expected", probe_n, per); break; }
        for (int k = 0; i > 0 && k < per; k += 2) {
            float ms = 0.0f;
            if (hipEventElapsedTime(&ms, probe_ev[k], probe_ev[k + 1]) == hipSuccess) { sum += ms; n++; }
        }
    }
    probe_kind = -1;
    for (auto &e : probe_ev) if (e) (void)hipEventDestroy(e);
    probe_ev.clear();
    CJ_HIP(hipStreamSynchronize(stream()));
    CJ_HIP(hipMemcpy(S.state, &saved, sizeof saved, hipMemcpyHostToDevice));
    if (rc) return rc;
    if (n == 0) return fail(CJ_ERR_HIP, "time in step: no interval measured");
    *avg_us = (float)(sum * 1000.0 / n);
    return CJ_OK;
}

// Time `reps` back-to-back eager launches of one kind of sequence s's step at
// its current position, on the engine's stream, between two HIP events. The
// launches rotate over the layers, so each reads weights the previous few did
// not (the model's weights are far larger than the 256 MB last-level cache:
// the timing is of HBM, not of a cached matrix). The step state is left as
// it was.
int Engine::time_kind(int s, int kind, int reps, float *avg_us, std::string &kernel) {
    if (s < 0 || s >= (int)seqs.size()) return fail(CJ_ERR_ARG, "sequence slot %d out of range", s);
    if (kind < K_EMBED || kind > K_MERGE || reps <= 0) return fail(CJ_ERR_ARG, "time: kind %d reps %d", kind, reps);
    const bool moe_kind = kind >= K_ROUTER && kind <= K_COMBINE, dense_kind = kind == K_GATE_UP || kind == K_DOWN;
    if ((n_experts == 0 && moe_kind) || (n_experts > 0 && dense_kind))
        return fail(CJ_ERR_ARG, "time: kind %d is not part of this model's step", kind);
    Seq &S = seqs[s];
    if (S.pos == 0) return fail(CJ_ERR_STATE, "time: prefill first");
    cj_step_state saved{};
    CJ_HIP(hipStreamSynchronize(stream()));
    CJ_HIP(hipMemcpy(&saved, S.state, sizeof saved, hipMemcpyDeviceToHost));
    only = kind;
    only_layer = 0;
    const uint64_t before = launch_count();
    launch_names_reset();
    int rc = enqueue_step(s);                     // one untimed launch
    if (!rc && launch_count() == before) rc = fail(CJ_ERR_ARG, "time: kind %d launches nothing in this model's step", kind);
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if (!rc && (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess))
        rc = fail(CJ_ERR_HIP, "time: event create");
    if (!rc) {
        kernel = launch_names();
        // the reps as the step runs them: captured into one graph and
        // replayed (eager launches when graphs are off, for profilers)
        hipGraphExec_t ge = nullptr;
        if (graphs) {
            CJ_HIP(hipStreamSynchronize(stream()));
            CJ_HIP(hipStreamBeginCapture(stream(), hipStreamCaptureModeThreadLocal));
            for (int i = 0; i < reps && !rc; i++) {
                only_layer = (i + 1) % (n_layers > 0 ? n_layers : 1);
                rc = enqueue_step(s);
            }
            hipGraph_t gr = nullptr;
            hipError_t ce = hipStreamEndCapture(stream(), &gr);
            if (!rc && ce != hipSuccess) rc = fail(CJ_ERR_HIP, "time: capture: %s", hipGetErrorString(ce));
            if (!rc && hipGraphInstantiate(&ge, gr, nullptr, nullptr, 0) != hipSuccess) {
                ge = nullptr;
                rc = fail(CJ_ERR_HIP, "time: graph instantiate");
            }
            if (gr) (void)hipGraphDestroy(gr);
            if (!rc) (void)hipGraphLaunch(ge, stream());   // warm replay
        }
        if (!rc) {
            (void)hipEventRecord(e0, stream());
            if (ge) (void)hipGraphLaunch(ge, stream());
            for (int i = 0; !ge && i < reps && !rc; i++) {
                only_layer = (i + 1) % (n_layers > 0 ? n_layers : 1);
                rc = enqueue_step(s);
            }
            (void)hipEventRecord(e1, stream());
            (void)hipEventSynchronize(e1);
            float ms = 0.0f;
            (void)hipEventElapsedTime(&ms, e0, e1);
            *avg_us = ms * 1000.0f / (float)reps;
        }
        if (ge) (void)hipGraphExecDestroy(ge);
    }
    only = -1;
    only_layer = 0;
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    CJ_HIP(hipStreamSynchronize(stream()));
    CJ_HIP(hipMemcpy(S.state, &saved, sizeof saved, hipMemcpyHostToDevice));
    return rc;
}

// ------------------------------------------------------------ scheduler
//
// Continuous batching over the sequence slots (Scheduler.stepOnce,
// sched/Scheduler.cajeta:414-605): each step admits requests into free
// slots — preempted ones first, in preemption order, then waiting ones in
// submission order (admitPhase, :1068-1150) — and feeds every running
// request: a prompt chunk of up to the chunk size, or the newest position
// of a decoding request (all of them as one batched step), or, for a sole
// running greedy request, the pipelined step (pipeFor/stepPipelined,
// :613-702). Each greedy token is consumed with the stop checks (stop
// tokens, then the budget); finished requests retire and free their slot
// and pages. A request whose next rows do not fit the page pool preempts
// the youngest running request, itself if it is the youngest (:496-512);
// a preempted request later resumes by recomputing its whole stream.
// Cancel takes effect between steps.

int Engine::submit(const int32_t *prompt, int n, int max_new, const int32_t *stops, int n_stops) {
    if (!prompt || n <= 0 || max_new <= 0) return fail(CJ_ERR_ARG, "submit: %d prompt tokens, max_new %d", n, max_new);
    // the slot must hold the prompt and one decode position (admitPhase's
    // tryDeviceKvRows(slot, totalLen + 1); nothing can make room for more)
    if (n + 1 > ctx)
        return fail(CJ_ERR_CAPACITY, "scheduler: the request needs %d positions of device KV, more than a sequence holds (%d)", n + 1, ctx);
    for (int i = 0; i < n; i++)
        if (prompt[i] < 0 || prompt[i] >= vocab) return fail(CJ_ERR_ARG, "submit: token %d outside the vocabulary", prompt[i]);
    Request r;
    r.all.assign(prompt, prompt + n);
    r.prompt_len = n;
    r.feed = n;
    r.max_new = max_new;
    // LlmEngine.defaultStops (LlmEngine.cajeta:458-474): the model's EOG set
    // unless the caller gave stop tokens (an empty list means none)
    if (n_stops < 0) r.stops.assign(eog.begin(), eog.end());
    else if (n_stops > 0) r.stops.assign(stops, stops + n_stops);
    reqs.push_back(std::move(r));
    return (int)reqs.size() - 1;
}

// Scheduler.soleRunning (:364-377): the one running request, else -1.
int Engine::sole_running() const {
    int found = -1;
    for (size_t i = 0; i < reqs.size(); i++)
        if (reqs[i].state == Request::RUNNING) {
            if (found >= 0) return -1;
            found = (int)i;
        }
    return found;
}

// Scheduler.youngestRunning (:1263-1276): the running request admitted last.
int Engine::youngest_running() const {
    int best = -1, bs = -1;
    for (size_t i = 0; i < reqs.size(); i++)
        if (reqs[i].state == Request::RUNNING && reqs[i].stamp > bs) {
            best = (int)i;
            bs = reqs[i].stamp;
        }
    return best;
}

int Engine::admit() {
    for (;;) {
        int pick = -1, best_pre = 0x7fffffff;
        for (size_t i = 0; i < reqs.size(); i++)
            if (reqs[i].state == Request::PREEMPTED && reqs[i].pre_stamp < best_pre) {
                pick = (int)i;
                best_pre = reqs[i].pre_stamp;
            }
        const bool resume = pick >= 0;
        if (pick < 0)
            for (size_t i = 0; i < reqs.size(); i++)
                if (reqs[i].state == Request::WAITING) { pick = (int)i; break; }
        if (pick < 0) return CJ_OK;
        int slot = -1;
        for (int s = 0; s < max_seqs; s++)
            if (slot_req[(size_t)s] < 0) { slot = s; break; }
        if (slot < 0) return CJ_OK;
        int rc = reset(slot);
        if (rc) return rc;
        Request &r = reqs[(size_t)pick];
        // the whole stream plus one decode position (tryDeviceKvRows(slot, totalLen + 1))
        const int64_t need = (int64_t)r.all.size() + 1;
        if (!pages_fit(slot, need)) {
            if (youngest_running() < 0)
                return fail(CJ_ERR_CAPACITY,
                            "scheduler: request %d needs %lld positions of device KV, more than the pool can hold with "
                            "nothing else running (%d pages of 64)", pick, (long long)need, kv_pages);
            return CJ_OK;
        }
        if ((rc = ensure_pages(slot, need))) return rc;
        slot_req[(size_t)slot] = pick;
        r.slot = slot;
        r.cached = 0;
        r.state = Request::RUNNING;
        r.stamp = ++stamp_n;
        if (resume) resumed_n++;
    }
}

void Engine::retire(Request &r, int finish) {
    if (r.slot >= 0) {
        release_pages(r.slot);
        slot_req[(size_t)r.slot] = -1;
    }
    r.slot = -1;
    r.state = Request::DONE;
    r.finish = finish;
}

// The greedy token the newest consumed position produced (Scheduler.consume,
// :705-760): appended, then the stops in the reference's order — a stop
// token, then the budget. A sequence whose slot has no position left for the
// next step also ends there (as a budget stop).
void Engine::consume(Request &r, int32_t tok) {
    r.all.push_back(tok);
    r.gen++;
    if (std::find(r.stops.begin(), r.stops.end(), tok) != r.stops.end()) retire(r, Request::FINISH_EOS);
    else if (r.gen >= r.max_new || (int)r.all.size() > ctx) retire(r, Request::FINISH_BUDGET);
}

// Scheduler.preempt (:1291-1315): the request's pages go back to the pool,
// its slot is freed, and it waits to resume by recomputing its stream (its
// generated ids stay). A pipelined step in flight for it is awaited and its
// token consumed first.
int Engine::preempt(int i) {
    Request &r = reqs[(size_t)i];
    int rc;
    if (pipe_in && pipe_req == i && (rc = finish_pipe())) return rc;
    if (r.state != Request::RUNNING) return CJ_OK;
    release_pages(r.slot);
    slot_req[(size_t)r.slot] = -1;
    r.slot = -1;
    r.cached = 0;
    r.feed = (int)r.all.size();
    r.state = Request::PREEMPTED;
    r.pre_stamp = ++stamp_n;
    preempted_n++;
    return CJ_OK;
}

// Scheduler.cancel (:288-315): false for an id never issued or already done.
int Engine::cancel(int i) {
    if (i < 0 || i >= (int)reqs.size()) return 0;
    Request &r = reqs[(size_t)i];
    if (r.state == Request::DONE) return 0;
    if (pipe_in && pipe_req == i && drain_pipe()) return CJ_ERR_HIP;
    retire(r, Request::FINISH_CANCEL);
    return 1;
}

// One decode step of slot s queued (its graph), its event recorded in
// pipe_ev[e]: the step consumes the id at the slot's position (written on
// the device by the previous step's pick) and its pick writes the next one.
int Engine::queue_pipe_step(int s, int e) {
    Seq &S = seqs[(size_t)s];
    int rc;
    if ((rc = ensure_pages(s, (int64_t)S.pos + 1))) return rc;
    if ((rc = run_step(s))) return rc;
    CJ_HIP(hipEventRecord(pipe_ev[e], stream()));
    pipe_pos[e] = S.pos;
    S.pos += 1;
    return CJ_OK;
}

// CausalLM.awaitStep (model/CausalLM.cajeta:1245-1256): wait for the oldest
// in-flight step alone (a later queued one keeps running) and read its token
// from the pinned mirror the pick wrote.
int Engine::await_pipe(int32_t *tok) {
    CJ_HIP(hipEventSynchronize(pipe_ev[pipe_out]));
    const Request &r = reqs[(size_t)pipe_req];
    *tok = __atomic_load_n(host_tok + (size_t)r.slot * (ctx + 2) + pipe_pos[pipe_out] + 1, __ATOMIC_ACQUIRE);
    if (*tok < 0 || *tok >= vocab) return fail(CJ_ERR_STATE, "pipelined step: token %d read back", *tok);
    return CJ_OK;
}

// Scheduler.pipeFor (:628-638): a sole running greedy request with one
// position to feed whose id the device already holds. (MoE models keep the
// synchronous step, which checks the router's status after every token.)
bool Engine::pipe_for(int i, const Request &r, int n) {
    if (pipe_in) return pipe_req == i;
    if (n != 1 || !graphs || n_experts > 0) return false;
    if (r.cached < r.feed) return false;
    return sole_running() == i;
}

// Scheduler.stepPipelined (:640-676). The first call seeds: the step is
// queued and no token is read. Each later call queues the speculative next
// step (unless this token must be the last by budget or context), then
// awaits the in-flight one and consumes its token; a finish leaves the
// speculative step queued, and retiring the request drains it.
int Engine::step_pipelined(int i, Request &r) {
    int rc;
    if (!pipe_in) {
        if (graphs && (rc = capture(r.slot))) return rc;
        if ((rc = queue_pipe_step(r.slot, 0))) return rc;
        pipe_in = true;
        pipe_out = 0;
        pipe_req = i;
        r.cached += 1;
        return CJ_OK;
    }
    Seq &S = seqs[(size_t)r.slot];
    const int in_e = pipe_out, out_e = 1 - in_e;
    const bool spec = r.gen + 1 < r.max_new && S.pos < ctx && pages_fit(r.slot, (int64_t)S.pos + 1);
    if (spec && (rc = queue_pipe_step(r.slot, out_e))) return rc;
    int32_t tok = 0;
    if ((rc = await_pipe(&tok))) return rc;
    consume(r, tok);
    if (r.state != Request::RUNNING) {   // retire released the slot, which drained the stream
        pipe_in = false;
        pipe_req = -1;
        return CJ_OK;
    }
    if (spec) {
        pipe_out = out_e;
        r.cached += 1;
    } else {
        pipe_in = false;
        pipe_req = -1;
    }
    return CJ_OK;
}

// Scheduler.finishPipe (:678-692): await the pending step, consume its
// token, and take the plain steps from here.
int Engine::finish_pipe() {
    if (!pipe_in) return CJ_OK;
    const int i = pipe_req;
    int32_t tok = 0;
    const int rc = await_pipe(&tok);
    pipe_in = false;
    pipe_req = -1;
    if (rc) return rc;
    Request &r = reqs[(size_t)i];
    if (r.state == Request::RUNNING) consume(r, tok);
    return CJ_OK;
}

// Scheduler.drainPipe (:694-702): let the pending step end (its token is
// not consumed) and forget the pipeline.
int Engine::drain_pipe() {
    if (!pipe_in) return CJ_OK;
    pipe_in = false;
    pipe_req = -1;
    CJ_HIP(hipEventSynchronize(pipe_ev[pipe_out]));
    return CJ_OK;
}

int Engine::step_once() {
    sched_steps++;
    int rc;
    if ((rc = admit())) return rc;
    // a pipeline serves one sole running request; the moment it is not sole,
    // its pending step is finished here and the plain steps take over
    if (pipe_in && sole_running() != pipe_req && (rc = finish_pipe())) return rc;
    const int cap = rows_prefill && chunk > 1 ? chunk : 512;   // prompt rows a request feeds per step
    std::vector<int> batch;                             // requests decoding one position
    for (size_t i = 0; i < reqs.size(); i++) {
        Request &r = reqs[i];
        if (r.state != Request::RUNNING) continue;
        // a pipelined step in flight has consumed the newest position already
        const int n = (int)r.all.size() - r.cached;
        const int m = std::min(n, cap);
        // per-item headroom: preempt younger requests until this item fits;
        // the youngest yields itself instead
        while (m > 0 && !pages_fit(r.slot, (int64_t)r.cached + m)) {
            const int v = youngest_running();
            if (v < 0) return fail(CJ_ERR_CAPACITY, "scheduler: no preemptable sequence");
            if ((rc = preempt(v))) return rc;
            batch.erase(std::remove(batch.begin(), batch.end(), v), batch.end());
            if (v == (int)i) break;
        }
        if (r.state != Request::RUNNING) continue;
        if (pipe_for((int)i, r, n)) {
            if ((rc = step_pipelined((int)i, r))) return rc;
            continue;
        }
        if (pipe_in && (rc = finish_pipe())) return rc;
        if (r.state != Request::RUNNING) continue;
        // one position whose id the device holds (the pick that produced it
        // wrote it into the slot's history): a row of the batched step
        if (n == 1 && r.cached >= r.feed) {
            batch.push_back((int)i);
            continue;
        }
        if ((rc = prefill(r.slot, r.all.data() + r.cached, m))) return rc;
        r.cached += m;
        if (r.cached == (int)r.all.size()) {
            // the stream's last row was consumed: its argmax is the next token
            int32_t tok = 0;
            CJ_HIP(hipMemcpy(&tok, seqs[(size_t)r.slot].tokens + seqs[(size_t)r.slot].pos, 4, hipMemcpyDeviceToHost));
            consume(r, tok);
        }
    }
    if (!batch.empty()) {
        std::vector<int32_t> slots(batch.size()), out(batch.size());
        for (size_t k = 0; k < batch.size(); k++) slots[k] = reqs[(size_t)batch[k]].slot;
        if ((rc = decode_batch(slots.data(), (int)slots.size(), 1, out.data()))) return rc;
        for (size_t k = 0; k < batch.size(); k++) {
            Request &r = reqs[(size_t)batch[k]];
            r.cached += 1;
            consume(r, out[k]);
        }
    }
    if ((rc = admit())) return rc;   // completions freed slots: same-step admission
    for (auto &r : reqs)
        if (r.state != Request::DONE) return 1;
    return 0;
}

}  // namespace cj

using cj::Engine;

namespace {
Engine *eng_of(int64_t h) { return (Engine *)(uintptr_t)h; }
}

extern "C" {

int64_t cj_engine_load(const int8_t *path, int32_t ctx, int32_t max_seqs) {
    return cj_engine_load_kv(path, ctx, max_seqs, 0, 0);
}

int64_t cj_engine_load_kv(const int8_t *path, int32_t ctx, int32_t max_seqs, int32_t kv_pages, int32_t kv_f32) {
    if (!cj::ready()) return cj::fail(CJ_ERR_STATE, "cj_init has not run"), 0;
    if (!path) return cj::fail(CJ_ERR_ARG, "cj_engine_load: null path"), 0;
    auto *e = new Engine();
    int rc;
    try {
        rc = e->load((const char *)path, ctx, max_seqs, kv_pages, kv_f32 != 0);
    } catch (const std::exception &x) {   // nothing may unwind through the C-ABI
        rc = cj::fail(CJ_ERR_IO, "model: %s", x.what());
    }
    if (rc) { std::string m = cj::last_error(); delete e; cj::fail(rc, "%s", m.c_str()); return 0; }
    return (int64_t)(uintptr_t)e;
}

int32_t cj_engine_close(int64_t h) {
    delete eng_of(h);
    return CJ_OK;
}

int32_t cj_engine_config(int64_t h, int64_t *out, int32_t n) {
    Engine *e = eng_of(h);
    if (!e) return cj::fail(CJ_ERR_STATE, "null engine");
    int64_t v[] = {e->n_layers, e->hidden, e->n_heads, e->n_kv, e->head_dim, e->ffn, e->vocab, e->ctx,
                   e->n_experts, e->n_used, e->wtype, e->head_type, e->expert_ffn, e->workers};
    for (int i = 0; i < n && i < (int)(sizeof v / sizeof v[0]); i++) out[i] = v[i];
    return CJ_OK;
}

int32_t cj_engine_submit(int64_t h, const int32_t *prompt, int32_t n, int32_t max_new) {
    Engine *e = eng_of(h);
    if (!e) return cj::fail(CJ_ERR_STATE, "null engine");
    return e->submit(prompt, n, max_new, nullptr, -1);
}

int32_t cj_engine_submit_stops(int64_t h, const int32_t *prompt, int32_t n, int32_t max_new, const int32_t *stops,
                               int32_t n_stops) {
    Engine *e = eng_of(h);
    if (!e) return cj::fail(CJ_ERR_STATE, "null engine");
    if (n_stops < 0 || (n_stops > 0 && !stops)) return cj::fail(CJ_ERR_ARG, "cj_engine_submit_stops: %d stop tokens", n_stops);
    return e->submit(prompt, n, max_new, stops, n_stops);
}

int32_t cj_engine_step_once(int64_t h) {
    Engine *e = eng_of(h);
    if (!e) return cj::fail(CJ_ERR_STATE, "null engine");
    return e->step_once();
}

int32_t cj_engine_run_all(int64_t h, int32_t max_steps) {
    Engine *e = eng_of(h);
    if (!e) return cj::fail(CJ_ERR_STATE, "null engine");
    if (max_steps <= 0) return cj::fail(CJ_ERR_ARG, "runAll: max_steps %d (a positive progress cap)", max_steps);
    for (int s = 0; s < max_steps; s++) {
        const int rc = e->step_once();
        if (rc <= 0) return rc;
    }
    return cj::fail(CJ_ERR_STATE, "scheduler: not done after %d steps", max_steps);
}

int32_t cj_engine_request(int64_t h, int32_t id, int32_t *tokens, int32_t cap, int32_t *state, int32_t *finish) {
    Engine *e = eng_of(h);
    if (!e || id < 0 || id >= (int)e->reqs.size()) return cj::fail(CJ_ERR_ARG, "cj_engine_request: unknown id %d", id);
    const cj::Request &r = e->reqs[(size_t)id];
    for (int i = 0; i < cap && i < r.gen; i++) tokens[i] = r.all[(size_t)(r.prompt_len + i)];
    if (state) *state = r.state;
    if (finish) *finish = r.finish;
    return (int32_t)r.gen;
}

int32_t cj_engine_cancel(int64_t h, int32_t id) {
    Engine *e = eng_of(h);
    if (!e) return cj::fail(CJ_ERR_STATE, "null engine");
    // Scheduler.cancel (:288-315): false for an id never issued or already done
    return e->cancel(id);
}

int32_t cj_engine_set_eog(int64_t h, const int32_t *ids, int32_t n) {
    Engine *e = eng_of(h);
    if (!e) return cj::fail(CJ_ERR_STATE, "null engine");
    e->eog.clear();
    for (int i = 0; i < n; i++) e->eog.insert(ids[i]);
    return CJ_OK;
}

int32_t cj_engine_reset(int64_t h, int32_t seq) {
    Engine *e = eng_of(h);
    return e ? e->reset(seq) : cj::fail(CJ_ERR_STATE, "null engine");
}
int32_t cj_engine_prefill(int64_t h, int32_t seq, const int32_t *tokens, int32_t n) {
    Engine *e = eng_of(h);
    return e ? e->prefill(seq, tokens, n) : cj::fail(CJ_ERR_STATE, "null engine");
}
int32_t cj_engine_decode(int64_t h, int32_t seq, int32_t steps, int32_t *out) {
    Engine *e = eng_of(h);
    return e ? e->decode(seq, steps, out) : cj::fail(CJ_ERR_STATE, "null engine");
}
int32_t cj_engine_decode_batch(int64_t h, const int32_t *slots, int32_t n, int32_t steps, int32_t *out) {
    Engine *e = eng_of(h);
    if (!e) return cj::fail(CJ_ERR_STATE, "null engine");
    if (!slots) return cj::fail(CJ_ERR_ARG, "cj_engine_decode_batch: no slots");
    return e->decode_batch(slots, n, steps, out);
}
int32_t cj_engine_set_cpu_threads(int64_t h, int32_t threads) {
    Engine *e = eng_of(h);
    if (!e) return cj::fail(CJ_ERR_STATE, "null engine");
    if (threads < 1 || threads > 65536) return cj::fail(CJ_ERR_ARG, "cpu threads %d (1..65536)", threads);
    if (threads == e->workers) return CJ_OK;
    CJ_HIP(hipStreamSynchronize(cj::stream()));
    e->workers = threads;
    // the captured steps hold the old split rule
    for (auto &sq : e->seqs)
        if (sq.graph) { (void)hipGraphExecDestroy(sq.graph); sq.graph = nullptr; }
    for (auto &g : e->batch_graphs)
        if (g) { (void)hipGraphExecDestroy(g); g = nullptr; }
    return CJ_OK;
}
int32_t cj_engine_set_prefill_chunk(int64_t h, int32_t rows) {
    Engine *e = eng_of(h);
    if (!e) return cj::fail(CJ_ERR_STATE, "null engine");
    if (rows < 0 || (rows > 1 && rows > e->rows_cap))
        return cj::fail(CJ_ERR_ARG, "prefill chunk %d (0..%d)", rows, e->rows_cap);
    e->chunk = rows;
    return CJ_OK;
}
int32_t cj_engine_logits(int64_t h, int32_t seq, float *out, int64_t n) {
    Engine *e = eng_of(h);
    if (!e || n > e->vocab) return cj::fail(CJ_ERR_ARG, "cj_engine_logits: n %lld", (long long)n);
    (void)seq;
    CJ_HIP(hipStreamSynchronize(cj::stream()));
    CJ_HIP(hipMemcpy(out, e->logits, (size_t)n * 4, hipMemcpyDeviceToHost));
    return CJ_OK;
}
int32_t cj_engine_preds(int64_t h, int32_t seq, int32_t *out, int32_t n) {
    Engine *e = eng_of(h);
    if (!e || seq < 0 || seq >= (int)e->seqs.size() || n > e->ctx) return cj::fail(CJ_ERR_ARG, "cj_engine_preds");
    CJ_HIP(hipStreamSynchronize(cj::stream()));
    CJ_HIP(hipMemcpy(out, e->seqs[seq].preds + 1, (size_t)n * 4, hipMemcpyDeviceToHost));
    return CJ_OK;
}
int32_t cj_engine_trace(int64_t h, int32_t what, float *out, int64_t n) {
    Engine *e = eng_of(h);
    if (!e || !out) return cj::fail(CJ_ERR_ARG, "cj_engine_trace: bad arguments");
    const int64_t qd = (int64_t)e->n_heads * e->head_dim;
    const float *src = nullptr;
    int64_t cap = 0;
    switch (what) {
    case 0: src = e->hs_last; cap = e->hidden; break;
    case 1: src = e->q; cap = qd; break;
    case 2: src = e->attn; cap = qd; break;
    case 3: src = e->act; cap = e->ffn; break;
    case 4: src = e->logits; cap = e->vocab; break;
    case 5: src = (const float *)e->act_pack; cap = ((int64_t)e->ffn + 255) / 256 * 80; break;
    case 6: src = e->r_logits; cap = e->r_logits ? (int64_t)e->batch_rows * e->vocab : 0; break;
    default: return cj::fail(CJ_ERR_ARG, "cj_engine_trace: unknown tap %d", what);
    }
    if (n > cap) return cj::fail(CJ_ERR_ARG, "cj_engine_trace: %lld > %lld", (long long)n, (long long)cap);
    CJ_HIP(hipStreamSynchronize(cj::stream()));
    CJ_HIP(hipMemcpy(out, src, (size_t)n * 4, hipMemcpyDeviceToHost));
    return CJ_OK;
}

float cj_engine_last_step_us(int64_t h) {
    Engine *e = eng_of(h);
    return e ? e->last_step_us : -1.0f;
}

int32_t cj_engine_time_kernel(int64_t h, int32_t seq, int32_t kind, int32_t reps, float *avg_us, int64_t *bytes,
                              int8_t *name, int32_t name_cap) {
    Engine *e = eng_of(h);
    if (!e || !avg_us || !bytes) return cj::fail(CJ_ERR_ARG, "cj_engine_time_kernel: bad arguments");
    std::string k;
    int rc = e->time_kind(seq, kind, reps, avg_us, k);
    if (rc) return rc;
    const int pos = e->seqs[seq].pos;
    const int w = e->layers.empty() ? 0 : e->layers[0].window;
    *bytes = e->kind_bytes(kind, w > 0 ? std::min(pos + 1, w) : pos + 1);
    if (name && name_cap > 0) {
        const size_t n = std::min<size_t>(k.size(), (size_t)name_cap - 1);
        memcpy(name, k.data(), n);
        name[n] = 0;
    }
    return CJ_OK;
}

int32_t cj_engine_time_kernel_in_step(int64_t h, int32_t seq, int32_t kind, int32_t steps, float *avg_us) {
    Engine *e = eng_of(h);
    if (!e || !avg_us) return cj::fail(CJ_ERR_ARG, "cj_engine_time_kernel_in_step: bad arguments");
    return e->time_in_step(seq, kind, steps, avg_us);
}

int32_t cj_engine_set_graphs(int64_t h, int32_t on) {
    Engine *e = eng_of(h);
    if (!e) return cj::fail(CJ_ERR_STATE, "null engine");
    e->graphs = on != 0;
    return CJ_OK;
}

int64_t cj_engine_step_bytes(int64_t h, int32_t count) {
    Engine *e = eng_of(h);
    if (!e || count <= 0) return cj::fail(CJ_ERR_ARG, "cj_engine_step_bytes: bad arguments");
    return e->step_bytes(count);
}

}  // extern "C"
