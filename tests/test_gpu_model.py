"""Model-level parity: the graph-captured decode step on the MI355X against
the CPU oracle's restatement of the reference CPU backend, on the same GGUF
bytes. Bars (the decode path's parity bar): greedy token ids identical; logits within
max-abs 1e-3 (f32 accumulation). A non-degeneracy control requires more than
one distinct generated token (T/BackendParityTest.cajeta:158-178)."""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(__file__), "golden", "gguf")
LOGIT_TOL = 1e-3


def say(*a):
    print(*a, flush=True)


def run_pair(pkg, path, image, prompt, n_gen, ctx, check_every=1, chunk=512, kv_f32=False):
    """Greedy-decode `prompt` + n_gen on both sides; compare every step. The
    prompt goes through each side's prefill (prefill chunks on dense head-size-
    128 models, decode steps otherwise). kv_f32: both sides keep f32 K/V."""
    from oracle.gguf_reader import GgufReader, oracle_model
    r = GgufReader(image if image is not None else path)
    om, cfg = oracle_model(r, ctx=ctx, kv_f32=kv_f32)
    opts = pkg.EngineOptions(path)
    opts.ctx = ctx
    opts.maxSeqs = 1
    opts.prefillChunk = chunk
    opts.kvF32 = kv_f32
    eng = pkg.LlmEngine.load(opts)
    try:
        eng.reset()
        eng.prefill(prompt)
        gpu_first = int(eng.preds(len(prompt))[-1])
        gpu_logits = [eng.logits()]
        gpu_toks = [gpu_first]
        for i in range(n_gen - 1):
            gpu_toks.append(int(eng.decode(1)[0]))
            if (i + 1) % check_every == 0:
                gpu_logits.append(eng.logits())
            else:
                gpu_logits.append(None)
        toks = list(prompt)
        t, lg = om.prefill(prompt, 0)
        ref_toks, ref_logits = [t], [lg]
        toks.append(t)
        for p in range(len(prompt), len(prompt) + n_gen - 1):
            t, lg = om.step(toks[p], p)
            ref_toks.append(t)
            ref_logits.append(lg)
            toks.append(t)
        worst, same = 0.0, True
        for g, o in zip(gpu_logits, ref_logits):
            if g is not None:
                worst = max(worst, float(np.max(np.abs(g - o))))
                same = same and np.array_equal(g.view(np.uint32), o.view(np.uint32))
        say("  logits max-abs %.3g, bit-identical %s" % (worst, same))
        run_pair.bit_identical = same
        return gpu_toks, ref_toks, worst
    finally:
        eng.close()
        om.close()


@pytest.mark.parametrize("name", ["toy-routable.gguf", "toy-routable-gqa8.gguf"])
def test_reference_toy_fixture_greedy_parity(gpu, name):
    say("model", name)
    rng = np.random.default_rng(5)
    prompt = rng.integers(0, 256, 12).tolist()
    g, o, err = run_pair(gpu, os.path.join(GOLD, name), None, prompt, 40, 256)
    assert g == o, "tokens differ: gpu %s oracle %s" % (g, o)
    assert err <= LOGIT_TOL, err
    assert len(set(g)) > 1


def test_split_gguf_decodes_as_the_whole_file(gpu, tmp_path):
    """The reference's toy GGUF split into three shards and loaded from the
    middle one decodes exactly as the oracle does on the unsplit file."""
    from gguf_split import split_gguf
    src = os.path.join(GOLD, "toy-routable.gguf")
    paths = split_gguf(src, str(tmp_path / "toy"), 3)
    rng = np.random.default_rng(7)
    prompt = rng.integers(0, 256, 10).tolist()
    g, o, err = run_pair(gpu, paths[1], src, prompt, 12, 256)
    assert g == o and run_pair.bit_identical, (g, o, err)


@pytest.mark.parametrize("key,moe", [("llama.feed_forward_length", False),
                                     ("llama.expert_feed_forward_length", True)])
def test_feed_forward_metadata_that_disagrees_with_the_tensors_is_refused(gpu, tmp_path, key, moe):
    """A GGUF whose FFN width key disagrees with its gate/up tensors' rows is
    refused by name at load, before any copy reads past a tensor."""
    spec = ("layers=1;hidden=256;heads=4;kv=2;hd=64;ffn=512;vocab=256;wtype=q8_0;head=q8_0;embd=q8_0;ctx=64" +
            (";experts=4;used=2;expert_ffn=512" if moe else ""))
    gpu.synth_gguf(spec, "mem:t_ffbad", 5)
    img = bytearray(gpu.image_bytes("t_ffbad").tobytes())
    gpu.image_free("t_ffbad")
    k = key.encode()
    at = img.find(len(k).to_bytes(8, "little") + k)
    assert at >= 0
    vt = at + 8 + len(k)
    assert int.from_bytes(img[vt:vt + 4], "little") == 4      # a u32 value
    img[vt + 4:vt + 8] = (768).to_bytes(4, "little")          # rows of gate/up stay 512
    path = tmp_path / "ffbad.gguf"
    path.write_bytes(bytes(img))
    opts = gpu.EngineOptions(str(path))
    opts.ctx, opts.maxSeqs = 64, 1
    with pytest.raises(gpu.LlmException) as e:
        gpu.LlmEngine.load(opts).close()
    assert "rows" in str(e.value), str(e.value)


def test_prefill_chunks_are_invisible(gpu):
    """A 45-token prompt as one chunk and as chunks of 7: chunking changes
    nothing (every row's arithmetic is the same), both against the oracle's
    prefill of the whole prompt."""
    say("prefill chunks")
    path = os.path.join(GOLD, "toy-routable.gguf")
    rng = np.random.default_rng(21)
    prompt = rng.integers(0, 256, 45).tolist()
    g1, o1, e1 = run_pair(gpu, path, None, prompt, 12, 256, chunk=512)
    b1 = run_pair.bit_identical
    g7, o7, e7 = run_pair(gpu, path, None, prompt, 12, 256, chunk=7)
    b7 = run_pair.bit_identical
    assert g1 == o1 and g7 == o7 and g1 == g7
    assert b1 and b7, (e1, e7)


def batch_case(gpu, path, image, prompts, steps, ctx, kv_f32=False):
    """Prefill every prompt into its own slot, decode all slots together;
    the oracle decodes each sequence alone with the batch's split rule."""
    from oracle.gguf_reader import GgufReader, oracle_model
    n = len(prompts)
    opts = gpu.EngineOptions(path)
    opts.ctx = ctx
    opts.maxSeqs = n
    opts.kvF32 = kv_f32
    eng = gpu.LlmEngine.load(opts)
    try:
        first = []
        for s, p in enumerate(prompts):
            eng.prefill(p, seq=s)
            first.append(int(eng.preds(len(p), seq=s)[-1]))
        out = eng.decodeBatch(list(range(n)), steps)
        last = eng.batchLogits()
    finally:
        eng.close()
    r = GgufReader(image if image is not None else path)
    worst, same = 0.0, True
    for s, p in enumerate(prompts):
        om, _ = oracle_model(r, ctx=ctx, attn_rows=n, kv_f32=kv_f32)
        t, _ = om.prefill(p, 0)
        toks, lg = [t], None
        for i in range(steps):
            t, lg = om.step(toks[-1], len(p) + i)
            toks.append(t)
        om.close()
        assert first[s] == toks[0], "slot %d first token" % s
        assert out[:, s].tolist() == toks[1:], "slot %d: gpu %s oracle %s" % (s, out[:, s].tolist(), toks[1:])
        worst = max(worst, float(np.max(np.abs(last[s] - lg))))
        same = same and np.array_equal(last[s].view(np.uint32), lg.view(np.uint32))
    say("  batch of %d: last-step logits max-abs %.3g, bit-identical %s" % (n, worst, same))
    return out, worst, same


@pytest.mark.parametrize("n", [3, 32])
def test_batched_decode_parity_toy_gqa8(gpu, n):
    """Batched decode (a row a sequence, the split rule over all rows' kv
    heads) on the reference's toy GGUF with 8 query heads a kv head."""
    say("batch toy gqa8", n)
    rng = np.random.default_rng(30 + n)
    prompts = [rng.integers(0, 256, int(rng.integers(2, 60))).tolist() for _ in range(n)]
    out, err, same = batch_case(gpu, os.path.join(GOLD, "toy-routable-gqa8.gguf"), None, prompts, 10, 256)
    assert err <= LOGIT_TOL and same
    assert len(set(out.ravel().tolist())) > 1


def synth(pkg, spec, name, seed):
    pkg.synth_gguf(spec, "mem:" + name, seed)
    return "mem:" + name, pkg.image_bytes(name)


def test_c1_config_literal_f32_kv_greedy_parity(gpu):
    """Benchmark configuration C1 as BASELINE.json states it: an f32 K/V cache (the
    reference's PagedKvCache mode) — 4 layers, d 512, 8/2 heads of 64, FFN 1408,
    V 32000, Q8_0, f32 embeddings; a 16-token prompt and 64 greedy tokens,
    logits bit for bit against the oracle's f32-K/V decode; then 5 slots
    decoding together in f32 K/V."""
    say("model c1 f32 K/V")
    path, img = synth(gpu, "c1", "t_c1f", 1234)
    rng = np.random.default_rng(11)
    prompt = rng.integers(0, 32000, 16).tolist()
    g, o, err = run_pair(gpu, path, img, prompt, 64, 128, kv_f32=True)
    assert g == o, "tokens differ at %d" % next(i for i, (a, b) in enumerate(zip(g, o)) if a != b)
    assert err <= LOGIT_TOL and run_pair.bit_identical, err
    assert len(set(g)) > 1
    prompts = [rng.integers(0, 32000, k).tolist() for k in (16, 3, 40, 9, 25)]
    out, err, same = batch_case(gpu, path, img, prompts, 6, 128, kv_f32=True)
    gpu.image_free("t_c1f")
    assert err <= LOGIT_TOL and same
    # the split-K models keep fp16 K/V: f32 is refused by name
    opts = gpu.EngineOptions(os.path.join(GOLD, "toy-routable.gguf"))
    opts.ctx = 64
    opts.maxSeqs = 1
    opts.kvF32 = True
    with pytest.raises(gpu.LlmException) as ex:
        gpu.LlmEngine.load(opts)
    assert "f32 K/V" in str(ex.value)


def test_c1_tiny_q8_0_greedy_parity(gpu):
    """Benchmark configuration C1: 4 layers, d 512, 8/2 heads of 64, FFN 1408, V 32000,
    Q8_0, f32 embeddings; 16-token prompt, 64 greedy tokens."""
    say("model c1")
    path, img = synth(gpu, "c1", "t_c1", 1234)
    rng = np.random.default_rng(11)
    prompt = rng.integers(0, 32000, 16).tolist()
    g, o, err = run_pair(gpu, path, img, prompt, 64, 128)
    gpu.image_free("t_c1")
    assert g == o, "tokens differ at %d" % next(i for i, (a, b) in enumerate(zip(g, o)) if a != b)
    assert err <= LOGIT_TOL, err
    assert len(set(g)) > 1
    # Q8_0 throughout and the two-pass attention: the same operations in the
    # same order as the restatement, so the logits are the same bits
    assert run_pair.bit_identical


def test_c3_shape_two_layers_greedy_parity(gpu):
    """Benchmark configuration C3's Llama-3-8B shapes (d 4096, 32/8 heads of 128, FFN
    14336, V 128256, Q4_K + Q6_K head, θ 500000) at two layers."""
    say("model c3x2")
    spec = "layers=2;hidden=4096;heads=32;kv=8;hd=128;ffn=14336;vocab=128256;eps=1e-5;theta=500000;" \
           "wtype=q4_k;head=q6_k;embd=q4_k;ctx=512"
    path, img = synth(gpu, spec, "t_c3x2", 77)
    rng = np.random.default_rng(3)
    prompt = rng.integers(0, 128256, 24).tolist()
    g, o, err = run_pair(gpu, path, img, prompt, 12, 256, check_every=3)
    gpu.image_free("t_c3x2")
    assert g == o
    assert err <= LOGIT_TOL, err
    assert run_pair.bit_identical


def test_in_step_timing_leaves_the_decode_unchanged(gpu):
    """The measurement seams (timing launches and in-step timing, which enqueue
    whole steps) leave the slot's state as it was: decoding on afterwards gives
    the tokens and logits of an engine that never timed anything."""
    say("in-step timing")
    spec = "layers=2;hidden=4096;heads=32;kv=8;hd=128;ffn=14336;vocab=128256;eps=1e-5;theta=500000;" \
           "wtype=q4_k;head=q6_k;embd=q4_k;ctx=256"
    path, img = synth(gpu, spec, "t_c3x2t", 79)
    prompt = np.random.default_rng(4).integers(0, 128256, 20).tolist()
    runs = []
    for timed in (False, True):
        opts = gpu.EngineOptions(path)
        opts.ctx, opts.maxSeqs = 256, 1
        eng = gpu.LlmEngine.load(opts)
        try:
            eng.reset()
            eng.prefill(prompt)
            toks = list(eng.decode(4))
            if timed:
                for kind in (1, 2, 3, 4, 5):
                    assert eng.timeKernelInStep(kind, 2) > 0.0
                assert eng.timeKernel(4, 8)[0] > 0.0
            toks += list(eng.decode(4))
            runs.append((toks, eng.logits()))
        finally:
            eng.close()
    gpu.image_free("t_c3x2t")
    assert runs[0][0] == runs[1][0]
    assert np.array_equal(runs[0][1].view(np.uint32), runs[1][1].view(np.uint32))


def test_c3_attention_at_the_benchmarked_context(gpu):
    """Benchmark configuration C3 at the context it is timed at: a 2048-token prompt
    through four 512-row prefill chunks, then 9 greedy steps at positions 2048 to
    2056 (2049 to 2057 keys a step), every step's logits bit for bit against the
    oracle, at the default 512 workers (64 splits a kv head) and at 16 (4
    splits, a 16-thread reference CPU run). The attention shapes are C3's (d 4096,
    32/8 heads of 128, θ 500000, Q4_K + Q6_K head, V 128256); two layers and a
    1024-wide FFN keep the oracle's 2048-row prefill to seconds, and the FFN
    width does not reach the context-dependent path (the 14336-wide FFN is
    checked above and at full depth)."""
    from oracle import oracle as O
    from oracle.gguf_reader import GgufReader, oracle_model
    say("model c3 ctx 2048")
    spec = "layers=2;hidden=4096;heads=32;kv=8;hd=128;ffn=1024;vocab=128256;eps=1e-5;theta=500000;" \
           "wtype=q4_k;head=q6_k;embd=q4_k;ctx=2304"
    path, img = synth(gpu, spec, "t_c3ctx", 91)
    rng = np.random.default_rng(21)
    prompt = rng.integers(0, 128256, 2048).tolist()
    n_gen, ctx = 9, 2304
    om, cfg = oracle_model(GgufReader(img), ctx=ctx)
    try:
        say("  oracle prefill of 2048 rows")
        first, first_lg = om.prefill(prompt, 0)
        ref = {}
        for w in (512, 16):
            # the KV planes of the prompt are kept; the steps overwrite 2048..
            om.set_workers(w)
            toks, lgs = [first], [first_lg]
            for p in range(len(prompt), len(prompt) + n_gen - 1):
                t, lg = om.step(toks[-1], p)
                toks.append(t)
                lgs.append(lg)
            ref[w] = (toks, lgs)
    finally:
        om.close()
    assert O.cpu_decode_splits(2049, 1, 8, 512) == 64 and O.cpu_decode_splits(2049, 1, 8, 16) == 4
    # the worker count reaches the logits' last bits: both counts are checked
    assert any(not np.array_equal(a.view(np.uint32), b.view(np.uint32)) for a, b in zip(ref[512][1], ref[16][1]))
    for w in (512, 16):
        say("  engine, %d workers" % w)
        opts = gpu.EngineOptions(path)
        opts.ctx, opts.maxSeqs, opts.cpuThreads = ctx, 1, w
        eng = gpu.LlmEngine.load(opts)
        try:
            eng.reset()
            eng.prefill(prompt)
            toks, lgs = [int(eng.preds(len(prompt))[-1])], [eng.logits()]
            for _ in range(n_gen - 1):
                toks.append(int(eng.decode(1)[0]))
                lgs.append(eng.logits())
        finally:
            eng.close()
        rt, rl = ref[w]
        assert toks == rt, (w, toks, rt)
        for i, (g, o) in enumerate(zip(lgs, rl)):
            assert np.array_equal(g.view(np.uint32), o.view(np.uint32)), \
                (w, i, float(np.max(np.abs(g - o))))
        assert len(set(toks)) > 1
    gpu.image_free("t_c3ctx")


@pytest.mark.parametrize("hd", [128, 64])
def test_rope_freqs_model_parity(gpu, hd):
    """A model carrying Llama-3.1's precomputed RoPE factors (`rope_freqs.weight`,
    hd/2 of them, 1 rising to 8 with a seeded wobble): every dimension's
    inverse frequency divided by its factor on both sides, through prefill
    chunks and decode steps, bit for bit."""
    say("model rope_freqs hd", hd)
    heads = 8 if hd == 128 else 16
    spec = "layers=2;hidden=1024;heads=%d;kv=2;hd=%d;ffn=2048;vocab=4096;eps=1e-5;theta=500000;" \
           "wtype=q4_k;head=q6_k;embd=q4_k;ctx=512;rope_freqs=1" % (heads, hd)
    path, img = synth(gpu, spec, "t_rf%d" % hd, 93)
    rng = np.random.default_rng(hd)
    prompt = rng.integers(0, 4096, 300).tolist()
    g, o, err = run_pair(gpu, path, img, prompt, 8, 512)
    gpu.image_free("t_rf%d" % hd)
    assert g == o
    assert run_pair.bit_identical, err


@pytest.mark.parametrize("heads,kv", [(8, 8), (8, 4), (16, 2)])
def test_prefill_attend_query_groups(gpu, heads, kv):
    """The prefill attend at head size 128 for 1, 2 and 8 query heads a kv
    head (the benchmark shapes have 4): a 300-token prompt through 128-row
    chunks (the last one partial), then decode steps, bit for bit."""
    say("prefill attend heads", heads, "kv", kv)
    name = "t_pfg%d" % (heads // kv)
    spec = "layers=1;hidden=1024;heads=%d;kv=%d;hd=128;ffn=1024;vocab=2048;eps=1e-5;theta=10000;" \
           "wtype=q8_0;head=q8_0;embd=q8_0;ctx=512" % (heads, kv)
    path, img = synth(gpu, spec, name, 95 + kv)
    rng = np.random.default_rng(heads * 10 + kv)
    prompt = rng.integers(0, 2048, 300).tolist()
    g, o, err = run_pair(gpu, path, img, prompt, 6, 512, chunk=128)
    gpu.image_free(name)
    assert g == o
    assert run_pair.bit_identical, err


def test_c4_shape_q8_0_two_layers_greedy_parity(gpu):
    """Benchmark configuration C4's Q8_0 weights on the 8B shapes, at two layers."""
    say("model c4x2")
    spec = "layers=2;hidden=4096;heads=32;kv=8;hd=128;ffn=14336;vocab=32000;eps=1e-5;theta=500000;" \
           "wtype=q8_0;head=q8_0;embd=q8_0;ctx=512"
    path, img = synth(gpu, spec, "t_c4x2", 78)
    rng = np.random.default_rng(4)
    prompt = rng.integers(0, 32000, 20).tolist()
    g, o, err = run_pair(gpu, path, img, prompt, 10, 256, check_every=3)
    gpu.image_free("t_c4x2")
    assert g == o
    assert err <= LOGIT_TOL, err
    assert run_pair.bit_identical


def test_c4_shape_q8_0_batched_decode_parity(gpu):
    """Benchmark configuration C4's batched decode at small scale: Q8_0 8B shapes at two
    layers, three sequences at different positions decoded together."""
    say("model c4x2 batch")
    spec = "layers=2;hidden=4096;heads=32;kv=8;hd=128;ffn=14336;vocab=32000;eps=1e-5;theta=500000;" \
           "wtype=q8_0;head=q8_0;embd=q8_0;ctx=512"
    path, img = synth(gpu, spec, "t_c4x2b", 81)
    rng = np.random.default_rng(8)
    prompts = [rng.integers(0, 32000, k).tolist() for k in (7, 30, 65)]
    out, err, same = batch_case(gpu, path, img, prompts, 6, 160)
    gpu.image_free("t_c4x2b")
    assert err <= LOGIT_TOL and same


def test_c5_moe_shape_two_layers_greedy_parity(gpu):
    """Benchmark configuration C5's gpt-oss-20b shapes (d 2880, 64/8 heads of 64, 32
    MXFP4 experts top-4 of FFN 2880, alternating 128-window attention) at two
    layers and a 32000 vocabulary."""
    say("model c5x2")
    spec = "layers=2;hidden=2880;heads=64;kv=8;hd=64;ffn=2880;vocab=32000;eps=1e-5;theta=150000;wtype=q8_0;" \
           "head=q8_0;embd=q8_0;experts=32;used=4;expert_ffn=2880;expert_type=mxfp4;swa=128;ctx=512"
    path, img = synth(gpu, spec, "t_c5x2", 79)
    rng = np.random.default_rng(6)
    prompt = rng.integers(0, 32000, 140).tolist()          # past the 128 window
    g, o, err = run_pair(gpu, path, img, prompt, 10, 256, check_every=3)
    gpu.image_free("t_c5x2")
    assert g == o
    assert err <= LOGIT_TOL, err
    assert run_pair.bit_identical


@pytest.mark.parametrize("expert_type", ["q8_0", "q4_0", "q4_k", "q6_k"])
def test_moe_expert_formats_greedy_and_batched_parity(gpu, expert_type):
    """MoE experts in the other GEMV formats (the benchmark models use MXFP4):
    Q8_0, Q4_K and Q6_K over int8 packs, Q4_0 over the f32 rows through the
    block-parallel GEMV, all indirected over the selections; 8 experts top-2
    at d 512, one sequence and a batch of three against the oracle, bit for
    bit."""
    say("model moe experts", expert_type)
    spec = ("layers=2;hidden=512;heads=8;kv=2;hd=64;ffn=512;vocab=2048;eps=1e-5;theta=10000;wtype=q8_0;"
            "head=q8_0;embd=q8_0;experts=8;used=2;expert_ffn=512;expert_type=%s;ctx=256" % expert_type)
    name = "t_moe_" + expert_type
    path, img = synth(gpu, spec, name, 91)
    rng = np.random.default_rng(23)
    prompt = rng.integers(0, 2048, 9).tolist()
    g, o, err = run_pair(gpu, path, img, prompt, 12, 128)
    assert g == o and run_pair.bit_identical, (g, o, err)
    prompts = [rng.integers(0, 2048, k).tolist() for k in (4, 11, 7)]
    out, err, same = batch_case(gpu, path, img, prompts, 5, 128)
    gpu.image_free(name)
    assert err <= LOGIT_TOL and same
    assert len(set(out.ravel().tolist())) > 1


def test_c3_shape_batched_decode_parity(gpu):
    """Benchmark configuration C3's formats in a batch: Q4_K projections on the int8
    matrix cores and the Q6_K head as the many-column GEMV, 5 slots at
    different positions, against the oracle decoding each alone."""
    say("model c3x2 batch 5")
    spec = "layers=2;hidden=4096;heads=32;kv=8;hd=128;ffn=14336;vocab=32000;eps=1e-5;theta=500000;" \
           "wtype=q4_k;head=q6_k;embd=q4_k;ctx=512"
    path, img = synth(gpu, spec, "t_c3x2b", 84)
    rng = np.random.default_rng(19)
    prompts = [rng.integers(0, 32000, k).tolist() for k in (5, 12, 40, 3, 70)]
    out, err, same = batch_case(gpu, path, img, prompts, 6, 160)
    gpu.image_free("t_c3x2b")
    assert err <= LOGIT_TOL and same
    assert len(set(out.ravel().tolist())) > 1


def test_c5_moe_shape_batched_decode_parity(gpu):
    """Benchmark configuration C5's batch-16 decode at two layers: 16 slots (two past the
    128 window) decode together — one router product and one top-k over the
    rows, one indirected gate|up and one down launch over all 64 selections,
    the two-pass attention as rows — every slot's tokens and last logits bit
    for bit against the oracle decoding it alone. The prompts go through
    prefill chunks of decode-attention rows."""
    say("model c5x2 batch 16")
    spec = "layers=2;hidden=2880;heads=64;kv=8;hd=64;ffn=2880;vocab=32000;eps=1e-5;theta=150000;wtype=q8_0;" \
           "head=q8_0;embd=q8_0;experts=32;used=4;expert_ffn=2880;expert_type=mxfp4;swa=128;ctx=512"
    path, img = synth(gpu, spec, "t_c5x2b", 83)
    rng = np.random.default_rng(16)
    lens = [int(rng.integers(2, 40)) for _ in range(14)] + [131, 150]
    prompts = [rng.integers(0, 32000, k).tolist() for k in lens]
    out, err, same = batch_case(gpu, path, img, prompts, 6, 256)
    gpu.image_free("t_c5x2b")
    assert err <= LOGIT_TOL and same
    assert len(set(out.ravel().tolist())) > 1


def test_c1_batched_decode_parity(gpu):
    """Benchmark configuration C1's shapes (head size 64, 4 query heads a kv head, the
    tanh-form GLU of the 1408-wide FFN) as a batch of 8 slots: the two-pass
    attention rows, every slot against the oracle decoding it alone."""
    say("model c1 batch 8")
    path, img = synth(gpu, "c1", "t_c1b", 1235)
    rng = np.random.default_rng(17)
    prompts = [rng.integers(0, 32000, int(rng.integers(2, 30))).tolist() for _ in range(8)]
    out, err, same = batch_case(gpu, path, img, prompts, 8, 128)
    gpu.image_free("t_c1b")
    assert err <= LOGIT_TOL and same
    assert len(set(out.ravel().tolist())) > 1


def test_c3_full_depth_greedy_parity(gpu):
    """Benchmark configuration C3 at its full depth (32 layers, the benchmarked model):
    a 40-token prompt through the prefill chunk, then 6 greedy steps; every
    step's logits bit for bit against the oracle."""
    say("model c3 full")
    path, img = synth(gpu, "c3", "t_c3full", 1)
    rng = np.random.default_rng(12)
    prompt = rng.integers(0, 128256, 40).tolist()
    g, o, err = run_pair(gpu, path, img, prompt, 7, 64)
    gpu.image_free("t_c3full")
    assert g == o
    assert err <= LOGIT_TOL, err
    assert run_pair.bit_identical


def test_c5_full_depth_greedy_parity(gpu):
    """Benchmark configuration C5 at its full depth (24 layers, 32 MXFP4 experts top-4,
    the 201,088 vocabulary): a 130-token prompt (past the 128 window) and 4
    greedy steps, logits bit for bit against the oracle."""
    say("model c5 full")
    path, img = synth(gpu, "c5", "t_c5full", 1)
    rng = np.random.default_rng(13)
    prompt = rng.integers(0, 201088, 130).tolist()
    g, o, err = run_pair(gpu, path, img, prompt, 5, 160, check_every=2)
    gpu.image_free("t_c5full")
    assert g == o
    assert err <= LOGIT_TOL, err
    assert run_pair.bit_identical


def oracle_stream(r, prompt, n_gen, ctx, stops=()):
    """The oracle's greedy continuation of `prompt`: the prompt through its
    prefill, then decode steps until n_gen ids or a stop token."""
    from oracle.gguf_reader import oracle_model
    om, _ = oracle_model(r, ctx=ctx)
    t, _ = om.prefill(prompt, 0)
    toks = [t]
    while len(toks) < n_gen and t not in stops:
        t, _ = om.step(toks[-1], len(prompt) + len(toks) - 1)
        toks.append(t)
    om.close()
    return toks


def test_scheduler_steps_interleave_requests_like_the_oracle(gpu):
    """LlmEngine.stepOnce is one scheduler step (Scheduler.stepOnce): with two
    sequence slots, four requests are admitted FIFO as slots free, decode
    together in batched steps, stop on their budget or a stop token, and a
    cancel between steps freezes one; every token stream equals the oracle's
    greedy continuation of that prompt alone."""
    from oracle.gguf_reader import GgufReader
    path = os.path.join(GOLD, "toy-routable-gqa8.gguf")
    r = GgufReader(path)
    ctx = 96
    P = gpu.Request
    prompts = {"a": [1, 2, 3, 4], "b": [5, 6, 7, 8, 9, 10, 11], "c": [9, 9, 40], "d": [3, 1, 4, 1, 5]}
    budget = {"a": 10, "b": 6, "c": 8, "d": 12}
    want = {k: oracle_stream(r, prompts[k], budget[k], ctx) for k in prompts}
    opts = gpu.EngineOptions(path)
    opts.ctx = ctx
    opts.maxSeqs = 2
    eng = gpu.LlmEngine.load(opts)
    try:
        ids = {k: eng.submitTokens(prompts[k], maxNew=budget[k], params=gpu.SampleParams(stopTokens=[]))
               for k in ("a", "b", "c", "d")}
        assert [ids[k] for k in "abcd"] == [0, 1, 2, 3]
        assert eng.request(ids["a"]).state == P.WAITING
        more, steps, seen_running = True, 0, []
        while more:
            more = eng.stepOnce()
            steps += 1
            st = {k: eng.request(ids[k]) for k in ids}
            seen_running.append(sorted(k for k in st if st[k].state == P.RUNNING))
            if steps == 1:
                # two slots: a and b admitted, the others wait
                assert st["a"].state == P.RUNNING and st["b"].state == P.RUNNING
                assert st["c"].state == P.WAITING and st["d"].state == P.WAITING
                assert len(st["a"].tokens) == 1 and len(st["b"].tokens) == 1
            if steps == 3:
                assert eng.cancel(ids["d"])          # a waiting request never admits
                assert not eng.cancel(ids["d"])      # already done
            if steps == 8:
                assert st["c"].state == P.RUNNING   # admitted in the step b finished
                assert eng.cancel(ids["a"])          # a running one: frozen where it is
            assert steps < 200
        got = {k: eng.request(ids[k]) for k in ids}
        say("  scheduler: %d steps; running sets %s" % (steps, seen_running))
        assert got["b"].tokens == want["b"] and got["b"].finishReason == P.FINISH_BUDGET
        assert got["c"].tokens == want["c"] and got["c"].finishReason == P.FINISH_BUDGET
        assert got["d"].tokens == [] and got["d"].finishReason == P.FINISH_CANCEL
        assert got["a"].finishReason == P.FINISH_CANCEL and len(got["a"].tokens) == 8
        assert got["a"].tokens == want["a"][:8]
        assert not eng.cancel(99)                    # never issued
        # a stop token ends the stream on that token (FINISH_EOS)
        stop = want["a"][3]
        e = eng.submitTokens(prompts["a"], maxNew=10, params=gpu.SampleParams(stopTokens=[stop]))
        eng.runAll(100)
        re_ = eng.request(e)
        assert re_.finishReason == P.FINISH_EOS and re_.tokens == want["a"][:want["a"].index(stop) + 1]
        # the model's end-of-generation set is the default stop set
        eng.setEog([stop])
        f = eng.submitTokens(prompts["a"], maxNew=10)
        eng.runAll(100)
        assert eng.request(f).tokens == re_.tokens
        with pytest.raises(gpu.LlmException):
            eng.submitTokens([1, 2], maxNew=2, params=gpu.SampleParams(temperature=0.7))
        with pytest.raises(gpu.LlmException):
            eng.submitTokens(list(range(ctx)), maxNew=2)   # no decode position left in a slot
    finally:
        eng.close()


def sched_run(pkg, eng, prompts, budgets, stops=None, watch=None):
    """Submit every prompt, step until done; returns {key: Request}. watch(step,
    states) sees every step's request states."""
    ids = {}
    for k in prompts:
        st = [] if stops is None or k not in stops else stops[k]
        ids[k] = eng.submitTokens(prompts[k], maxNew=budgets[k], params=pkg.SampleParams(stopTokens=st))
    steps, more = 0, True
    while more:
        more = eng.stepOnce()
        steps += 1
        if watch:
            watch(steps, {k: eng.request(ids[k]) for k in ids})
        assert steps < 2000
    return {k: eng.request(ids[k]) for k in ids}


def test_scheduler_feeds_the_prompt_row_a_chunk_left(gpu):
    """A prompt one row longer than whole prefill chunks (chunk + 1, 2·chunk + 1):
    its last prompt row is fed from the host in the next step, not taken for a
    decode row (the chunk's pick has already written its own guess into that
    position), so every stream equals the oracle's greedy continuation."""
    from oracle.gguf_reader import GgufReader
    path = os.path.join(GOLD, "toy-routable-gqa8.gguf")
    r = GgufReader(path)
    ctx = 96
    prompts = {"a": [1, 2, 3, 4, 5], "b": [5, 6, 7, 8, 9, 10, 11, 12, 13], "c": [9, 9, 40, 7]}
    budget = {"a": 6, "b": 5, "c": 7}
    want = {k: oracle_stream(r, prompts[k], budget[k], ctx) for k in prompts}
    opts = gpu.EngineOptions(path)
    opts.ctx = ctx
    opts.maxSeqs = 3
    opts.prefillChunk = 4
    eng = gpu.LlmEngine.load(opts)
    try:
        got = sched_run(gpu, eng, prompts, budget)
        for k in prompts:
            assert got[k].tokens == want[k], (k, got[k].tokens, want[k])
        # alone (the pipelined step takes over once its prompt is in)
        e = eng.submitTokens(prompts["b"], maxNew=5, params=gpu.SampleParams(stopTokens=[]))
        eng.runAll(100)
        assert eng.request(e).tokens == want["b"]
    finally:
        eng.close()


def test_scheduler_pipelines_a_sole_greedy_request(gpu):
    """A sole running greedy request takes the pipelined step
    (Scheduler.stepPipelined): the seed step queues a decode step and emits no
    token, each later step queues the next before reading the last, a stop
    token ends the stream on that token (the queued step drained) and a budget
    on its last token; a second request arriving mid-stream finishes the
    pipeline and both go on batched. Every stream equals the oracle's."""
    from oracle.gguf_reader import GgufReader
    path = os.path.join(GOLD, "toy-routable.gguf")
    r = GgufReader(path)
    ctx = 128
    P = gpu.Request
    prompt = [7, 3, 99, 12, 1, 200]
    want = oracle_stream(r, prompt, 20, ctx)
    opts = gpu.EngineOptions(path)
    opts.ctx = ctx
    opts.maxSeqs = 2
    eng = gpu.LlmEngine.load(opts)
    try:
        counts = []
        got = sched_run(gpu, eng, {"a": prompt}, {"a": 9}, watch=lambda s, st: counts.append(len(st["a"].tokens)))
        assert got["a"].tokens == want[:9] and got["a"].finishReason == P.FINISH_BUDGET
        # prefill emits token 1; the seed emits none; then one a step
        assert counts[:4] == [1, 1, 2, 3], counts
        stop = want[5]
        got = sched_run(gpu, eng, {"a": prompt}, {"a": 20}, stops={"a": [stop]})
        assert got["a"].finishReason == P.FINISH_EOS and got["a"].tokens == want[:want.index(stop) + 1]
        # a second request mid-stream: the pipeline's pending token is consumed, then batched steps
        other = [4, 4, 8]
        want_b = oracle_stream(r, other, 6, ctx)
        a = eng.submitTokens(prompt, maxNew=12, params=gpu.SampleParams(stopTokens=[]))
        for _ in range(5):
            eng.stepOnce()
        b = eng.submitTokens(other, maxNew=6, params=gpu.SampleParams(stopTokens=[]))
        eng.runAll(200)
        assert eng.request(a).tokens == want[:12]
        assert eng.request(b).tokens == want_b
        # cancel while a step is in flight
        c = eng.submitTokens(prompt, maxNew=15, params=gpu.SampleParams(stopTokens=[]))
        for _ in range(4):
            eng.stepOnce()
        n = len(eng.request(c).tokens)
        assert eng.cancel(c)
        rc = eng.request(c)
        assert rc.finishReason == P.FINISH_CANCEL and rc.tokens == want[:n]
    finally:
        eng.close()


def test_scheduler_preempts_when_the_kv_pool_runs_dry(gpu):
    """A K/V pool smaller than every slot at full context (CausalLM's
    numBlocks): when a request's next rows do not fit, the youngest running
    request is preempted (Scheduler.preempt), its pages freed, and it resumes
    later by recomputing its whole stream. On a head-size-64 model the
    recompute's prefill rows run the decode step's attention, so every
    stream equals the oracle's uninterrupted greedy continuation; a request
    that cannot fit the pool with nothing else running is refused."""
    say("scheduler preemption")
    spec = ("layers=2;hidden=256;heads=4;kv=2;hd=64;ffn=512;vocab=512;eps=1e-5;theta=10000;wtype=q8_0;"
            "head=q8_0;embd=q8_0;ctx=256")
    path, img = synth(gpu, spec, "t_preempt", 17)
    from oracle.gguf_reader import GgufReader
    r = GgufReader(img)
    ctx = 256
    rng = np.random.default_rng(31)
    prompts = {k: rng.integers(0, 512, n).tolist() for k, n in (("a", 50), ("b", 40), ("c", 30))}
    budget = {"a": 60, "b": 70, "c": 50}
    want = {k: oracle_stream(r, prompts[k], budget[k], ctx) for k in prompts}
    opts = gpu.EngineOptions(path)
    opts.ctx = ctx
    opts.maxSeqs = 3
    opts.kvBlocks = 5           # 320 positions for three streams of 100-120
    eng = gpu.LlmEngine.load(opts)
    P = gpu.Request
    try:
        seen = set()
        got = sched_run(gpu, eng, prompts, budget,
                        watch=lambda s, st: seen.update(k for k in st if st[k].state == P.PREEMPTED))
        assert seen, "no request was preempted"
        say("  preempted: %s" % sorted(seen))
        for k in prompts:
            assert got[k].tokens == want[k], k
            assert got[k].finishReason == P.FINISH_BUDGET
    finally:
        eng.close()
    opts.kvBlocks = 2           # 128 positions: a 200-token prompt never fits
    eng = gpu.LlmEngine.load(opts)
    try:
        eng.submitTokens(rng.integers(0, 512, 200).tolist(), maxNew=4, params=gpu.SampleParams(stopTokens=[]))
        with pytest.raises(gpu.LlmException) as ex:
            eng.runAll(50)
        assert "pool" in str(ex.value)
    finally:
        eng.close()
        gpu.image_free("t_preempt")


def test_router_status_is_raised_by_batched_and_row_paths(gpu, tmp_path):
    """A MoE router whose logits are not finite raises in the call that
    routed them (MoeFfn.routeFromLogits throws): the embedding row of the
    token the model predicts first is made NaN, so the prefill is clean and
    the first decode routes NaN — through the batched decode (decodeBatch and
    stepOnce) and through prefill rows (a prompt holding that token)."""
    say("router status")
    spec = ("layers=2;hidden=512;heads=8;kv=2;hd=64;ffn=512;vocab=1024;eps=1e-5;theta=10000;wtype=q8_0;"
            "head=q8_0;embd=q8_0;experts=8;used=2;expert_ffn=512;expert_type=q8_0;ctx=128")
    path, img = synth(gpu, spec, "t_nanroute", 41)
    prompt = [3, 17, 250, 9, 77]
    opts = gpu.EngineOptions(path)
    opts.ctx = 128
    opts.maxSeqs = 2
    eng = gpu.LlmEngine.load(opts)
    eng.reset()
    eng.prefill(prompt)
    t0 = int(eng.preds(len(prompt))[-1])
    eng.close()
    assert t0 not in prompt
    from oracle.gguf_reader import GgufReader
    buf = np.array(img, np.uint8)
    gpu.image_free("t_nanroute")
    rd = GgufReader(buf)
    ty, dims, rows, cols, data = rd.tensors["token_embd.weight"]
    rb = cols // 32 * 34
    row = data[t0 * rb:(t0 + 1) * rb].reshape(-1, 34)
    row[:, 0:2] = np.frombuffer(np.float16(np.nan).tobytes(), np.uint8)   # every block scale NaN
    f = tmp_path / "nanroute.gguf"
    buf.tofile(str(f))
    opts = gpu.EngineOptions(str(f))
    opts.ctx = 128
    opts.maxSeqs = 2
    eng = gpu.LlmEngine.load(opts)
    try:
        for s in (0, 1):
            eng.reset(s)
            eng.prefill(prompt, s)
        with pytest.raises(gpu.LlmException) as ex:
            eng.decodeBatch([0, 1], 1)
        assert "not finite" in str(ex.value)
        eng.reset(0)
        with pytest.raises(gpu.LlmException):
            eng.prefill(prompt + [t0, 5], 0)         # prefill rows route the NaN row
        eng.reset(0)
        eng.reset(1)
        for _ in range(2):
            eng.submitTokens(prompt, maxNew=4, params=gpu.SampleParams(stopTokens=[]))
        with pytest.raises(gpu.LlmException):
            eng.runAll(20)
    finally:
        eng.close()
