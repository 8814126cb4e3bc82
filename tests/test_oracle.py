"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each restated function is checked against something other than its own
formula: the reference's golden vectors (dequant), IEEE/numpy (fp16),
closed forms and invariants (packs, argmax, splits, row permutation) and a
float64 brute force (GEMVs, RMSNorm, RoPE, SiLU, attention, routing, and a
whole toy-model forward). test_planted_mistakes_are_caught rebuilds the
oracle with one deliberate mistake at a time (OR_PLANT) and shows the check
for that function fails on it.

Runs on the CPU (no GPU marker)."""
import math
import os
import struct
import subprocess

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
GOLD = os.path.join(HERE, "golden")


# ------------------------------------------------------------------ helpers

def rand_blocks(O, ty, nblocks, rng):
    """Valid random blocks of a format: random bytes with sane scales."""
    be, bb = O.BLOCK[ty]
    raw = rng.integers(0, 256, size=(nblocks, bb), dtype=np.uint8)

    def f16(vals):
        return np.asarray(vals, np.float16).view(np.uint8).reshape(-1, 2)
    if ty in (O.Q8_0, O.Q4_0):
        raw[:, 0:2] = f16(rng.uniform(0.001, 0.01, nblocks))
    elif ty == O.Q4_K:
        raw[:, 0:2] = f16(rng.uniform(0.0005, 0.002, nblocks))
        raw[:, 2:4] = f16(rng.uniform(0.0005, 0.002, nblocks))
    elif ty == O.Q6_K:
        raw[:, 208:210] = f16(rng.uniform(0.0001, 0.001, nblocks))
    elif ty == O.MXFP4:
        raw[:, 0] = rng.integers(118, 126, nblocks)
    return raw.reshape(-1)


def unpack(O, xp, n, per32):
    """The values a 320-byte pack stands for: q · scale (block layout of
    Quant.q8kPackPad / q8kPack32Pad: 256 int8, 8 int32 sums, scale(s) at 288)."""
    out = np.zeros(n, np.float64)
    for b in range((n + 255) // 256):
        blk = xp[b * 320:(b + 1) * 320]
        q = blk[:256].view(np.int8).astype(np.float64)
        if per32:
            s = np.repeat(blk[288:320].view(np.float32).astype(np.float64), 32)
        else:
            s = np.full(256, blk[288:292].view(np.float32)[0], np.float64)
        m = min(256, n - 256 * b)
        out[256 * b:256 * b + m] = (q * s)[:m]
    return out


def golden(name):
    d = os.path.join(GOLD, "kquant")
    return np.fromfile(os.path.join(d, name + ".bin"), np.uint8), np.fromfile(os.path.join(d, name + ".f32"), np.float32)


def rel_err(got, ref):
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / (np.max(np.abs(ref)) + 1e-30))


# ------------------------------------------------- checks (also run on plants)

def check_dequant_golden(O):
    """Dequant of the reference's golden blocks (gguf-py of real Llama-3.1-8B
    blocks, F/gguf/kquant) is bit-exact."""
    bad = []
    for name, ty in (("q4_k", O.Q4_K), ("q6_k", O.Q6_K), ("q8_0", O.Q8_0), ("q4_0", O.Q4_0)):
        raw, ref = golden(name)
        got = O.dequant(ty, raw)
        if not np.array_equal(got.view(np.uint32), ref.view(np.uint32)):
            bad.append(name)
    b = open(os.path.join(GOLD, "mxfp4", "mxfp4_ref.bin"), "rb").read()
    _, nb = struct.unpack("<ii", b[:8])
    raw = np.frombuffer(b[8:8 + nb * 17], np.uint8)
    ref = np.frombuffer(b[8 + nb * 17:], np.float32)
    if not np.array_equal(O.dequant(O.MXFP4, raw).view(np.uint32), ref.view(np.uint32)):
        bad.append("mxfp4")
    return not bad, bad


def check_matvec(O, ty, rows=24, cols=1024, seed=3):
    """GEMV against a float64 product of the dequantised weights with the
    values the activation pack stands for (the int8 formats) or with x (the
    f32-activation formats): only fp32 accumulation rounding may differ."""
    rng = np.random.default_rng(seed + ty)
    be, bb = O.BLOCK[ty]
    if ty == O.F32:          # the MoE router's plain f32 rows
        raw = rng.standard_normal(rows * cols).astype(np.float32).view(np.uint8)
    else:
        raw = rand_blocks(O, ty, rows * cols // be, rng)
    x = rng.standard_normal(cols).astype(np.float32)
    W = O.dequant(ty, raw).astype(np.float64).reshape(rows, cols)
    if ty in (O.Q4_0, O.MXFP4, O.F32):
        got = O.matvec(ty, raw, rows, cols, x)
        ref = W @ x.astype(np.float64)
    else:
        per32 = ty == O.Q8_0
        xp = O.q8k_pack(x, per32=per32)
        got = O.matvec_packed(ty, raw, rows, cols, xp)
        ref = W @ unpack(O, xp, cols, per32)
    e = rel_err(got, ref)
    return e < 2e-6, e


def check_mxfp4_q8(O):
    """The MXFP4 device Q8 form. The activation quant: closed forms (the
    block maximum maps to ±127, exact halves away from zero, an all-zero
    block to zeros with scale 0) and, on random blocks, every value within
    half a step of its code. The mat-vec: against a float64 product of the
    dequantised weights (pinned by mxfp4_ref.bin) with the values the codes
    stand for — only f32 accumulation rounding may differ — and against the
    unquantised x within the quantisation bound Σ|w|·d/2."""
    bad = []
    x = np.zeros(96, np.float32)
    x[0], x[1], x[2], x[3], x[4] = 127.0, 2.5, -2.5, 0.5, -126.5
    x[33], x[40] = -254.0, 127.0          # block 1: scale 2, 127 -> 63.5 -> 64
    xq, xd = O.mxfp4_quant_act(x)
    if list(xq[:5]) != [127, 3, -3, 1, -127] or xd[0] != np.float32(1.0):
        bad.append(("block 0", list(xq[:5]), float(xd[0])))
    if xq[33] != -127 or xq[40] != 64 or xd[1] != np.float32(2.0):
        bad.append(("block 1", int(xq[33]), int(xq[40]), float(xd[1])))
    if np.any(xq[64:]) or xd[2] != 0.0:
        bad.append(("zero block", float(xd[2])))
    rng = np.random.default_rng(39)
    for rows, cols in ((24, 2880), (8, 32), (5, 1056), (3, 4096)):
        xr = (rng.standard_normal(cols) * rng.uniform(0.1, 10, cols // 32).repeat(32)).astype(np.float32)
        xq, xd = O.mxfp4_quant_act(xr)
        step = np.repeat(xd.astype(np.float64), 32)
        xhat = xq.astype(np.float64) * step
        if np.max(np.abs(xhat - xr) - step / 2) > 1e-6 * np.max(np.abs(xr)) or \
                np.any(np.abs(xq.reshape(-1, 32)).max(1) != 127):
            bad.append(("quant bound", cols))
        raw = rand_blocks(O, O.MXFP4, rows * cols // 32, rng)
        W = O.dequant(O.MXFP4, raw).astype(np.float64).reshape(rows, cols)
        got = O.matvec_mxfp4_q8(raw, rows, cols, xr)
        e = rel_err(got, W @ xhat)
        if e > 2e-6:
            bad.append(("dot", rows, cols, e))
        lim = np.abs(W) @ (step / 2) + 1e-5 * np.max(np.abs(W @ xhat))
        if np.any(np.abs(got - W @ xr.astype(np.float64)) > lim):
            bad.append(("bound", rows, cols))
    return not bad, bad


def check_rmsnorm(O):
    bad = []
    for n, scale in ((4096, 1.0), (2880, 1.0), (512, 3e-3)):   # the last: eps matters
        rng = np.random.default_rng(n)
        x = (rng.standard_normal(n) * scale).astype(np.float32)
        w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        for form in (0, 1):
            got = O.rmsnorm(x, w, 1e-5, form)
            xd = x.astype(np.float64)
            wd = w.astype(np.float64) + (1.0 if form else 0.0)
            ref = xd / np.sqrt(np.mean(xd * xd) + 1e-5) * wd
            e = rel_err(got, ref)
            if e > 1e-6:
                bad.append((n, form, e))
    return not bad, bad


def check_rope(O):
    bad = []
    for hd, theta, pos in ((128, 500000.0, 2047), (64, 10000.0, 37), (128, 10000.0, 0)):
        rng = np.random.default_rng(hd + pos)
        nh = 3
        t = rng.standard_normal(nh * hd).astype(np.float32)
        inv = O.inv_freq(hd, theta)
        got = O.rope(t.copy(), nh, hd, pos, inv)
        half = hd // 2
        invd = theta ** (-np.arange(half, dtype=np.float64) * 2.0 / hd)
        ang = pos * invd
        z = t.reshape(nh, hd).astype(np.float64)
        zc = (z[:, :half] + 1j * z[:, half:]) * np.exp(1j * ang)
        ref = np.concatenate([zc.real, zc.imag], axis=1).ravel()
        e = rel_err(got, ref)
        if e > 2e-5 or (pos == 0 and not np.array_equal(got, t)):
            bad.append((hd, pos, e))
    return not bad, bad


def check_rope_freqs(O):
    """A model's rope_freqs factors: each inverse frequency θ^(−2d/hd)
    divided by its factor (a zero factor leaves it), against float64; a
    count other than hd/2 refused."""
    bad = []
    for hd, theta in ((128, 500000.0), (64, 10000.0)):
        half = hd // 2
        c = dict(n_layers=1, hidden=hd, n_heads=1, n_kv=1, head_dim=hd, ffn=256, vocab=8, ctx=8, eps=1e-5,
                 theta=theta, kv_f32=0, workers=512, n_experts=0, n_used=0, norm_topk=1, expert_ffn=256,
                 swa_window=0, attn_rows=0, w_scale=0.0, swa_pattern=2)
        m = O.Model(c)
        rng = np.random.default_rng(hd)
        f = (1.0 + 7.0 * np.arange(half) / (half - 1)) * (1.0 + 0.05 * rng.standard_normal(half))
        f = f.astype(np.float32)
        f[3] = 0.0
        m.set_rope_freqs(f)
        got = m.trace(5, half).astype(np.float64)
        ref = theta ** (-np.arange(half, dtype=np.float64) * 2.0 / hd)
        ref = np.where(f != 0, ref / np.where(f != 0, f.astype(np.float64), 1.0), ref)
        e = float(np.max(np.abs(got - ref) / ref))
        if e > 1e-6:
            bad.append((hd, e))
        try:
            m.set_rope_freqs(f[:-1])
            bad.append((hd, "short factor list accepted"))
        except ValueError:
            pass
        m.close()
    return not bad, bad


def check_argmax(O):
    v = np.array([0.5, 3.0, -1.0, 3.0, 2.0, 3.0], np.float32)
    cases = [(v, 1), (np.zeros(7, np.float32), 0), (np.array([-5, -2, -2], np.float32), 1)]
    bad = [(list(a), O.argmax(a), want) for a, want in cases if O.argmax(a) != want]
    return not bad, bad


def check_glu_structure(O):
    """gluCpuKernel: 16-wide tanh chunks across each 4096-wide work block, the
    block's remainder in the exp form; tanh form within 4e-6 of the exp form
    (the reference's stated bound for its rational tanh)."""
    rng = np.random.default_rng(5)
    n = 4096 + 4096 + 40            # two whole blocks, then 40 (two chunks + 8)
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    t = O.glu(g, u, "tanh")
    ex = O.glu(g, u, "exp")
    tail = slice(8192 + 32, n)
    same_tail = np.array_equal(t[tail].view(np.uint32), ex[tail].view(np.uint32))
    # inside whole chunks the rational form is used: it differs from exp somewhere
    last15 = slice(4096 - 15, 4096)
    chunk_used = not np.array_equal(t[last15].view(np.uint32), ex[last15].view(np.uint32))
    close = float(np.max(np.abs(t - ex))) < 4e-6 * 16
    return same_tail and chunk_used and close, (same_tail, chunk_used, close)


def attention_ref(q, k, v, nh, nkv, hd, count, scale):
    qd = q.reshape(nh, hd).astype(np.float64)
    kd = k[:count].reshape(count, nkv, hd).astype(np.float64)
    vd = v[:count].reshape(count, nkv, hd).astype(np.float64)
    out = np.zeros((nh, hd))
    for h in range(nh):
        kv = h // (nh // nkv)
        s = kd[:, kv, :] @ qd[h] * scale
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ vd[:, kv, :]
    return out.ravel()


def check_attention(O):
    bad = []
    for nh, nkv, hd, count, mode in ((8, 2, 128, 300, 0), (32, 8, 128, 2049, 0), (8, 2, 64, 257, 1),
                                     (64, 8, 64, 130, 1), (8, 1, 128, 1, 0)):
        rng = np.random.default_rng(count + hd)
        q = rng.standard_normal(nh * hd).astype(np.float32)
        k = rng.standard_normal((count, nkv * hd)).astype(np.float16)
        v = rng.standard_normal((count, nkv * hd)).astype(np.float16)
        scale = float(np.float32(1.0 / math.sqrt(hd)))
        splits = O.cpu_decode_splits(count, 1, nkv, 512) if mode == 0 else 1
        got = O.attend(q, k.view(np.uint16), v.view(np.uint16), nh, nkv, hd, count, splits, scale, mode)
        e = rel_err(got, attention_ref(q, k, v, nh, nkv, hd, count, scale))
        if e > 2e-5:
            bad.append((nh, nkv, hd, count, mode, e))
    return not bad, bad


def prefill_ref(q, k, v, nh, nkv, hd, start, rows, window, scale):
    """float64 causal attention of rows at positions start.. over planes that
    hold every row's K/V (row r sees positions [t0, start + r])."""
    out = np.zeros((rows, nh * hd))
    kd = k.astype(np.float64).reshape(-1, nkv, hd)
    vd = v.astype(np.float64).reshape(-1, nkv, hd)
    qd = q.astype(np.float64).reshape(rows, nh, hd)
    for r in range(rows):
        count = start + r + 1
        t0 = count - window if window and count > window else 0
        for h in range(nh):
            g = h // (nh // nkv)
            s_ = kd[t0:count, g, :] @ qd[r, h] * scale
            p = np.exp(s_ - s_.max())
            out[r, h * hd:(h + 1) * hd] = (p / p.sum()) @ vd[t0:count, g, :]
    return out.ravel()


def check_prefill_attention(O):
    """The prefill attend (one pass a row and head, q pre-scaled) against
    float64 causal softmax attention, over offsets, GQA groups and a window."""
    bad = []
    hd = 128
    for nh, nkv, start, rows, window in ((8, 2, 0, 37, 0), (32, 8, 100, 20, 0), (4, 1, 5, 9, 6), (8, 8, 0, 3, 0),
                                         (16, 2, 300, 64, 0)):
        rng = np.random.default_rng(start + rows + nh)
        count = start + rows
        q = (rng.standard_normal(rows * nh * hd) * 2).astype(np.float32)
        k = rng.standard_normal((count, nkv * hd)).astype(np.float16)
        v = rng.standard_normal((count, nkv * hd)).astype(np.float16)
        scale = float(np.float32(1.0 / math.sqrt(hd)))
        got = O.prefill_attend(q, k.view(np.uint16), v.view(np.uint16), nh, nkv, hd, start, rows, window, scale)
        e = rel_err(got, prefill_ref(q, k, v, nh, nkv, hd, start, rows, window, scale))
        if e > 2e-5:
            bad.append((nh, nkv, start, rows, window, e))
    return not bad, bad


def check_reference_cpu_goldens(O):
    """The reference CPU backend's own recorded outputs, bit for bit: the
    decode prep at hd 128 (QK-norm + RoPE, QkPrepTest.run(32, 4, 128, true))
    and at hd 64 (the generic qkPrepKernel, QkPrepTest.run(6, 2, 64, true)),
    the split merge + per-256 pack (reducePackGolden, 32 heads × 8 splits),
    the two-pass scores after the combine's in-place softmax exps
    (TreeSiteReferenceTest.attnScoreKernelStaysWithinItsBar: 32 heads, 4 kv
    heads, hd 128, 256 positions) and the router mat-vec + top-8 of 128
    (routerTopKKernelStaysWithinItsBar: logits, picks and weights)."""
    from reference_goldens import cpu_golden_rows, qkprep_fill, reduce_pack_partials, spread
    g = cpu_golden_rows()
    bad = []
    q, k = O.qk_prep128(qkprep_fill(32 * 128, 1), qkprep_fill(4 * 128, 2), qkprep_fill(128, 4), qkprep_fill(128, 5),
                        qkprep_fill(64, 6), 32, 4, True, 1e-6, 0, 11)
    q64, k64 = O.qk_prep(qkprep_fill(6 * 64, 1), qkprep_fill(2 * 64, 2), qkprep_fill(64, 4), qkprep_fill(64, 5),
                         qkprep_fill(32, 6), 6, 2, 64, True, 1e-6, 0, 11)
    for name, got in (("h32kv4d128-q", q), ("h32kv4d128-k", k), ("h6kv2d64-q", q64), ("h6kv2d64-k", k64)):
        want = g[("qkPrepKernel", name)]
        if not np.array_equal(got.view(np.uint32), want.view(np.uint32)):
            bad.append((name, int((got != want).sum())))
    nh, nkv, hd, count = 32, 4, 128, 256
    kq = spread(count * nkv * hd, 5).astype(np.float16)
    sc = O.attn_scores(spread(nh * hd, 3), kq.view(np.uint16), nh, nkv, hd, count,
                       float(np.float32(1) / np.sqrt(np.float32(hd))), softmax=True)
    want = g[("attnScoreKernel", "h32kv4d128c256")]
    if not np.array_equal(sc.reshape(-1).view(np.uint32), want.view(np.uint32)):
        bad.append(("h32kv4d128c256", int((sc.reshape(-1) != want).sum())))
    lg, sel, wt = O.router_topk(spread(128 * 2048, 7), spread(2048, 11), 128, 2048, 8, True, 0.0)
    for name, got in (("logits", lg), ("sel", sel.astype(np.float32)), ("w", wt)):
        want = g[("routerTopKKernel", "e128h2048k8-" + name)]
        if not np.array_equal(got.view(np.uint32), want.view(np.uint32)):
            bad.append(("e128h2048k8-" + name, int((got != want).sum())))
    out = O.attn_merge(reduce_pack_partials(), 32, 8, 128)
    pk = O.q8k_pack(out, per32=False, npad=4096).view(np.int8).astype(np.float32)
    want = g[("attnReducePackQ8Kernel", "h32s8")]
    if not np.array_equal(pk, want):
        bad.append(("h32s8", int((pk != want).sum())))
    return not bad, bad


def check_moe_route(O):
    """MoeFfn.routeFromLogits against float64: softmax over every expert,
    top-k by probability with ties to the lower index, renormalised by the
    sum, scaled by expert_weights_scale (neither 0 nor 1); non-finite logits
    are refused."""
    bad = []
    rng = np.random.default_rng(4)
    for ne, k, scale in ((32, 4, 0.0), (128, 8, 0.0), (32, 4, 2.5)):
        lg = rng.standard_normal(ne).astype(np.float32)
        lg[5] = lg[6] = np.float32(lg.max() + 1)          # a tie: the lower index first
        sel, w = O.moe_route(lg, k, norm=True, w_scale=scale)
        p = np.exp(lg.astype(np.float64) - lg.max())
        p /= p.sum()
        order = sorted(range(ne), key=lambda i: (-p[i], i))[:k]
        want = p[order] / p[order].sum() * (scale if scale else 1.0)
        if list(sel) != order or rel_err(w, want) > 1e-6:
            bad.append((ne, k, scale, list(sel), order))
        _, w1 = O.moe_route(lg, k, norm=True, w_scale=1.0)   # a scale of 1 changes nothing
        _, w0 = O.moe_route(lg, k, norm=True, w_scale=0.0)
        if not np.array_equal(w1, w0):
            bad.append(("scale 1", ne))
    nan = np.full(8, np.nan, np.float32)
    try:
        O.moe_route(nan, 2, norm=True)
        bad.append("non-finite logits routed")
    except ValueError:
        pass
    return not bad, bad


def moe_toy(O, seed=11):
    """A small gpt-oss-like MoE decoder bound straight into the oracle (no
    GGUF): 2 layers, hidden 256, 8 query / 2 kv heads of 64, vocab 512, 8
    experts top-3 (MXFP4 gate/up/down, an f32 router), f32 attention, head
    and embeddings, f32 norms, an 8-position window on layer 0 (pattern 2).
    Every product reads f32 activations, so no int8 pack can round one way
    in f32 and the other in float64: the comparison is of the layer
    composition at f32 accumulation rounding."""
    rng = np.random.default_rng(seed)
    c = dict(n_layers=2, hidden=256, n_heads=8, n_kv=2, head_dim=64, ffn=256, vocab=512, ctx=32, eps=1e-5,
             theta=10000.0, kv_f32=0, workers=512, n_experts=8, n_used=3, norm_topk=1, expert_ffn=256,
             swa_window=8, attn_rows=0, w_scale=0.0, swa_pattern=2)
    H, E, F = c["hidden"], c["n_experts"], c["expert_ffn"]
    qd, kvd = c["n_heads"] * c["head_dim"], c["n_kv"] * c["head_dim"]

    def mx(rows, cols):
        raw = rand_blocks(O, O.MXFP4, rows * cols // 32, rng).reshape(-1, 17)
        raw[:, 0] = rng.integers(118, 121, raw.shape[0])
        return (O.MXFP4, raw.reshape(-1), rows, cols)

    def f32(rows, cols, scale, base=0.0):
        v = (base + scale * rng.standard_normal(rows * cols)).astype(np.float32)
        return (O.F32, v.view(np.uint8), rows, cols)

    t = {"token_embd.weight": f32(c["vocab"], H, 1.0), "output_norm.weight": f32(1, H, 0.05, 1.0),
         "output.weight": f32(c["vocab"], H, 0.06)}
    for l in range(c["n_layers"]):
        p = "blk.%d." % l
        t.update({p + "attn_norm.weight": f32(1, H, 0.05, 1.0), p + "ffn_norm.weight": f32(1, H, 0.05, 1.0),
                  p + "attn_q.weight": f32(qd, H, 0.15), p + "attn_k.weight": f32(kvd, H, 0.15),
                  p + "attn_v.weight": f32(kvd, H, 0.06), p + "attn_output.weight": f32(H, qd, 0.06),
                  p + "ffn_gate_inp.weight": f32(E, H, 0.3),
                  p + "ffn_gate_exps.weight": mx(E * F, H), p + "ffn_up_exps.weight": mx(E * F, H),
                  p + "ffn_down_exps.weight": mx(E * H, F)})
    return c, t


def q8_32(v):
    """The values the MXFP4 experts' per-32 activation codes stand for, in
    float64: q = round-half-away(v·127/max|v|) per block, times max|v|/127."""
    b = v.reshape(-1, 32)
    amax = np.abs(b).max(1, keepdims=True)
    inv = np.where(amax > 0, 127.0 / np.where(amax > 0, amax, 1.0), 0.0)
    q = np.sign(b) * np.floor(np.abs(b) * inv + 0.5)
    return (q * amax / 127.0).ravel()


def moe_forward64(O, c, t, toks):
    """float64 forward of moe_toy's model over `toks` (positions 0..): f16
    K/V, the window clamp
    from = p + 1 - w (PagedKvCache.attendRow), routing on f64 probabilities,
    the experts' inputs at their per-32 codes' values (the MXFP4 Q8 form)."""
    H, nh, nkv, hd, eps = c["hidden"], c["n_heads"], c["n_kv"], c["head_dim"], c["eps"]
    E, K, F = c["n_experts"], c["n_used"], c["expert_ffn"]
    W = {k: O.dequant(ty, raw).astype(np.float64).reshape(rows, cols) for k, (ty, raw, rows, cols) in t.items()}

    def lin(name, xv):
        return W[name] @ xv

    def norm(xv, w):
        return xv / np.sqrt(np.mean(xv * xv) + eps) * w.ravel()

    half = hd // 2
    invd = c["theta"] ** (-np.arange(half, dtype=np.float64) * 2.0 / hd)

    def rope(v, n, pos):
        z = v.reshape(n, hd)
        zc = (z[:, :half] + 1j * z[:, half:]) * np.exp(1j * pos * invd)
        return np.concatenate([zc.real, zc.imag], 1).ravel()

    kc = [[] for _ in range(c["n_layers"])]
    vc = [[] for _ in range(c["n_layers"])]
    out = []
    for pos, tok in enumerate(toks):
        hs = W["token_embd.weight"][tok].copy()
        for l in range(c["n_layers"]):
            p = "blk.%d." % l
            xn = norm(hs, W[p + "attn_norm.weight"])
            q = rope(lin(p + "attn_q.weight", xn), nh, pos)
            k = rope(lin(p + "attn_k.weight", xn), nkv, pos)
            v = lin(p + "attn_v.weight", xn)
            # K/V stored as fp16 of the f32 value the step computes
            kc[l].append(k.astype(np.float32).astype(np.float16).astype(np.float64))
            vc[l].append(v.astype(np.float32).astype(np.float16).astype(np.float64))
            win = c["swa_window"] if (l + 1) % c["swa_pattern"] else 0
            t0 = pos + 1 - win if win and pos + 1 > win else 0
            Kk, Vv = np.array(kc[l][t0:]), np.array(vc[l][t0:])
            ao = np.zeros(nh * hd)
            for h in range(nh):
                g = h // (nh // nkv)
                sc = Kk[:, g * hd:(g + 1) * hd] @ q[h * hd:(h + 1) * hd] / math.sqrt(hd)
                pr = np.exp(sc - sc.max())
                ao[h * hd:(h + 1) * hd] = (pr / pr.sum()) @ Vv[:, g * hd:(g + 1) * hd]
            hs = hs + lin(p + "attn_output.weight", ao)
            xn = norm(hs, W[p + "ffn_norm.weight"])
            lg = W[p + "ffn_gate_inp.weight"] @ xn
            pr = np.exp(lg - lg.max())
            pr /= pr.sum()
            sel = sorted(range(E), key=lambda i: (-pr[i], i))[:K]
            wts = pr[sel] / pr[sel].sum()
            y = np.zeros(H)
            xq = q8_32(xn)
            for e, we in zip(sel, wts):
                gg = W[p + "ffn_gate_exps.weight"][e * F:(e + 1) * F] @ xq
                uu = W[p + "ffn_up_exps.weight"][e * F:(e + 1) * F] @ xq
                y += we * (W[p + "ffn_down_exps.weight"][e * H:(e + 1) * H] @ q8_32(gg / (1 + np.exp(-gg)) * uu))
            hs = hs + y
        out.append(lin("output.weight", norm(hs, W["output_norm.weight"])))
    return out


def check_moe_model(O):
    """The oracle's whole MoE decode step (router, top-k, renormalisation,
    MXFP4 experts, SiLU·up, down, weighted combine, a sliding window on
    alternate layers) against moe_forward64, past the window's length."""
    c, t = moe_toy(O)
    m = O.Model(c)
    for name, (ty, raw, rows, cols) in t.items():
        m.bind(name, ty, raw, rows, cols)
    toks = [3, 141, 59, 26, 5, 77, 200, 13, 9, 300, 42, 7, 99, 1]
    ref = moe_forward64(O, c, t, toks)
    worst = 0.0
    for pos, tok in enumerate(toks):
        _, lg = m.step(tok, pos)
        worst = max(worst, float(np.max(np.abs(lg - ref[pos])) / np.max(np.abs(ref[pos]))))
    m.close()
    return worst < 1e-4, worst


def check_unpermute(O):
    """Checkpoint.unpermuteRows undoes the GGUF llama q/k row permutation:
    HF row (h, a, b) sits at GGUF row (h, b, a) — built here by reshape."""
    nh, hd, rb = 4, 16, 3
    rows = nh * hd
    hf = np.arange(rows * rb, dtype=np.uint8).reshape(rows, rb) % 251
    gg = hf.reshape(nh, 2, hd // 2, rb).swapaxes(1, 2).reshape(rows, rb)
    got = O.unpermute_rows(gg.ravel(), rows, rb, nh).reshape(rows, rb)
    return np.array_equal(got, hf), None


# ------------------------------------------------------------------- tests

def test_dequant_matches_reference_goldens(O):
    ok, bad = check_dequant_golden(O)
    assert ok, bad


def test_f16_conversions_match_ieee(O):
    h = np.arange(65536, dtype=np.uint16)
    got = O.f16_bits_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(4000) * 10, rng.standard_normal(2000) * 1e-5,
                        rng.standard_normal(1000) * 7e4,
                        # exact ties between halves round to even
                        (np.arange(1, 200) + 0.5).astype(np.float32) * np.float32(2.0 ** -10),
                        [0.0, -0.0, 65504.0, 65520.0, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26]]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(O.f32_to_f16_bits(x), want)


@pytest.mark.parametrize("per32", [False, True])
def test_pack_closed_form(O, per32):
    # round half away from zero at exact halves; amax 127 makes the step 1
    x = np.zeros(256, np.float32)
    x[0], x[1], x[2], x[3], x[4] = 127.0, 2.5, -2.5, 0.5, -1.5
    if per32:
        x[32:64] = 127.0
        x[33], x[34] = 3.5, -3.5
    xp = O.q8k_pack(x, per32=per32)
    q = xp[:256].view(np.int8)
    assert list(q[:5]) == [127, 3, -3, 1, -2]
    if per32:
        assert q[33] == 4 and q[34] == -4
    sums = xp[256:288].view(np.int32)
    assert np.array_equal(sums, q.astype(np.int32).reshape(8, 32).sum(1))
    if per32:
        sc = xp[288:320].view(np.float32)
        assert sc[0] == np.float32(1.0) and sc[1] == np.float32(1.0) and np.all(sc[2:] == 0)
    else:
        assert xp[288:292].view(np.float32)[0] == np.float32(1.0)
        assert not xp[292:320].any()
    # a zero block packs to zero with scale 0; a random block reconstructs to half a step
    z = O.q8k_pack(np.zeros(300, np.float32), per32=per32)
    assert not z.any()
    rng = np.random.default_rng(9)
    r = rng.standard_normal(700).astype(np.float32)
    rp = O.q8k_pack(r, per32=per32)
    step = np.max(np.abs(r)) / 127
    assert np.max(np.abs(unpack(O, rp, 700, per32) - r)) <= step * 0.5000001


@pytest.mark.parametrize("ty", [8, 2, 12, 14, 39, 0])
def test_matvec_against_float64(O, ty):
    ok, e = check_matvec(O, ty)
    assert ok, e


def test_rmsnorm_against_float64(O):
    ok, bad = check_rmsnorm(O)
    assert ok, bad


def test_rmsnorm_sums_in_the_device_decode_order(O):
    """Widths that are not whole 256s (gpt-oss's 2880) take the reference's
    rmsnormRowF32 order through Prim.rmsnormDevice (L/model/Prim.cajeta:
    742-775, :1440-1450; the resident layer's fallback, CausalLM.cajeta:3643,
    :3819): 256 lane partials over x[j + 256k] in k order, then the halving
    tree. The input is chosen so that element order gives other bits, so the
    test tells the two apart."""
    for n in (2880, 4096, 300):
        rng = np.random.default_rng(n + 9)
        x = (rng.standard_normal(n) * np.exp(rng.standard_normal(n))).astype(np.float32)
        w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        p = np.zeros(256, np.float32)
        for k in range(0, n, 256):
            seg = x[k:k + 256]
            p[:seg.size] = p[:seg.size] + seg * seg
        s = 128
        while s:
            p[:s] = p[:s] + p[s:2 * s]
            s //= 2
        lanes = p[0]
        seq = np.float32(0)
        for v in x:
            seq = np.float32(seq + v * v)
        assert lanes != seq, n          # the orders differ on this input
        scale = np.float32(1) / np.sqrt(lanes / np.float32(n) + np.float32(1e-5))
        want = x * scale * w
        got = O.rmsnorm(x, w, 1e-5, 0)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), n


def test_rope_against_complex_rotation(O):
    ok, bad = check_rope(O)
    assert ok, bad


def check_expf(O):
    """or_expf is the reference CPU backend's Math.exp, glibc's expf: equal
    to the C library's expf bit for bit on a sample spanning the whole range
    (normal and subnormal results, the overflow and underflow edges, ±0) —
    the restatement was compared over every f32 input when it was written —
    and within 0.51 ulp of exp (glibc's bound)."""
    import ctypes
    libm = ctypes.CDLL("libm.so.6")
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    rng = np.random.default_rng(7)
    xs = np.concatenate([rng.uniform(-104.5, 89.0, 60000), rng.uniform(-1, 1, 20000), rng.uniform(-20, 20, 20000),
                         [0.0, -0.0, 1.0, -1.0, 1e-8, 88.72283, 88.722839, -103.972, -103.97208, -87.4, 0.693147]]
                        ).astype(np.float32)
    got = O.expf(xs)
    want = np.array([libm.expf(float(v)) for v in xs], np.float32)
    bad = int(np.sum(got.view(np.uint32) != want.view(np.uint32)))
    ref = np.exp(xs.astype(np.float64))
    fin = np.isfinite(ref) & (ref < 3e38) & (ref > 1.2e-38)
    ulp = np.spacing(ref[fin].astype(np.float32)).astype(np.float64)
    worst = float(np.max(np.abs(got[fin] - ref[fin]) / ulp))
    return bad == 0 and worst <= 0.51, (bad, worst)


def test_expf_is_glibc_expf(O):
    ok, detail = check_expf(O)
    assert ok, detail
    assert O.expf(np.float32(-105.0))[0] == 0.0 and np.isinf(O.expf(np.float32(89.0))[0])


def test_exp_table_is_two_to_the_i_over_32(O):
    """The table behind or_expf (and the kernels' exp): 2^(i/32) correctly
    rounded to f64, less i·2^47 in its bit pattern, for i < 32."""
    from decimal import Decimal, getcontext
    getcontext().prec = 60
    t = O.exp2_table()
    for i in range(32):
        v = float(Decimal(2) ** (Decimal(i) / Decimal(32)))
        bits = struct.unpack("<Q", struct.pack("<d", v))[0]
        assert int(t[i]) == (bits - (i << 47)) & 0xFFFFFFFFFFFFFFFF, i


def check_router_topk(O):
    """routerTopKKernel beyond its recorded row: equal logits (two identical
    router rows) are picked lower index first; the weights are the float64
    softmax of the logits renormalised over the picks, to f32 rounding; a
    w_scale multiplies them; the logits are a float64 product to 1e-5."""
    rng = np.random.default_rng(21)
    E, H, k = 40, 512, 6
    w = (rng.standard_normal((E, H)) * 0.05).astype(np.float32)
    w[9] = w[4] = (np.abs(w[4]) * 2).astype(np.float32)       # experts 4 and 9: the same, large logit
    x = np.abs(rng.standard_normal(H)).astype(np.float32)
    lg, sel, wt = O.router_topk(w, x, E, H, k, True, 0.0)
    ref = w.astype(np.float64) @ x.astype(np.float64)
    bad = []
    if np.max(np.abs(lg - ref)) > 1e-5 * np.max(np.abs(ref)):
        bad.append("logits")
    if list(sel[:2]) != [4, 9]:
        bad.append(("tie order", list(sel[:2])))
    p = np.exp(lg.astype(np.float64) - lg.max())
    want = p[sel] / p[sel].sum()
    if np.max(np.abs(wt - want)) > 1e-6:
        bad.append(("weights", float(np.max(np.abs(wt - want)))))
    if list(sel) != list(np.argsort(-lg, kind="stable")[:k]):
        bad.append(("picks", list(sel)))
    _, _, ws = O.router_topk(w, x, E, H, k, True, 2.5)
    if not np.array_equal(ws, (wt * np.float32(2.5)).astype(np.float32)):
        bad.append("w_scale")
    return not bad, bad


def test_router_topk(O):
    ok, bad = check_router_topk(O)
    assert ok, bad


def test_silu_forms(O):
    rng = np.random.default_rng(2)
    g = (rng.standard_normal(5000) * 5).astype(np.float32)
    u = rng.standard_normal(5000).astype(np.float32)
    gd = g.astype(np.float64)
    ref = gd / (1 + np.exp(-gd)) * u
    assert rel_err(O.glu(g, u, "exp"), ref) < 1e-6
    ok, detail = check_glu_structure(O)
    assert ok, detail


def test_argmax_first_occurrence(O):
    ok, bad = check_argmax(O)
    assert ok, bad


def test_attention_against_float64(O):
    ok, bad = check_attention(O)
    assert ok, bad


def test_prefill_attention_against_float64(O):
    ok, bad = check_prefill_attention(O)
    assert ok, bad


def test_prefill_first_row_is_the_decode_attention(O):
    """At one position the prefill attend is softmax over one key: the output
    is that key's V row exactly (weight exp(0) = 1, l = 1), as the decode
    form's is."""
    rng = np.random.default_rng(9)
    nh, nkv, hd = 8, 2, 128
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal((1, nkv * hd)).astype(np.float16)
    v = rng.standard_normal((1, nkv * hd)).astype(np.float16)
    got = O.prefill_attend(q, k.view(np.uint16), v.view(np.uint16), nh, nkv, hd, 0, 1, 0, 0.088)
    want = np.repeat(v.astype(np.float32).reshape(nkv, 1, hd), nh // nkv, axis=1).ravel()
    assert np.array_equal(got, want)


def test_model_prefill_matches_decode_steps(O):
    """A prefill chunk through the many-row forward (prefill attend) against
    the same prompt as decode steps (split-K attend), on the reference's toy
    GGUF: the attention forms round differently, so the logits agree to the
    packs' rounding and the greedy token is the same; the K/V the chunk
    leaves continue decoding to the same tokens."""
    from oracle.gguf_reader import GgufReader, oracle_model
    r = GgufReader(os.path.join(GOLD, "gguf", "toy-routable.gguf"))
    a, _ = oracle_model(r, ctx=64)
    b, _ = oracle_model(r, ctx=64)
    toks = [3, 141, 59, 26, 5, 77, 200, 13, 9]
    ta, la = a.prefill(toks, 0)
    for p, t in enumerate(toks):
        tb, lb = b.step(t, p)
    assert ta == tb
    assert float(np.max(np.abs(la - lb)) / np.max(np.abs(lb))) < 1e-4
    ga, gb = [ta], [tb]
    for i in range(6):
        ga.append(a.step(ga[-1], len(toks) + i)[0])
        gb.append(b.step(gb[-1], len(toks) + i)[0])
    assert ga == gb
    # a chunk split in two: the same bits (the rows' arithmetic does not
    # depend on the chunking)
    c, _ = oracle_model(r, ctx=64)
    c.prefill(toks[:4], 0)
    tc, lc = c.prefill(toks[4:], 4)
    assert tc == ta and np.array_equal(lc.view(np.uint32), la.view(np.uint32))
    for m in (a, b, c):
        m.close()


def test_reference_cpu_backend_goldens(O):
    ok, bad = check_reference_cpu_goldens(O)
    assert ok, bad


def test_decode_splits_closed_form(O):
    # two work items a worker over the kv heads, within [1, min(64, count)]
    assert O.cpu_decode_splits(2049, 1, 8, 512) == 64
    assert O.cpu_decode_splits(2049, 1, 8, 16) == 4
    assert O.cpu_decode_splits(3, 1, 8, 512) == 3
    assert O.cpu_decode_splits(100, 1, 8, 1) == 1
    assert O.cpu_decode_splits(100, 2, 8, 24) == 3


def test_rope_freqs_factors(O):
    ok, bad = check_rope_freqs(O)
    assert ok, bad


def test_mxfp4_device_q8_form(O):
    ok, bad = check_mxfp4_q8(O)
    assert ok, bad


def test_moe_route_against_float64(O):
    ok, bad = check_moe_route(O)
    assert ok, bad


def test_moe_model_forward_against_float64(O):
    """The MoE layer composition and the sliding window, at model level."""
    ok, worst = check_moe_model(O)
    print("moe forward: worst relative logit difference %.3g" % worst)
    assert ok, worst


def test_attention_with_f32_kv_against_float64(O):
    """The config-literal f32 K/V planes (the reference's non-resident
    PagedKvCache path) through both decode forms and the prefill attend."""
    bad = []
    for nh, nkv, hd, count, mode in ((8, 2, 128, 300, 0), (8, 2, 64, 70, 1)):
        rng = np.random.default_rng(count)
        q = rng.standard_normal(nh * hd).astype(np.float32)
        k = rng.standard_normal((count, nkv * hd)).astype(np.float32)
        v = rng.standard_normal((count, nkv * hd)).astype(np.float32)
        scale = float(np.float32(1.0 / math.sqrt(hd)))
        splits = O.cpu_decode_splits(count, 1, nkv, 512) if mode == 0 else 1
        got = O.attend(q, k, v, nh, nkv, hd, count, splits, scale, mode, kv_f32=True)
        e = rel_err(got, attention_ref(q, k, v, nh, nkv, hd, count, scale))
        if e > 2e-5:
            bad.append((hd, mode, e))
    rng = np.random.default_rng(5)
    nh, nkv, hd, start, rows = 8, 2, 128, 10, 12
    q = rng.standard_normal(rows * nh * hd).astype(np.float32)
    k = rng.standard_normal((start + rows, nkv * hd)).astype(np.float32)
    v = rng.standard_normal((start + rows, nkv * hd)).astype(np.float32)
    got = O.prefill_attend(q, k, v, nh, nkv, hd, start, rows, 0, 0.088, kv_f32=True)
    e = rel_err(got, prefill_ref(q, k, v, nh, nkv, hd, start, rows, 0, 0.088))
    if e > 2e-5:
        bad.append(("prefill", e))
    assert not bad, bad


def test_unpermute_rows_inverts_the_gguf_permutation(O):
    ok, _ = check_unpermute(O)
    assert ok


def test_gguf_reader_reads_the_reference_toy_fixtures():
    from oracle.gguf_reader import GgufReader, model_config
    for name, nkv in (("toy-routable.gguf", 1), ("toy-routable-gqa8.gguf", None)):
        r = GgufReader(os.path.join(GOLD, "gguf", name))
        cfg = model_config(r)
        assert cfg["hidden"] == 512 and cfg["head_dim"] == 128 and cfg["n_layers"] == 2
        if nkv:
            assert cfg["n_kv"] == nkv
        assert "token_embd.weight" in r.tensors and "blk.1.ffn_down.weight" in r.tensors


def test_toy_model_forward_against_float64(O):
    """The oracle's whole decode step against a float64 forward of the same
    GGUF (weights dequantised, activations through the same int8 packs, fp16
    K/V): the layer composition — norms, RoPE, GQA, residuals, SwiGLU, head —
    agrees to the packs' rounding."""
    from oracle.gguf_reader import GgufReader, oracle_model
    r = GgufReader(os.path.join(GOLD, "gguf", "toy-routable.gguf"))
    om, cfg = oracle_model(r, ctx=16)
    L, H, nh, nkv, hd = cfg["n_layers"], cfg["hidden"], cfg["n_heads"], cfg["n_kv"], cfg["head_dim"]
    eps, theta, V = cfg["eps"], cfg["theta"], cfg["vocab"]

    def t(name, unperm=0):
        ty, dims, rows, cols, data = r.tensors[name]
        raw = np.ascontiguousarray(data)
        if ty == O.F32:
            return raw.view(np.float32).astype(np.float64).reshape(rows, cols) if rows > 1 else \
                raw.view(np.float32).astype(np.float64).ravel()
        if unperm:
            be, bb = O.BLOCK[ty]
            raw = O.unpermute_rows(raw, rows, cols // be * bb, unperm)
        return O.dequant(ty, raw).astype(np.float64).reshape(rows, cols)

    def lin(name, xv, unperm=0):
        ty = r.tensors[name][0]
        Wm = t(name, unperm)
        if ty in (O.Q4_0, O.MXFP4, O.F32):
            return Wm @ xv
        x32 = xv.astype(np.float32)
        return Wm @ unpack(O, O.q8k_pack(x32, per32=(ty == O.Q8_0)), x32.size, ty == O.Q8_0)

    def norm(xv, w):
        return xv / np.sqrt(np.mean(xv * xv) + eps) * w

    half = hd // 2
    invd = theta ** (-np.arange(half, dtype=np.float64) * 2.0 / hd)

    def rope(v, n, pos):
        z = v.reshape(n, hd)
        zc = (z[:, :half] + 1j * z[:, half:]) * np.exp(1j * pos * invd)
        return np.concatenate([zc.real, zc.imag], 1).ravel()

    emb = t("token_embd.weight")
    head = "output.weight" if "output.weight" in r.tensors else "token_embd.weight"
    toks = [3, 141, 59, 26, 5]
    kc = [[] for _ in range(L)]
    vc = [[] for _ in range(L)]
    worst = 0.0
    for pos, tok in enumerate(toks):
        hs = emb[tok].copy()
        for l in range(L):
            p = "blk.%d." % l
            xn = norm(hs, t(p + "attn_norm.weight"))
            q = rope(lin(p + "attn_q.weight", xn, nh), nh, pos)
            k = rope(lin(p + "attn_k.weight", xn, nkv), nkv, pos)
            v = lin(p + "attn_v.weight", xn)
            kc[l].append(k.astype(np.float16).astype(np.float64))
            vc[l].append(v.astype(np.float16).astype(np.float64))
            K, Vv = np.array(kc[l]), np.array(vc[l])
            ao = np.zeros(nh * hd)
            for h in range(nh):
                g = h // (nh // nkv)
                s = K[:, g * hd:(g + 1) * hd] @ q[h * hd:(h + 1) * hd] / math.sqrt(hd)
                pr = np.exp(s - s.max())
                ao[h * hd:(h + 1) * hd] = (pr / pr.sum()) @ Vv[:, g * hd:(g + 1) * hd]
            hs = hs + lin(p + "attn_output.weight", ao)
            xn = norm(hs, t(p + "ffn_norm.weight"))
            gg, uu = lin(p + "ffn_gate.weight", xn), lin(p + "ffn_up.weight", xn)
            hs = hs + lin(p + "ffn_down.weight", gg / (1 + np.exp(-gg)) * uu)
        ref = lin(head, norm(hs, t("output_norm.weight")))
        _, logits = om.step(tok, pos)
        worst = max(worst, float(np.max(np.abs(logits - ref)) / np.max(np.abs(ref))))
    om.close()
    print("toy forward: worst relative logit difference %.3g" % worst)
    assert worst < 1e-4, worst


# ------------------------------------------------------- planted mistakes

PLANTS = {
    1: ("Q4_K GEMV without the min term", lambda O: check_matvec(O, O.Q4_K)),
    2: ("RoPE with a sign error", check_rope),
    3: ("argmax keeps the last maximum", check_argmax),
    4: ("Q4_K 6-bit scale from the wrong byte", check_dequant_golden),
    5: ("RMSNorm without eps", check_rmsnorm),
    6: ("tanh-form SiLU chunks stepped by one", check_glu_structure),
    7: ("split-K without the rescale on a new max", check_attention),
    8: ("q/k rows unpermuted with the halves swapped", check_unpermute),
    9: ("prefill scores from one lane partial", check_prefill_attention),
    10: ("QK-norm 32-sums folded from the end", check_reference_cpu_goldens),
    11: ("router ties keep the higher expert index", check_moe_route),
    12: ("router weights not renormalised", check_moe_route),
    13: ("sliding window one position short", check_moe_model),
    14: ("MoE model without the renormalisation", check_moe_model),
    15: ("MXFP4 activation codes at half scale", check_mxfp4_q8),
    16: ("MXFP4 high nibbles against the low activation half", check_mxfp4_q8),
    17: ("rope_freqs factors multiplied, not divided", check_rope_freqs),
    18: ("device router ties keep the higher expert index", check_router_topk),
    19: ("generic QK-norm wave lanes summed in order", check_reference_cpu_goldens),
    20: ("device router lanes summed in order", check_reference_cpu_goldens),
    21: ("exp's polynomial without its cubic term", check_expf),
}
# 14 is plant 12 again, caught at model level as well (the tie order of plant
# 11 needs an exact tie, which only check_moe_route constructs)
PLANT_DEFINE = {14: 12}


@pytest.mark.parametrize("plant", sorted(PLANTS))
def test_planted_mistakes_are_caught(O, tmp_path, plant):
    what, check = PLANTS[plant]
    so = str(tmp_path / ("liboracle_plant%d.so" % plant))
    subprocess.check_call(["gcc", "-O2", "-std=gnu11", "-fPIC", "-fopenmp", "-ffp-contract=off", "-fno-fast-math",
                           "-DOR_PLANT=%d" % PLANT_DEFINE.get(plant, plant), "-shared", "-o", so,
                           os.path.join(ROOT, "oracle", "oracle.c"), "-lm"])
    assert check(O)[0], "the check must pass on the real oracle first"
    prev = O.use(O.load(so))
    try:
        ok, detail = check(O)
    finally:
        O.use(prev)
    assert not ok, "planted mistake not caught: %s (%s)" % (what, detail)
