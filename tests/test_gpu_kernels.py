"""Kernel-level parity: each launch-seam entry point of the C-ABI on the
MI355X against the CPU oracle on the same seeded inputs. Integer/byte work
(dequant, packs, argmax, fp16 appends, routing ids) is bit-exact; float
reductions are held to the tolerance written in each test."""
import struct

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def rand_blocks(O, ty, nblocks, rng):
    """Valid random blocks of a format: random bytes with sane scales."""
    be, bb = O.BLOCK[ty]
    raw = rng.integers(0, 256, size=(nblocks, bb), dtype=np.uint8)
    def f16(vals):
        return np.asarray(vals, np.float16).view(np.uint8).reshape(-1, 2)
    if ty == O.Q8_0 or ty == O.Q4_0:
        raw[:, 0:2] = f16(rng.uniform(0.001, 0.01, nblocks))
    elif ty == O.Q4_K:
        raw[:, 0:2] = f16(rng.uniform(0.0005, 0.002, nblocks))
        raw[:, 2:4] = f16(rng.uniform(0.0005, 0.002, nblocks))
    elif ty == O.Q6_K:
        raw[:, 208:210] = f16(rng.uniform(0.0001, 0.001, nblocks))
    elif ty == O.MXFP4:
        raw[:, 0] = rng.integers(118, 126, nblocks)
    return raw.reshape(-1)


def golden(name):
    import os
    here = os.path.join(os.path.dirname(__file__), "golden", "kquant")
    return np.fromfile(os.path.join(here, name + ".bin"), np.uint8), np.fromfile(os.path.join(here, name + ".f32"), np.float32)


FORMATS = [("q8_0", 8), ("q4_0", 2), ("q4_k", 12), ("q6_k", 14), ("mxfp4", 39)]


@pytest.mark.parametrize("name,ty", [f for f in FORMATS if f[0] != "mxfp4"])
def test_dequant_file_layout_matches_golden(gpu, O, name, ty):
    say("dequant golden", name)
    raw, ref = golden(name)
    be, bb = O.BLOCK[ty]
    rows, cols = 1, ref.size
    src, out = gpu.Buffer.of(raw), gpu.Buffer(ref.size * 4)
    gpu.native.check(gpu.native.lib().cj_dequant(out.h, src.h, ty, rows, cols, 0), "dequant")
    got = out.download(np.float32, ref.size)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_dequant_mxfp4_matches_golden(gpu, O):
    import os
    b = open(os.path.join(os.path.dirname(__file__), "golden", "mxfp4", "mxfp4_ref.bin"), "rb").read()
    _, nb = struct.unpack("<ii", b[:8])
    raw = np.frombuffer(b[8:8 + nb * 17], np.uint8)
    ref = np.frombuffer(b[8 + nb * 17:], np.float32)
    src, out = gpu.Buffer.of(raw), gpu.Buffer(ref.size * 4)
    gpu.native.check(gpu.native.lib().cj_dequant(out.h, src.h, 39, 1, ref.size, 0), "dequant")
    assert np.array_equal(out.download(np.float32, ref.size).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("name,ty", FORMATS)
def test_prepared_layout_dequant_is_bit_exact(gpu, O, name, ty):
    say("prepared dequant", name)
    rng = np.random.default_rng(ty)
    rows, cols = 37, 2048
    be, bb = O.BLOCK[ty]
    raw = rand_blocks(O, ty, rows * cols // be, rng)
    ref = O.dequant(ty, raw)
    lib = gpu.native.lib()
    prb = lib.cj_prepared_row_bytes(ty, cols)
    src, dst, out = gpu.Buffer.of(raw), gpu.Buffer(prb * rows), gpu.Buffer(rows * cols * 4)
    gpu.native.check(lib.cj_prepare_weight(dst.h, src.h, ty, rows, cols), "prepare")
    gpu.native.check(lib.cj_dequant(out.h, dst.h, ty, rows, cols, 1), "dequant prepared")
    assert np.array_equal(out.download(np.float32, rows * cols).view(np.uint32), ref.view(np.uint32))
    gpu.native.check(lib.cj_dequant(out.h, src.h, ty, rows, cols, 0), "dequant file")
    assert np.array_equal(out.download(np.float32, rows * cols).view(np.uint32), ref.view(np.uint32))


def tie_vector(rng, n):
    """Values with exact .5 ties after the pack's scaling (amax 127 per block)."""
    x = (rng.integers(-126, 126, n) + 0.5).astype(np.float32)
    x[::256] = 127.0
    return x


@pytest.mark.parametrize("per32", [0, 1])
@pytest.mark.parametrize("n", [256, 1408, 4096, 14336])
def test_pack_is_bit_exact(gpu, O, per32, n):
    say("pack", n, per32)
    rng = np.random.default_rng(n + per32)
    npad = (n + 255) // 256 * 256
    for x in (rng.standard_normal(n).astype(np.float32), tie_vector(rng, n), np.zeros(n, np.float32)):
        xb, ob = gpu.Buffer.of(x), gpu.Buffer(npad // 256 * 320)
        gpu.native.check(gpu.native.lib().cj_q8k_pack(ob.h, xb.h, 1, n, npad, per32), "pack")
        got = ob.download(np.uint8, npad // 256 * 320)
        ref = O.q8k_pack(x, per32=bool(per32), npad=npad)
        assert np.array_equal(got, ref)


@pytest.mark.parametrize("dim", [512, 4096, 2880])
@pytest.mark.parametrize("per32", [0, 1])
def test_rmsnorm_pack(gpu, O, dim, per32):
    """Whole 256s: the CPU row form's 256-lane tree; other widths: the host
    floor's element-order sum. The kernel makes the same adds and a correctly
    rounded sqrt and divide, so the same bits, over many rows (a 1-ulp error
    in the scale shows on a fraction of rows only)."""
    say("rmsnorm_pack", dim, per32)
    rng = np.random.default_rng(dim + per32)
    npad = (dim + 255) // 256 * 256
    w = (1 + 0.02 * rng.standard_normal(dim)).astype(np.float32)
    wb, ob, pb = gpu.Buffer.of(w), gpu.Buffer(dim * 4), gpu.Buffer(npad // 256 * 320)
    lib = gpu.native.lib()
    for row in range(48):
        x = (rng.standard_normal(dim) * rng.uniform(0.05, 8)).astype(np.float32)
        xb = gpu.Buffer.of(x)
        gpu.native.check(lib.cj_rmsnorm_pack(ob.h, pb.h, xb.h, wb.h, dim, 1e-5, 0, per32), "rmsnorm_pack")
        got = ob.download(np.float32, dim)
        ref = O.rmsnorm(x, w, 1e-5)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), "row %d" % row
        assert np.array_equal(pb.download(np.uint8, npad // 256 * 320), O.q8k_pack(ref, per32=bool(per32), npad=npad))
        xb.free()


def matvec_case(gpu, O, ty, rows, cols, seed, accum=False):
    rng = np.random.default_rng(seed)
    be, bb = O.BLOCK[ty]
    raw = rand_blocks(O, ty, rows * cols // be, rng)
    x = rng.standard_normal(cols).astype(np.float32)
    lib = gpu.native.lib()
    prb = lib.cj_prepared_row_bytes(ty, cols)
    src, w = gpu.Buffer.of(raw), gpu.Buffer(prb * rows)
    gpu.native.check(lib.cj_prepare_weight(w.h, src.h, ty, rows, cols), "prepare")
    if ty in (O.Q4_0, O.MXFP4):
        act = gpu.Buffer.of(x)
        ref = O.matvec(ty, raw, rows, cols, x)
    else:
        xp = O.q8k_pack(x, per32=(ty == O.Q8_0))
        act = gpu.Buffer.of(xp)
        ref = O.matvec_packed(ty, raw, rows, cols, xp)
    y0 = rng.standard_normal(rows).astype(np.float32) if accum else np.zeros(rows, np.float32)
    y = gpu.Buffer.of(y0)
    gpu.native.check(lib.cj_matvec(ty, y.h, w.h, act.h, rows, cols, 0, int(accum)), "matvec")
    got = y.download(np.float32, rows)
    if accum:
        ref = (y0 + ref).astype(np.float32)
    return got, ref, raw, x


@pytest.mark.parametrize("name,ty", FORMATS)
@pytest.mark.parametrize("rows,cols", [(300, 512), (1024, 4096), (96, 14336), (70, 2880), (32800, 96), (40, 2880)])
def test_matvec_matches_oracle(gpu, O, name, ty, rows, cols):
    if cols % 256 and ty in (12, 14):
        pytest.skip("K-quant rows are whole 256-element blocks")
    say("matvec", name, rows, cols)
    got, ref, raw, x = matvec_case(gpu, O, ty, rows, cols, rows + cols + ty)
    # int8 formats: integer sub-block dots, then the f32 fold over blocks in
    # the reference's block order; f32-activation formats: the row summed in
    # the reference's element order. The same bits either way.
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), \
        "%s %dx%d: %d rows differ" % (name, rows, cols, int((got != ref).sum()))


@pytest.mark.parametrize("rows,cols", [(32, 2880), (64, 6144), (3, 6176), (40, 14336), (7, 96)])
def test_matvec_f32_rows_match_oracle(gpu, O, rows, cols):
    """The f32 GEMV (the MoE router's product) at up to 64 rows: a workgroup a
    row, whose adder wave walks the row's element-order chain across its
    lanes — rows of one tile (up to 6144 columns, the tile run alone) and of
    several (2, 3 tiles) — bit for bit the oracle's column-order dot."""
    say("matvec f32", rows, cols)
    rng = np.random.default_rng(rows * 31 + cols)
    w = (rng.standard_normal(rows * cols) * 0.05).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    lib = gpu.native.lib()
    wb, xb = gpu.Buffer.of(w), gpu.Buffer.of(x)
    yb = gpu.Buffer.of(np.zeros(rows, np.float32))
    gpu.native.check(lib.cj_matvec(O.F32, yb.h, wb.h, xb.h, rows, cols, 0, 0), "matvec f32")
    got = yb.download(np.float32, rows)
    ref = O.matvec(O.F32, w.view(np.uint8), rows, cols, x)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), \
        "f32 %dx%d: %d rows differ" % (rows, cols, int((got != ref).sum()))
    # a row that is not whole 32-element blocks is refused, not truncated
    assert lib.cj_matvec(O.F32, yb.h, wb.h, xb.h, 1, cols - 4, 0, 0) == gpu.native.CJ_ERR_ARG


@pytest.mark.parametrize("name,ty", [("q4_k", 12), ("q8_0", 8)])
def test_matvec_accumulate_store(gpu, O, name, ty):
    got, ref, _, _ = matvec_case(gpu, O, ty, 512, 4096, 7, accum=True)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("rows,cols,accum", [(5760, 2880, 0), (2880, 2880, 1), (24, 32, 0), (40, 96, 0),
                                             (7, 4096, 1), (9, 4128, 0), (33, 8192, 0), (11520, 2880, 0)])
def test_matvec_mxfp4_q8_matches_oracle(gpu, O, rows, cols, accum):
    """The MXFP4 device Q8 form (the engine's MoE experts): per-32 activation
    codes, the integer block dots over 32 lanes and their butterfly, bit for
    bit the oracle's restatement; 1 to 4 blocks a lane a sweep, and more
    sweeps past 4096 columns. Activations with a spread of block scales and
    exact zeros (an all-zero block quantizes to zeros with scale 0)."""
    say("mxfp4 q8", rows, cols, accum)
    rng = np.random.default_rng(rows * 7 + cols)
    raw = rand_blocks(O, O.MXFP4, rows * cols // 32, rng)
    x = (rng.standard_normal(cols) * rng.uniform(0.05, 5, cols // 32).repeat(32)).astype(np.float32)
    x[:32] = 0.0
    lib = gpu.native.lib()
    prb = lib.cj_prepared_row_bytes(O.MXFP4, cols)
    src, w = gpu.Buffer.of(raw), gpu.Buffer(prb * rows)
    gpu.native.check(lib.cj_prepare_weight(w.h, src.h, O.MXFP4, rows, cols), "prepare")
    y0 = rng.standard_normal(rows + 3).astype(np.float32)
    xb, y = gpu.Buffer.of(x), gpu.Buffer.of(y0)
    gpu.native.check(lib.cj_matvec_mxfp4_q8(y.h, w.h, xb.h, rows, cols, 3, accum), "matvec_mxfp4_q8")
    got = y.download(np.float32, rows + 3)
    ref = O.matvec_mxfp4_q8(raw, rows, cols, x)
    if accum:
        ref = (y0[3:] + ref).astype(np.float32)
    assert np.array_equal(got[:3].view(np.uint32), y0[:3].view(np.uint32)), "y_off prefix touched"
    assert np.array_equal(got[3:].view(np.uint32), ref.view(np.uint32)), \
        "%dx%d: %d rows differ" % (rows, cols, int((got[3:] != ref).sum()))


def test_matvec_refuses_short_buffers(gpu, O):
    lib = gpu.native.lib()
    w, act, y = gpu.Buffer(1024), gpu.Buffer(320), gpu.Buffer(16)
    rc = lib.cj_matvec(12, y.h, w.h, act.h, 64, 256, 0, 0)
    assert rc == -1 and "weight" in gpu.native.last_error()


@pytest.mark.parametrize("form", [0, 1])
@pytest.mark.parametrize("n,per32", [(14336, 0), (1408, 1), (512, 0)])
def test_glu_pack(gpu, O, form, n, per32):
    say("glu", n, form, per32)
    rng = np.random.default_rng(n + form)
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    npad = (n + 255) // 256 * 256
    gb, ub, ob, pb = gpu.Buffer.of(g), gpu.Buffer.of(u), gpu.Buffer(n * 4), gpu.Buffer(npad // 256 * 320)
    gpu.native.check(gpu.native.lib().cj_glu(ob.h, pb.h, gb.h, ub.h, n, form, per32), "glu")
    got = ob.download(np.float32, n)
    ref = O.glu(g, u, "tanh" if form else "exp")
    # the rational tanh is fma/div (correctly rounded both sides); the exp
    # form runs the same written-out expf on both sides: the same bits
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    # the pack of the device's own values is the oracle's pack of them, bit for bit
    assert np.array_equal(pb.download(np.uint8, npad // 256 * 320), O.q8k_pack(got, per32=bool(per32), npad=npad))


@pytest.mark.parametrize("n", [5, 1024, 128256, 201088])
def test_argmax_first_occurrence(gpu, O, n):
    rng = np.random.default_rng(n)
    v = rng.standard_normal(n).astype(np.float32)
    v[n // 3] = 9.0
    v[(2 * n) // 3] = 9.0          # a tie later: the smaller index wins
    vb, tb = gpu.Buffer.of(v), gpu.Buffer(16)
    gpu.native.check(gpu.native.lib().cj_argmax_row(tb.h, 1, vb.h, n), "argmax")
    assert int(tb.download(np.int32, 4)[1]) == O.argmax(v) == n // 3


def to_paged(plane, n_kv, hd, pages):
    """position-major [ctx][n_kv·hd] fp16 -> page-blocked head-major planes"""
    ctx = plane.shape[0]
    out = np.zeros((pages, n_kv, 64, hd), np.uint16)
    for p in range(ctx):
        out[p // 64, :, p % 64, :] = plane[p].reshape(n_kv, hd)
    return out.reshape(-1)


@pytest.mark.parametrize("hd,n_q,n_kv", [(128, 32, 8), (128, 4, 1), (128, 8, 1), (64, 8, 2), (64, 64, 8), (128, 8, 8)])
@pytest.mark.parametrize("count,frm,workers", [(1, 0, 512), (37, 0, 16), (300, 5, 16), (2049, 0, 512), (130, 70, 3),
                                               (4133, 3, 512), (6300, 70, 512)])
def test_attend_matches_oracle(gpu, O, hd, n_q, n_kv, count, frm, workers):
    say("attend", hd, n_q, n_kv, count, frm, workers)
    rng = np.random.default_rng(count * 7 + hd + n_q)
    pages = (frm + count + 63) // 64 + 1
    ctx = pages * 64
    kf = (rng.standard_normal((ctx, n_kv * hd))).astype(np.float32)
    vf = (rng.standard_normal((ctx, n_kv * hd))).astype(np.float32)
    k16, v16 = kf.astype(np.float16).view(np.uint16), vf.astype(np.float16).view(np.uint16)
    q = rng.standard_normal(n_q * hd).astype(np.float32)
    scale = np.float32(1.0 / np.sqrt(hd))
    # a shuffled page table
    tab = rng.permutation(pages).astype(np.int32)
    kp = np.zeros((pages * 64, n_kv * hd), np.uint16); vp = np.zeros_like(kp)
    for p in range(ctx):
        row = tab[p // 64] * 64 + p % 64
        kp[row] = k16[p]; vp[row] = v16[p]
    kb, vb = gpu.Buffer.of(to_paged(kp, n_kv, hd, pages)), gpu.Buffer.of(to_paged(vp, n_kv, hd, pages))
    qb, tb = gpu.Buffer.of(q), gpu.Buffer.of(tab)
    part = gpu.Buffer(n_q * max(64 * (hd + 2), count) * 4)
    out, cnt = gpu.Buffer(n_q * hd * 4), gpu.Buffer(4 * n_kv)
    cnt.zero()
    lib = gpu.native.lib()
    gpu.native.check(lib.cj_attend(part.h, out.h, qb.h, kb.h, vb.h, tb.h, 0, cnt.h, n_q, n_kv, hd, count, frm,
                                   workers, float(scale)), "attend")
    got = out.download(np.float32, n_q * hd)
    split = hd == 128 and n_q in (4 * n_kv, 8 * n_kv)
    spl = O.cpu_decode_splits(count, 1, n_kv, workers) if split else 1
    assert lib.cj_decode_splits(count, n_kv, workers) == O.cpu_decode_splits(count, 1, n_kv, workers)
    ref = O.attend(q, k16[frm:frm + count], v16[frm:frm + count], n_q, n_kv, hd, count, spl, float(scale),
                   0 if split else 1)
    # the reference CPU backend's operation order on both sides: the same bits
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), np.abs(got - ref).max()
    if split:
        # the merge kernel over the same partials gives the same output
        out2 = gpu.Buffer(n_q * hd * 4)
        gpu.native.check(lib.cj_attn_merge(out2.h, 0, part.h, n_q, hd, spl, 0), "merge")
        assert np.array_equal(out2.download(np.float32, n_q * hd).view(np.uint32), got.view(np.uint32))
        assert np.array_equal(cnt.download(np.int32, n_kv), np.zeros(n_kv, np.int32))


@pytest.mark.parametrize("hd,n_q,n_kv,theta", [(128, 32, 8, 500000.0), (64, 8, 2, 10000.0)])
def test_qk_prep_rope_and_append(gpu, O, hd, n_q, n_kv, theta):
    rng = np.random.default_rng(hd)
    ctx = 256
    pos = 131
    q = rng.standard_normal(n_q * hd).astype(np.float32)
    k = rng.standard_normal(n_kv * hd).astype(np.float32)
    v = rng.standard_normal(n_kv * hd).astype(np.float32)
    pages = ctx // 64
    lib = gpu.native.lib()
    qb, kb, vb = gpu.Buffer.of(q), gpu.Buffer.of(k), gpu.Buffer.of(v)
    kc, vc = gpu.Buffer(pages * n_kv * 64 * hd * 2), gpu.Buffer(pages * n_kv * 64 * hd * 2)
    kc.zero(); vc.zero()
    rope = gpu.Buffer(ctx * hd * 4)
    gpu.native.check(lib.cj_rope_table(rope.h, hd, theta, ctx), "rope_table")
    tab = gpu.Buffer.of(np.arange(pages, dtype=np.int32))
    gpu.native.check(lib.cj_qk_prep(qb.h, kb.h, vb.h, kc.h, vc.h, 0, 0, rope.h, tab.h, 0, n_q, n_kv, hd, 0, 1e-5, 0, pos),
                     "qk_prep")
    inv = O.inv_freq(hd, theta)
    qr, kr = O.rope(q, n_q, hd, pos, inv), O.rope(k, n_kv, hd, pos, inv)
    assert np.array_equal(qb.download(np.float32, q.size).view(np.uint32), qr.view(np.uint32))
    kcache = kc.download(np.uint16, pages * n_kv * 64 * hd).reshape(pages, n_kv, 64, hd)
    vcache = vc.download(np.uint16, pages * n_kv * 64 * hd).reshape(pages, n_kv, 64, hd)
    assert np.array_equal(kcache[pos // 64, :, pos % 64, :].reshape(-1), O.f32_to_f16_bits(kr))
    assert np.array_equal(vcache[pos // 64, :, pos % 64, :].reshape(-1), O.f32_to_f16_bits(v))


@pytest.mark.parametrize("ne,k", [(32, 4), (128, 8), (8, 2), (200, 4), (256, 8)])
def test_moe_route(gpu, O, ne, k):
    rng = np.random.default_rng(ne)
    rows = 5
    lg = rng.standard_normal((rows, ne)).astype(np.float32)
    lg[2, 3] = lg[2, 5] = 7.0                     # tie: the lower index first
    lg[3, :] = 0.5                                # every probability equal: 0, 1, ..., k-1
    lg[4, ne - 1] = lg[4, ne - 2] = 9.0           # a tie at the top across lanes
    lb, sb, wb = gpu.Buffer.of(lg), gpu.Buffer(rows * k * 4), gpu.Buffer(rows * k * 4)
    gpu.native.check(gpu.native.lib().cj_moe_route(sb.h, wb.h, lb.h, rows, ne, k, 1, 0.0, 0), "route")
    sel = sb.download(np.int32, rows * k).reshape(rows, k)
    w = wb.download(np.float32, rows * k).reshape(rows, k)
    for r in range(rows):
        rs, rw = O.moe_route(lg[r], k, True)
        assert np.array_equal(sel[r], rs)
        assert np.allclose(w[r], rw, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("ty", [0, 8, 12, 14])
def test_embed_row(gpu, O, ty):
    rng = np.random.default_rng(ty)
    hidden, vocab = 512, 40
    be, bb = O.BLOCK[ty]
    if ty == 0:
        raw = rng.standard_normal(vocab * hidden).astype(np.float32).view(np.uint8)
    else:
        raw = rand_blocks(O, ty, vocab * hidden // be, rng)
    tb, ob = gpu.Buffer.of(raw), gpu.Buffer(hidden * 4)
    gpu.native.check(gpu.native.lib().cj_embed_row(ob.h, tb.h, ty, hidden, 33), "embed")
    rb = hidden // be * bb
    ref = O.dequant(ty, raw[33 * rb:34 * rb])
    assert np.array_equal(ob.download(np.float32, hidden).view(np.uint32), ref.view(np.uint32))


def test_embed_row_from_a_device_token_slot(gpu, O):
    """cj_embed_row_slot reads the id the previous argmax left in a device
    slot (EmbedKernel.embedRowLaunchNoSync); an id naming no row writes zeros
    and raises the status word instead of reading past the table."""
    rng = np.random.default_rng(3)
    hidden, vocab = 512, 40
    raw = rand_blocks(O, 12, vocab * hidden // 256, rng)
    tb, ob = gpu.Buffer.of(raw), gpu.Buffer(hidden * 4)
    toks = gpu.Buffer.of(np.array([5, 33, vocab, -1], np.int32))
    st = gpu.Buffer.of(np.zeros(1, np.int32))
    lib = gpu.native.lib()
    gpu.native.check(lib.cj_embed_row_slot(ob.h, tb.h, 12, hidden, vocab, toks.h, 1, st.h), "embed slot")
    rb = hidden // 256 * 144
    ref = O.dequant(12, raw[33 * rb:34 * rb])
    assert np.array_equal(ob.download(np.float32, hidden).view(np.uint32), ref.view(np.uint32))
    assert st.download(np.int32, 1)[0] == 0
    for slot in (2, 3):
        gpu.native.check(lib.cj_embed_row_slot(ob.h, tb.h, 12, hidden, vocab, toks.h, slot, st.h), "embed slot")
        assert not ob.download(np.float32, hidden).any()
        assert st.download(np.int32, 1)[0] == 1
    # extents: a slot past the token buffer is refused on the host
    assert lib.cj_embed_row_slot(ob.h, tb.h, 12, hidden, vocab, toks.h, 4, 0) == gpu.native.CJ_ERR_ARG


def test_kernel_registry_answers_reference_names(gpu):
    for name in ("q4kQ8WaveMatVecKernel", "q6kQ8WaveMatVecKernel", "q80Q8WaveMatVecKernel", "q8kPackKernel",
                 "rmsnormPackRowF32", "gluPackF32", "qkPrepKernel", "attnFlashDecodeGqa4Kernel",
                 "attnFlashDecodeGqa8Kernel", "attnReducePackQ8Kernel", "argmaxRowKernel", "embedRowQ4kKernel",
                 "routerTopKKernel", "mxfp4MatVecKernel", "attnScoreKernel"):
        assert gpu.KernelCap.usable(name), name
    assert not gpu.KernelCap.usable("iq2xxsQ8WaveMatVecKernel")
    # names whose semantics this backend does not serve are refused: the
    # fused MoE id kernels (their combine, Q4_K experts), CPU-backend kernels
    # (the 8-row interleave products among them) and the MXFP4 activation
    # quant as a launch of its own (here it is a GEMV's prologue, and no
    # kernel writes the codes a following launch would read)
    for name in ("q4kQ8IdDownCombineKernel", "q4kQ8IdGateUpGluKernel", "attnDecodeCpuGqaKernel",
                 "attnPrefillCpuGqaKernel", "q4kQ8X8RowsKernel", "q80Q8X8RowsKernel", "mxfp4QuantActKernel"):
        assert not gpu.KernelCap.usable(name), name
    gpu.KernelCap.setOverride("q4kQ8WaveMatVecKernel", False)
    assert not gpu.KernelCap.usable("q4kQ8WaveMatVecKernel")
    gpu.KernelCap.clearOverrides()
    assert gpu.KernelCap.usable("q4kQ8WaveMatVecKernel")


@pytest.mark.parametrize("name,ty", [("q8_0", 8), ("q4_k", 12), ("q6_k", 14), ("q4_0", 2)])
@pytest.mark.parametrize("rows,cols,ncols", [(300, 512, 1), (1024, 4096, 4), (64, 1408, 8), (272, 4096, 17),
                                             (96, 14336, 16), (160, 2048, 70), (100, 1408, 80), (40, 512, 33),
                                             (130, 768, 200), (37, 4096, 5), (48, 2560, 24)])
def test_matmul_columns_equal_matvec(gpu, O, name, ty, rows, cols, ncols):
    """The batched product (int8 matrix cores for Q8_0 and Q4_K, the
    many-column GEMV for Q6_K and Q4_0): every output column is the one-column
    product of its activation pack (Q4_0: of its f32 column), bit for bit
    (integer sub-block dots are exact; the float fold runs in the reference's
    block order; Q4_0's block dots in its element order)."""
    if ty in (O.Q4_K, O.Q6_K) and cols % 256:
        pytest.skip("K-quant rows are whole 256-element blocks")
    say("matmul", name, rows, cols, ncols)
    rng = np.random.default_rng(rows * 7 + cols + ncols + ty)
    be, bb = O.BLOCK[ty]
    raw = rand_blocks(O, ty, rows * cols // be, rng)
    lib = gpu.native.lib()
    prb = lib.cj_prepared_row_bytes(ty, cols)
    src, w = gpu.Buffer.of(raw), gpu.Buffer(prb * rows)
    gpu.native.check(lib.cj_prepare_weight(w.h, src.h, ty, rows, cols), "prepare")
    npad = (cols + 255) // 256 * 256
    f32cols = ty == O.Q4_0
    used = cols * 4 if f32cols else npad // 256 * 320
    stride = used + 64                                  # a gap between columns the kernel must skip
    packs = np.zeros((ncols, stride), np.uint8)
    for c in range(ncols):
        x = (rng.standard_normal(cols) * rng.uniform(0.1, 4)).astype(np.float32)
        packs[c, :used] = x.view(np.uint8) if f32cols else O.q8k_pack(x, per32=(ty == O.Q8_0), npad=npad)
    ystride, yoff = rows + 5, 3
    y0 = rng.standard_normal((ncols, ystride)).astype(np.float32)
    xb = gpu.Buffer.of(packs.reshape(-1))
    for accum in (0, 1):
        yb = gpu.Buffer.of(y0.reshape(-1))
        gpu.native.check(lib.cj_matmul(ty, yb.h, w.h, xb.h, rows, cols, ncols, stride, ystride, yoff, accum), "matmul")
        got = yb.download(np.float32, ncols * ystride).reshape(ncols, ystride)
        for c in range(ncols):
            ref = (O.matvec(ty, raw, rows, cols, packs[c, :used].view(np.float32)) if f32cols
                   else O.matvec_packed(ty, raw, rows, cols, packs[c, :used]))
            if accum:
                ref = (y0[c, yoff:yoff + rows] + ref).astype(np.float32)
            assert np.array_equal(got[c, yoff:yoff + rows].view(np.uint32), ref.view(np.uint32)), \
                "%s column %d accum %d: %d rows differ" % (name, c, accum, int((got[c, yoff:yoff + rows] != ref).sum()))
            # outside the column's rows nothing is written
            assert np.array_equal(got[c, :yoff], y0[c, :yoff]) and np.array_equal(got[c, yoff + rows:], y0[c, yoff + rows:])
        yb.free()


@pytest.mark.parametrize("name,ty", [("q8_0", 8), ("q4_0", 2), ("q4_k", 12), ("q6_k", 14)])
@pytest.mark.parametrize("rows,cols", [(4096, 4096), (14336, 4096), (4096, 14336), (128256, 4096)])
def test_c2_shapes_match_oracle(gpu, O, name, ty, rows, cols):
    """The C2 microbenchmark's shapes and kernels, outputs checked: the
    batch-1 GEMV and the 16-column product (the launches bench.py times),
    every output bit for bit the oracle's mat-vec of its column."""
    say("c2 shape", name, rows, cols)
    rng = np.random.default_rng(rows + cols + ty)
    be, bb = O.BLOCK[ty]
    raw = rand_blocks(O, ty, rows * cols // be, rng)
    lib = gpu.native.lib()
    prb = lib.cj_prepared_row_bytes(ty, cols)
    src, w = gpu.Buffer.of(raw), gpu.Buffer(prb * rows)
    gpu.native.check(lib.cj_prepare_weight(w.h, src.h, ty, rows, cols), "prepare")
    src.free()
    B = 16
    x = rng.standard_normal((B, cols)).astype(np.float32)
    f32cols = ty == O.Q4_0
    if f32cols:
        act, stride = gpu.Buffer.of(x.reshape(-1)), cols * 4
    else:
        packs = np.stack([O.q8k_pack(x[c], per32=(ty == O.Q8_0)) for c in range(B)])
        act, stride = gpu.Buffer.of(packs.reshape(-1)), packs.shape[1]
    refs = [O.matvec(ty, raw, rows, cols, x[c]) for c in range(B)]
    y = gpu.Buffer(B * rows * 4)
    gpu.native.check(lib.cj_matvec(ty, y.h, w.h, act.h, rows, cols, 0, 0), "matvec")
    got = y.download(np.float32, rows)
    assert np.array_equal(got.view(np.uint32), refs[0].view(np.uint32)), \
        "%s %dx%d batch 1: %d rows differ" % (name, rows, cols, int((got != refs[0]).sum()))
    gpu.native.check(lib.cj_matmul(ty, y.h, w.h, act.h, rows, cols, B, stride, rows, 0, 0), "matmul")
    got = y.download(np.float32, B * rows).reshape(B, rows)
    for c in range(B):
        assert np.array_equal(got[c].view(np.uint32), refs[c].view(np.uint32)), \
            "%s %dx%d batch %d column %d: %d rows differ" % (name, rows, cols, B, c, int((got[c] != refs[c]).sum()))
    for b in (w, act, y):
        b.free()


def test_matmul_refuses_short_buffers(gpu, O):
    lib = gpu.native.lib()
    prb = lib.cj_prepared_row_bytes(12, 256)
    w, xp, y = gpu.Buffer(prb * 64), gpu.Buffer(320 * 3), gpu.Buffer(64 * 4 * 4)
    assert lib.cj_matmul(12, y.h, w.h, xp.h, 64, 256, 4, 320, 64, 0, 0) == -1
    assert "activation" in gpu.native.last_error()
    assert lib.cj_matmul(6, y.h, w.h, xp.h, 64, 256, 1, 320, 64, 0, 0) == -1


def test_qk_prep_with_norm_matches_the_reference_cpu_golden(gpu, O):
    """QK-norm + RoPE + K/V append at hd 128 against the reference CPU
    backend's recorded q and k (QkPrepTest.run(32, 4, 128, true): position
    11, eps 1e-6, the test's own inv-frequency fill), bit for bit; the RoPE
    table holds f32 cos/sin of pos·inv (glibc cosf/sinf reproduce the
    recording)."""
    import ctypes
    from reference_goldens import cpu_golden_rows, qkprep_fill
    g = cpu_golden_rows()
    n_q, n_kv, hd, pos = 32, 4, 128, 11
    q, k, v = qkprep_fill(n_q * hd, 1), qkprep_fill(n_kv * hd, 2), qkprep_fill(n_kv * hd, 3)
    qw, kw, inv = qkprep_fill(hd, 4), qkprep_fill(hd, 5), qkprep_fill(hd // 2, 6)
    libm = ctypes.CDLL("libm.so.6")
    libm.cosf.restype = libm.sinf.restype = ctypes.c_float
    libm.cosf.argtypes = libm.sinf.argtypes = [ctypes.c_float]
    tab = np.zeros((pos + 1, hd // 2, 2), np.float32)
    for d in range(hd // 2):
        ang = float(np.float32(pos) * inv[d])
        tab[pos, d] = (libm.cosf(ang), libm.sinf(ang))
    lib = gpu.native.lib()
    qb, kb, vb = gpu.Buffer.of(q), gpu.Buffer.of(k), gpu.Buffer.of(v)
    qwb, kwb, rope = gpu.Buffer.of(qw), gpu.Buffer.of(kw), gpu.Buffer.of(tab.reshape(-1))
    kc, vc = gpu.Buffer(n_kv * 64 * hd * 2), gpu.Buffer(n_kv * 64 * hd * 2)
    pg = gpu.Buffer.of(np.zeros(1, np.int32))
    gpu.native.check(lib.cj_qk_prep(qb.h, kb.h, vb.h, kc.h, vc.h, qwb.h, kwb.h, rope.h, pg.h, 0, n_q, n_kv, hd, 1,
                                    1e-6, 0, pos), "qk_prep")
    gq, gk = qb.download(np.float32, q.size), kb.download(np.float32, k.size)
    assert np.array_equal(gq.view(np.uint32), g[("qkPrepKernel", "h32kv4d128-q")].view(np.uint32))
    assert np.array_equal(gk.view(np.uint32), g[("qkPrepKernel", "h32kv4d128-k")].view(np.uint32))
    kcache = kc.download(np.uint16, n_kv * 64 * hd).reshape(n_kv, 64, hd)
    assert np.array_equal(kcache[:, pos % 64, :].reshape(-1), O.f32_to_f16_bits(gk))


def test_attn_merge_pack_matches_the_reference_cpu_golden(gpu, O):
    """The split merge + per-256 q8 pack of 32 heads × 8 splits against the
    reference CPU backend's recorded bytes (reducePackGolden), bit for bit."""
    from reference_goldens import cpu_golden_rows, reduce_pack_partials
    want = cpu_golden_rows()[("attnReducePackQ8Kernel", "h32s8")]
    n_q, hd, splits = 32, 128, 8
    part = np.zeros((n_q, 64, hd + 2), np.float32)
    part[:, :splits, :] = reduce_pack_partials().reshape(n_q, splits, hd + 2)
    pb, ob, packed = gpu.Buffer.of(part.reshape(-1)), gpu.Buffer(n_q * hd * 4), gpu.Buffer(n_q * hd // 256 * 320)
    gpu.native.check(gpu.native.lib().cj_attn_merge(ob.h, packed.h, pb.h, n_q, hd, splits, 0), "merge")
    got = packed.download(np.uint8, n_q * hd // 256 * 320).view(np.int8).astype(np.float32)
    assert np.array_equal(got, want)


def test_router_topk_matches_the_reference_cpu_golden(gpu, O):
    """routerTopKKernel's launch (the router mat-vec and its top-k in one)
    against the reference CPU backend's recorded e128h2048k8 logits, picks and
    weights (TreeSiteReferenceTest.routerTopKKernelStaysWithinItsBar: 128
    experts, 2048 columns, top-8, renormalised), bit for bit, and against the
    oracle on a case with an exact tie and a w_scale; the counter is left
    zero for the next launch."""
    from reference_goldens import cpu_golden_rows, spread
    g = cpu_golden_rows()
    lib = gpu.native.lib()

    def run(w, x, E, H, k, norm, scale):
        wb, xb = gpu.Buffer.of(w.reshape(-1)), gpu.Buffer.of(x)
        lg, sel, wt = gpu.Buffer(E * 4), gpu.Buffer(k * 4), gpu.Buffer(k * 4)
        ctr = gpu.Buffer.of(np.zeros(4, np.int32))
        gpu.native.check(lib.cj_router_topk(sel.h, wt.h, lg.h, wb.h, xb.h, ctr.h, E, H, k, int(norm), scale), "router")
        out = lg.download(np.float32, E), sel.download(np.int32, k), wt.download(np.float32, k)
        assert ctr.download(np.int32, 1)[0] == 0
        return out

    say("router top-k e128h2048k8")
    w, x = spread(128 * 2048, 7), spread(2048, 11)
    lg, sel, wt = run(w, x, 128, 2048, 8, True, 0.0)
    assert np.array_equal(lg.view(np.uint32), g[("routerTopKKernel", "e128h2048k8-logits")].view(np.uint32))
    assert np.array_equal(sel.astype(np.float32), g[("routerTopKKernel", "e128h2048k8-sel")])
    assert np.array_equal(wt.view(np.uint32), g[("routerTopKKernel", "e128h2048k8-w")].view(np.uint32))
    rng = np.random.default_rng(21)
    E, H, k = 40, 512, 6
    w = (rng.standard_normal((E, H)) * 0.05).astype(np.float32)
    w[9] = w[4] = (np.abs(w[4]) * 2).astype(np.float32)
    x = np.abs(rng.standard_normal(H)).astype(np.float32)
    for norm, scale in ((True, 2.5), (False, 0.0)):
        got = run(w, x, E, H, k, norm, scale)
        want = O.router_topk(w, x, E, H, k, norm, scale)
        for a, b in zip(got, want):
            assert np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))
        assert list(got[1][:2]) == [4, 9]


def test_attn_scores_match_the_reference_cpu_golden(gpu, O):
    """attnScoreKernel's launch (the two-pass decode attention's score pass)
    at the reference's recorded shape — 32 query heads, 4 kv heads of 128,
    256 positions, TreeSiteReferenceTest.attnScoreKernelStaysWithinItsBar's
    inputs — bit for bit against the oracle's scores, whose softmax exps are
    the recorded row bit for bit (tests/test_oracle.py); the K rows sit in
    this backend's paged layout, the pages in a shuffled order."""
    from reference_goldens import spread
    say("attention scores h32kv4d128c256")
    nh, nkv, hd, count = 32, 4, 128, 256
    q = spread(nh * hd, 3)
    kh = spread(count * nkv * hd, 5).astype(np.float16).reshape(count, nkv, hd)
    pages = np.array([3, 0, 2, 1], np.int32)             # position block j lives in page pages[j]
    plane = np.zeros((4, nkv, 64, hd), np.float16)
    for t in range(count):
        plane[pages[t // 64], :, t % 64, :] = kh[t]
    scale = float(np.float32(1) / np.sqrt(np.float32(hd)))
    qb, kb, tb, sb = gpu.Buffer.of(q), gpu.Buffer.of(plane.view(np.uint16).reshape(-1)), gpu.Buffer.of(pages), \
        gpu.Buffer(nh * count * 4)
    gpu.native.check(gpu.native.lib().cj_attn_scores(sb.h, qb.h, kb.h, tb.h, 0, nh, nkv, hd, count, 0, scale), "scores")
    got = sb.download(np.float32, nh * count)
    want = O.attn_scores(q, kh.reshape(count, nkv * hd).view(np.uint16), nh, nkv, hd, count, scale)
    assert np.array_equal(got.view(np.uint32), want.reshape(-1).view(np.uint32))


def test_qk_prep_hd64_with_norm_matches_the_reference_cpu_golden(gpu, O):
    """QK-norm + RoPE at head size 64 — the generic qkPrepKernel, whose norm
    sums in 32-lane waves from the adjacent lane up — against the reference
    CPU backend's recorded q and k (QkPrepTest.run(6, 2, 64, true)), bit for
    bit, and the fp16 K row appended."""
    import ctypes
    from reference_goldens import cpu_golden_rows, qkprep_fill
    g = cpu_golden_rows()
    n_q, n_kv, hd, pos = 6, 2, 64, 11
    q, k, v = qkprep_fill(n_q * hd, 1), qkprep_fill(n_kv * hd, 2), qkprep_fill(n_kv * hd, 3)
    qw, kw, inv = qkprep_fill(hd, 4), qkprep_fill(hd, 5), qkprep_fill(hd // 2, 6)
    libm = ctypes.CDLL("libm.so.6")
    libm.cosf.restype = libm.sinf.restype = ctypes.c_float
    libm.cosf.argtypes = libm.sinf.argtypes = [ctypes.c_float]
    tab = np.zeros((pos + 1, hd // 2, 2), np.float32)
    for d in range(hd // 2):
        ang = float(np.float32(pos) * inv[d])
        tab[pos, d] = (libm.cosf(ang), libm.sinf(ang))
    lib = gpu.native.lib()
    qb, kb, vb = gpu.Buffer.of(q), gpu.Buffer.of(k), gpu.Buffer.of(v)
    qwb, kwb, rope = gpu.Buffer.of(qw), gpu.Buffer.of(kw), gpu.Buffer.of(tab.reshape(-1))
    kc, vc = gpu.Buffer(n_kv * 64 * hd * 2), gpu.Buffer(n_kv * 64 * hd * 2)
    pg = gpu.Buffer.of(np.zeros(1, np.int32))
    gpu.native.check(lib.cj_qk_prep(qb.h, kb.h, vb.h, kc.h, vc.h, qwb.h, kwb.h, rope.h, pg.h, 0, n_q, n_kv, hd, 1,
                                    1e-6, 0, pos), "qk_prep")
    gq, gk = qb.download(np.float32, q.size), kb.download(np.float32, k.size)
    assert np.array_equal(gq.view(np.uint32), g[("qkPrepKernel", "h6kv2d64-q")].view(np.uint32))
    assert np.array_equal(gk.view(np.uint32), g[("qkPrepKernel", "h6kv2d64-k")].view(np.uint32))
    kcache = kc.download(np.uint16, n_kv * 64 * hd).reshape(n_kv, 64, hd)
    assert np.array_equal(kcache[:, pos % 64, :].reshape(-1), O.f32_to_f16_bits(gk))


def test_allocating_argmax_refuses_a_graph_capture(gpu):
    """cj_argmax_row may grow its scratch (a synchronize, an allocation and a
    memset, none of which a capture may record): it refuses while the stream
    is capturing and leaves the capture intact; the allocation-free entry
    point serves there."""
    lib = gpu.native.lib()
    v = gpu.Buffer.of(np.arange(5000, dtype=np.float32))
    tb = gpu.Buffer.of(np.full(2, -1, np.int32))
    gpu.native.check(lib.cj_graph_begin(), "graph begin")
    rc = lib.cj_argmax_row(tb.h, 0, v.h, 5000)
    msg = gpu.native.last_error()
    rc2 = lib.cj_argmax_row_noalloc(tb.h, 1, v.h, 5000)
    gh = lib.cj_graph_end()
    assert rc == gpu.native.CJ_ERR_STATE and "capturing" in msg
    assert rc2 == 0 and gh > 0
    gpu.native.check(lib.cj_graph_launch(gh), "graph launch")
    gpu.native.check(lib.cj_stream_sync(), "sync")
    assert list(tb.download(np.int32, 2)) == [-1, 4999]
    gpu.native.check(lib.cj_graph_free(gh), "graph free")
    gpu.native.check(lib.cj_argmax_row(tb.h, 0, v.h, 5000), "argmax")
    assert tb.download(np.int32, 1)[0] == 4999
