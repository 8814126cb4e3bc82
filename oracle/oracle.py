"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker. The product never imports it.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, MXFP4 = 0, 1, 2, 8, 12, 14, 39
BLOCK = {F32: (1, 4), F16: (1, 2), Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144),
         Q6_K: (256, 210), MXFP4: (32, 17)}


def build():
    subprocess.check_call(["make", "-s", "-C", HERE])


_lib = None


class Config(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in
                ("n_layers", "hidden", "n_heads", "n_kv", "head_dim", "ffn", "vocab", "ctx")] + \
               [("eps", ctypes.c_float), ("theta", ctypes.c_float)] + \
               [(n, ctypes.c_int32) for n in
                ("kv_f32", "workers", "n_experts", "n_used", "norm_topk", "expert_ffn", "swa_window", "attn_rows")] + \
               [("w_scale", ctypes.c_float), ("swa_pattern", ctypes.c_int32)]


def load(path):
    """A configured handle on an oracle build at `path`."""
    L = ctypes.CDLL(path)
    _configure(L)
    return L


def use(L):
    """Route the wrappers below through library `L` (None: the default build);
    returns the previous one. Tests use it for planted-mistake builds."""
    global _lib
    prev, _lib = _lib, L
    return prev


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = load(LIB_PATH)
    return _lib


def _configure(L):
    if True:
        P, I64, I32, F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
        sig = {
            "or_block_bytes": (I32, [I32]), "or_block_elems": (I32, [I32]),
            "or_f16_to_f32": (F, [ctypes.c_uint16]), "or_f32_to_f16": (ctypes.c_uint16, [F]),
            "or_dequant": (I32, [I32, P, I64, P]),
            "or_q8k_pack": (None, [P, I64, I64, P]), "or_q8k_pack32": (None, [P, I64, I64, P]),
            "or_matvec": (I32, [I32, P, I64, I64, P, P, P]),
            "or_mxfp4_quant_act": (None, [P, I64, P, P]),
            "or_matvec_mxfp4_q8": (I32, [P, I64, I64, P, P]),
            "or_rmsnorm": (None, [P, P, I64, F, I32, P]),
            "or_glu_exp": (None, [P, P, I64, P]), "or_glu_tanh": (None, [P, P, I64, P]),
            "or_inv_freq": (None, [I32, F, P]), "or_rope": (None, [P, I32, I32, I32, P]),
            "or_argmax": (I32, [P, I64]), "or_moe_route": (I32, [P, I32, I32, I32, F, P, P]),
            "or_unpermute_rows": (None, [P, P, I64, I64, I32]),
            "or_attend": (None, [P, P, P, I32, I32, I32, I32, I32, I32, F, I32, P]),
            "or_cpu_decode_splits": (I32, [I32, I32, I32, I32]),
            "or_prefill_attend": (None, [P, P, P, I32, I32, I32, I32, I32, I32, I32, F, P]),
            "or_attn_merge": (None, [P, I32, I32, I32, P]),
            "or_qk_prep128": (I32, [P, P, P, P, P, I32, I32, I32, F, I32, I32]),
            "or_qk_prep": (I32, [P, P, P, P, P, I32, I32, I32, I32, F, I32, I32]),
            "or_router_topk": (None, [P, P, I32, I32, I32, I32, F, P, P, P]),
            "or_attn_scores": (None, [P, P, I32, I32, I32, I32, I32, F, I32, P]),
            "or_exp2_table": (None, [P]),
            "or_model_prefill": (I32, [P, P, I32, I32, P]),
            "or_expf": (F, [F]),
            "or_model_new": (P, [ctypes.POINTER(Config)]), "or_model_free": (None, [P]),
            "or_model_bind": (I32, [P, ctypes.c_char_p, I32, P, I64, I64]),
            "or_model_step": (I32, [P, I32, I32, P]), "or_model_reset": (None, [P]),
            "or_model_set_workers": (None, [P, I32]),
            "or_model_set_rope_freqs": (I32, [P, P, I32]),
            "or_model_threads": (I32, []),
            "or_model_trace": (I64, [P, I32, P, I64]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def dequant(ty, raw):
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    be, bb = BLOCK[ty]
    nb = raw.size // bb
    out = np.empty(nb * be, np.float32)
    assert lib().or_dequant(ty, _p(raw), nb, _p(out)) == 0
    return out


def f32_to_f16_bits(x):
    x = np.asarray(x, np.float32).ravel()
    return np.array([lib().or_f32_to_f16(float(v)) for v in x], np.uint16)


def f16_bits_to_f32(h):
    h = np.asarray(h, np.uint16).ravel()
    return np.array([lib().or_f16_to_f32(int(v)) for v in h], np.float32)


def q8k_pack(x, per32=False, npad=None):
    x = np.ascontiguousarray(x, np.float32)
    n = x.size
    npad = npad or (n + 255) // 256 * 256
    out = np.zeros(npad // 256 * 320, np.uint8)
    (lib().or_q8k_pack32 if per32 else lib().or_q8k_pack)(_p(x), n, npad, _p(out))
    return out


def matvec(ty, w, rows, cols, x):
    """y = W x the way the reference CPU backend computes it for format `ty`
    (packing x first where that format reads int8 activations)."""
    w = np.ascontiguousarray(w, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.float32)
    xp = np.zeros(1, np.uint8)
    if ty in (Q4_K, Q6_K):
        xp = q8k_pack(x)
    elif ty == Q8_0:
        xp = q8k_pack(x, per32=True)
    assert lib().or_matvec(ty, _p(w), rows, cols, _p(xp), _p(x), _p(y)) == 0
    return y


def mxfp4_quant_act(x):
    """The per-32 activation quant of the MXFP4 device Q8 form: (int8 codes, scales)."""
    x = np.ascontiguousarray(x, np.float32)
    xq = np.empty(x.size, np.int8)
    xd = np.empty(x.size // 32, np.float32)
    lib().or_mxfp4_quant_act(_p(x), x.size, _p(xq), _p(xd))
    return xq, xd


def matvec_mxfp4_q8(w, rows, cols, x):
    """y = W x in the MXFP4 device Q8 form (activation quant, then the
    32-lane integer dot and butterfly)."""
    w = np.ascontiguousarray(w, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.float32)
    assert lib().or_matvec_mxfp4_q8(_p(w), rows, cols, _p(x), _p(y)) == 0
    return y


def matvec_packed(ty, w, rows, cols, xp):
    w = np.ascontiguousarray(w, np.uint8)
    xp = np.ascontiguousarray(xp, np.uint8)
    y = np.empty(rows, np.float32)
    dummy = np.zeros(1, np.float32)
    assert lib().or_matvec(ty, _p(w), rows, cols, _p(xp), _p(dummy), _p(y)) == 0
    return y


def rmsnorm(x, w, eps=1e-5, form=0):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    lib().or_rmsnorm(_p(x), _p(w), x.size, eps, form, _p(out))
    return out


def glu(g, u, form="exp"):
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    out = np.empty_like(g)
    (lib().or_glu_exp if form == "exp" else lib().or_glu_tanh)(_p(g), _p(u), g.size, _p(out))
    return out


def inv_freq(hd, theta):
    out = np.empty(hd // 2, np.float32)
    lib().or_inv_freq(hd, theta, _p(out))
    return out


def rope(t, nheads, hd, pos, inv):
    t = np.array(t, np.float32, copy=True)
    inv = np.ascontiguousarray(inv, np.float32)
    lib().or_rope(_p(t), nheads, hd, pos, _p(inv))
    return t


def argmax(v):
    v = np.ascontiguousarray(v, np.float32)
    return lib().or_argmax(_p(v), v.size)


def moe_route(logits, k, norm=True, w_scale=0.0):
    logits = np.ascontiguousarray(logits, np.float32)
    sel = np.empty(k, np.int32)
    w = np.empty(k, np.float32)
    rc = lib().or_moe_route(_p(logits), logits.size, k, int(norm), float(w_scale), _p(sel), _p(w))
    if rc != 0:
        raise ValueError("moe router: logits are not finite")
    return sel, w


def unpermute_rows(src, rows, row_bytes, n_head):
    src = np.ascontiguousarray(src, np.uint8)
    dst = np.empty_like(src)
    lib().or_unpermute_rows(_p(src), _p(dst), rows, row_bytes, n_head)
    return dst


def attend(q, kplane, vplane, n_h, n_kv, hd, count, splits, scale, mode, kv_f32=False):
    q = np.ascontiguousarray(q, np.float32)
    kplane = np.ascontiguousarray(kplane)
    vplane = np.ascontiguousarray(vplane)
    out = np.empty(n_h * hd, np.float32)
    lib().or_attend(_p(q), _p(kplane), _p(vplane), int(kv_f32), n_h, n_kv, hd, count, splits,
                    scale, mode, _p(out))
    return out


def expf(x):
    """The written-out f32 exp the restatement (and the kernels) use."""
    return np.array([lib().or_expf(float(v)) for v in np.asarray(x, np.float32).ravel()], np.float32)


def prefill_attend(q, kplane, vplane, n_h, n_kv, hd, start, rows, window, scale, kv_f32=False):
    q = np.ascontiguousarray(q, np.float32)
    out = np.empty(rows * n_h * hd, np.float32)
    lib().or_prefill_attend(_p(q), _p(np.ascontiguousarray(kplane)), _p(np.ascontiguousarray(vplane)), int(kv_f32),
                            n_h, n_kv, hd, start, rows, window, scale, _p(out))
    return out


def attn_merge(part, n_h, splits, hd):
    """Merge split partials [n_h][splits][hd+2] in the reference's order."""
    part = np.ascontiguousarray(part, np.float32)
    out = np.empty(n_h * hd, np.float32)
    lib().or_attn_merge(_p(part), n_h, splits, hd, _p(out))
    return out


def qk_prep128(q, k, qw, kw, inv, n_h, n_kv, norm, eps, form, pos):
    """The CPU decode prep at head size 128: QK-norm (optional) and RoPE."""
    q = np.array(q, np.float32, copy=True)
    k = np.array(k, np.float32, copy=True)
    lib().or_qk_prep128(_p(q), _p(k), _p(np.ascontiguousarray(qw, np.float32)), _p(np.ascontiguousarray(kw, np.float32)),
                        _p(np.ascontiguousarray(inv, np.float32)), n_h, n_kv, int(norm), float(eps), int(form), int(pos))
    return q, k


def qk_prep(q, k, qw, kw, inv, n_h, n_kv, hd, norm, eps, form, pos):
    """The generic qkPrepKernel at any head size (head size 128: the CPU kernel)."""
    q = np.array(q, np.float32)
    k = np.array(k, np.float32)
    rc = lib().or_qk_prep(_p(q), _p(k), _p(np.asarray(qw, np.float32)), _p(np.asarray(kw, np.float32)),
                          _p(np.asarray(inv, np.float32)), n_h, n_kv, hd, int(norm), float(eps), form, pos)
    assert rc == 0
    return q, k


def router_topk(w, x, experts, cols, used, norm_topk=True, w_scale=0.0):
    """routerTopKKernel: (logits, sel, weights)."""
    w = np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    lg = np.zeros(experts, np.float32)
    sel = np.zeros(used, np.int32)
    wt = np.zeros(used, np.float32)
    lib().or_router_topk(_p(w), _p(x), experts, cols, used, int(norm_topk), float(w_scale), _p(lg), _p(sel), _p(wt))
    return lg, sel, wt


def attn_scores(q, kplane, n_h, n_kv, hd, count, scale, softmax=False, kv_f32=False):
    """attnScoreKernel's scores [n_h][count] over a position-major K plane
    (fp16 bits, or f32); softmax: attnCombineKernel's in-place exp(s − max)."""
    q = np.ascontiguousarray(q, np.float32)
    kplane = np.ascontiguousarray(kplane)
    out = np.zeros((n_h, count), np.float32)
    lib().or_attn_scores(_p(q), _p(kplane), int(kv_f32), n_h, n_kv, hd, count, float(scale), int(softmax), _p(out))
    return out


def exp2_table():
    t = np.zeros(32, np.uint64)
    lib().or_exp2_table(_p(t))
    return t


def cpu_decode_splits(count, rows, n_kv, workers):
    return lib().or_cpu_decode_splits(count, rows, n_kv, workers)


class Model:
    """The whole-model decode restatement over tensors bound by GGUF name."""

    def __init__(self, cfg: dict):
        c = Config()
        for k, v in cfg.items():
            setattr(c, k, v)
        self.cfg = c
        self._keep = []
        self.h = lib().or_model_new(ctypes.byref(c))

    def bind(self, name, ty, data, rows, cols):
        data = np.ascontiguousarray(data)
        self._keep.append(data)
        rc = lib().or_model_bind(self.h, name.encode(), ty, _p(data), rows, cols)
        if rc != 0:
            raise KeyError(name)

    def step(self, token, pos, want_logits=True):
        lg = np.empty(self.cfg.vocab, np.float32) if want_logits else None
        t = lib().or_model_step(self.h, token, pos, _p(lg) if want_logits else None)
        return t, lg

    def prefill(self, tokens, start, want_logits=True):
        """A prefill chunk at positions start.. (the many-row forward); the
        greedy token and logits of its last row."""
        t = np.ascontiguousarray(tokens, np.int32)
        lg = np.empty(self.cfg.vocab, np.float32) if want_logits else None
        tok = lib().or_model_prefill(self.h, _p(t), int(t.size), int(start), _p(lg) if want_logits else None)
        return tok, lg

    def reset(self):
        lib().or_model_reset(self.h)

    def set_rope_freqs(self, factors):
        """A model's rope_freqs.weight factors (head_dim/2 of them)."""
        f = np.ascontiguousarray(factors, np.float32)
        self._keep.append(f)
        if lib().or_model_set_rope_freqs(self.h, _p(f), int(f.size)) != 0:
            raise ValueError("rope_freqs has %d entries; expected %d (headDim/2)" % (f.size, self.cfg.head_dim // 2))

    def set_workers(self, workers):
        """The split rule's worker count for the steps that follow (KV kept)."""
        lib().or_model_set_workers(self.h, int(workers))
        self.cfg.workers = int(workers)

    def trace(self, what, n):
        out = np.empty(n, np.float32)
        k = lib().or_model_trace(self.h, what, _p(out), n)
        return out[:k]

    def close(self):
        if self.h:
            lib().or_model_free(self.h)
            self.h = None

    def __del__(self):
        self.close()
