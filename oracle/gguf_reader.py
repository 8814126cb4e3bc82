"""A GGUF v2/v3 reader for the checker side (TEST INFRASTRUCTURE ONLY).

Independent of the product's C++ reader, so a parsing mistake on either side
shows up as a disagreement. Follows io/GgufFile.cajeta (alignment :773-777)
of the reference for the header, metadata and tensor table.
"""
import struct

import numpy as np

from . import oracle as O

_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q", 11: "<q", 12: "<d"}


class GgufReader:
    def __init__(self, data):
        if isinstance(data, (str, bytes)) and not isinstance(data, (bytes, bytearray)):
            data = np.memmap(data, dtype=np.uint8, mode="r")
        self.buf = np.asarray(data, dtype=np.uint8)
        self.at = 0
        magic, ver = self._u32(), self._u32()
        if magic != 0x46554747 or ver not in (2, 3):
            raise ValueError("not a GGUF v2/v3 image")
        nt, nkv = self._u64(), self._u64()
        self.meta = {}
        for _ in range(nkv):
            k = self._str()
            self.meta[k] = self._value(self._u32())
        self.tensors = {}
        order = []
        for _ in range(nt):
            name = self._str()
            nd = self._u32()
            dims = [self._u64() for _ in range(nd)]
            ty = self._u32()
            off = self._u64()
            order.append((name, dims, ty, off))
        align = int(self.meta.get("general.alignment", 32)) or 32
        base = (self.at + align - 1) // align * align
        for name, dims, ty, off in order:
            be, bb = O.BLOCK[ty]
            cols = dims[0]
            rows = int(np.prod(dims[1:])) if len(dims) > 1 else 1
            nbytes = cols // be * bb * rows
            self.tensors[name] = (ty, dims, rows, cols, self.buf[base + off: base + off + nbytes])

    def _take(self, n):
        b = self.buf[self.at:self.at + n].tobytes()
        self.at += n
        return b

    def _u32(self):
        return struct.unpack("<I", self._take(4))[0]

    def _u64(self):
        return struct.unpack("<Q", self._take(8))[0]

    def _str(self):
        return self._take(self._u64()).decode("utf-8", errors="replace")

    def _value(self, ty):
        if ty in _SCALAR:
            fmt = _SCALAR[ty]
            return struct.unpack(fmt, self._take(struct.calcsize(fmt)))[0]
        if ty == 8:
            return self._str()
        if ty == 9:
            et, n = self._u32(), self._u64()
            return [self._value(et) for _ in range(n)]
        raise ValueError("unknown GGUF value type %d" % ty)


def model_config(r, workers=512, kv_f32=False, ctx=None, attn_rows=1):
    """The oracle's config from GGUF metadata (model/ModelConfig.cajeta:172-320)."""
    m = r.meta
    arch = m["general.architecture"]
    kp = arch + "."
    hidden = int(m[kp + "embedding_length"])
    heads = int(m[kp + "attention.head_count"])
    emb = r.tensors["token_embd.weight"]
    cfg = dict(
        n_layers=int(m[kp + "block_count"]), hidden=hidden, n_heads=heads,
        n_kv=int(m.get(kp + "attention.head_count_kv", heads)),
        head_dim=int(m.get(kp + "attention.key_length", m.get(kp + "rope.dimension_count", hidden // heads))),
        ffn=int(m[kp + "feed_forward_length"]), vocab=int(m.get(kp + "vocab_size", emb[2])),
        ctx=int(ctx or m.get(kp + "context_length", 4096)),
        eps=float(m.get(kp + "attention.layer_norm_rms_epsilon", 1e-5)),
        theta=float(m.get(kp + "rope.freq_base", 10000.0)),
        kv_f32=int(kv_f32), workers=int(workers),
        n_experts=int(m.get(kp + "expert_count", 0)), n_used=int(m.get(kp + "expert_used_count", 0)),
        norm_topk=int(m.get(kp + "expert_weights_norm", 1)),
        expert_ffn=int(m.get(kp + "expert_feed_forward_length", m[kp + "feed_forward_length"])),
        swa_window=int(m.get(kp + "attention.sliding_window", 0)),
        attn_rows=int(attn_rows),
        w_scale=float(m.get(kp + "expert_weights_scale", 0.0)),
        swa_pattern=int(m.get(kp + "attention.sliding_window_pattern", 2)),
    )
    return cfg


def oracle_model(r, **kw):
    """Bind every tensor of a GGUF into the oracle model, llama q/k rows
    un-permuted to HF order (Checkpoint.unpermuteRows, io/Checkpoint.cajeta:236-274)."""
    cfg = model_config(r, **kw)
    m = O.Model(cfg)
    arch = r.meta["general.architecture"]
    for name, (ty, dims, rows, cols, data) in r.tensors.items():
        d = np.ascontiguousarray(data)
        if arch == "llama" and (name.endswith("attn_q.weight") or name.endswith("attn_k.weight")):
            nh = cfg["n_heads"] if name.endswith("attn_q.weight") else cfg["n_kv"]
            be, bb = O.BLOCK[ty]
            d = O.unpermute_rows(d, rows, cols // be * bb, nh)
        if name == "output.weight" or name.startswith("token_embd") or name.startswith("output_norm") or \
                name.startswith("blk."):
            m.bind(name, ty, d, rows, cols)
    if "output.weight" not in r.tensors:
        ty, dims, rows, cols, data = r.tensors["token_embd.weight"]
        m.bind("output.weight", ty, np.ascontiguousarray(data), rows, cols)
    if "rope_freqs.weight" in r.tensors:   # ModelConfig, model/ModelConfig.cajeta:307-316
        ty, dims, rows, cols, data = r.tensors["rope_freqs.weight"]
        if ty != O.F32:
            raise ValueError("rope_freqs.weight is type %d, not f32" % ty)
        m.set_rope_freqs(np.frombuffer(np.ascontiguousarray(data).tobytes(), np.float32))
    return m, cfg
