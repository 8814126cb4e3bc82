"""Write a GGUF as a split model the way llama.cpp's gguf-split lays one out
(and the reference's GgufFile reads it, io/GgufFile.cajeta:45-55): shard k
of n is <base>-%05d-of-%05d.gguf (numbered from 1); shard 1 keeps the
model's metadata and adds split.no / split.count / split.tensors.count, the
others carry only those three keys; every shard has its own tensor
directory over its own tensors and its own aligned data section."""
import struct

import numpy as np

_FIXED = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}
_BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 8: (32, 34), 12: (256, 144), 14: (256, 210), 39: (32, 17), 30: (1, 2)}


def _skip_value(b, at, ty):
    if ty in _FIXED:
        return at + _FIXED[ty]
    if ty == 8:
        (n,) = struct.unpack_from("<Q", b, at)
        return at + 8 + n
    if ty == 9:
        et, cnt = struct.unpack_from("<IQ", b, at)
        at += 12
        for _ in range(cnt):
            at = _skip_value(b, at, et)
        return at
    raise ValueError("GGUF value type %d" % ty)


def _str(s):
    e = s.encode()
    return struct.pack("<Q", len(e)) + e


def _kv_i32(key, v):
    return _str(key) + struct.pack("<Ii", 5, v)


def _kv_u16(key, v):
    return _str(key) + struct.pack("<IH", 2, v)


def split_gguf(src, prefix, n):
    """Split GGUF file `src` into n shards named prefix-%05d-of-%05d.gguf;
    returns their paths."""
    b = open(src, "rb").read()
    magic, ver, nt, nkv = struct.unpack_from("<IIQQ", b, 0)
    assert magic == 0x46554747 and ver in (2, 3)
    at = 24
    kv_start = at
    align = 32
    for _ in range(nkv):
        (kl,) = struct.unpack_from("<Q", b, at)
        key = b[at + 8:at + 8 + kl].decode()
        at += 8 + kl
        (ty,) = struct.unpack_from("<I", b, at)
        at += 4
        if key == "general.alignment":
            align = struct.unpack_from("<I", b, at)[0]
        at = _skip_value(b, at, ty)
    kv_raw = b[kv_start:at]
    tensors = []
    for _ in range(nt):
        (nl,) = struct.unpack_from("<Q", b, at)
        name = b[at + 8:at + 8 + nl].decode()
        at += 8 + nl
        (nd,) = struct.unpack_from("<I", b, at)
        dims = struct.unpack_from("<%dQ" % nd, b, at + 4)
        ty, off = struct.unpack_from("<IQ", b, at + 4 + 8 * nd)
        at += 4 + 8 * nd + 12
        be, bb = _BLOCK[ty]
        nbytes = int(np.prod(dims)) // be * bb
        tensors.append((name, dims, ty, off, nbytes))
    data0 = (at + align - 1) // align * align
    parts = [tensors[k::n] for k in range(n)]
    paths = []
    for k, part in enumerate(parts):
        keys = _kv_u16("split.no", k) + _kv_u16("split.count", n) + _kv_i32("split.tensors.count", nt)
        kvs, nkeys, al = (kv_raw + keys, nkv + 3, align) if k == 0 else (keys, 3, 32)
        infos, blobs, off = b"", [], 0
        for name, dims, ty, src_off, nbytes in part:
            infos += _str(name) + struct.pack("<I", len(dims)) + struct.pack("<%dQ" % len(dims), *dims)
            infos += struct.pack("<IQ", ty, off)
            blobs.append(b[data0 + src_off:data0 + src_off + nbytes])
            off = (off + nbytes + al - 1) // al * al
        head = struct.pack("<IIQQ", magic, 3, len(part), nkeys) + kvs + infos
        head += b"\0" * ((-len(head)) % al)
        out = bytearray(head)
        for blob in blobs:
            out += blob
            out += b"\0" * ((-len(out)) % al)
        p = "%s-%05d-of-%05d.gguf" % (prefix, k + 1, n)
        open(p, "wb").write(bytes(out))
        paths.append(p)
    return paths
