"""The C-ABI library: it loads, exports every symbol include/cajeta_mi355x.h
declares (and the ctypes table binds exactly those), and its code object
holds every kernel the runtime registers. No compute calls (no GPU here)."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    src = open(os.path.join(ROOT, "include", "cajeta_mi355x.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(cj_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol(pkg):
    lib = pkg.native.lib()
    names = declared()
    assert len(names) > 40
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(pkg.native.SIGNATURES) == names


def test_code_object_holds_the_registered_kernels(pkg):
    # the code object is a clang offload bundle around the gfx950 ELF; the
    # kernel symbol names are NUL-terminated strings of its string table
    blob = open(pkg.native.HSACO_PATH, "rb").read()
    assert blob.startswith(b"__CLANG_OFFLOAD_BUNDLE__") and b"gfx950" in blob
    syms = set(m.decode() for m in re.findall(rb"(cj_[a-z0-9_]+)\x00", blob))
    src = open(os.path.join(ROOT, "cajeta-llm_amd", "csrc", "runtime", "runtime.cpp")).read()
    table = src[src.index("static const char *kernels[]"):]
    table = table[:table.index("};")]
    registered = re.findall(r'"(cj_[a-z0-9_]+)"', table)
    assert len(registered) >= 30
    missing = [k for k in registered if k not in syms]
    assert not missing, missing


def test_calls_without_init_fail_loudly(pkg):
    lib = pkg.native.lib()
    assert lib.cj_buf_alloc(64) == 0
    assert "cj_init" in pkg.native.last_error()
    assert lib.cj_matvec(12, 0, 0, 0, 1, 256, 0, 0) < 0


def test_prepared_row_bytes(pkg):
    lib = pkg.native.lib()
    assert lib.cj_prepared_row_bytes(12, 4096) == 16 * 144
    assert lib.cj_prepared_row_bytes(14, 4096) == 16 * 210          # 16 blocks: no pad
    assert lib.cj_prepared_row_bytes(8, 512) == 16 * 34
    assert lib.cj_prepared_row_bytes(8, 1408) == 44 * 32 + 96       # 88 bytes of scales, padded to 96
    assert lib.cj_prepared_row_bytes(39, 2880) == 90 * 16 + 96
    assert lib.cj_prepared_row_bytes(12, 1000) < 0


def _gguf_info(pkg, path):
    import ctypes
    nt, ns = ctypes.c_int64(0), ctypes.c_int64(0)
    rc = pkg.native.lib().cj_gguf_info(path.encode(), ctypes.byref(nt), ctypes.byref(ns))
    return rc, nt.value, ns.value


def test_split_gguf_opens_as_one_model(pkg, tmp_path):
    """A model split into <base>-%05d-of-%05d.gguf shards opens from any
    shard as the whole directory (io/GgufFile.cajeta:45-55, :467-560); a
    missing shard is refused by name."""
    from gguf_split import split_gguf
    src = os.path.join(os.path.dirname(__file__), "golden", "gguf", "toy-routable.gguf")
    rc, n_one, s_one = _gguf_info(pkg, src)
    assert rc == 0 and s_one == 1 and n_one > 3
    paths = split_gguf(src, str(tmp_path / "toy"), 3)
    for p in paths:
        rc, n, s = _gguf_info(pkg, p)
        assert (rc, n, s) == (0, n_one, 3), p
    os.remove(paths[2])
    rc, _, _ = _gguf_info(pkg, paths[0])
    assert rc != 0
    msg = pkg.native.last_error()
    assert "missing" in msg and "00003-of-00003" in msg, msg


def _gguf(kvs=b"", nkv=0, tensors=(), data=b"", align=32):
    """A GGUF v3 image from raw key/value bytes and (name, dims, type, offset) tensors."""
    import struct
    s = lambda x: struct.pack("<Q", len(x)) + x
    head = struct.pack("<IIQQ", 0x46554747, 3, len(tensors), nkv) + kvs
    for name, dims, ty, off in tensors:
        head += s(name.encode()) + struct.pack("<I", len(dims)) + struct.pack("<%dQ" % len(dims), *dims)
        head += struct.pack("<IQ", ty, off)
    head += b"\0" * ((-len(head)) % align)
    return head + data


def test_crafted_gguf_headers_are_refused_not_trusted(pkg, tmp_path):
    """Header values that would wrap an extent check (a huge string length, a
    huge tensor offset, an element count past int64, a zero dimension,
    deeply nested arrays) are refused with a message; none reads past the
    file or unwinds through the C-ABI."""
    import struct
    ok = _gguf(tensors=[("t", (32, 2), 0, 0)], data=b"\0" * 256)
    cases = {
        "ok": ok,
        "string length": struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + struct.pack("<Q", 2 ** 64 - 8) + b"key",
        "tensor offset": _gguf(tensors=[("t", (32, 2), 0, 2 ** 64 - 16)], data=b"\0" * 256),
        "element count": _gguf(tensors=[("t", (2 ** 40, 2 ** 40), 0, 0)], data=b"\0" * 256),
        "zero dimension": _gguf(tensors=[("t", (32, 0), 0, 0)], data=b"\0" * 256),
        "byte size": _gguf(tensors=[("t", (2 ** 61, 2), 0, 0)], data=b"\0" * 256),
        "past the end": _gguf(tensors=[("t", (64, 2), 0, 0)], data=b"\0" * 256),
        "nested arrays": _gguf(kvs=struct.pack("<Q", 1) + b"k" + struct.pack("<I", 9)
                               + b"".join(struct.pack("<IQ", 9, 1) for _ in range(64)) + struct.pack("<IQ", 5, 0),
                               nkv=1),
        "alignment": _gguf(kvs=struct.pack("<Q", 17) + b"general.alignment" + struct.pack("<II", 4, 2 ** 31), nkv=1),
    }
    for name, blob in cases.items():
        p = tmp_path / ("%s.gguf" % name.replace(" ", "_"))
        p.write_bytes(blob)
        rc, nt, _ = _gguf_info(pkg, str(p))
        if name == "ok":
            assert rc == 0 and nt == 1, pkg.native.last_error()
        else:
            assert rc == pkg.native.CJ_ERR_IO, (name, rc)
            assert pkg.native.last_error(), name
