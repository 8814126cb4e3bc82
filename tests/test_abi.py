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
