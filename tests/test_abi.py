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
