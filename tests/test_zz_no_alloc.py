"""cj_argmax_row_noalloc: the allocation-free argmax (its scratch is a static
device array) gives what cj_argmax_row gives, on two calls in a row, the
second with a smaller input, and refuses sizes beyond its limit."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

NOALLOC_MAX = 1 << 22


def test_noalloc_argmax_equals_the_allocating_entry_point(gpu):
    lib = gpu.native.lib()
    rng = np.random.default_rng(12)
    for n in (201088, 32000):       # the second call is smaller: the shared scratch keeps the first's partials
        print("noalloc argmax n=%d" % n, flush=True)
        v = rng.standard_normal(n).astype(np.float32)
        top = np.float32(v.max() + 1)
        v[n // 3] = v[n - 5] = top   # a tie: the first occurrence wins
        vb = gpu.Buffer.of(v)
        tb = gpu.Buffer.of(np.full(4, -7, np.int32))
        gpu.native.check(lib.cj_argmax_row(tb.h, 1, vb.h, n), "argmax")
        gpu.native.check(lib.cj_argmax_row_noalloc(tb.h, 2, vb.h, n), "argmax noalloc")
        t = tb.download(np.int32, 4)
        assert t[2] == t[1] == n // 3, (n, t)
        assert t[0] == -7 and t[3] == -7
    # beyond the static scratch: refused before anything is launched
    assert lib.cj_argmax_row_noalloc(tb.h, 0, vb.h, NOALLOC_MAX + 1) == gpu.native.CJ_ERR_ARG
    assert "static scratch" in gpu.native.last_error()
    assert lib.cj_argmax_row_noalloc(tb.h, 4, vb.h, 100) == gpu.native.CJ_ERR_ARG   # row outside the token buffer
