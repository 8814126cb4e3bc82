"""Inputs and recorded outputs of the reference's own golden tests
(tests/golden/wave): the rows its CPU backend recorded, and the input
generators of the tests that recorded them."""
import os

import numpy as np

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def cpu_golden_rows():
    """The reference's recorded CPU-backend outputs (tests/golden/wave)."""
    out = {}
    for line in open(os.path.join(GOLD, "wave", "cpu_rows.tsv")):
        be, kern, tag, n, vals = line.rstrip("\n").split("\t")
        bits = np.array([int(v) for v in vals.split(",")], np.int64).astype(np.uint32)
        assert be == "cpu" and bits.size == int(n)
        out[(kern, tag)] = bits.view(np.float32)
    return out


def qkprep_fill(n, seed):
    """QkPrepTest.fill: ((i·37 + seed) mod 101 − 50) / 17 in f32."""
    i = np.arange(n, dtype=np.int64)
    return ((((i * 37 + seed) % 101) - 50).astype(np.float32) / np.float32(17.0)).astype(np.float32)


def reduce_pack_partials():
    """WorkgroupReduceGoldenTest.reducePackGolden's partials: 32 heads × 8
    splits × (128 accumulators, max, sum)."""
    i = np.arange(32 * 8 * 130, dtype=np.int64)
    slot, seg = i % 130, i // 130
    acc = ((((i * 13) % 29) - 14).astype(np.float32) / np.float32(8.0))
    m = (seg % 5).astype(np.float32) * np.float32(0.25) - np.float32(0.5)
    l = np.float32(1.0) + (seg % 3).astype(np.float32) * np.float32(0.5)
    return np.where(slot < 128, acc, np.where(slot == 128, m, l)).astype(np.float32)


def spread(n, seed):
    """TreeSiteReferenceTest.spread (AttnKernelTest.spread's generator): an
    int32 linear congruential state s ← s·1103515245 + 12345 (wrapping), made
    non-negative (the state keeps the negation), then ((s mod 2000) − 1000) / 700
    in f32."""
    out = np.empty(n, np.float32)
    s = seed
    for i in range(n):
        s = (s * 1103515245 + 12345) & 0xFFFFFFFF
        if s >= 0x80000000:
            s -= 1 << 32
        if s < 0:
            s = -s
            if s == 1 << 31:      # 0 − INT_MIN wraps to INT_MIN
                s = -(1 << 31)
        m = int(np.fmod(s, 2000)) if s < 0 else s % 2000
        out[i] = np.float32(np.float32(m) - np.float32(1000.0)) / np.float32(700.0)
    return out
