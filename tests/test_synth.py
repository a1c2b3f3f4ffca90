"""The synthetic generator: the reference LCG stream and the block layouts."""
import numpy as np

from chatokf_amd import synth
from chatokf_amd.formats import Q8_0, Q2_0, Q4_K, IQ2_XXS, row_bytes


def lcg_ref(seed, n):
    # LLM/Qwen/QwenMetalSelfTest.swift:5-14, one step at a time
    s = (seed + 0x9E3779B97F4A7C15) % 2**64
    out = []
    for _ in range(n):
        s = (s * 6364136223846793005 + 1442695040888963407) % 2**64
        out.append(s >> 33)
    return out


def test_lcg_matches_reference_stream():
    for seed in (0, 1, 1003, 2**63 + 5):
        g = synth.LCG(seed)
        a = list(g.u32(37)) + list(g.u32(1000))  # continuation across calls
        assert a == lcg_ref(seed, 1037)


def test_uniform_and_normal_ranges():
    g = synth.LCG(3)
    u = g.uniform(1e-3, 1e-2, 10000)
    assert u.min() >= 1e-3 and u.max() < 1e-2
    z = synth.LCG(4).normal(200000)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01


def test_layouts_and_determinism():
    for t, K in ((Q8_0, 2048), (Q2_0, 2048), (Q4_K, 512), (IQ2_XXS, 512)):
        a = synth.weights(t, 3, K, 9)
        b = synth.weights(t, 3, K, 9)
        assert a.size == 3 * row_bytes(t, K) and np.array_equal(a, b)
    w = synth.q8_0(4, 64, 1).reshape(-1, 34)
    q = w[:, 2:].view(np.int8)
    assert q.min() >= -127
    d = w[:, :2].copy().view(np.float16).astype(np.float32)
    assert d.min() >= np.float16(1e-3) and d.max() <= np.float16(1e-2)
    c = synth.q2_0(8, 128, 2).reshape(-1, 34)[:, 2:]
    codes = np.stack([(c >> s) & 3 for s in (0, 2, 4, 6)])
    assert codes.max() == 2 and set(np.unique(codes)) == {0, 1, 2}
