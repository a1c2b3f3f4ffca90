"""GPU parity: the HIP library (through its C ABI) against the CPU oracle.

Bars (written in each test): dequantized weights bit-identical; matvec and
narrow (N = 2..5) outputs within max|gpu - ref| / max|ref| <= 1e-4 (the
reference's relative metric, LLM/Qwen/QwenMetalSelfTest.swift:441-445, at
the gate its own gemv self-test applies, :580), the activations being
carried at fp32 precision as the reference's gemv reads them
(LLM/metal/Kernels.metal:46-52, :1681-1690); tile GEMM outputs (fp16
activation tiles, as the reference's gemm_mm stages them, Kernels.metal:282)
within 1e-3, the north-star tolerance; narrow-N vs N x gemv within 1e-5
(QwenMetalSelfTest.swift:478-483).
"""
import ctypes
import functools
import sys

import numpy as np
import pytest

import oracle
from chatokf_amd import synth
from chatokf_amd.formats import (Q8_0, Q2_0, Q4_K, IQ2_XXS, Q4_0, IQ4_NL, Q5_K, Q6_K, IQ4_XS, IQ2_XS, IQ2_S,  # noqa
                                 IQ3_XXS, IQ3_S, IQ1_S, IQ1_M, F32, F16, BF16, Q2_K, Q3_K, NAMES, row_bytes)

torch = pytest.importorskip("torch")
import chatokf_amd as ok  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = 1e-3      # tile GEMM (fp16 activation tiles)
TOL_MV = 1e-4   # matvec / narrow: QwenMetalSelfTest.swift:580


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def rel(got, ref):
    return float(np.abs(got.astype(np.float64) - ref).max() / np.abs(ref).max())


@functools.lru_cache(maxsize=None)
def weights(t, M, K, seed):
    return synth.weights(t, M, K, seed)


@functools.lru_cache(maxsize=None)
def acts(N, K, seed):
    return synth.activations(N, K, seed)


def run_gemm(enc, t, M, K, w, X, tile=False):
    N = X.shape[0]
    wd, Xd = dev(w), dev(X)
    Y = torch.full((N, M), float("nan"), device="cuda")
    qt = ok.QuantTensor(wd, K, M, t)
    if tile:
        enc.gemm_tile(qt, Xd, Y, N)
    elif N == 1:
        enc.gemv(qt, Xd, Y)
    else:
        enc.gemm(qt, Xd, Y, N)
    enc.sync()
    return host(Y)


# ------------------------------------------------------------------ dequant
DQ_CASES = [(Q8_0, 6, 2048), (Q2_0, 6, 6144), (Q4_K, 4, 5120), (IQ2_XXS, 4, 5120), (Q4_0, 6, 4096),
            (IQ4_NL, 6, 4096), (Q5_K, 4, 5120), (Q6_K, 4, 5120), (IQ4_XS, 4, 5120)] + \
    [(t, 4, 5120) for t in (IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S, IQ1_M, Q2_K, Q3_K, F32, F16, BF16)]


@pytest.mark.parametrize("t,M,K", DQ_CASES, ids=[NAMES[c[0]] for c in DQ_CASES])
def test_dequant_row_bit_exact(enc, t, M, K):
    say("dequant", NAMES[t], M, K)
    w = weights(t, M, K, 101)
    wd = dev(w)
    rb = row_bytes(t, K)
    for m in range(M):
        out = torch.full((K,), float("nan"), device="cuda")
        enc.dequant_row(ok.QuantTensor(wd, K, 1, t, off=m * rb), out, K)
        got = host(out)
        ref = oracle.dequant(t, w[m * rb:(m + 1) * rb], K)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (NAMES[t], m)


def test_dequant_row_q2_0_code3(enc):
    w = synth.q2_0(2, 512, 55, codes=4)
    out = torch.empty(512, device="cuda")
    enc.dequant_row(ok.QuantTensor(dev(w), 512, 1, Q2_0, off=row_bytes(Q2_0, 512)), out, 512)
    ref = oracle.dequant(Q2_0, w[row_bytes(Q2_0, 512):], 512)
    assert np.array_equal(host(out), ref)


# ------------------------------------------------------------------ matvec
# The BASELINE.json decode configs at their full shapes: (name, type, M, K, seed)
FULL_GEMV = [
    ("q8_0 2048x2048", Q8_0, 2048, 2048, 1001),
    ("q2_0 gate 6144x2048", Q2_0, 6144, 2048, 1002),
    ("q2_0 down 2048x6144", Q2_0, 2048, 6144, 1102),
    ("q4_k 17408x5120", Q4_K, 17408, 5120, 1003),
    ("q4_k 5120x17408", Q4_K, 5120, 17408, 1103),
    ("iq2_xxs 17408x5120", IQ2_XXS, 17408, 5120, 1004),
    # formats past the scope's four, at the 27B FFN shapes
    ("q5_k 17408x5120", Q5_K, 17408, 5120, 1005),
    ("q6_k 5120x17408", Q6_K, 5120, 17408, 1006),
    ("iq4_xs 17408x5120", IQ4_XS, 17408, 5120, 1007),
    ("iq3_xxs 17408x5120", IQ3_XXS, 17408, 5120, 1008),
    ("iq1_s 6144x2048", IQ1_S, 6144, 2048, 1009),
]


@pytest.mark.parametrize("name,t,M,K,seed", FULL_GEMV, ids=[c[0] for c in FULL_GEMV])
def test_gemv_full_config(enc, name, t, M, K, seed):
    say("gemv", name)
    w = weights(t, M, K, seed)
    x = acts(1, K, seed + 1000)
    ref = oracle.matvec(t, w, K, M, x[0]).astype(np.float64)
    got = run_gemm(enc, t, M, K, w, x)[0]
    r = rel(got, ref)
    say("  rel", r)
    assert r <= TOL_MV


# Shapes that exercise tails: M not a multiple of the rows per workgroup, a
# single block per row, K not a multiple of 64 units.
EDGE = [(Q8_0, 1, 32), (Q8_0, 3, 96), (Q8_0, 4099, 2080), (Q2_0, 5, 128), (Q2_0, 4097, 384),
        (Q4_K, 1, 256), (Q4_K, 7, 768), (Q4_K, 4101, 2304), (Q4_K, 1000, 8192), (Q4_K, 13, 8448), (IQ2_XXS, 2, 256), (IQ2_XXS, 4103, 1280), (IQ2_XXS, 301, 8192),
        (Q4_0, 1, 32), (Q4_0, 4099, 2080), (Q4_0, 2048, 4096), (IQ4_NL, 3, 96), (IQ4_NL, 4099, 2080),
        (IQ4_NL, 2048, 4096), (Q5_K, 1, 256), (Q5_K, 4101, 2304), (Q6_K, 3, 256), (Q6_K, 4099, 1280),
        (IQ4_XS, 2, 512), (IQ4_XS, 4103, 2304)] + \
    [(t, M, K) for t in (IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S, IQ1_M, Q2_K, Q3_K) for M, K in ((3, 256), (4101, 1280))] + \
    [(t, M, K) for t in (F32, F16, BF16) for M, K in ((3, 32), (4101, 1056))]


def l1_rows(t, w, K, M, x):
    """Per-row sum_i |w_i x_i| in float64: the scale fp32 summation error is
    relative to when a row's dot product cancels."""
    rb = row_bytes(t, K)
    W = np.stack([oracle.dequant(t, w[m * rb:(m + 1) * rb], K) for m in range(M)]).astype(np.float64)
    return np.abs(W) @ np.abs(x.astype(np.float64))


@pytest.mark.parametrize("t,M,K", EDGE)
def test_gemv_edges(enc, t, M, K):
    say("gemv edge", NAMES[t], M, K)
    w = weights(t, M, K, 7)
    x = acts(1, K, 8)
    ref = oracle.matvec(t, w, K, M, x[0]).astype(np.float64)
    got = run_gemm(enc, t, M, K, w, x)[0]
    r = rel(got, ref)
    say("  rel", r)
    # the reference's metric at its gemv gate, for every shape
    assert r <= TOL_MV
    # every row within fp32-summation distance of the oracle, measured
    # against the row's sum of |w x| (meaningful also where a row cancels)
    if M <= 64:
        assert (np.abs(got - ref) <= 2e-6 * l1_rows(t, w, K, M, x[0]) + 1e-30).all()


# Activations of any fp32 magnitude: each 32-weight group carries its own
# power-of-two scale, so tiny, huge and mixed-magnitude vectors keep the
# reference's fp32 relative precision (no fp16 overflow or underflow).
@pytest.mark.parametrize("t", [Q8_0, Q2_0, Q4_K, IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S, IQ1_M, Q2_K, Q3_K,
                               F32], ids=lambda t: NAMES[t])
@pytest.mark.parametrize("scale", ["1e-20", "1e-5", "1e5", "1e20", "mixed"])
def test_gemv_activation_range(enc, t, scale):
    M, K = 1030, 2048
    say("gemv range", NAMES[t], scale)
    w = weights(t, M, K, 31)
    x = acts(1, K, 32).copy()
    if scale == "mixed":
        x *= (10.0 ** np.random.default_rng(33).uniform(-8, 8, K)).astype(np.float32)
    else:
        x *= np.float32(float(scale))
    ref = oracle.matvec(t, w, K, M, x[0]).astype(np.float64)
    got = run_gemm(enc, t, M, K, w, x)[0]
    say("  rel", rel(got, ref))
    assert np.isfinite(got).all()
    assert rel(got, ref) <= TOL_MV
    for N in (2, 5):  # the narrow kernels stage the same way
        X = np.repeat(x, N, axis=0)
        assert rel(run_gemm(enc, t, M, K, w, X)[N - 1], ref) <= TOL_MV


def test_gemv_nan_propagates(enc):
    # a NaN activation makes every output NaN, as fp32 products do
    t, M, K = Q4_K, 300, 1024
    w = weights(t, M, K, 34)
    x = acts(1, K, 35).copy()
    x[0, 517] = np.nan
    assert np.isnan(run_gemm(enc, t, M, K, w, x)[0]).all()


def test_gemv_weight_offset(enc):
    # the weight window + 64-bit offset of WeightRef (MetalContext.swift:4-11)
    t, M, K = Q4_K, 64, 1024
    w = weights(t, M, K, 9)
    pad = 4096
    buf = np.zeros(pad + w.size, np.uint8)
    buf[pad:] = w
    x = acts(1, K, 10)
    y = torch.empty(M, device="cuda")
    enc.gemv(ok.QuantTensor(dev(buf), K, M, t, off=pad), dev(x), y)
    ref = oracle.matvec(t, w, K, M, x[0]).astype(np.float64)
    assert rel(host(y), ref) <= TOL_MV


# ------------------------------------------------------------------ narrow N = 2..5
@pytest.mark.parametrize("t", [Q8_0, Q2_0, Q4_K, IQ2_XXS, Q4_0, IQ4_NL, Q5_K, Q6_K, IQ4_XS, IQ2_XS, IQ2_S,
                               IQ3_XXS, IQ3_S, IQ1_S, IQ1_M, Q2_K, Q3_K, F32, F16, BF16], ids=lambda t: NAMES[t])
@pytest.mark.parametrize("N", [2, 3, 4, 5])
def test_narrow_matches_oracle_and_gemv(enc, t, N):
    M, K = 1030, 2048
    say("narrow", NAMES[t], N)
    w = weights(t, M, K, 13)
    X = acts(N, K, 14)
    ref = oracle.matmul(t, w, K, M, X).astype(np.float64)
    got = run_gemm(enc, t, M, K, w, X)
    say("  rel", rel(got, ref))
    assert rel(got, ref) <= TOL_MV
    for n in range(N):
        g1 = run_gemm(enc, t, M, K, w, X[n:n + 1])[0]
        assert rel(got[n], g1.astype(np.float64)) <= 1e-5


def test_iq2_xxs_mtp_verify_full_config(enc):
    # BASELINE config 4 at M = 4: W 17408 x 5120, X 4 x 5120
    t, M, K = IQ2_XXS, 17408, 5120
    w = weights(t, M, K, 1004)
    X = acts(4, K, 2004)
    ref = oracle.matmul(t, w, K, M, X).astype(np.float64)
    r = rel(run_gemm(enc, t, M, K, w, X), ref)
    say("iq2_xxs M=4 rel", r)
    assert r <= TOL_MV


MM_FMTS = [Q4_K, Q5_K, IQ4_XS, Q8_0, IQ3_XXS, IQ3_S, IQ2_XS, IQ2_S, IQ1_S, IQ1_M, Q2_K, Q3_K]


@pytest.mark.parametrize("t", MM_FMTS, ids=lambda t: NAMES[t])
@pytest.mark.parametrize("N", [2, 3, 4])
def test_narrow_mm_full_config(enc, t, N):
    # 17408 x 5120 with 2..4 columns (the matrix-core narrow kernels; Q8_0 from 3)
    M, K = 17408, 5120
    w = weights(t, M, K, 1003)
    X = acts(N, K, 2006)
    ref = oracle.matmul(t, w, K, M, X).astype(np.float64)
    r = rel(run_gemm(enc, t, M, K, w, X), ref)
    say(NAMES[t], "N", N, "rel", r)
    assert r <= TOL_MV


# the same kernels on ragged shapes: rows that leave a partial row quad per
# workgroup, K whose 64-weight units leave a partial last step
@pytest.mark.parametrize("t", MM_FMTS, ids=lambda t: NAMES[t])
@pytest.mark.parametrize("M,K,N", [(4101, 2304, 4), (4099, 1280, 3), (5000, 768, 2), (4097, 6144, 4)])
def test_narrow_mm_edges(enc, t, M, K, N):
    say("narrow mm", NAMES[t], M, K, N)
    w = weights(t, M, K, 41)
    X = acts(N, K, 42)
    ref = oracle.matmul(t, w, K, M, X).astype(np.float64)
    got = run_gemm(enc, t, M, K, w, X)
    assert rel(got, ref) <= TOL_MV
    for n in range(N):  # each column as its own matvec
        assert rel(got[n], run_gemm(enc, t, M, K, w, X[n:n + 1])[0].astype(np.float64)) <= 1e-5


# ------------------------------------------- one workgroup per CU (wide)
# With OKF_GEMV_WIDE=1 every single-matrix matvec / narrow call that the
# one-workgroup-per-CU kernel takes goes through it (the automatic policy
# sends it large IQ2_XXS matrices only).  The shapes cover M below the grid
# size, rows per workgroup that do not divide evenly, K whose units leave a
# partial last step, and slot ranges that cross row boundaries; IQ2_XXS
# with 2..4 columns takes the matrix-core variant (row quads).
WIDE = [(IQ2_XXS, 3, 256, 1), (IQ2_XXS, 257, 1280, 2), (IQ2_XXS, 1000, 5120, 4), (IQ2_XXS, 4103, 1280, 1),
        (IQ2_XXS, 2048, 2304, 5), (IQ2_XXS, 300, 17408, 1), (IQ2_XXS, 3, 256, 2), (IQ2_XXS, 4103, 1280, 3),
        (IQ2_XXS, 300, 5120, 4), (IQ2_XXS, 2049, 2048, 2), (Q2_0, 1000, 2048, 1), (Q2_0, 2048, 6144, 2),
        (Q2_0, 5, 384, 3), (Q4_K, 4101, 2304, 1), (Q4_K, 100, 17408, 1), (Q8_0, 4099, 2080, 1),
        (Q4_0, 1030, 2048, 4), (IQ4_NL, 1030, 2048, 5)]


@pytest.fixture(scope="module")
def enc_wide():
    import os
    os.environ["OKF_GEMV_WIDE"] = "1"
    try:
        e = ok.Enc(0)
    finally:
        del os.environ["OKF_GEMV_WIDE"]
    yield e
    e.close()


@pytest.mark.parametrize("t,M,K,N", WIDE)
def test_wide_matches_oracle_and_default(enc, enc_wide, t, M, K, N):
    say("wide", NAMES[t], M, K, N)
    w = weights(t, M, K, 21)
    X = acts(N, K, 22)
    ref = oracle.matmul(t, w, K, M, X).astype(np.float64)
    got = run_gemm(enc_wide, t, M, K, w, X)
    say("  rel", rel(got, ref))
    assert rel(got, ref) <= TOL_MV
    assert rel(got, run_gemm(enc, t, M, K, w, X).astype(np.float64)) <= 1e-5


# ---------------------------------------------- add + RMSNorm, argmax
# n: vector path (multiple of 4, <= 8192), scalar paths (odd n, n > 8192, a
# pointer off 16-byte alignment); rows as decode (1) and MTP verify (5)
NORM = [(2048, 1, 0), (5120, 5, 0), (6144, 3, 0), (10000, 2, 0), (1001, 3, 0), (2048, 2, 1)]


@pytest.mark.parametrize("n,rows,skew", NORM)
@pytest.mark.parametrize("add", [True, False], ids=["add", "plain"])
def test_add_rmsnorm_matches_oracle(enc, n, rows, skew, add):
    say("add_rmsnorm", n, rows, skew, add)
    rng = np.random.default_rng(n + rows)
    x = rng.standard_normal((rows, n)).astype(np.float32) * 4
    r = rng.standard_normal((rows, n)).astype(np.float32) if add else None
    w = rng.uniform(0.5, 1.5, n).astype(np.float32)
    xs, ref = oracle.add_rmsnorm(x, r, w, 1e-6)
    buf = torch.zeros(rows * n + skew, device="cuda")
    xd = buf[skew:].view(rows, n)
    xd.copy_(dev(x))
    yd = torch.full((rows, n), float("nan"), device="cuda")
    enc.add_rmsnorm(xd, None if r is None else dev(r), dev(w), yd, n, rows, 1e-6)
    got_x, got_y = host(xd), host(yd)
    assert np.array_equal(got_x, xs)  # one fp32 add per element (or untouched)
    assert np.abs(got_y - ref).max() <= 1e-5 * np.abs(ref).max()  # summation order only


ARGMAX = [(248320, 1, 0), (248320, 5, 0), (1, 1, 0), (1003, 3, 0), (8192 * 3 + 5, 2, 1), (100000, 4, 0)]


@pytest.mark.parametrize("n,rows,skew", ARGMAX)
def test_argmax_rows_matches_oracle(enc, n, rows, skew):
    say("argmax", n, rows, skew)
    rng = np.random.default_rng(n * 7 + rows)
    x = rng.standard_normal((rows, n)).astype(np.float32)
    if n > 16:
        x[0, n // 3] = x[0, n - 2] = 9.0  # a tie across chunks: the lower index wins
        x[0, 5] = np.nan
    if rows > 1:
        x[1, :] = np.nan  # nothing wins: 0
    if rows > 2:
        x[2, :] = -np.inf
        x[2, n - 1] = -1e30
    ref = oracle.argmax_rows(x)
    buf = torch.zeros(rows * n + skew, device="cuda")
    xd = buf[skew:].view(rows, n)
    xd.copy_(dev(x))
    out = torch.full((rows,), -7, dtype=torch.int32, device="cuda")
    enc.argmax_rows(xd, n, rows, out)
    assert np.array_equal(host(out), ref)


def test_argmax_repeated_calls_reset_counters(enc):
    # the single-launch argmax counts finished workgroups per row and the last
    # one resets the count: back-to-back calls of different shapes stay right
    rng = np.random.default_rng(77)
    for n, rows in ((248320, 2), (5000, 5), (248320, 1), (1025, 3)):
        x = rng.standard_normal((rows, n)).astype(np.float32)
        out = torch.full((rows,), -7, dtype=torch.int32, device="cuda")
        enc.argmax_rows(dev(x), n, rows, out)
        assert np.array_equal(host(out), oracle.argmax_rows(x))


@pytest.mark.parametrize("nbytes", [16, 16 * 1000 + 16 * 7, 50135040])
def test_stream_read_xor(enc, nbytes):
    # the calibration read touches every byte exactly once: its xor of all
    # 32-bit words equals numpy's, folded into the value already in out
    rng = np.random.default_rng(nbytes)
    a = rng.integers(0, 2**32, size=nbytes // 4, dtype=np.uint32)
    out = torch.tensor([0x5A5A5A5A], dtype=torch.int32, device="cuda")
    enc.stream_read(dev(a.view(np.int32)), nbytes, out)
    want = np.bitwise_xor.reduce(a) ^ np.uint32(0x5A5A5A5A)
    assert int(host(out)[0]) & 0xFFFFFFFF == int(want)


# ------------------------------------------------------------ reserve
def test_reserve_then_no_allocation():
    # okf_ctx_reserve sizes the scratch once; the Q4_K tile GEMM and argmax
    # then run without any device allocation, and a call beyond the
    # reservation is refused rather than growing the scratch
    e = ok.Enc(0)
    try:
        t, M, K, N = Q4_K, 512, 2048, 64
        w, X = dev(weights(t, M, K, 41)), dev(acts(N, K, 42))
        Y = torch.empty((N, M), device="cuda")
        xa = torch.randn(3, 100000, device="cuda")
        out = torch.empty(3, dtype=torch.int32, device="cuda")
        X2 = dev(acts(2 * N, K, 43))
        Y2 = torch.empty((2 * N, M), device="cuda")
        e.reserve(N * K, 100000, 3)
        qt = ok.QuantTensor(w, K, M, t)
        # one call of each first: the HIP runtime loads a kernel's code object
        # at its first launch (device memory that is not ours)
        e.gemm(qt, X, Y, N)
        e.argmax_rows(xa, 100000, 3, out)
        e.sync()
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        for _ in range(3):
            e.gemm(qt, X, Y, N)
            e.argmax_rows(xa, 100000, 3, out)
            e.gemm(qt, X[:N // 2], Y[:N // 2], N // 2)
        e.sync()
        assert torch.cuda.mem_get_info()[0] == free0
        with pytest.raises(ok.OkfError) as err:
            e.gemm(qt, X2, Y2, 2 * N)
        assert err.value.status == ok.OKF_E_SHAPE
        with pytest.raises(ok.OkfError):
            e.argmax_rows(xa, 100000, 4, out)  # (4 rows > 3 reserved)
        ref = oracle.matmul(t, weights(t, M, K, 41), K, M, acts(N, K, 42)).astype(np.float64)
        assert rel(host(Y), ref) <= TOL
        assert np.array_equal(host(out), oracle.argmax_rows(host(xa)))
    finally:
        e.close()


# ------------------------------------------------------------ SiLU-gated FFN
def test_silu_mul_matches_oracle(enc):
    a = np.random.default_rng(4).standard_normal(6144).astype(np.float32) * 3
    b = np.random.default_rng(5).standard_normal(6144).astype(np.float32)
    ad, bd = dev(a), dev(b)
    enc.silu_mul(ad, bd, 6144)
    got, ref = host(ad), oracle.silu_mul(a, b).astype(np.float64)
    # device exp: a few ulp from the C library's expf
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-6)


SILU_CASES = [(Q2_0, 2048, 6144, 1102), (Q8_0, 300, 2048, 81), (Q4_K, 260, 2304, 82), (IQ4_NL, 96, 512, 85),
              (IQ2_XXS, 129, 1536, 83), (Q2_0, 130, 1024, 84), (Q5_K, 100, 768, 86), (Q6_K, 70, 512, 87),
              (IQ4_XS, 90, 1024, 88), (IQ2_S, 70, 512, 89), (IQ1_M, 50, 768, 90), (Q3_K, 60, 512, 91),
              (BF16, 40, 1024, 92)]


@pytest.mark.parametrize("t,M,K,seed", SILU_CASES)
def test_gemv_silu_matches_silu_mul_then_matvec(enc, t, M, K, seed):
    # QwenMetalEngine.swift:924-928: siluMul(gate, up) then gemv(down)
    w = weights(t, M, K, seed)
    g, u = acts(1, K, seed + 1)[0] * 2, acts(1, K, seed + 2)[0]
    ref = oracle.matvec(t, w, K, M, oracle.silu_mul(g, u)).astype(np.float64)
    gd, ud = dev(g), dev(u)
    y = torch.full((M,), float("nan"), device="cuda")
    enc.gemv_silu(ok.QuantTensor(dev(w), K, M, t), gd, ud, y)
    got = host(y)
    say("gemv_silu", NAMES[t], M, K, rel(got, ref))
    # (silu's device exp and reciprocal are within a few ulp of the C library's)
    assert rel(got, ref) <= TOL_MV
    assert np.array_equal(host(gd), g)  # gate is not modified
    # the two-call form: silu_mul in place, then gemv
    enc.silu_mul(gd, ud, K)
    y2 = torch.full((M,), float("nan"), device="cuda")
    enc.gemv(ok.QuantTensor(dev(w), K, M, t), gd, y2)
    assert rel(got, host(y2).astype(np.float64)) <= 1e-5


# The Bonsai-shape Q2_0 matvecs on the integer matrix cores (K 2048 and
# 6144) at row counts that leave the last workgroups partial or empty, and
# R = ceil(M / CUs) rows a workgroup from 1 to 16: with OKF_Q2_KS=1 (the
# default) a K-6144 workgroup of at most 8 rows runs its tile as two K
# halves side by side, with 0 it repeats rows in the tile's spare columns.
# Both against the oracle, plain and with the SiLU-gated activations.
@pytest.fixture(scope="module", params=["1", "0"], ids=["ks", "noks"])
def enc_q2ks(request):
    import os
    os.environ["OKF_Q2_KS"] = request.param
    try:
        e = ok.Enc(0)
    finally:
        del os.environ["OKF_Q2_KS"]
    yield e
    e.close()


@pytest.mark.parametrize("M,K", [(2048, 6144), (2000, 6144), (1100, 6144), (37, 6144), (3000, 6144),
                                 (4000, 2048), (100, 2048), (6143, 2048)])
@pytest.mark.parametrize("silu", [False, True], ids=["plain", "silu"])
def test_q2_0_matrix_core_rows(enc_q2ks, M, K, silu):
    say("q2_0 matrix-core rows", M, K, "silu" if silu else "plain")
    w = weights(Q2_0, M, K, 61)
    g, u = acts(1, K, 62)[0] * 2, acts(1, K, 63)[0]
    x = oracle.silu_mul(g, u) if silu else g
    ref = oracle.matvec(Q2_0, w, K, M, x).astype(np.float64)
    y = torch.full((M,), float("nan"), device="cuda")
    qt = ok.QuantTensor(dev(w), K, M, Q2_0)
    if silu:
        enc_q2ks.gemv_silu(qt, dev(g), dev(u), y)
    else:
        enc_q2ks.gemv(qt, dev(g), y)
    got = host(y)
    r = rel(got, ref)
    say("  rel", r)
    assert r <= TOL_MV
    if M <= 64:
        assert (np.abs(got - ref) <= 2e-6 * l1_rows(Q2_0, w, K, M, x) + 1e-30).all()


# ------------------------------------------------------------ FFN block
# okf_ffn: gate and up on x (one grid), then down on silu(gate) * up
# (QwenMetalEngine.swift:918-929); against the oracle's three matvecs.
FFN = [(Q2_0, Q2_0, Q2_0, 6144, 2048, 1002), (Q4_K, Q4_K, Q4_K, 768, 512, 31), (IQ2_XXS, IQ2_XXS, IQ2_XXS, 512, 1280, 32),
       (Q8_0, Q8_0, Q8_0, 320, 2080, 33), (Q2_0, Q2_0, Q2_0, 256, 1024, 34),
       (Q4_K, Q4_K, Q8_0, 512, 768, 35),  # (down's format differs)
       (Q4_K, Q8_0, Q2_0, 256, 512, 36),  # (gate's and up's formats differ: no pairing)
       (Q2_0, Q2_0, Q8_0, 224, 1024, 37),
       (Q2_0, Q2_0, Q2_0, 8192, 4096, 38), (Q2_0, Q2_0, Q2_0, 384, 640, 39)]


@pytest.mark.parametrize("tg,tu,td,H,D,seed", FFN)
def test_ffn_matches_oracle(enc, tg, tu, td, H, D, seed):
    say("ffn", NAMES[tg], NAMES[td], H, D)
    wg, wu, wd = weights(tg, H, D, seed), weights(tu, H, D, seed + 1), weights(td, D, H, seed + 2)
    qg, qu, qd = (ok.QuantTensor(dev(w), k, m, t) for w, k, m, t in ((wg, D, H, tg), (wu, D, H, tu), (wd, H, D, td)))
    for rep in range(2):
        x = acts(1, D, seed + 10 + rep)[0]
        g, u = (torch.full((H,), float("nan"), device="cuda") for _ in range(2))
        y = torch.full((D,), float("nan"), device="cuda")
        enc.ffn(qg, qu, qd, dev(x), g, u, y)
        enc.sync()
        rg = oracle.matvec(tg, wg, D, H, x)
        ru = oracle.matvec(tu, wu, D, H, x)
        rh = oracle.silu_mul(rg, ru)
        ry = oracle.matvec(td, wd, H, D, rh).astype(np.float64)
        # g holds silu(gate) * up after the call (the reference's in-place siluMul)
        assert rel(host(g), rh.astype(np.float64)) <= TOL_MV
        assert rel(host(u), ru.astype(np.float64)) <= TOL_MV
        r = rel(host(y), ry)
        say("  rel", r)
        assert r <= TOL_MV


# The all-Q2_0 FFN runs as one cooperative launch (gate and up, a grid-wide
# barrier, down); OKF_FFN_FUSED=0 keeps the two launches.  Both compute every
# unit exactly and differ only in the order of the fp32 partial sums, and
# each is deterministic: a second call gives the same bits.
@pytest.fixture(scope="module")
def enc_ffn2():
    import os
    os.environ["OKF_FFN_FUSED"] = "0"
    try:
        e = ok.Enc(0)
    finally:
        del os.environ["OKF_FFN_FUSED"]
    yield e
    e.close()


# The one-launch FFN captured into a HIP graph on the context's stream and
# replayed: its grid barrier keeps its state in counters that only grow, so
# every replay must synchronise as a fresh launch does.  Each replay runs on
# a new x (written into the captured buffer), with eager calls between the
# replays, and must give the eager call's bits for that x.
@pytest.mark.parametrize("fused", ["1", "2"])
def test_ffn_graph_replay(fused):
    # fused "1": okf_ffn's default at this shape (two matrix-core launches);
    # "2": the one launch with its grid barrier, whose epochs live on the
    # device, so replays of one captured launch keep agreeing
    import os
    os.environ["OKF_FFN_FUSED"] = fused
    try:
        enc = ok.Enc(0)
    finally:
        del os.environ["OKF_FFN_FUSED"]
    try:
        _ffn_graph_replay(enc)
    finally:
        enc.close()


def _ffn_graph_replay(enc):
    hip = ctypes.CDLL("libamdhip64.so")
    vp = ctypes.c_void_p
    H, D = 6144, 2048
    wg, wu, wd = weights(Q2_0, H, D, 51), weights(Q2_0, H, D, 52), weights(Q2_0, D, H, 53)
    qg, qu, qd = (ok.QuantTensor(dev(w), k, m, Q2_0) for w, k, m in ((wg, D, H), (wu, D, H), (wd, H, D)))
    x = dev(acts(1, D, 60)[0])
    g, u = torch.zeros(H, device="cuda"), torch.zeros(H, device="cuda")
    y = torch.zeros(D, device="cuda")
    ge, ue, ye = torch.zeros(H, device="cuda"), torch.zeros(H, device="cuda"), torch.zeros(D, device="cuda")
    enc.ffn(qg, qu, qd, x, g, u, y)  # (first call outside the capture)
    enc.sync()
    st = vp(enc.stream)
    graph, exe = vp(), vp()
    assert hip.hipStreamBeginCapture(st, 0) == 0  # hipStreamCaptureModeGlobal
    enc.ffn(qg, qu, qd, x, g, u, y)
    assert hip.hipStreamEndCapture(st, ctypes.byref(graph)) == 0
    assert hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
    try:
        for rep in range(4):
            say("ffn graph replay", rep)
            x.copy_(dev(acts(1, D, 70 + rep)[0]))
            torch.cuda.synchronize()
            enc.ffn(qg, qu, qd, x, ge, ue, ye)  # eager, same x
            enc.sync()
            g.fill_(float("nan"))
            y.fill_(float("nan"))
            torch.cuda.synchronize()
            assert hip.hipGraphLaunch(exe, st) == 0
            assert hip.hipStreamSynchronize(st) == 0
            for a, b in ((g, ge), (u, ue), (y, ye)):
                assert np.array_equal(host(a), host(b))
    finally:
        hip.hipGraphExecDestroy(exe)
        hip.hipGraphDestroy(graph)


# The tile GEMM of a non-Q4_K format captured into a HIP graph on a fresh,
# unreserved context: the capture must not allocate or synchronise (its
# scratch cannot grow while the stream is captured, so it runs without the
# K split and the fp16 copy of X), and every replay must match the oracle and
# the replays must agree bit for bit.  Eager calls run between the replays
# (they may grow the scratch; the graph keeps its own launches).
@pytest.mark.parametrize("t,M,K,N", [(Q8_0, 512, 1024, 64), (Q2_0, 2048, 1024, 300)])
def test_tile_gemm_graph_capture_unreserved(t, M, K, N):
    hip = ctypes.CDLL("libamdhip64.so")
    vp = ctypes.c_void_p
    e = ok.Enc(0)
    try:
        say("tile gemm graph capture", NAMES[t], M, K, N)
        w = weights(t, M, K, 91)
        qw = ok.QuantTensor(dev(w), K, M, t)
        X = acts(N, K, 92)
        Xd = dev(X)
        Y = torch.full((N, M), float("nan"), device="cuda")
        Ye = torch.zeros((N, M), device="cuda")
        st = vp(e.stream)
        graph, exe = vp(), vp()
        assert hip.hipStreamBeginCapture(st, 0) == 0
        e.gemm(qw, Xd, Y, N)
        assert hip.hipStreamEndCapture(st, ctypes.byref(graph)) == 0
        assert hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        ref = oracle.matmul(t, w, K, M, X).astype(np.float64)
        try:
            outs = []
            for rep in range(3):
                Y.fill_(float("nan"))
                torch.cuda.synchronize()
                assert hip.hipGraphLaunch(exe, st) == 0
                assert hip.hipStreamSynchronize(st) == 0
                outs.append(host(Y))
                e.gemm(qw, Xd, Ye, N)  # eager between the replays
                e.sync()
                assert rel(host(Ye), ref) <= TOL
            for o in outs:
                assert rel(o, ref) <= TOL
                assert np.array_equal(o, outs[0])
        finally:
            hip.hipGraphExecDestroy(exe)
            hip.hipGraphDestroy(graph)
    finally:
        e.close()


# The grid barrier's bounded wait, forced from the host: OKF_FFN_STALL=1
# makes the next launch's barrier wait for one arrival more than the grid
# has, OKF_FFN_SPIN a short poll limit.  Every workgroup still finishes; the
# call must fail loudly (NaN in y, never a plausible wrong value), and the
# next call on the same context must give the normal result, bit for bit.
@pytest.mark.parametrize("mfma", ["1", "0"])
def test_ffn_barrier_timeout_is_loud_and_recovers(mfma):
    # The master's barrier wait is forced to give up (it waits for one arrival
    # more than the grid has, polls bounded from the host): every workgroup of
    # that launch must fail (NaN in every output row), the next okf_sync must
    # report OKF_E_TIMEOUT once, and the next launch must match a clean context
    # of the same kernel (mfma "1": ffn_mfma_kernel, "0": ffn_fused_kernel).
    import os

    def ctx(stall):
        env = {"OKF_FFN_MFMA": mfma, "OKF_FFN_FUSED": "2"}
        if stall:
            env.update(OKF_FFN_STALL="1", OKF_FFN_SPIN="2000")
        os.environ.update(env)
        try:
            return ok.Enc(0)
        finally:
            for k in env:
                del os.environ[k]

    e, clean = ctx(True), ctx(False)
    try:
        H, D = 6144, 2048
        wg, wu, wd = weights(Q2_0, H, D, 81), weights(Q2_0, H, D, 82), weights(Q2_0, D, H, 83)
        qg, qu, qd = (ok.QuantTensor(dev(w), k, m, Q2_0) for w, k, m in ((wg, D, H), (wu, D, H), (wd, H, D)))
        x = dev(acts(1, D, 84)[0])
        outs, codes = [], []
        for en in (e, e, clean):
            say("ffn barrier time-out", mfma, len(outs))
            g, u = torch.zeros(H, device="cuda"), torch.zeros(H, device="cuda")
            y = torch.zeros(D, device="cuda")
            en.ffn(qg, qu, qd, x, g, u, y)
            try:
                en.sync()
                codes.append(ok.OKF_OK)
            except ok.OkfError as err:
                codes.append(err.status)
            outs.append(host(y))
        assert codes == [ok.OKF_E_TIMEOUT, ok.OKF_OK, ok.OKF_OK]
        assert np.isnan(outs[0]).all()
        assert np.array_equal(outs[1], outs[2])
        # a failure not yet collected by okf_sync is reported by the next okf_ffn
        e2 = ctx(True)
        try:
            y = torch.zeros(D, device="cuda")
            g, u = torch.zeros(H, device="cuda"), torch.zeros(H, device="cuda")
            e2.ffn(qg, qu, qd, x, g, u, y)
            torch.cuda.synchronize()
            with pytest.raises(ok.OkfError) as err:
                e2.ffn(qg, qu, qd, x, g, u, y)
            assert err.value.status == ok.OKF_E_TIMEOUT
            e2.ffn(qg, qu, qd, x, g, u, y)
            e2.sync()
            assert np.array_equal(host(y), outs[2])
        finally:
            e2.close()
    finally:
        e.close()
        clean.close()


@pytest.fixture(scope="module")
def enc_ffn1():
    # okf_ffn as one launch wherever it fits (at the Bonsai shape the default
    # takes the two matrix-core launches)
    import os
    os.environ["OKF_FFN_FUSED"] = "2"
    try:
        e = ok.Enc(0)
    finally:
        del os.environ["OKF_FFN_FUSED"]
    yield e
    e.close()


@pytest.mark.parametrize("H,D,seed", [(6144, 2048, 1002), (8192, 4096, 38), (384, 640, 39), (128, 128, 40)])
def test_ffn_one_launch_matches_two(enc_ffn1, enc_ffn2, H, D, seed):
    say("ffn one launch", H, D)
    wg, wu, wd = weights(Q2_0, H, D, seed), weights(Q2_0, H, D, seed + 1), weights(Q2_0, D, H, seed + 2)
    qg, qu, qd = (ok.QuantTensor(dev(w), k, m, Q2_0) for w, k, m in ((wg, D, H), (wu, D, H), (wd, H, D)))
    x = dev(acts(1, D, seed + 10)[0])
    outs = []
    for e in (enc_ffn1, enc_ffn1, enc_ffn2):
        g, u = (torch.full((H,), float("nan"), device="cuda") for _ in range(2))
        y = torch.full((D,), float("nan"), device="cuda")
        e.ffn(qg, qu, qd, x, g, u, y)
        e.sync()
        outs.append([host(v).astype(np.float64) for v in (g, u, y)])
    for a, b in zip(outs[0], outs[1]):
        assert np.array_equal(a, b)
    for a, b in zip(outs[0], outs[2]):
        assert rel(a, b) <= 1e-5


@pytest.mark.parametrize("tg,tu,H,D,seed", [(Q2_0, Q2_0, 6144, 2048, 51), (Q2_0, Q2_0, 40, 1024, 52),
                                            (Q2_0, Q2_0, 45, 384, 56), (Q4_K, Q4_K, 7, 256, 57),
                                            (Q4_K, Q4_K, 1000, 768, 53), (IQ2_XXS, IQ2_XXS, 72, 512, 54),
                                            (Q8_0, Q4_0, 96, 256, 55)])
def test_gemv_gate_up_matches_oracle(enc, tg, tu, H, D, seed):
    # gate and up in one grid (rows paired per workgroup, any M), g = silu(gate) * up
    say("gate_up", NAMES[tg], NAMES[tu], H, D)
    wg, wu = weights(tg, H, D, seed), weights(tu, H, D, seed + 1)
    qg, qu = ok.QuantTensor(dev(wg), D, H, tg), ok.QuantTensor(dev(wu), D, H, tu)
    x = acts(1, D, seed + 2)[0]
    g, u = (torch.full((H,), float("nan"), device="cuda") for _ in range(2))
    enc.gemv_gate_up(qg, qu, dev(x), g, u)
    rg, ru = oracle.matvec(tg, wg, D, H, x), oracle.matvec(tu, wu, D, H, x)
    assert rel(host(u), ru.astype(np.float64)) <= TOL_MV
    assert rel(host(g), oracle.silu_mul(rg, ru).astype(np.float64)) <= TOL_MV


# ------------------------------------------------------------ parallel group
def test_parallel_group_matches_single_calls(enc):
    # MetalEnc.parallel { gate; up } (QwenMetalEngine.swift:918-923) plus more
    # matrices than one launch takes, of two formats and two K: every output
    # equals its single okf_gemv within float reassociation.
    cases = [(Q2_0, 6144, 2048, 1002), (Q2_0, 6144, 2048, 1202), (Q8_0, 300, 2048, 61),
             (Q2_0, 200, 2048, 62), (Q2_0, 130, 1024, 63), (Q2_0, 64, 2048, 64), (Q2_0, 96, 2048, 65),
             (Q8_0, 40, 2048, 66), (Q4_K, 1000, 2048, 67), (Q4_K, 37, 2048, 68), (Q4_K, 300, 1024, 69)]
    xs = {K: dev(acts(1, K, 70 + K)) for K in (1024, 2048)}
    ws, ys, singles = [], [], []
    for t, M, K, seed in cases:
        w = dev(weights(t, M, K, seed))
        ws.append(ok.QuantTensor(w, K, M, t))
        ys.append(torch.full((M,), float("nan"), device="cuda"))
        y1 = torch.full((M,), float("nan"), device="cuda")
        enc.gemv(ws[-1], xs[K], y1)
        singles.append(y1)
    with enc.parallel():
        for q, y in zip(ws, ys):
            enc.gemv(q, xs[q.K], y)
    enc.sync()
    for (t, M, K, seed), y, y1 in zip(cases, ys, singles):
        got, one = host(y), host(y1)
        ref = oracle.matvec(t, weights(t, M, K, seed), K, M, acts(1, K, 70 + K)[0]).astype(np.float64)
        say("group", NAMES[t], M, K, rel(got, ref))
        assert rel(got, ref) <= TOL_MV
        assert rel(got, one.astype(np.float64)) <= 1e-5


# ------------------------------------------------------------------ tile GEMM
# (The metric is relative to max|ref| over the output, so every case keeps
# enough outputs for that maximum to be representative; a single dot product
# can cancel to near zero, where fp16 staging error is not bounded by 1e-3.)
# The Q4_K kernel (256-row x 128-token tiles, one per CU) runs the tiles
# beyond whole rounds of 256 as 16 thin pieces each (64 rows x 32 tokens,
# whole K): the small cases are all thin pieces (M and N not multiples of the
# piece, K of 1 superblock leaves wavefronts without steps); (8192, 512,
# 1024) is exactly 256 whole tiles with eight N tiles per row block, grouped
# four to an XCD.
TILE = [(Q8_0, 300, 2048, 37), (Q2_0, 130, 1024, 129), (Q4_K, 260, 2304, 77), (IQ2_XXS, 129, 1536, 6),
        (Q4_K, 1, 256, 64), (Q8_0, 5, 96, 200), (Q4_K, 4224, 256, 512), (Q4_K, 1000, 512, 300),
        (Q4_K, 8192, 512, 1024),
        (Q4_0, 300, 2048, 37), (IQ4_NL, 130, 1024, 70), (Q5_K, 200, 1024, 40), (Q6_K, 129, 768, 33),
        (IQ4_XS, 260, 1280, 90), (Q2_0, 300, 2048, 300), (Q8_0, 130, 1024, 257), (IQ3_XXS, 260, 768, 256)] + [(t, 130, 768, 41) for t in (IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S, IQ1_M, Q2_K, Q3_K, F32,
                                                                F16, BF16)]


@pytest.mark.parametrize("t,M,K,N", TILE)
def test_tile_gemm_matches_oracle(enc, t, M, K, N):
    say("tile", NAMES[t], M, K, N)
    w = weights(t, M, K, 17)
    X = acts(N, K, 18)
    ref = oracle.matmul(t, w, K, M, X).astype(np.float64)
    got = run_gemm(enc, t, M, K, w, X, tile=True)
    assert rel(got, ref) <= TOL
    if N > 5 and not narrow_chunks(t, M, N, K):  # the auto path takes the tile past the narrow chunks
        assert np.array_equal(run_gemm(enc, t, M, K, w, X), got)


# From N = 256 the tile GEMM of the other formats converts X to fp16 once
# per call; the rounding is the one its loader applies per tile, so with
# OKF_GEMM_XH=0 (rounded per tile) the results are the same bits.
@pytest.fixture(scope="module")
def enc_noxh():
    import os
    os.environ["OKF_GEMM_XH"] = "0"
    try:
        e = ok.Enc(0)
    finally:
        del os.environ["OKF_GEMM_XH"]
    yield e
    e.close()


@pytest.mark.parametrize("t,M,K,N", [(Q2_0, 300, 2048, 300), (Q8_0, 130, 1024, 257), (Q6_K, 260, 768, 512)])
def test_tile_fp16_x_same_bits(enc, enc_noxh, t, M, K, N):
    say("tile fp16 x", NAMES[t], M, K, N)
    w = weights(t, M, K, 23)
    X = acts(N, K, 24)
    assert np.array_equal(run_gemm(enc, t, M, K, w, X, tile=True), run_gemm(enc_noxh, t, M, K, w, X, tile=True))


# The auto path for 5 < N <= narrow_max: consecutive narrow launches of up
# to narrow_cols columns (okf_quant.hip's narrow_max / narrow_cols).
SMALL_MAX = {Q8_0: 6, Q5_K: 6, Q6_K: 8, IQ4_XS: 8}  # M < 4096
NARROW_MAX = {Q4_K: 7, IQ2_XXS: 12, Q4_0: 8, IQ4_NL: 8, Q8_0: 5, Q6_K: 5, Q2_0: 5, F32: 5, F16: 5, BF16: 5}
NARROW_COLS = {IQ2_XXS: 4, Q4_0: 4, IQ4_NL: 4}


def mm_fits(t, M, K):
    return t in MM_FMTS and t != Q8_0 and K <= 6144 and K % 64 == 0 and M >= 4096


MM_MAX = {Q4_K: 16, Q3_K: 8}


def narrow_cols(t, M, K):
    return 4 if t in NARROW_COLS or mm_fits(t, M, K) else 5


def narrow_max(t, M, K):
    if M < 4096:
        return SMALL_MAX.get(t, 5)
    return MM_MAX.get(t, 12) if mm_fits(t, M, K) else NARROW_MAX.get(t, 12)


def narrow_chunks(t, M, N, K):
    first = 5 if t == IQ2_XXS or mm_fits(t, M, K) else 6
    return first <= N <= narrow_max(t, M, K)


CHUNKS = [(Q8_0, 300, 2048, 6), (Q6_K, 129, 768, 8), (IQ4_XS, 300, 1024, 7), (Q5_K, 130, 1024, 6),
          (IQ2_XXS, 4100, 1280, 12), (IQ2_XXS, 4097, 2048, 5), (Q4_K, 4100, 2048, 5), (Q4_K, 4100, 8192, 7),
          (Q4_K, 4200, 2304, 16), (Q5_K, 4100, 1024, 9), (IQ4_XS, 4100, 1024, 6), (IQ3_S, 4100, 1024, 12),
          (IQ1_M, 4099, 768, 9), (Q3_K, 4100, 1280, 8), (Q2_K, 4200, 1024, 11), (IQ2_S, 4096, 512, 12),
          (IQ1_S, 4097, 1536, 5), (Q4_0, 4100, 2048, 8), (IQ3_XXS, 4100, 768, 10)]


@pytest.mark.parametrize("t,M,K,N", CHUNKS)
def test_small_n_narrow_chunks(enc, t, M, K, N):
    say("chunks", NAMES[t], M, K, N)
    assert narrow_chunks(t, M, N, K)
    w = weights(t, M, K, 19)
    X = acts(N, K, 20)
    ref = oracle.matmul(t, w, K, M, X).astype(np.float64)
    got = run_gemm(enc, t, M, K, w, X)
    assert rel(got, ref) <= TOL_MV
    nc = narrow_cols(t, M, K)
    for c0 in range(0, N, nc):
        assert np.array_equal(got[c0:c0 + nc], run_gemm(enc, t, M, K, w, X[c0:c0 + nc]))


# With OKF_GEMM_KS=k the leftover tiles are split over k K ranges of whole
# superblocks instead (partial tiles added by a second kernel in K order):
# 2..9 ways, odd superblock counts leave the odd K half empty.
@pytest.fixture(scope="module")
def enc_ksplit():
    import os
    os.environ["OKF_GEMM_KS"] = "5"
    try:
        e = ok.Enc(0)
    finally:
        del os.environ["OKF_GEMM_KS"]
    yield e
    e.close()


@pytest.mark.parametrize("M,K,N", [(260, 2304, 77), (4224, 256, 512), (1000, 512, 300), (17408, 2560, 512)])
def test_q4_k_ksplit_matches_thin(enc, enc_ksplit, M, K, N):
    say("ksplit", M, K, N)
    w = weights(Q4_K, M, K, 21)
    X = acts(N, K, 22)
    ref = oracle.matmul(Q4_K, w, K, M, X).astype(np.float64) if M * N <= 300_000 else None
    got = run_gemm(enc_ksplit, Q4_K, M, K, w, X)
    thin = run_gemm(enc, Q4_K, M, K, w, X)
    if ref is not None:
        assert rel(got, ref) <= TOL
    assert rel(got, thin.astype(np.float64)) <= 1e-3


def test_q4_k_pp512_full_config(enc):
    # X 512 x 5120 . W(17408 x 5120, Q4_K) -> Y 512 x 17408.
    t, M, K, N = Q4_K, 17408, 5120, 512
    w = weights(t, M, K, 1003)
    X = acts(N, K, 2005)
    got = run_gemm(enc, t, M, K, w, X)
    assert np.isfinite(got).all()
    # the full oracle GEMM (512 sequential matvecs, GQ.matmul :159-169)
    ref = oracle.matmul(t, w, K, M, X).astype(np.float64)
    r = rel(got, ref)
    say("pp512 rel", r)
    assert r <= TOL
    # every token against the independent gemv kernel
    wd = dev(w)
    Xd = dev(X)
    y = torch.empty((N, M), device="cuda")
    qt = ok.QuantTensor(wd, K, M, t)
    for n in range(N):
        enc.gemv(qt, Xd[n], y[n])
    enc.sync()
    r2 = rel(got, host(y).astype(np.float64))
    say("pp512 vs gemv rel", r2)
    assert r2 <= TOL


# ------------------------------------------------------------------ failure handling
def test_injected_fault_launches_nothing(enc):
    t, M, K = Q8_0, 64, 256
    w = dev(weights(t, M, K, 3))
    x = dev(acts(1, K, 4))
    y = torch.full((M,), 7.0, device="cuda")
    enc.set_fault_rate(1.0, 5)
    try:
        with pytest.raises(ok.OkfError) as e:
            enc.gemv(ok.QuantTensor(w, K, M, t), x, y)
        assert e.value.status == ok.OKF_E_INJECTED
    finally:
        enc.set_fault_rate(0.0, 0)
    enc.sync()
    assert (host(y) == 7.0).all()
    enc.gemv(ok.QuantTensor(w, K, M, t), x, y)
    enc.sync()
    assert not (host(y) == 7.0).all()


# ------------------------------------------------------------------ embedding gather
@pytest.mark.parametrize("t", [Q8_0, Q2_0, Q4_K, IQ2_XXS, Q4_0, IQ4_NL, Q5_K, Q6_K, IQ4_XS, IQ2_XS, IQ2_S,
                               IQ3_XXS, IQ3_S, IQ1_S, IQ1_M, Q2_K, Q3_K, F32, F16, BF16], ids=lambda t: NAMES[t])
def test_embed_batch_bit_exact(enc, t):
    # embedBatch (MetalEnc.swift:1096-1146) vs the oracle's dequant of each row
    M, K = 300, 2048
    w = weights(t, M, K, 91)
    ids = np.array([0, 299, 17, 17, 150, 1, 298, 64], np.int32)
    out = torch.full((len(ids), K), float("nan"), device="cuda")
    enc.embed_batch(ok.QuantTensor(dev(w), K, M, t), dev(ids), len(ids), out)
    got = host(out)
    rb = row_bytes(t, K)
    for n, i in enumerate(ids):
        ref = oracle.dequant(t, w[i * rb:(i + 1) * rb], K)
        assert np.array_equal(got[n].view(np.uint32), ref.view(np.uint32)), (NAMES[t], n, i)


def test_embed_batch_clamps_ids(enc):
    M, K = 8, 256
    w = weights(Q4_K, M, K, 92)
    ids = np.array([-5, 8, 1000], np.int32)
    out = torch.empty((3, K), device="cuda")
    enc.embed_batch(ok.QuantTensor(dev(w), K, M, Q4_K), dev(ids), 3, out)
    got = host(out)
    rb = row_bytes(Q4_K, K)
    assert np.array_equal(got[0], oracle.dequant(Q4_K, w[:rb], K))
    assert np.array_equal(got[1], oracle.dequant(Q4_K, w[7 * rb:8 * rb], K))
    assert np.array_equal(got[2], got[1])


# ------------------------------------------------------------------ GGUF weights
def test_gguf_upload_then_gemv(enc, tmp_path):
    # GGUF(path:) + the MetalContext weight window: a tensor read from a file,
    # made device-resident, then used through its okf_weight
    import ggufw as gw
    w4 = weights(Q4_K, 96, 1024, 93)
    w2 = weights(Q2_0, 64, 512, 94)
    path = tmp_path / "m.gguf"
    gw.write(path, [("general.alignment", gw.U32, 32)],
             [("a.weight", [1024, 96], Q4_K, w4.tobytes()), ("b.weight", [512, 64], Q2_0, w2.tobytes())])
    with ok.GGUF(str(path)) as g:
        base = g.upload(enc)
        try:
            for name, t, M, K, w in (("a.weight", Q4_K, 96, 1024, w4), ("b.weight", Q2_0, 64, 512, w2)):
                x = acts(1, K, 95)
                y = torch.full((M,), float("nan"), device="cuda")
                enc.gemv(g.weight(name, base), dev(x), y)
                ref = oracle.matvec(t, w, K, M, x[0]).astype(np.float64)
                assert rel(host(y), ref) <= TOL_MV
        finally:
            enc.sync()
            enc._lib.okf_gguf_free_device(enc.h, ctypes.c_void_p(base))
