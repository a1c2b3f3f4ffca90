"""Seeded synthetic weights and activations for the benchmark configurations.

The pseudo-random source is the reference's 64-bit LCG
(``LLM/Qwen/QwenMetalSelfTest.swift:5-14``): ``s = seed + 0x9E3779B97F4A7C15``,
then per draw ``s = s * 6364136223846793005 + 1442695040888963407`` and
``u32 = s >> 33`` (so a draw holds 31 random bits).  The stream is produced vectorised with a jump-ahead
(doubling) construction, so gigabyte-sized tensors take seconds.

Derived draws (fixed here, the reference has none of them):

* byte          = low 8 bits of a u32;
* U(a, b)       = a + (b - a) * u32 / 2**31, computed in float64;
* fp16 scale    = U(a, b) rounded to nearest-even binary16 (the stored bits
  are the ground truth);
* N(0, 1)       = Box-Muller on two consecutive u32:
  ``sqrt(-2 ln((u0 + 0.5) / 2**31)) * cos(2 pi u1 / 2**31)``, then float32.

Block layouts follow the reference decoders: Q8_0 ``{f16 d; i8 qs[32]}``
(``LLM/Gemma/Gemma4Quant.swift:51-69``), Q2_0 ``{f16 d; u8 qs[32]}`` per 128
weights (``LLM/Base/Quant.swift:2-25``), Q4_K ``{f16 d; f16 dmin; u8 scales[12];
u8 qs[128]}`` (``LLM/Quantize/KQuants.swift:103-125``), IQ2_XXS
``{f16 d; u16 qs[32]}`` (``LLM/Quantize/IQ2XXS.swift:34-54``).
"""
from __future__ import annotations

import numpy as np

from .formats import (Q8_0, Q2_0, Q4_K, IQ2_XXS, Q4_0, IQ4_NL, Q5_K, Q6_K, IQ4_XS, IQ2_XS, IQ2_S, IQ3_XXS,
                      IQ3_S, IQ1_S, IQ1_M, F32, F16, BF16, Q2_K, Q3_K, row_bytes)

_A = 6364136223846793005
_C = 1442695040888963407
_GOLD = 0x9E3779B97F4A7C15
_MASK = (1 << 64) - 1


class LCG:
    """Sequential stream of the reference LCG; ``u32(n)`` continues it."""

    def __init__(self, seed: int):
        self.s = (seed + _GOLD) & _MASK

    def u32(self, n: int) -> np.ndarray:
        n = int(n)
        if n <= 0:
            return np.zeros(0, np.uint32)
        out = np.empty(n, np.uint64)
        with np.errstate(over="ignore"):
            out[0] = np.uint64((self.s * _A + _C) & _MASK)
            filled, a_l, c_l = 1, _A, _C  # (a_l, c_l): the filled-length step
            while filled < n:
                take = min(filled, n - filled)
                out[filled:filled + take] = out[:take] * np.uint64(a_l) + np.uint64(c_l)
                # compose the transform with itself: L -> 2L steps
                a_l, c_l = (a_l * a_l) & _MASK, (c_l * a_l + c_l) & _MASK
                filled += take
            self.s = int(out[-1])
            return (out >> np.uint64(33)).astype(np.uint32)

    def uniform(self, a: float, b: float, n: int) -> np.ndarray:
        return a + (b - a) * (self.u32(n).astype(np.float64) / 2147483648.0)

    def f16(self, a: float, b: float, n: int) -> np.ndarray:
        return self.uniform(a, b, n).astype(np.float16)

    def bytes(self, n: int) -> np.ndarray:
        return (self.u32(n) & 0xFF).astype(np.uint8)

    def normal(self, n: int) -> np.ndarray:
        u = self.u32(2 * n).astype(np.float64).reshape(n, 2)
        r = np.sqrt(-2.0 * np.log((u[:, 0] + 0.5) / 2147483648.0))
        return (r * np.cos(2.0 * np.pi * u[:, 1] / 2147483648.0)).astype(np.float32)


def _f16_bytes(v: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(v.astype(np.float16)).view(np.uint8).reshape(-1, 2)


def q8_0(M: int, K: int, seed: int, d_range=(1e-3, 1e-2)) -> np.ndarray:
    """M rows of Q8_0: d ~ U(d_range) as fp16, qs uniform integers in [-127, 127]."""
    nb = M * (K // 32)
    g = LCG(seed)
    d = g.f16(*d_range, nb)
    qs = ((g.u32(nb * 32) % 255).astype(np.int16) - 127).astype(np.int8)
    blk = np.empty((nb, 34), np.uint8)
    blk[:, :2] = _f16_bytes(d)
    blk[:, 2:] = qs.view(np.uint8).reshape(nb, 32)
    return blk.reshape(-1)


def nibble32(M: int, K: int, seed: int, d_range=(1e-3, 1e-2)) -> np.ndarray:
    """M rows of 18-byte 32-weight blocks (Q4_0 / IQ4_NL): d ~ U(d_range) as
    fp16, the 16 code bytes uniform random."""
    nb = M * (K // 32)
    g = LCG(seed)
    d = g.f16(*d_range, nb)
    blk = np.empty((nb, 18), np.uint8)
    blk[:, :2] = _f16_bytes(d)
    blk[:, 2:] = g.bytes(nb * 16).reshape(nb, 16)
    return blk.reshape(-1)


def q2_0(M: int, K: int, seed: int, d_range=(0.01, 0.05), codes=3) -> np.ndarray:
    """M rows of Q2_0 (Bonsai ternary): codes uniform in {0..codes-1}, d ~ U."""
    nb = M * (K // 128)
    g = LCG(seed)
    d = g.f16(*d_range, nb)
    c = (g.u32(nb * 128) % codes).astype(np.uint8).reshape(nb, 32, 4)
    packed = c[:, :, 0] | (c[:, :, 1] << 2) | (c[:, :, 2] << 4) | (c[:, :, 3] << 6)
    blk = np.empty((nb, 34), np.uint8)
    blk[:, :2] = _f16_bytes(d)
    blk[:, 2:] = packed
    return blk.reshape(-1)


def q4_k(M: int, K: int, seed: int, d_range=(1e-3, 1e-2)) -> np.ndarray:
    """M rows of Q4_K: d, dmin ~ U(d_range) fp16; scales[12], qs[128] uniform bytes."""
    nb = M * (K // 256)
    g = LCG(seed)
    d = g.f16(*d_range, nb)
    dmin = g.f16(*d_range, nb)
    rest = g.bytes(nb * 140).reshape(nb, 140)
    blk = np.empty((nb, 144), np.uint8)
    blk[:, 0:2] = _f16_bytes(d)
    blk[:, 2:4] = _f16_bytes(dmin)
    blk[:, 4:] = rest
    return blk.reshape(-1)


def iq2_xxs(M: int, K: int, seed: int, d_range=(1e-3, 1e-2)) -> np.ndarray:
    """M rows of IQ2_XXS: d ~ U(d_range) fp16; the 64 qs bytes uniform."""
    nb = M * (K // 256)
    g = LCG(seed)
    d = g.f16(*d_range, nb)
    blk = np.empty((nb, 66), np.uint8)
    blk[:, :2] = _f16_bytes(d)
    blk[:, 2:] = g.bytes(nb * 64).reshape(nb, 64)
    return blk.reshape(-1)


def q5_k(M: int, K: int, seed: int, d_range=(1e-3, 1e-2)) -> np.ndarray:
    """M rows of Q5_K: d, dmin ~ U(d_range) fp16; scales[12], qh[32], qs[128]
    uniform bytes."""
    nb = M * (K // 256)
    g = LCG(seed)
    d = g.f16(*d_range, nb)
    dmin = g.f16(*d_range, nb)
    blk = np.empty((nb, 176), np.uint8)
    blk[:, 0:2] = _f16_bytes(d)
    blk[:, 2:4] = _f16_bytes(dmin)
    blk[:, 4:] = g.bytes(nb * 172).reshape(nb, 172)
    return blk.reshape(-1)


def q6_k(M: int, K: int, seed: int, d_range=(1e-4, 1e-3)) -> np.ndarray:
    """M rows of Q6_K: ql[128], qh[64], int8 scales[16] uniform bytes; d at
    byte 208 ~ U(d_range) fp16 (scales reach +-128, so d is smaller)."""
    nb = M * (K // 256)
    g = LCG(seed)
    d = g.f16(*d_range, nb)
    blk = np.empty((nb, 210), np.uint8)
    blk[:, :208] = g.bytes(nb * 208).reshape(nb, 208)
    blk[:, 208:] = _f16_bytes(d)
    return blk.reshape(-1)


def iq4_xs(M: int, K: int, seed: int, d_range=(1e-4, 1e-3)) -> np.ndarray:
    """M rows of IQ4_XS: d ~ U(d_range) fp16; scales_h, scales_l[4] and
    qs[128] uniform bytes."""
    nb = M * (K // 256)
    g = LCG(seed)
    d = g.f16(*d_range, nb)
    blk = np.empty((nb, 136), np.uint8)
    blk[:, :2] = _f16_bytes(d)
    blk[:, 2:] = g.bytes(nb * 134).reshape(nb, 134)
    return blk.reshape(-1)


def _d_first(nbytes):
    """256-weight blocks of `nbytes`: fp16 d ~ U(d_range) first, the rest uniform bytes."""
    def gen(M: int, K: int, seed: int, d_range=(1e-3, 1e-2)) -> np.ndarray:
        nb = M * (K // 256)
        g = LCG(seed)
        d = g.f16(*d_range, nb)
        blk = np.empty((nb, nbytes), np.uint8)
        blk[:, :2] = _f16_bytes(d)
        blk[:, 2:] = g.bytes(nb * (nbytes - 2)).reshape(nb, nbytes - 2)
        return blk.reshape(-1)
    gen.__doc__ = f"M rows of {nbytes}-byte superblocks: d ~ U(d_range) fp16, the rest uniform bytes."
    return gen


def iq1_m(M: int, K: int, seed: int, d_range=(1e-3, 1e-2)) -> np.ndarray:
    """M rows of IQ1_M: qs, qh and the scale fields uniform; the fp16 d ~
    U(d_range) spread over the top nibbles of the four scale shorts
    (IQ1M.scale, LLM/Quantize/IQ2XXS.swift:63-72)."""
    nb = M * (K // 256)
    g = LCG(seed)
    d = g.f16(*d_range, nb).view(np.uint16).astype(np.uint16)
    blk = g.bytes(nb * 56).reshape(nb, 56)
    sc = blk[:, 48:56].copy().view(np.uint16).reshape(nb, 4) & np.uint16(0x0FFF)
    for i in range(4):
        sc[:, i] |= ((d >> np.uint16(4 * i)) & np.uint16(0xF)) << np.uint16(12)
    blk[:, 48:56] = sc.view(np.uint8).reshape(nb, 8)
    return blk.reshape(-1)


def _d_last(nbytes, nd):
    """256-weight blocks of `nbytes` with `nd` fp16 scales ~ U(d_range) at the
    end (Q2_K: d, dmin; Q3_K: d), the rest uniform bytes."""
    def gen(M: int, K: int, seed: int, d_range=(1e-3, 1e-2)) -> np.ndarray:
        nb = M * (K // 256)
        g = LCG(seed)
        blk = np.empty((nb, nbytes), np.uint8)
        blk[:, :nbytes - 2 * nd] = g.bytes(nb * (nbytes - 2 * nd)).reshape(nb, nbytes - 2 * nd)
        for i in range(nd):
            blk[:, nbytes - 2 * (nd - i):nbytes - 2 * (nd - i) + 2] = _f16_bytes(g.f16(*d_range, nb))
        return blk.reshape(-1)
    gen.__doc__ = f"M rows of {nbytes}-byte K-quant superblocks: {nd} fp16 scale(s) at the end, the rest uniform."
    return gen


def dense(kind):
    """M rows of plain weights (f32, f16 or bf16): N(0, 1) / 16 from the LCG."""
    def gen(M: int, K: int, seed: int) -> np.ndarray:
        v = (LCG(seed).normal(M * K) / 16).astype(np.float32)
        if kind == "f32":
            return v.view(np.uint8)
        if kind == "f16":
            return v.astype(np.float16).view(np.uint8)
        return (v.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)  # bf16: the upper half
    return gen


GENERATORS = {Q8_0: q8_0, Q2_0: q2_0, Q4_K: q4_k, IQ2_XXS: iq2_xxs, Q4_0: nibble32, IQ4_NL: nibble32,
              Q5_K: q5_k, Q6_K: q6_k, IQ4_XS: iq4_xs, IQ2_XS: _d_first(74), IQ2_S: _d_first(82),
              IQ3_XXS: _d_first(98), IQ3_S: _d_first(110), IQ1_S: _d_first(50), IQ1_M: iq1_m,
              Q2_K: _d_last(84, 2), Q3_K: _d_last(110, 1), F32: dense("f32"), F16: dense("f16"),
              BF16: dense("bf16")}


def weights(ggml_type: int, M: int, K: int, seed: int) -> np.ndarray:
    w = GENERATORS[ggml_type](M, K, seed)
    assert w.size == M * row_bytes(ggml_type, K)
    return w


def activations(N: int, K: int, seed: int) -> np.ndarray:
    """X[N][K] ~ N(0, 1), float32, row-major."""
    return LCG(seed).normal(N * K).reshape(N, K)
