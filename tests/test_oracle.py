"""Pins the CPU oracle (oracle/okf_oracle.c) before anything is checked against it.

Every check here is independent of the oracle's own code: the reference's
table data (tests/golden/iq2xxs_tables.json, extracted from two copies in the
reference), hand-built blocks with closed-form answers, an independent
vectorised numpy decoder, float64 brute force, and invariants.
"""
import json
import os
import re

import numpy as np
import pytest

import oracle
from chatokf_amd import synth
from chatokf_amd.formats import (Q8_0, Q2_0, Q4_K, IQ2_XXS, Q4_0, IQ4_NL, Q5_K, Q6_K, IQ4_XS, IQ2_XS, IQ2_S,  # noqa: E501
                                 IQ3_XXS, IQ3_S, IQ1_S, IQ1_M, F32, F16, BF16, Q2_K, Q3_K)

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLD = json.load(open(os.path.join(ROOT, "tests", "golden", "iq2xxs_tables.json")))
GRID = np.array([int(v, 16) for v in GOLD["iq2xxs_grid"]], dtype=np.uint64)
KSIGNS = np.array(GOLD["ksigns"], dtype=np.uint8)
IQG = json.load(open(os.path.join(ROOT, "tests", "golden", "iq_grids.json")))
G = {k: np.array([int(v, 16) for v in IQG[k]], dtype=np.uint64) for k in
     ("iq1s", "iq2xs", "iq2s", "iq3xxs", "iq3s")}


def _f16(v):
    return np.frombuffer(np.float16(v).tobytes(), np.uint8)


# ------------------------------------------------------------------ tables
def _inc_grid(path, name):
    text = open(path).read()
    body = text[text.index(name):]
    body = body[body.index("{") + 1: body.index("}")]
    return [int(t.rstrip("ull"), 16) for t in re.findall(r"0x[0-9a-fA-F]+ull", body)]


@pytest.mark.parametrize("path,name", [
    ("oracle/iq2xxs_grid.inc", "okf_ref_iq2xxs_grid"),
    ("chatokf_amd/csrc/iq2xxs_grid.inc", "okf_iq2xxs_grid_host"),
])
def test_grid_tables_match_reference(path, name):
    assert _inc_grid(os.path.join(ROOT, path), name) == [int(v) for v in GRID]


@pytest.mark.parametrize("name", ["iq1s", "iq2xs", "iq2s", "iq3xxs", "iq3s"])
@pytest.mark.parametrize("path,prefix", [("oracle/iq_grids.inc", "okf_ref_"),
                                         ("chatokf_amd/csrc/iq_grids.inc", "okf_host_")])
def test_iq_grids_match_reference(name, path, prefix):
    """The C tables against the fixture made from the reference's two copies
    (Swift and IQTables.h, which tests/golden/make_iq_grids.py checks agree)."""
    text = open(os.path.join(ROOT, path)).read()
    body = text[text.index(prefix + name + "_grid"):]
    body = body[body.index("{") + 1: body.index("}")]
    vals = [int(t, 16) for t in re.findall(r"0x([0-9a-fA-F]+)", body)]
    assert vals == [int(v) for v in G[name]]


def test_iq_grid_invariants():
    # magnitudes: IQ2_XS / IQ2_S grid bytes are from {8, 25, 43}, IQ3 bytes
    # take 8 levels (IQ3_XXS 4 + 8i with 62 on top, IQ3_S the odd 1..15), IQ1
    # digits are ternary (0, 1, 2) in the nibbles 8 (j % 4) + 4 (j / 4)
    for k in ("iq2xs", "iq2s"):
        b = set(int(v) >> (8 * j) & 255 for v in G[k] for j in range(8))
        assert b <= {8, 25, 43}
        assert len(set(int(v) for v in G[k])) == len(G[k])  # distinct entries
    for k, levels in (("iq3xxs", {4, 12, 20, 28, 36, 44, 52, 62}), ("iq3s", set(range(1, 16, 2)))):
        b = set(int(v) >> (8 * j) & 255 for v in G[k] for j in range(4))
        assert b == levels
        assert len(set(int(v) for v in G[k])) == len(G[k])
    dig = set(int(v) >> (8 * (j % 4) + 4 * (j // 4)) & 15 for v in G["iq1s"] for j in range(8))
    assert dig <= {0, 1, 2}
    assert all((int(v) & 0xF0F0F0F0) >> 4 <= 0x02020202 for v in G["iq1s"])
    assert len(set(int(v) for v in G["iq1s"])) == 2048


def test_oracle_ksigns_match_reference():
    text = open(os.path.join(ROOT, "oracle/iq2xxs_grid.inc")).read()
    body = text[text.index("okf_ref_ksigns"):]
    body = body[body.index("{") + 1: body.index("}")]
    assert [int(t) for t in re.findall(r"\d+", body)] == GOLD["ksigns"]
    assert GOLD["kmask"] == [1 << j for j in range(8)]


def test_ksigns_is_even_parity_completion():
    # The eighth sign bit makes the number of negated weights even; the HIP
    # kernels compute it this way instead of loading the table.
    for i in range(128):
        par = bin(i).count("1") & 1
        assert KSIGNS[i] == i | (par << 7)


def test_grid_magnitudes():
    mags = {(int(e) >> (8 * j)) & 0xFF for e in GRID for j in range(8)}
    assert mags == {0x08, 0x19, 0x2B}
    assert len(set(int(e) for e in GRID)) == 256


@pytest.mark.skipif(not os.path.isdir("/root/reference/LLM"), reason="reference checkout absent")
def test_golden_fixture_is_current(tmp_path):
    import subprocess
    import sys
    env = dict(os.environ)
    out = tmp_path / "t.json"
    script = os.path.join(ROOT, "tests/golden/make_iq2_tables.py")
    # regenerate into a temp copy of the script dir
    src = open(script).read().replace('HERE = os.path.dirname(os.path.abspath(__file__))',
                                      f'HERE = {str(tmp_path)!r}')
    p = tmp_path / "mk.py"
    p.write_text(src)
    subprocess.run([sys.executable, str(p)], check=True, env=env, capture_output=True)
    assert json.load(open(tmp_path / "iq2xxs_tables.json")) == GOLD


# ------------------------------------------------------------------ sizes
def test_row_bytes_match_rowByteCount():
    # GGUF.rowByteCount, LLM/Base/GGUF.swift:160-188, at the BASELINE shapes
    cases = [(Q8_0, 2048, 2176), (Q2_0, 2048, 544), (Q2_0, 6144, 1632),
             (Q4_K, 5120, 2880), (Q4_K, 17408, 9792), (IQ2_XXS, 5120, 1320)]
    for t, n, want in cases:
        assert oracle.row_bytes(t, n) == want
    with pytest.raises(ValueError):
        oracle.row_bytes(Q4_K, 100)


def test_f16_conversion_exact():
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits[::7]], np.float32)
    r = ref[::7]
    nan = np.isnan(r)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), r[~nan].view(np.uint32))


# ------------------------------------------------------------------ known answers
def test_q8_0_known_answer():
    qs = np.array(list(range(-127, 128, 8)), np.int8)  # 32 values
    assert qs.size == 32
    blk = np.concatenate([_f16(1.0), qs.view(np.uint8)])
    assert np.array_equal(oracle.dequant(Q8_0, blk, 32), qs.astype(np.float32))
    blk = np.concatenate([_f16(0.5), qs.view(np.uint8)])
    assert np.array_equal(oracle.dequant(Q8_0, blk, 32), qs.astype(np.float32) * 0.5)


def test_q2_0_known_answer():
    # byte 0b11100100 holds codes 0, 1, 2, 3 (LSB first) -> -d, 0, d, 2d
    qs = np.full(32, 0b11100100, np.uint8)
    blk = np.concatenate([_f16(0.25), qs])
    want = np.tile(np.array([-0.25, 0.0, 0.25, 0.5], np.float32), 32)
    assert np.array_equal(oracle.dequant(Q2_0, blk, 128), want)


def test_q4_k_known_answer_scale_paths():
    # d = 1, dmin = 2.  Scale bytes s[0..11]:
    #   s[0..3] = 0x45 -> j<4: sc = 0x45 & 63 = 5; top bits 01 feed j>=4 sc
    #   s[4..7] = 0x83 -> j<4: mn = 3;            top bits 10 feed j>=4 mn
    #   s[8..11] = 0x7A -> j>=4: sc = 0xA | (1 << 4) = 26, mn = 7 | (2 << 4) = 39
    hdr = np.concatenate([_f16(1.0), _f16(2.0), np.array([0x45] * 4 + [0x83] * 4 + [0x7A] * 4, np.uint8)])
    qs = (np.arange(128) % 16 | ((15 - np.arange(128) % 16) << 4)).astype(np.uint8)
    w = oracle.dequant(Q4_K, np.concatenate([hdr, qs]), 256)
    for sb in range(8):
        sc, mn = (5, 3) if sb < 4 else (26, 39)
        g, hi = sb // 2, sb % 2
        for l in range(32):
            q = int(qs[g * 32 + l])
            nib = (q >> 4) if hi else (q & 15)
            assert w[sb * 32 + l] == np.float32(sc * nib - 2.0 * mn)


def test_iq2_xxs_known_answer():
    d = _f16(1.0)
    sub = []
    # sub-block 0: grid 0 (all 8s), signs 0 (+), scale 0 -> db = 1/8 -> all 1.0
    sub.append((0, 0, 0))
    # sub-block 1: grid 1 (byte 0 = 0x2b), signs idx 127 (all -), scale 15 -> db = 3.875
    sub.append((0x01010101, 0x7F | (0x7F << 7) | (0x7F << 14) | (0x7F << 21), 15))
    while len(sub) < 8:
        sub.append((0, 0, 0))
    qs = []
    for a0, s, sc in sub:
        a1 = s | (sc << 28)
        qs += list(np.array([a0, a1], np.uint32).view(np.uint8))
    w = oracle.dequant(IQ2_XXS, np.concatenate([d, np.array(qs, np.uint8)]), 256)
    assert np.array_equal(w[:32], np.ones(32, np.float32))
    row = np.array([-43.0] + [-8.0] * 7, np.float32) * np.float32(3.875)
    assert np.array_equal(w[32:64], np.tile(row, 4))


# ------------------------------------------------------------------ numpy decoders
def np_dequant(t, w, M, K):
    """Independent vectorised decoders (array arithmetic in float32)."""
    if t == Q8_0:
        b = w.reshape(M, K // 32, 34)
        d = b[:, :, :2].copy().view(np.float16).astype(np.float32)
        q = b[:, :, 2:].view(np.int8).astype(np.float32)
        return (q * d).reshape(M, K)
    if t == Q2_0:
        b = w.reshape(M, K // 128, 34)
        d = b[:, :, :2].copy().view(np.float16).astype(np.float32)
        qs = b[:, :, 2:]
        codes = np.stack([(qs >> s) & 3 for s in (0, 2, 4, 6)], -1).reshape(M, K // 128, 128)
        return ((codes.astype(np.float32) - 1) * d).reshape(M, K)
    if t == Q4_K:
        b = w.reshape(M, K // 256, 144)
        d = b[:, :, 0:2].copy().view(np.float16).astype(np.float32)[..., 0]
        dm = b[:, :, 2:4].copy().view(np.float16).astype(np.float32)[..., 0]
        s = b[:, :, 4:16].astype(np.uint32)
        sc = np.zeros((M, K // 256, 8), np.uint32)
        mn = np.zeros_like(sc)
        sc[..., :4] = s[..., 0:4] & 63
        mn[..., :4] = s[..., 4:8] & 63
        sc[..., 4:] = (s[..., 8:12] & 15) | ((s[..., 0:4] >> 6) << 4)
        mn[..., 4:] = (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)
        qs = b[:, :, 16:].reshape(M, K // 256, 4, 32)
        nib = np.stack([qs & 15, qs >> 4], 3).reshape(M, K // 256, 8, 32).astype(np.float32)
        d1 = d[..., None] * sc.astype(np.float32)
        o1 = dm[..., None] * mn.astype(np.float32)
        return (d1[..., None] * nib - o1[..., None]).reshape(M, K)
    if t == IQ2_XXS:
        b = w.reshape(M, K // 256, 66)
        d = b[:, :, 0:2].copy().view(np.float16).astype(np.float32)[..., 0]
        a = b[:, :, 2:].copy().view(np.uint32).reshape(M, K // 256, 8, 2)
        a0, a1 = a[..., 0], a[..., 1]
        db = d[..., None] * (np.float32(0.5) + (a1 >> 28).astype(np.float32)) * np.float32(0.25)
        out = np.empty((M, K // 256, 8, 4, 8), np.float32)
        for l in range(4):
            e = GRID[(a0 >> (8 * l)) & 255]
            sg = KSIGNS[(a1 >> (7 * l)) & 127]
            for j in range(8):
                g = ((e >> np.uint64(8 * j)) & np.uint64(255)).astype(np.float32)
                s = np.where(sg & (1 << j), np.float32(-1), np.float32(1))
                out[..., l, j] = db * g * s
        return out.reshape(M, K)
    if t == Q5_K:
        b = w.reshape(M, K // 256, 176)
        d = b[:, :, 0:2].copy().view(np.float16).astype(np.float32)[..., 0]
        dm = b[:, :, 2:4].copy().view(np.float16).astype(np.float32)[..., 0]
        s = b[:, :, 4:16].astype(np.uint32)
        sc = np.concatenate([s[..., 0:4] & 63, (s[..., 8:12] & 15) | ((s[..., 0:4] >> 6) << 4)], -1)
        mn = np.concatenate([s[..., 4:8] & 63, (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)], -1)
        qh = b[:, :, 16:48]
        qs = b[:, :, 48:].reshape(M, K // 256, 4, 32)
        q = np.empty((M, K // 256, 8, 32), np.float32)
        for g in range(4):  # group g: sub-blocks 2g (low nibbles) and 2g + 1 (high)
            q[:, :, 2 * g] = (qs[:, :, g] & 15) + 16 * ((qh >> (2 * g)) & 1)
            q[:, :, 2 * g + 1] = (qs[:, :, g] >> 4) + 16 * ((qh >> (2 * g + 1)) & 1)
        d1 = d[..., None] * sc.astype(np.float32)
        o1 = dm[..., None] * mn.astype(np.float32)
        return (d1[..., None] * q - o1[..., None]).reshape(M, K)
    if t == Q6_K:
        b = w.reshape(M, K // 256, 210)
        ql, qh = b[:, :, 0:128].astype(np.int32), b[:, :, 128:192].astype(np.int32)
        sc = b[:, :, 192:208].view(np.int8).astype(np.float32)
        d = b[:, :, 208:210].copy().view(np.float16).astype(np.float32)[..., 0]
        out = np.empty((M, K // 256, 2, 4, 32), np.float32)
        for n in range(2):
            lo, hi = ql[:, :, 64 * n:64 * n + 32], ql[:, :, 64 * n + 32:64 * n + 64]
            h = qh[:, :, 32 * n:32 * n + 32]
            quads = [(lo & 15), (hi & 15), (lo >> 4), (hi >> 4)]
            for r in range(4):
                q = quads[r] | (((h >> (2 * r)) & 3) << 4)
                s = np.repeat(sc[:, :, 8 * n + 2 * r:8 * n + 2 * r + 2], 16, axis=-1)
                out[:, :, n, r] = d[..., None] * s * (q - 32).astype(np.float32)
        return out.reshape(M, K)
    if t == IQ4_XS:
        b = w.reshape(M, K // 256, 136)
        d = b[:, :, 0:2].copy().view(np.float16).astype(np.float32)[..., 0]
        sh = b[:, :, 2:4].copy().view(np.uint16)[..., 0].astype(np.int32)
        sl = b[:, :, 4:8].astype(np.int32)
        qs = b[:, :, 8:].reshape(M, K // 256, 8, 16)
        out = np.empty((M, K // 256, 8, 32), np.float32)
        for ib in range(8):
            ls = ((sl[..., ib // 2] >> (4 * (ib % 2))) & 15) | (((sh >> (2 * ib)) & 3) << 4)
            dl = d * (ls - 32).astype(np.float32)
            out[:, :, ib, :16] = dl[..., None] * IQ4NL_TABLE[qs[:, :, ib] & 15]
            out[:, :, ib, 16:] = dl[..., None] * IQ4NL_TABLE[qs[:, :, ib] >> 4]
        return out.reshape(M, K)
    if t in (IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S, IQ1_M):
        return np.stack([_np_iq(t, w.reshape(M, -1)[m]) for m in range(M)])
    if t == F32:
        return w.view(np.float32).reshape(M, K).copy()
    if t == F16:
        return w.view(np.float16).astype(np.float32).reshape(M, K)
    if t == BF16:
        return (w.view(np.uint16).astype(np.uint32) << 16).view(np.float32).reshape(M, K)
    if t == Q2_K:
        b = w.reshape(M, K // 256, 84)
        d = b[:, :, 80:82].copy().view(np.float16).astype(np.float32)
        dm = b[:, :, 82:84].copy().view(np.float16).astype(np.float32)
        sc = b[:, :, :16].astype(np.float32)
        out = np.empty((M, K // 256, 2, 4, 2, 16), np.float32)
        for n in range(2):
            for s in range(4):
                for h in range(2):
                    i = n * 8 + s * 2 + h
                    q = (b[:, :, 16 + 32 * n + 16 * h:32 + 32 * n + 16 * h] >> (2 * s)) & 3
                    dl = d[..., 0] * (b[:, :, i] & 15).astype(np.float32)
                    ml = dm[..., 0] * (b[:, :, i] >> 4).astype(np.float32)
                    out[:, :, n, s, h] = dl[..., None] * q.astype(np.float32) - ml[..., None]
        return out.reshape(M, K)
    if t == Q3_K:
        b = w.reshape(M, K // 256, 110).astype(np.int64)
        d = w.reshape(M, K // 256, 110)[:, :, 108:110].copy().view(np.float16).astype(np.float32)[..., 0]
        # the 16 6-bit scales: low nibble from byte i (i < 8) or the high
        # nibble of byte i - 8, top two bits from byte 8 + i % 4 at 2 (i // 4)
        sc = np.empty((M, K // 256, 16), np.int64)
        for i in range(16):
            lo = (b[:, :, 96 + (i % 8)] >> (4 * (i // 8))) & 15
            hi = (b[:, :, 104 + i % 4] >> (2 * (i // 4))) & 3
            sc[:, :, i] = (lo | (hi << 4)) - 32
        out = np.empty((M, K // 256, 2, 4, 2, 16), np.float32)
        for n in range(2):
            for s in range(4):
                for h in range(2):
                    q = (b[:, :, 32 + 32 * n + 16 * h:48 + 32 * n + 16 * h] >> (2 * s)) & 3
                    bump = np.where(b[:, :, 16 * h:16 * h + 16] & (1 << (4 * n + s)), 0, 4).astype(np.float32)
                    dl = d * sc[:, :, n * 8 + s * 2 + h].astype(np.float32)
                    out[:, :, n, s, h] = dl[..., None] * (q.astype(np.float32) - bump)
        return out.reshape(M, K)
    if t in (Q4_0, IQ4_NL):
        b = w.reshape(M, K // 32, 18)
        d = b[:, :, :2].copy().view(np.float16).astype(np.float32)
        q = np.concatenate([b[:, :, 2:] & 15, b[:, :, 2:] >> 4], -1)  # j, j + 16
        v = q.astype(np.float32) - 8 if t == Q4_0 else IQ4NL_TABLE[q]
        return (v * d).reshape(M, K)
    raise ValueError(t)


def _g8(entry, nbytes):
    return [(int(entry) >> (8 * j)) & 255 for j in range(nbytes)]


def _np_iq(t, row):
    """One row of the grid formats, superblock by superblock, written from the
    ggml block layouts (float32 array arithmetic, the reference's order)."""
    f32, out = np.float32, []
    for b in row.reshape(-1, len(row) // (len(row) // {IQ2_XS: 74, IQ2_S: 82, IQ3_XXS: 98, IQ3_S: 110,
                                                         IQ1_S: 50, IQ1_M: 56}[t])):
        b = b.astype(np.int64)
        w = np.zeros(256, np.float32)
        d = np.frombuffer(bytes(np.uint8(b[:2])), np.float16)[0].astype(f32) if t != IQ1_M else None
        sgn = lambda s, j: f32(-1) if (int(s) >> j) & 1 else f32(1)  # noqa: E731
        for ib in range(8):
            if t in (IQ2_XS, IQ2_S):
                sc = b[66 + ib] if t == IQ2_XS else b[74 + ib]
                db = [d * (f32(0.5) + f32(sc & 15)) * f32(0.25), d * (f32(0.5) + f32(sc >> 4)) * f32(0.25)]
                for l in range(4):
                    if t == IQ2_XS:
                        q = b[2 + 2 * (ib * 4 + l)] | (b[3 + 2 * (ib * 4 + l)] << 8)
                        g, s = _g8(G["iq2xs"][q & 511], 8), KSIGNS[q >> 9]
                    else:
                        g = _g8(G["iq2s"][b[2 + ib * 4 + l] | ((b[66 + ib] << (8 - 2 * l)) & 0x300)], 8)
                        s = b[34 + ib * 4 + l]
                    for j in range(8):
                        w[ib * 32 + l * 8 + j] = sgn(s, j) * (db[l // 2] * f32(g[j]))
            elif t == IQ3_XXS:
                aux = int(b[66 + 4 * ib]) | int(b[67 + 4 * ib]) << 8 | int(b[68 + 4 * ib]) << 16 | int(b[69 + 4 * ib]) << 24
                db = d * (f32(0.5) + f32(aux >> 28)) * f32(0.5)
                for l in range(4):
                    s = KSIGNS[(aux >> (7 * l)) & 127]
                    g = _g8(G["iq3xxs"][b[2 + ib * 8 + 2 * l]], 4) + _g8(G["iq3xxs"][b[3 + ib * 8 + 2 * l]], 4)
                    for j in range(8):
                        w[ib * 32 + l * 8 + j] = sgn(s, j) * (db * f32(g[j]))
            elif t == IQ3_S:
                sc = b[106 + ib // 2] >> (4 * (ib % 2)) & 15
                db = d * f32(1 + 2 * sc)
                qh = b[66 + ib]
                for l in range(4):
                    g = (_g8(G["iq3s"][b[2 + ib * 8 + 2 * l] | ((qh << (8 - 2 * l)) & 256)], 4)
                         + _g8(G["iq3s"][b[3 + ib * 8 + 2 * l] | ((qh << (7 - 2 * l)) & 256)], 4))
                    s = b[74 + ib * 4 + l]
                    for j in range(8):
                        w[ib * 32 + l * 8 + j] = sgn(s, j) * (db * f32(g[j]))
            else:  # IQ1_S / IQ1_M: digits n in {0, 1, 2}, w = dl (n - 1 + delta)
                if t == IQ1_S:
                    h = int(b[34 + 2 * ib]) | int(b[35 + 2 * ib]) << 8
                    dls = [d * f32(2 * ((h >> 12) & 7) + 1)] * 2
                    hb = [(h >> (3 * l)) & 7 for l in range(4)]
                    neg = [h >> 15] * 4
                    qs = b[2 + ib * 4: 6 + ib * 4]
                else:
                    sc = [int(b[48 + 2 * i]) | int(b[49 + 2 * i]) << 8 for i in range(4)]
                    bits = (sc[0] >> 12) | ((sc[1] >> 8) & 0xF0) | ((sc[2] >> 4) & 0xF00) | (sc[3] & 0xF000)
                    dm = np.array([bits], np.uint16).view(np.float16)[0].astype(f32)
                    s = sc[ib // 2] >> (6 * (ib % 2))
                    dls = [dm * f32(2 * (s & 7) + 1), dm * f32(2 * ((s >> 3) & 7) + 1)]
                    h = [int(b[32 + 2 * ib]), int(b[33 + 2 * ib])]
                    hb = [h[l // 2] & 7 if l % 2 == 0 else (h[l // 2] >> 4) & 7 for l in range(4)]
                    neg = [(h[l // 2] >> (3 if l % 2 == 0 else 7)) & 1 for l in range(4)]
                    qs = b[ib * 4: ib * 4 + 4]
                for l in range(4):
                    e = int(G["iq1s"][int(qs[l]) | (hb[l] << 8)])
                    delta = f32(-0.125) if neg[l] else f32(0.125)
                    for j in range(8):
                        n = (e >> (8 * (j % 4) + 4 * (j // 4))) & 15
                        w[ib * 32 + l * 8 + j] = dls[l // 2] * (f32(n) - f32(1) + delta)
        out.append(w)
    return np.concatenate(out)


# IQ4_NL's 16 non-linear levels, as published with the format (ggml's
# kvalues_iq4nl); the golden test checks them against the reference's copy.
IQ4NL_TABLE = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113],
                       np.float32)

SMALL = [(Q8_0, 64, 256), (Q2_0, 64, 512), (Q4_K, 32, 512), (IQ2_XXS, 32, 512), (Q4_0, 64, 256),
         (IQ4_NL, 64, 256), (Q5_K, 32, 512), (Q6_K, 32, 512), (IQ4_XS, 32, 512), (IQ2_XS, 8, 512),
         (IQ2_S, 8, 512), (IQ3_XXS, 8, 512), (IQ3_S, 8, 512), (IQ1_S, 8, 512), (IQ1_M, 8, 512),
         (Q2_K, 16, 512), (Q3_K, 16, 512), (F32, 16, 256), (F16, 16, 256), (BF16, 16, 256)]


@pytest.mark.parametrize("t,M,K", SMALL)
def test_oracle_dequant_matches_numpy(t, M, K):
    w = synth.weights(t, M, K, 77)
    ref = np_dequant(t, w, M, K)
    rb = oracle.row_bytes(t, K)
    for m in range(M):
        got = oracle.dequant(t, w[m * rb:(m + 1) * rb], K)
        assert np.array_equal(got.view(np.uint32), ref[m].view(np.uint32)), m


def test_q2_0_code3_decodes_to_2d():
    w = synth.q2_0(4, 256, 5, codes=4)
    ref = np_dequant(Q2_0, w, 4, 256)
    got = np.concatenate([oracle.dequant(Q2_0, w[m * 68:(m + 1) * 68], 256) for m in range(4)])
    assert np.array_equal(got, ref.reshape(-1))
    d = w.reshape(-1, 34)[:, :2].copy().view(np.float16).astype(np.float32)
    assert np.any(ref.reshape(-1, 128) == 2 * d)  # some code 3 was drawn


# ------------------------------------------------------------------ matvec/matmul
@pytest.mark.parametrize("t,M,K", SMALL + [(Q2_0, 48, 6144 // 4), (Q4_K, 16, 4096)])
def test_matvec_matches_float64(t, M, K):
    w = synth.weights(t, M, K, 11)
    x = synth.activations(1, K, 12)[0]
    W = np_dequant(t, w, M, K).astype(np.float64)
    ref = W @ x.astype(np.float64)
    y = oracle.matvec(t, w, K, M, x)
    assert np.abs(y - ref).max() / np.abs(ref).max() < 2e-6


@pytest.mark.parametrize("t,M,K", SMALL)
def test_matmul_is_column_matvecs(t, M, K):
    w = synth.weights(t, M, K, 21)
    X = synth.activations(3, K, 22)
    Y = oracle.matmul(t, w, K, M, X)
    for n in range(3):
        y = oracle.matvec(t, w, K, M, X[n])
        if t in (Q8_0, Q4_0):  # block-reuse matmul sums in another order
            assert np.abs(Y[n] - y).max() <= 1e-5 * np.abs(y).max()
        else:  # GQ.matmul runs the matvec itself
            assert np.array_equal(Y[n], y)


def test_matvec_thread_count_does_not_change_bits():
    w = synth.weights(Q4_K, 37, 1024, 31)
    x = synth.activations(1, 1024, 32)[0]
    a = oracle.matvec(Q4_K, w, 1024, 37, x, threads=1)
    b = oracle.matvec(Q4_K, w, 1024, 37, x, threads=7)
    assert np.array_equal(a, b)


def test_matvec_linear_in_x():
    w = synth.weights(IQ2_XXS, 16, 512, 41)
    x = synth.activations(1, 512, 42)[0]
    a = oracle.matvec(IQ2_XXS, w, 512, 16, x)
    b = oracle.matvec(IQ2_XXS, w, 512, 16, 2 * x)  # exact: scaling by 2
    assert np.array_equal(2 * a, b)
    c = oracle.matvec(IQ2_XXS, w, 512, 16, -x)
    assert np.array_equal(-a, c)


def test_silu_mul_known_values_and_float64():
    # Swift silu (LLM/Base/Kernels.swift:3): x / (1 + expf(-x)), times b
    a = np.array([0.0, 1.0, -1.0, 20.0, -20.0, 88.0, -88.0, 0.5], np.float32)
    b = np.array([3.0, 1.0, 1.0, 1.0, 1.0, 2.0, 2.0, -4.0], np.float32)
    got = oracle.silu_mul(a, b)
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    ref = a64 / (1.0 + np.exp(-a64)) * b64
    assert got[0] == 0.0
    assert np.allclose(got, ref, rtol=2e-7, atol=1e-30)
    assert abs(got[3] - 20.0) < 1e-5 and abs(got[4]) < 1e-7
    rng = np.random.default_rng(3)
    x = rng.standard_normal(4096).astype(np.float32) * 4
    y = rng.standard_normal(4096).astype(np.float32)
    x64 = x.astype(np.float64)
    assert np.allclose(oracle.silu_mul(x, y), x64 / (1 + np.exp(-x64)) * y, rtol=1e-6, atol=1e-7)


def test_add_rmsnorm_closed_forms():
    # a constant row c with eps = 0 normalizes to exactly 1 (c / sqrt(c^2))
    x = np.full((2, 64), 3.0, np.float32)
    xs, y = oracle.add_rmsnorm(x, None, np.ones(64, np.float32), 0.0)
    assert np.array_equal(xs, x) and np.array_equal(y, np.ones((2, 64), np.float32))
    # residual add is one fp32 add per element; the norm matches float64
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 2048)).astype(np.float32)
    r = rng.standard_normal((5, 2048)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 2048).astype(np.float32)
    xs, y = oracle.add_rmsnorm(x, r, w, 1e-6)
    assert np.array_equal(xs, x + r)
    s = (x + r).astype(np.float64)
    ref = s / np.sqrt((s * s).mean(axis=1, keepdims=True) + 1e-6) * w
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()
    # scale invariance with eps = 0: rmsnorm(2x) == rmsnorm(x)
    _, y1 = oracle.add_rmsnorm(x, None, w, 0.0)
    _, y2 = oracle.add_rmsnorm(2 * x, None, w, 0.0)
    assert np.allclose(y1, y2, rtol=1e-6, atol=0)


def _argmax_ref(x):
    # numpy's argmax takes the first maximum; NaN never wins, a row with
    # nothing above -inf gives 0
    z = np.where(np.isnan(x), -np.inf, x)
    return np.argmax(z, axis=-1).astype(np.int32)


def test_argmax_rows_ties_nan_and_brute_force():
    x = np.array([[1, 3, 3, 2], [np.nan, 5, np.nan, 5], [np.nan] * 4, [-np.inf] * 4, [0, -np.inf, np.nan, 0]],
                 np.float32)
    assert oracle.argmax_rows(x).tolist() == [1, 1, 0, 0, 0]
    rng = np.random.default_rng(4)
    x = rng.integers(-50, 50, (7, 1000)).astype(np.float32)  # many ties
    x[2, ::7] = np.nan
    assert np.array_equal(oracle.argmax_rows(x), _argmax_ref(x))


def test_q4_0_and_iq4_nl_known_answer():
    # d = 1: byte j holds codes for weights j (low nibble) and j + 16 (high)
    d = np.array([1.0], np.float16).view(np.uint8)
    qs = np.array([(j & 15) | ((15 - (j & 15)) << 4) for j in range(16)], np.uint8)
    blk = np.concatenate([d, qs])
    w = oracle.dequant(Q4_0, blk, 32)
    assert np.array_equal(w[:16], np.arange(16, dtype=np.float32) - 8)
    assert np.array_equal(w[16:], 15 - np.arange(16, dtype=np.float32) - 8)
    w = oracle.dequant(IQ4_NL, blk, 32)
    assert np.array_equal(w[:16], IQ4NL_TABLE)
    assert np.array_equal(w[16:], IQ4NL_TABLE[::-1])


def test_q5_k_q6_k_iq4_xs_known_answer():
    # Q5_K, d = 1, dmin = 0, sub-block 0 scale 1: w[l] = (nibble | qh bit 0 << 4)
    blk = np.zeros(176, np.uint8)
    blk[0:2] = _f16(1.0)
    blk[4] = 1
    blk[48:80] = np.arange(32) & 15
    blk[16 + 16:16 + 32] = 1  # qh bit 0 for l >= 16
    w = oracle.dequant(Q5_K, blk, 256)
    assert np.array_equal(w[:32], np.arange(32, dtype=np.float32))
    assert np.array_equal(w[32:], np.zeros(224, np.float32))  # other scales 0
    # Q6_K, d = 1: zero codes give -32 * scale, and each 16 weights of
    # (n, r) take their own scale scales[n*8 + 2r + l/16]
    blk = np.zeros(210, np.uint8)
    blk[192:208] = np.arange(1, 17)
    blk[208:210] = _f16(1.0)
    w = oracle.dequant(Q6_K, blk, 256)
    assert np.array_equal(w, -32 * np.repeat(np.arange(1, 17), 16).astype(np.float32))
    blk[0:192] = 0xFF  # every code 63: w = scale * 31
    w = oracle.dequant(Q6_K, blk, 256)
    assert np.array_equal(w, 31 * np.repeat(np.arange(1, 17), 16).astype(np.float32))
    # IQ4_XS, d = 1: ls = 33 everywhere (low nibbles 1, high bits 2) gives
    # dl = 1, so the weights are the levels; ls = 0 gives dl = -32
    blk = np.zeros(136, np.uint8)
    blk[0:2] = _f16(1.0)
    blk[2:4] = np.array([0xAAAA], np.uint16).view(np.uint8)
    blk[4:8] = 0x11
    blk[8:136] = np.tile(np.array([j | ((15 - j) << 4) for j in range(16)], np.uint8), 8)
    w = oracle.dequant(IQ4_XS, blk, 256).reshape(8, 32)
    assert np.array_equal(w[:, :16], np.tile(IQ4NL_TABLE, (8, 1)))
    assert np.array_equal(w[:, 16:], np.tile(IQ4NL_TABLE[::-1], (8, 1)))
    blk[2:8] = 0
    w = oracle.dequant(IQ4_XS, blk, 256).reshape(8, 32)
    assert np.array_equal(w[:, :16], np.tile(-32 * IQ4NL_TABLE, (8, 1)))


def test_grid_formats_known_answer():
    f32 = np.float32
    # IQ2_XS, d = 1, scales 0 -> db = 1/8; index 0 (all 8s) with sign index 0
    # -> 1.0; index 1 (byte 0 is 43) with sign index 127 (all eight negated)
    blk = np.zeros(74, np.uint8)
    blk[0:2] = _f16(1.0)
    blk[2:4] = np.array([1 | (127 << 9)], np.uint16).view(np.uint8)  # group 0: index 1, signs 127
    blk[66] = 0x20  # sub-block 0: low scale 0 (groups 0, 1), high scale 2 (groups 2, 3)
    w = oracle.dequant(IQ2_XS, blk, 256)
    assert np.array_equal(w[:8], -f32(0.125) * np.array([43] + [8] * 7, f32))  # byte j = weight j
    assert np.array_equal(w[8:16], np.ones(8, f32))
    assert np.array_equal(w[16:32], np.full(16, f32(2.5 * 0.25 * 8)))  # (0.5 + 2) / 4 * 8
    # IQ2_S: the grid index takes bits 2l.. of qh as bits 8, 9; signs are bytes
    blk = np.zeros(82, np.uint8)
    blk[0:2] = _f16(1.0)
    blk[2] = 1  # group 0 low index 1 ...
    blk[66] = 0b01  # ... plus qh bits 0-1 = 1 -> index 257
    blk[34] = 0x81  # signs of group 0: weights 0 and 7
    w = oracle.dequant(IQ2_S, blk, 256)
    g = _g8(G["iq2s"][257], 8)
    assert np.array_equal(w[:8], np.array([(-1 if j in (0, 7) else 1) * 0.125 * g[j] for j in range(8)], f32))
    # IQ3_XXS, d = 1, aux = 0 -> db = 1/4; index 0 (all 4s) -> 1.0; aux scale
    # 15 -> db = 15.5 / 2
    blk = np.zeros(98, np.uint8)
    blk[0:2] = _f16(1.0)
    blk[66 + 4:70 + 4] = np.array([15 << 28], np.uint32).view(np.uint8)
    w = oracle.dequant(IQ3_XXS, blk, 256)
    assert np.array_equal(w[:32], np.ones(32, f32))
    assert np.array_equal(w[32:64], np.full(32, f32(15.5 * 0.5 * 4)))
    # IQ3_S, d = 1, scale nibble 0 -> db = 1; index 0 (all 1s); sign byte
    # 0xFF negates its group; qh bit 0 lifts the first index of group 0 to 256
    blk = np.zeros(110, np.uint8)
    blk[0:2] = _f16(1.0)
    blk[74 + 1] = 0xFF
    w = oracle.dequant(IQ3_S, blk, 256)
    assert np.array_equal(w[:8], np.ones(8, f32)) and np.array_equal(w[8:16], -np.ones(8, f32))
    blk[66] = 1
    w = oracle.dequant(IQ3_S, blk, 256)
    assert np.array_equal(w[:4], np.array(_g8(G["iq3s"][256], 4), f32))
    # IQ1_S, d = 1: grid 0 (all digits 0) -> -1 + 1/8; h = 0x8000 | 7 << 12 ->
    # dl = 15, delta = -1/8; index 1 has digit 2 at j = 0 -> dl (1 + delta)
    blk = np.zeros(50, np.uint8)
    blk[0:2] = _f16(1.0)
    blk[36:38] = np.array([0x8000 | (7 << 12)], np.uint16).view(np.uint8)  # sub-block 1
    blk[2 + 4] = 1  # sub-block 1, group 0: index 1
    w = oracle.dequant(IQ1_S, blk, 256)
    assert np.array_equal(w[:32], np.full(32, f32(-0.875)))
    assert w[32] == f32(15 * 0.875) and np.array_equal(w[33:64], np.full(31, f32(-15 * 1.125)))
    # IQ1_M: d = 1.0 (0x3C00) spread over the top nibbles of the scale shorts
    blk = np.zeros(56, np.uint8)
    blk[48:56] = np.array([0x0000, 0x0000, 0xC000, 0x3000], np.uint16).view(np.uint8)
    w = oracle.dequant(IQ1_M, blk, 256)
    assert np.array_equal(w, np.full(256, f32(-0.875)))


def test_q2_k_q3_k_dense_known_answer():
    f32 = np.float32
    # Q2_K, d = 1, dmin = 1/2: scale byte 0x13 -> dl = 3, ml = 1/2; codes
    # 0..3 in the first byte's four 2-bit fields go to weights 0, 32, 64, 96
    blk = np.zeros(84, np.uint8)
    blk[0] = blk[2] = blk[4] = blk[6] = 0x13
    blk[16] = 0b11100100  # codes 0, 1, 2, 3
    blk[80:82], blk[82:84] = _f16(1.0), _f16(0.5)
    w = oracle.dequant(Q2_K, blk, 256)
    assert [w[0], w[32], w[64], w[96]] == [f32(-0.5), f32(2.5), f32(5.5), f32(8.5)]
    assert w[1] == f32(-0.5) and w[16] == 0  # weights 16..31 take scale byte 1 = 0
    # Q3_K, d = 1: scale 32 + 2 (low nibble 2, top bits 2) gives dl = 2;
    # hmask bit set -> no bump, clear -> code - 4
    blk = np.zeros(110, np.uint8)
    blk[96] = 0x02
    blk[104] = 0b10  # top bits of scale 0
    blk[32] = 3
    blk[0] = 1  # hmask bit 0 of weight 0
    blk[108:110] = _f16(1.0)
    w = oracle.dequant(Q3_K, blk, 256)
    assert w[0] == f32(6) and w[1] == f32(-8)  # 2 * 3 and 2 * (0 - 4)
    # dense: f16 1.5, bf16 0x3FC0 = 1.5, f32 as stored
    assert oracle.dequant(F16, np.tile(_f16(1.5), 32), 32)[0] == f32(1.5)
    assert oracle.dequant(BF16, np.tile(np.array([0xC0, 0x3F], np.uint8), 32), 32)[0] == f32(1.5)
    v = np.arange(32, dtype=np.float32) / 7
    assert np.array_equal(oracle.dequant(F32, v.view(np.uint8), 32), v)


def test_iq4_nl_table_matches_reference_golden():
    """IQ4_NL.kvalues (LLM/Gemma/Gemma4Quant.swift:8-11), cross-checked against
    the Metal header's copy by tests/golden/make_iq2_tables.py."""
    assert np.array_equal(np.array(GOLD["kvalues_iq4nl"], np.float32), IQ4NL_TABLE)
    assert np.all(np.diff(IQ4NL_TABLE) > 0) and IQ4NL_TABLE[0] == -127 and IQ4NL_TABLE[-1] == 113
