// okf_decode.h -- bit-exact decoders of one 32-weight unit per format.
//
// A "unit" is 32 consecutive weights of a row: Q8_0 one block, Q2_0 a quarter
// block, Q4_K and IQ2_XXS one sub-block.  These produce exactly the fp32
// values of the reference's CPU decoders: every product and difference is
// rounded separately (no contraction), in the reference's order.
#pragma once
#include "okf_common.h"

namespace okf {

#pragma clang fp contract(off)

// Q8_0.dequant, LLM/Gemma/Gemma4Quant.swift:55-68: w = Float(q) * d.
__device__ __forceinline__ void decode_unit_q8_0(const uint8_t *row, uint32_t u, float *w) {
    const uint8_t *b = row + (uint64_t)u * 34;
    float d = h2f(ldu<uint16_t>(b));
    uint32_t q[8];
    *(uint4 *)&q[0] = ldu<uint4>(b + 2);
    *(uint4 *)&q[4] = ldu<uint4>(b + 18);
#pragma unroll
    for (int j = 0; j < 32; j++) {
        int v = (int8_t)byte_of(q[j >> 2], j & 3);
        w[j] = (float)v * d;
    }
}

// Q2_0.dequant, LLM/Base/Quant.swift:10-25: w = Float(code - 1) * d with the
// 2-bit codes LSB-first; unit u covers weights 32*(u&3).. of block u>>2.
__device__ __forceinline__ void decode_unit_q2_0(const uint8_t *row, uint32_t u, float *w) {
    const uint8_t *b = row + (uint64_t)(u >> 2) * 34;
    float d = h2f(ldu<uint16_t>(b));
    uint2 q = ldu<uint2>(b + 2 + (u & 3) * 8);
#pragma unroll
    for (int j = 0; j < 32; j++) {
        uint32_t dw = j < 16 ? q.x : q.y;
        int code = (int)((dw >> (2 * (j & 15))) & 3);
        w[j] = (float)(code - 1) * d;
    }
}

// KQuant.scaleMin (LLM/Quantize/KQuants.swift:86-101) for sub-block j, from the
// three scale words of a Q4_K header (bytes 4..15: sy = s0..s3, sz = s4..s7,
// sw = s8..s11).
__device__ __forceinline__ void q4k_scale_min(uint32_t sy, uint32_t sz, uint32_t sw, uint32_t j,
                                              uint32_t &sc, uint32_t &mn) {
    uint32_t jj = j & 3;
    uint32_t by = byte_of(sy, jj), bz = byte_of(sz, jj);
    if (j < 4) {
        sc = by & 63;
        mn = bz & 63;
    } else {
        uint32_t bw = byte_of(sw, jj);
        sc = (bw & 0xF) | ((by >> 6) << 4);
        mn = (bw >> 4) | ((bz >> 6) << 4);
    }
}

// Scales/mins of the sub-block pair (2g, 2g + 1) that share code bytes 32g..
__device__ __forceinline__ void q4k_scale_min_pair(uint4 hdr, uint32_t g, uint32_t &sc0,
                                                   uint32_t &mn0, uint32_t &sc1, uint32_t &mn1) {
    q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * g, sc0, mn0);
    q4k_scale_min(hdr.y, hdr.z, hdr.w, 2 * g + 1, sc1, mn1);
}

// KQuant.q4K, LLM/Quantize/KQuants.swift:104-125, sub-block j = u & 7 of
// superblock u >> 3: w[l] = (d * sc) * Float(nibble) - dmin * m.
__device__ __forceinline__ void decode_unit_q4_k(const uint8_t *row, uint32_t u, float *w) {
    const uint8_t *b = row + (uint64_t)(u >> 3) * 144;
    uint4 hdr = ldu<uint4>(b);
    uint32_t j = u & 7, g = j >> 1, hi = j & 1;
    uint32_t sc, mn;
    q4k_scale_min(hdr.y, hdr.z, hdr.w, j, sc, mn);
    float d = h2f(hdr.x & 0xFFFF), dmin = h2f(hdr.x >> 16);
    float d1 = d * (float)sc, o1 = dmin * (float)mn;
    uint32_t q[8];
    *(uint4 *)&q[0] = ldu<uint4>(b + 16 + g * 32);
    *(uint4 *)&q[4] = ldu<uint4>(b + 32 + g * 32);
#pragma unroll
    for (int l = 0; l < 32; l++) {
        uint32_t nib = (byte_of(q[l >> 2], l & 3) >> (hi * 4)) & 0xF;
        w[l] = d1 * (float)nib - o1;
    }
}

// IQ2XXS.dequant, LLM/Quantize/IQ2XXS.swift:34-54, sub-block ib = u & 7 of
// superblock u >> 3: db = d * (0.5 + (a1 >> 28)) * 0.25; w = db * g * sign.
// grid is the 256-entry table (two u32 per entry, low word first).
__device__ __forceinline__ void decode_unit_iq2_xxs(const uint8_t *row, uint32_t u, float *w,
                                                    const uint2 *grid) {
    const uint8_t *b = row + (uint64_t)(u >> 3) * 66;
    float d = h2f(ldu<uint16_t>(b));
    uint2 a = ldu<uint2>(b + 2 + (u & 7) * 8);
    float db = d * (0.5f + (float)(a.y >> 28)) * 0.25f;
#pragma unroll
    for (int l = 0; l < 4; l++) {
        uint2 e = grid[byte_of(a.x, l)];
        uint32_t s = iq2_signs((a.y >> (7 * l)) & 127);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            float g = (float)byte_of(j < 4 ? e.x : e.y, j & 3);
            float sg = (s >> j) & 1 ? -1.0f : 1.0f;
            w[l * 8 + j] = db * g * sg;
        }
    }
}

// Q4_0.dequant, LLM/Gemma/Gemma4Quant.swift:30-49: byte j of the block gives
// w[j] = (Float(b & 0xF) - 8) * d and w[j + 16] = (Float(b >> 4) - 8) * d.
__device__ __forceinline__ void decode_unit_q4_0(const uint8_t *row, uint32_t u, float *w) {
    const uint8_t *b = row + (uint64_t)u * 18;
    float d = h2f(ldu<uint16_t>(b));
    uint32_t q[4];
    *(uint4 *)&q[0] = ldu<uint4>(b + 2);
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const uint32_t v = byte_of(q[j >> 2], j & 3);
        w[j] = ((float)(v & 15) - 8.0f) * d;
        w[j + 16] = ((float)(v >> 4) - 8.0f) * d;
    }
}

// IQ4_NL.dequant, Gemma4Quant.swift:13-27: w = kvalues[nibble] * d, the same
// nibble placement as Q4_0.
__device__ __forceinline__ void decode_unit_iq4_nl(const uint8_t *row, uint32_t u, float *w) {
    const uint8_t *b = row + (uint64_t)u * 18;
    float d = h2f(ldu<uint16_t>(b));
    uint32_t q[4];
    *(uint4 *)&q[0] = ldu<uint4>(b + 2);
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const uint32_t v = byte_of(q[j >> 2], j & 3);
        w[j] = (float)iq4nl_level(v & 15) * d;
        w[j + 16] = (float)iq4nl_level(v >> 4) * d;
    }
}

// KQuant.q5K, LLM/Quantize/KQuants.swift:127-155, sub-block j = u & 7 of
// superblock u >> 3: code group g = j >> 1 (bytes 48 + 32 g ..), low
// nibbles for even j, high for odd; the fifth bit is bit j of qh[l] (bytes
// 16..47); w = (d * sc) * Float(q) - dmin * m.
__device__ __forceinline__ void decode_unit_q5_k(const uint8_t *row, uint32_t u, float *w) {
    const uint8_t *b = row + (uint64_t)(u >> 3) * 176;
    const uint4 hdr = ldu<uint4>(b);
    const uint32_t j = u & 7, g = j >> 1, hi = j & 1;
    uint32_t sc, mn;
    q4k_scale_min(hdr.y, hdr.z, hdr.w, j, sc, mn);
    const float d = h2f(hdr.x & 0xFFFF), dmin = h2f(hdr.x >> 16);
    const float d1 = d * (float)sc, o1 = dmin * (float)mn;
    uint32_t q[8], h[8];
    *(uint4 *)&q[0] = ldu<uint4>(b + 48 + g * 32);
    *(uint4 *)&q[4] = ldu<uint4>(b + 64 + g * 32);
    *(uint4 *)&h[0] = ldu<uint4>(b + 16);
    *(uint4 *)&h[4] = ldu<uint4>(b + 32);
#pragma unroll
    for (int l = 0; l < 32; l++) {
        const uint32_t nib = (byte_of(q[l >> 2], l & 3) >> (hi * 4)) & 0xF;
        const uint32_t hb = (byte_of(h[l >> 2], l & 3) >> j) & 1;
        w[l] = d1 * (float)(nib + 16 * hb) - o1;
    }
}

// KQuant.q6K, LLM/Quantize/KQuants.swift:157-176, 32-weight group u & 7 =
// (n, r) of superblock u >> 3: weight n*128 + r*32 + l is the low (r < 2) or
// high nibble of ql[n*64 + l] (r even) or ql[n*64 + 32 + l] (r odd), with
// bits 2r, 2r + 1 of qh[n*32 + l] on top; w = d * Float(s) * Float(q - 32),
// s = int8 scales[n*8 + 2r + l/16], d at byte 208.
__device__ __forceinline__ void decode_unit_q6_k(const uint8_t *row, uint32_t u, float *w) {
    const uint8_t *b = row + (uint64_t)(u >> 3) * 210;
    const uint32_t n = (u >> 2) & 1, r = u & 3;
    const float d = h2f(ldu<uint16_t>(b + 208));
    uint32_t q[8], h[8];
    const uint8_t *qb = b + n * 64 + (r & 1) * 32;
    *(uint4 *)&q[0] = ldu<uint4>(qb);
    *(uint4 *)&q[4] = ldu<uint4>(qb + 16);
    *(uint4 *)&h[0] = ldu<uint4>(b + 128 + n * 32);
    *(uint4 *)&h[4] = ldu<uint4>(b + 144 + n * 32);
    const uint2 sc2 = make_uint2(byte_of(ldu<uint16_t>(b + 192 + n * 8 + 2 * r), 0),
                                 byte_of(ldu<uint16_t>(b + 192 + n * 8 + 2 * r), 1));
#pragma unroll
    for (int l = 0; l < 32; l++) {
        const uint32_t nib = (byte_of(q[l >> 2], l & 3) >> ((r >> 1) * 4)) & 0xF;
        const uint32_t hb = (byte_of(h[l >> 2], l & 3) >> (2 * r)) & 3;
        const int s = (int8_t)(l < 16 ? sc2.x : sc2.y);
        w[l] = d * (float)s * (float)((int)(nib | (hb << 4)) - 32);
    }
}

// IQX.iq4XS, LLM/Quantize/IQ3.swift:118-133, sub-block ib = u & 7 of
// superblock u >> 3: ls = (nibble ib of scales_l) | (bits 2 ib of scales_h)
// << 4, dl = d * Float(ls - 32), w = dl * level(nibble) with the IQ4_NL
// levels, low nibbles of qs[ib*16 + j] for j < 16, high for j + 16.
__device__ __forceinline__ void decode_unit_iq4_xs(const uint8_t *row, uint32_t u, float *w) {
    const uint8_t *b = row + (uint64_t)(u >> 3) * 136;
    const uint32_t ib = u & 7;
    const float d = h2f(ldu<uint16_t>(b));
    const uint32_t sh = ldu<uint16_t>(b + 2), sl = b[4 + ib / 2];
    const int ls = (int)(((sl >> (4 * (ib & 1))) & 0xF) | (((sh >> (2 * ib)) & 3) << 4));
    const float dl = d * (float)(ls - 32);
    uint32_t q[4];
    *(uint4 *)&q[0] = ldu<uint4>(b + 8 + ib * 16);
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const uint32_t v = byte_of(q[j >> 2], j & 3);
        w[j] = dl * (float)iq4nl_level(v & 15);
        w[j + 16] = dl * (float)iq4nl_level(v >> 4);
    }
}

// IQX.sign (LLM/Quantize/IQ3.swift:9-11): bit j of the sign byte negates.
__device__ __forceinline__ float iq_sign(uint32_t signs, int j, float v) { return (signs >> j) & 1 ? -v : v; }

// IQX.iq2XS / IQX.iq2S (LLM/Quantize/IQ3.swift:14-57), sub-block ib = u & 7:
// db = d * (0.5 + nibble) * 0.25 (low nibble for groups 0, 1, high for 2, 3);
// w = sign(db * grid byte j).
template <bool S>
__device__ __forceinline__ void decode_unit_iq2_xs_s(const uint8_t *row, uint32_t u, float *w,
                                                     const uint8_t *fg) {
    const uint8_t *b = row + (uint64_t)(u >> 3) * (S ? 82 : 74);
    const uint32_t ib = u & 7;
    const float d = h2f(ldu<uint16_t>(b));
    const uint32_t sc = b[(S ? 74 : 66) + ib];
    const float db0 = d * (0.5f + (float)(sc & 0xF)) * 0.25f, db1 = d * (0.5f + (float)(sc >> 4)) * 0.25f;
    const uint64_t *grid = (const uint64_t *)fg;
#pragma unroll
    for (int l = 0; l < 4; l++) {
        uint64_t e;
        uint32_t signs;
        if constexpr (S) {
            const uint32_t qh = b[66 + ib];
            e = grid[b[2 + ib * 4 + l] | ((qh << (8 - 2 * l)) & 0x300)];
            signs = b[34 + ib * 4 + l];
        } else {
            const uint32_t q = ldu<uint16_t>(b + 2 + (ib * 4 + l) * 2);
            e = grid[q & 511];
            signs = iq2_signs(q >> 9);
        }
        const float dl = l < 2 ? db0 : db1;
#pragma unroll
        for (int j = 0; j < 8; j++) w[l * 8 + j] = iq_sign(signs, j, dl * (float)((e >> (8 * j)) & 0xFF));
    }
}

// IQX.iq3XXS / IQX.iq3S (LLM/Quantize/IQ3.swift:60-115), sub-block ib = u & 7.
template <bool S>
__device__ __forceinline__ void decode_unit_iq3(const uint8_t *row, uint32_t u, float *w, const uint8_t *fg) {
    const uint8_t *b = row + (uint64_t)(u >> 3) * (S ? 110 : 98);
    const uint32_t ib = u & 7;
    const float d = h2f(ldu<uint16_t>(b));
    const uint32_t *grid = (const uint32_t *)fg;
    float db;
    uint32_t aux = 0, qh = 0;
    if constexpr (S) {
        const uint32_t sc = (b[106 + ib / 2] >> (4 * (ib & 1))) & 0xF;
        db = d * (float)(1 + 2 * sc);
        qh = b[66 + ib];
    } else {
        aux = ldu<uint32_t>(b + 66 + ib * 4);
        db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
    }
#pragma unroll
    for (int l = 0; l < 4; l++) {
        const uint32_t i1 = b[2 + ib * 8 + 2 * l], i2 = b[3 + ib * 8 + 2 * l];
        uint32_t g1, g2, signs;
        if constexpr (S) {
            g1 = grid[i1 | ((qh << (8 - 2 * l)) & 256)];
            g2 = grid[i2 | ((qh << (7 - 2 * l)) & 256)];
            signs = b[74 + ib * 4 + l];
        } else {
            g1 = grid[i1];
            g2 = grid[i2];
            signs = iq2_signs((aux >> (7 * l)) & 127);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            w[l * 8 + j] = iq_sign(signs, j, db * (float)((g1 >> (8 * j)) & 0xFF));
            w[l * 8 + j + 4] = iq_sign(signs, j + 4, db * (float)((g2 >> (8 * j)) & 0xFF));
        }
    }
}

// IQ1.dequant (LLM/Quantize/IQ1.swift:44-66) and IQ1M.dequant
// (LLM/Quantize/IQ2XXS.swift:63-98), sub-block ib = u & 7: w = dl (n - 1 +
// delta) with the grid's ternary digit n at bit 8 (j % 4) + 4 (j / 4).
template <bool M>
__device__ __forceinline__ void decode_unit_iq1(const uint8_t *row, uint32_t u, float *w, const uint8_t *fg) {
    const uint8_t *b = row + (uint64_t)(u >> 3) * (M ? 56 : 50);
    const uint32_t ib = u & 7;
    const uint32_t *grid = (const uint32_t *)fg;
    float dls[2];
    uint32_t hb[4], neg[4];
    const uint8_t *qs;
    if constexpr (M) {
        uint32_t sc[4];
#pragma unroll
        for (int i = 0; i < 4; i++) sc[i] = ldu<uint16_t>(b + 48 + i * 2);
        const uint32_t bits = (sc[0] >> 12) | ((sc[1] >> 8) & 0x00f0) | ((sc[2] >> 4) & 0x0f00) | (sc[3] & 0xf000);
        const float d = h2f((uint16_t)bits);
        const uint32_t s = sc[ib / 2] >> (6 * (ib & 1));
        dls[0] = d * (float)(2 * (s & 7) + 1);
        dls[1] = d * (float)(2 * ((s >> 3) & 7) + 1);
        const uint32_t h0 = b[32 + ib * 2], h1 = b[33 + ib * 2];
        hb[0] = h0 & 7; hb[1] = (h0 >> 4) & 7; hb[2] = h1 & 7; hb[3] = (h1 >> 4) & 7;
        neg[0] = (h0 >> 3) & 1; neg[1] = h0 >> 7; neg[2] = (h1 >> 3) & 1; neg[3] = h1 >> 7;
        qs = b + ib * 4;
    } else {
        const float d = h2f(ldu<uint16_t>(b));
        const uint32_t h = ldu<uint16_t>(b + 34 + ib * 2);
        dls[0] = dls[1] = d * (float)(2 * ((h >> 12) & 7) + 1);
#pragma unroll
        for (int l = 0; l < 4; l++) {
            hb[l] = (h >> (3 * l)) & 7;
            neg[l] = h >> 15;
        }
        qs = b + 2 + ib * 4;
    }
#pragma unroll
    for (int l = 0; l < 4; l++) {
        const uint32_t e = grid[qs[l] | (hb[l] << 8)];
        const float delta = neg[l] ? -0.125f : 0.125f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t n = (e >> (8 * (j % 4) + 4 * (j / 4))) & 0xF;
            w[l * 8 + j] = dls[l / 2] * ((float)n - 1.0f + delta);
        }
    }
}

// KQuant.q2K (LLM/Quantize/KQuants.swift:9-36), 32-weight group j = u & 7 of
// superblock u >> 3 ({u8 scales[16]; u8 qs[64]; half d, dmin}): n = j / 4,
// bit field 2 (j % 4) of code bytes 16 + 32 n .., scale bytes 2 j, 2 j + 1
// (16 weights each); w = (d * (sc & 15)) * q - dmin * (sc >> 4).
__device__ __forceinline__ void decode_unit_q2_k(const uint8_t *row, uint32_t u, float *w) {
    const uint8_t *b = row + (uint64_t)(u >> 3) * 84;
    const uint32_t j = u & 7, n = j >> 2, sh = 2 * (j & 3);
    const float d = h2f(ldu<uint16_t>(b + 80)), dmin = h2f(ldu<uint16_t>(b + 82));
    uint32_t q[8];
    *(uint4 *)&q[0] = ldu<uint4>(b + 16 + 32 * n);
    *(uint4 *)&q[4] = ldu<uint4>(b + 32 + 32 * n);
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const uint32_t sc = b[2 * j + h];
        const float dl = d * (float)(sc & 0xF), ml = dmin * (float)(sc >> 4);
#pragma unroll
        for (int l = 0; l < 16; l++)
            w[16 * h + l] = dl * (float)((byte_of(q[(16 * h + l) >> 2], l & 3) >> sh) & 3) - ml;
    }
}

// KQuant.q3K (LLM/Quantize/KQuants.swift:38-83), group j = u & 7 ({u8
// hmask[32]; u8 qs[64]; u8 scales[12]; half d}): scale i = 2 j + h has its
// low nibble in byte i (i < 8) or the high nibble of byte i - 8 and its top
// bits at 2 (i / 4) of byte 8 + i % 4 (the reference's aux shuffle);
// w = (d * (scale - 32)) * (q - (hmask bit n * 4 + j % 4 of byte l ? 0 : 4)).
__device__ __forceinline__ void decode_unit_q3_k(const uint8_t *row, uint32_t u, float *w) {
    const uint8_t *b = row + (uint64_t)(u >> 3) * 110;
    const uint32_t j = u & 7, n = j >> 2, sh = 2 * (j & 3), hb = 4 * n + (j & 3);
    const float dall = h2f(ldu<uint16_t>(b + 108));
    uint32_t q[8], hm[8];
    *(uint4 *)&q[0] = ldu<uint4>(b + 32 + 32 * n);
    *(uint4 *)&q[4] = ldu<uint4>(b + 48 + 32 * n);
    *(uint4 *)&hm[0] = ldu<uint4>(b);
    *(uint4 *)&hm[4] = ldu<uint4>(b + 16);
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const uint32_t i = n * 8 + (j & 3) * 2 + h;
        const uint32_t lo = (b[96 + (i & 7)] >> (4 * (i >> 3))) & 0xF, hi = (b[104 + (i & 3)] >> (2 * (i >> 2))) & 3;
        const float dl = dall * (float)((int)(lo | (hi << 4)) - 32);
#pragma unroll
        for (int l = 0; l < 16; l++) {
            const uint32_t at = 16 * h + l;
            const float bump = (byte_of(hm[at >> 2], at & 3) >> hb) & 1 ? 0.0f : 4.0f;
            w[at] = dl * ((float)((byte_of(q[at >> 2], at & 3) >> sh) & 3) - bump);
        }
    }
}

// GQ.element (LLM/Gemma/Gemma4Quant.swift:302-316): 32 plain weights.
template <int F>
__device__ __forceinline__ void decode_unit_dense(const uint8_t *row, uint32_t u, float *w) {
    if constexpr (F == F32) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint4 v = ldu<uint4>(row + (uint64_t)u * 128 + 16 * i);
            w[4 * i] = __builtin_bit_cast(float, v.x);
            w[4 * i + 1] = __builtin_bit_cast(float, v.y);
            w[4 * i + 2] = __builtin_bit_cast(float, v.z);
            w[4 * i + 3] = __builtin_bit_cast(float, v.w);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint4 v = ldu<uint4>(row + (uint64_t)u * 64 + 16 * i);
            const uint32_t d4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t lo = d4[k] & 0xFFFF, hi = d4[k] >> 16;
                w[8 * i + 2 * k] = F == F16 ? h2f((uint16_t)lo) : __builtin_bit_cast(float, lo << 16);
                w[8 * i + 2 * k + 1] = F == F16 ? h2f((uint16_t)hi) : __builtin_bit_cast(float, hi << 16);
            }
        }
    }
}

// The grid formats' decoders take fg, the format's own grid (gt_off<F>()
// bytes into the buffer of all the grids, or a copy of it in LDS).
template <int F>
__device__ __forceinline__ void decode_unit_fg(const uint8_t *row, uint32_t u, float *w, const uint8_t *fg) {
    if constexpr (F == IQ2_XS || F == IQ2_S) decode_unit_iq2_xs_s<F == IQ2_S>(row, u, w, fg);
    else if constexpr (F == IQ3_XXS || F == IQ3_S) decode_unit_iq3<F == IQ3_S>(row, u, w, fg);
    else if constexpr (F == IQ1_S || F == IQ1_M) decode_unit_iq1<F == IQ1_M>(row, u, w, fg);
}

// gt: the grid tables of the grid formats (GT_* offsets), in device memory
template <int F>
__device__ __forceinline__ void decode_unit(const uint8_t *row, uint32_t u, float *w,
                                            const uint2 *grid, const uint8_t *gt = nullptr) {
    if constexpr (F == Q8_0) decode_unit_q8_0(row, u, w);
    else if constexpr (F == Q2_0) decode_unit_q2_0(row, u, w);
    else if constexpr (F == Q4_K) decode_unit_q4_k(row, u, w);
    else if constexpr (F == Q4_0) decode_unit_q4_0(row, u, w);
    else if constexpr (F == IQ4_NL) decode_unit_iq4_nl(row, u, w);
    else if constexpr (F == Q5_K) decode_unit_q5_k(row, u, w);
    else if constexpr (F == Q6_K) decode_unit_q6_k(row, u, w);
    else if constexpr (F == IQ4_XS) decode_unit_iq4_xs(row, u, w);
    else if constexpr (F == IQ2_XS || F == IQ2_S || F == IQ3_XXS || F == IQ3_S || F == IQ1_S || F == IQ1_M)
        decode_unit_fg<F>(row, u, w, gt + gt_off(F));
    else if constexpr (F == Q2_K) decode_unit_q2_k(row, u, w);
    else if constexpr (F == Q3_K) decode_unit_q3_k(row, u, w);
    else if constexpr (F == F32 || F == F16 || F == BF16) decode_unit_dense<F>(row, u, w);
    else decode_unit_iq2_xxs(row, u, w, grid);
}

#pragma clang fp contract(on)

}  // namespace okf
