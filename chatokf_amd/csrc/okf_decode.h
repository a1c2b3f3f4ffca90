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

template <int F>
__device__ __forceinline__ void decode_unit(const uint8_t *row, uint32_t u, float *w,
                                            const uint2 *grid) {
    if constexpr (F == Q8_0) decode_unit_q8_0(row, u, w);
    else if constexpr (F == Q2_0) decode_unit_q2_0(row, u, w);
    else if constexpr (F == Q4_K) decode_unit_q4_k(row, u, w);
    else if constexpr (F == Q4_0) decode_unit_q4_0(row, u, w);
    else if constexpr (F == IQ4_NL) decode_unit_iq4_nl(row, u, w);
    else if constexpr (F == Q5_K) decode_unit_q5_k(row, u, w);
    else if constexpr (F == Q6_K) decode_unit_q6_k(row, u, w);
    else if constexpr (F == IQ4_XS) decode_unit_iq4_xs(row, u, w);
    else decode_unit_iq2_xxs(row, u, w, grid);
}

#pragma clang fp contract(on)

}  // namespace okf
