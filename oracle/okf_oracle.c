/*
 * okf_oracle.c -- CPU restatement of ChatOKF's quantized matvec/matmul and
 * block decoders.  TEST INFRASTRUCTURE ONLY (checker + CPU baseline); the
 * product never links it.  See okf_oracle.h for what pins each function.
 *
 * Build: oracle/Makefile (-O2 -ffp-contract=off -fno-fast-math).
 */
#define _GNU_SOURCE
#include "okf_oracle.h"

#include <pthread.h>
#include <sched.h>
#include <stdlib.h>
#include <math.h>
#include <string.h>

#include "iq2xxs_grid.inc"
#include "iq_grids.inc"

#if defined(__FP_FAST_FMAF) || defined(__FAST_MATH__)
#error "the oracle must be built without fast-math"
#endif

/* ------------------------------------------------------------------ */
/* scalar helpers                                                      */

float okf_ref_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: renormalise */
            int e = -1;
            do {
                man <<= 1;
                e++;
            } while ((man & 0x400) == 0);
            man &= 0x3ff;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static inline uint16_t ld16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline uint32_t ld32(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
static inline float ldh(const uint8_t *p) { return okf_ref_f16_to_f32(ld16(p)); }

/* ------------------------------------------------------------------ */
/* sizes: LLM/Base/GGUF.swift:160-188, GQ.blockElems Gemma4Quant.swift:77-87 */

static int block_geom(int32_t type, uint32_t *elems, uint32_t *bytes) {
    switch (type) {
    case OKF_REF_Q8_0: *elems = 32; *bytes = 34; return 0;
    case OKF_REF_Q4_0: *elems = 32; *bytes = 18; return 0;
    case OKF_REF_IQ4_NL: *elems = 32; *bytes = 18; return 0;
    case OKF_REF_Q2_0: *elems = 128; *bytes = 34; return 0;
    case OKF_REF_Q4_K: *elems = 256; *bytes = 144; return 0;
    case OKF_REF_Q5_K: *elems = 256; *bytes = 176; return 0;
    case OKF_REF_Q6_K: *elems = 256; *bytes = 210; return 0;
    case OKF_REF_IQ4_XS: *elems = 256; *bytes = 136; return 0;
    case OKF_REF_IQ2_XS: *elems = 256; *bytes = 74; return 0;
    case OKF_REF_IQ2_S: *elems = 256; *bytes = 82; return 0;
    case OKF_REF_IQ3_XXS: *elems = 256; *bytes = 98; return 0;
    case OKF_REF_IQ3_S: *elems = 256; *bytes = 110; return 0;
    case OKF_REF_IQ1_S: *elems = 256; *bytes = 50; return 0;
    case OKF_REF_IQ1_M: *elems = 256; *bytes = 56; return 0;
    case OKF_REF_Q2_K: *elems = 256; *bytes = 84; return 0;
    case OKF_REF_Q3_K: *elems = 256; *bytes = 110; return 0;
    case OKF_REF_F32: *elems = 32; *bytes = 128; return 0;
    case OKF_REF_F16: case OKF_REF_BF16: *elems = 32; *bytes = 64; return 0;
    case OKF_REF_IQ2_XXS: *elems = 256; *bytes = 66; return 0;
    default: return -1;
    }
}

int okf_ref_row_bytes(int32_t type, uint64_t n, uint64_t *out) {
    uint32_t e, b;
    if (block_geom(type, &e, &b) || n % e) return -1;
    *out = n / e * b;
    return 0;
}

/* ------------------------------------------------------------------ */
/* decoders                                                            */

/* Q8_0.dequant, LLM/Gemma/Gemma4Quant.swift:55-68: w = Float(q) * d */
static void dq_q8_0(const uint8_t *p, uint64_t n, float *out) {
    for (uint64_t b = 0; b < n / 32; b++, p += 34, out += 32) {
        float d = ldh(p);
        for (int j = 0; j < 32; j++) out[j] = (float)(int8_t)p[2 + j] * d;
    }
}

/* Q4_0.dequant, LLM/Gemma/Gemma4Quant.swift:30-49: byte j of the 16 gives
 * w[j] = (Float(b & 0xF) - 8) * d and w[j + 16] = (Float(b >> 4) - 8) * d */
static void dq_q4_0(const uint8_t *p, uint64_t n, float *out) {
    for (uint64_t b = 0; b < n / 32; b++, p += 18, out += 32) {
        float d = ldh(p);
        for (int j = 0; j < 16; j++) {
            out[j] = ((float)(p[2 + j] & 0xF) - 8) * d;
            out[j + 16] = ((float)(p[2 + j] >> 4) - 8) * d;
        }
    }
}

/* IQ4_NL.kvalues, LLM/Gemma/Gemma4Quant.swift:8-11 (the format's table) */
static const float iq4nl_values[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                       1,    13,   25,  38,  53,  69,  89,  113};

/* IQ4_NL.dequant, Gemma4Quant.swift:13-27: w = kvalues[nibble] * d */
static void dq_iq4_nl(const uint8_t *p, uint64_t n, float *out) {
    for (uint64_t b = 0; b < n / 32; b++, p += 18, out += 32) {
        float d = ldh(p);
        for (int j = 0; j < 16; j++) {
            out[j] = iq4nl_values[p[2 + j] & 0xF] * d;
            out[j + 16] = iq4nl_values[p[2 + j] >> 4] * d;
        }
    }
}

/* Q2_0.dequant, LLM/Base/Quant.swift:10-25: w = Float(code - 1) * d,
 * code j = (qs[j >> 2] >> 2(j & 3)) & 3 */
static void dq_q2_0(const uint8_t *p, uint64_t n, float *out) {
    for (uint64_t b = 0; b < n / 128; b++, p += 34, out += 128) {
        float d = ldh(p);
        const uint8_t *qs = p + 2;
        for (int j = 0; j < 128; j++) {
            int code = (qs[j >> 2] >> ((j & 3) << 1)) & 3;
            out[j] = (float)(code - 1) * d;
        }
    }
}

/* KQuant.scaleMin, LLM/Quantize/KQuants.swift:86-101 (ggml get_scale_min_k4):
 * s(i) is byte 4 + i of the block. */
static void scale_min(const uint8_t *b, int j, float *sc_out, float *mn_out) {
    const uint8_t *s = b + 4;
    uint8_t sc, mn;
    if (j < 4) {
        sc = s[j] & 63;
        mn = s[j + 4] & 63;
    } else {
        sc = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
        mn = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
    *sc_out = (float)sc;
    *mn_out = (float)mn;
}

/* KQuant.q4K, LLM/Quantize/KQuants.swift:104-125 */
static void dq_q4_k_block(const uint8_t *b, float *out) {
    float d = ldh(b), dmin = ldh(b + 2);
    int y = 0, qoff = 16, isc = 0;
    for (int it = 0; it < 4; it++) {
        float s1, m1, s2, m2;
        scale_min(b, isc, &s1, &m1);
        scale_min(b, isc + 1, &s2, &m2);
        float d1 = d * s1, o1 = dmin * m1;
        float d2 = d * s2, o2 = dmin * m2;
        for (int l = 0; l < 32; l++) {
            uint8_t q = b[qoff + l];
            out[y + l] = d1 * (float)(q & 0xF) - o1;
            out[y + 32 + l] = d2 * (float)(q >> 4) - o2;
        }
        y += 64;
        qoff += 32;
        isc += 2;
    }
}

/* KQuant.q2K, LLM/Quantize/KQuants.swift:9-36:
 * { u8 scales[16]; u8 qs[64]; half d; half dmin } */
static void dq_q2_k_block(const uint8_t *b, float *out) {
    float d = ldh(b + 80), dmin = ldh(b + 82);
    int y = 0, qoff = 16, isc = 0;
    for (int n = 0; n < 2; n++) {
        for (int shift = 0; shift < 8; shift += 2)
            for (int half = 0; half < 2; half++) {
                uint8_t sc = b[isc++];
                float dl = d * (float)(sc & 0xF), ml = dmin * (float)(sc >> 4);
                for (int l = 0; l < 16; l++) out[y++] = dl * (float)((b[qoff + half * 16 + l] >> shift) & 3) - ml;
            }
        qoff += 32;
    }
}

/* KQuant.q3K, LLM/Quantize/KQuants.swift:38-83:
 * { u8 hmask[32]; u8 qs[64]; u8 scales[12]; half d }; the 16 6-bit scales
 * are unpacked from the 12 bytes as the reference's aux shuffle does */
static void dq_q3_k_block(const uint8_t *b, float *out) {
    float dall = ldh(b + 108);
    uint32_t aux[4] = {ld32(b + 96), ld32(b + 100), ld32(b + 104), 0};
    const uint32_t km1 = 0x03030303u, km2 = 0x0f0f0f0fu, tmp = aux[2];
    aux[2] = ((aux[0] >> 4) & km2) | (((tmp >> 4) & km1) << 4);
    aux[3] = ((aux[1] >> 4) & km2) | (((tmp >> 6) & km1) << 4);
    aux[0] = (aux[0] & km2) | (((tmp >> 0) & km1) << 4);
    aux[1] = (aux[1] & km2) | (((tmp >> 2) & km1) << 4);
    int8_t scales[16];
    for (int i = 0; i < 4; i++)
        for (int j = 0; j < 4; j++) scales[i * 4 + j] = (int8_t)((aux[i] >> (8 * j)) & 0xFF);
    int y = 0, qoff = 32, isc = 0;
    uint8_t m = 1;
    for (int n = 0; n < 2; n++) {
        for (int shift = 0; shift < 8; shift += 2) {
            for (int half = 0; half < 2; half++) {
                float dl = dall * (float)((int)scales[isc++] - 32);
                for (int l = 0; l < 16; l++) {
                    int at = half * 16 + l;
                    float bump = (b[at] & m) ? 0.0f : 4.0f;
                    out[y++] = dl * ((float)((b[qoff + at] >> shift) & 3) - bump);
                }
            }
            m <<= 1;
        }
        qoff += 32;
    }
}

/* GQ.element, LLM/Gemma/Gemma4Quant.swift:302-316: f32, f16 and bf16 (the
 * upper half of an f32) weights */
static float dense_element(int32_t type, const uint8_t *p, uint64_t i) {
    if (type == OKF_REF_F32) {
        float v;
        memcpy(&v, p + i * 4, 4);
        return v;
    }
    if (type == OKF_REF_F16) return okf_ref_f16_to_f32(ld16(p + i * 2));
    uint32_t bits = (uint32_t)ld16(p + i * 2) << 16;
    float v;
    memcpy(&v, &bits, 4);
    return v;
}

/* KQuant.q5K, LLM/Quantize/KQuants.swift:127-155: as q4K with a fifth bit
 * from qh[l] (bytes 16..47), bit 2 it for the low nibble of code group it
 * and bit 2 it + 1 for its high nibble. */
static void dq_q5_k_block(const uint8_t *b, float *out) {
    float d = ldh(b), dmin = ldh(b + 2);
    int y = 0, qoff = 48, isc = 0;
    uint8_t u1 = 1, u2 = 2;
    for (int it = 0; it < 4; it++) {
        float s1, m1, s2, m2;
        scale_min(b, isc, &s1, &m1);
        scale_min(b, isc + 1, &s2, &m2);
        float d1 = d * s1, o1 = dmin * m1;
        float d2 = d * s2, o2 = dmin * m2;
        for (int l = 0; l < 32; l++) {
            uint8_t q = b[qoff + l], h = b[16 + l];
            float lo = (float)((q & 0xF) + ((h & u1) ? 16 : 0));
            float hi = (float)((q >> 4) + ((h & u2) ? 16 : 0));
            out[y + l] = d1 * lo - o1;
            out[y + 32 + l] = d2 * hi - o2;
        }
        y += 64;
        qoff += 32;
        isc += 2;
        u1 <<= 2;
        u2 <<= 2;
    }
}

/* KQuant.q6K, LLM/Quantize/KQuants.swift:157-176: ql[128], qh[64],
 * int8 scales[16], d at 208; weight n*128 + r*32 + l has the low nibble
 * (r < 2) or high nibble (r >= 2) of ql[n*64 + l] (r even) or
 * ql[n*64 + 32 + l] (r odd), and bits 2r.. of qh[n*32 + l] on top;
 * w = d * s * (q - 32) with s = scales[n*8 + 2r + l/16]. */
static void dq_q6_k_block(const uint8_t *b, float *out) {
    float d = ldh(b + 208);
    for (int n = 0; n < 2; n++)
        for (int l = 0; l < 32; l++) {
            int h = b[128 + n * 32 + l], a = b[n * 64 + l], c = b[n * 64 + l + 32];
            for (int r = 0; r < 4; r++) {
                int byte = (r % 2) == 0 ? a : c;
                int nib = r < 2 ? (byte & 0xF) : (byte >> 4);
                int q = nib | (((h >> (2 * r)) & 3) << 4);
                int s = (int8_t)b[192 + n * 8 + 2 * r + l / 16];
                out[n * 128 + r * 32 + l] = d * (float)s * (float)(q - 32);
            }
        }
}

/* IQX.iq4XS, LLM/Quantize/IQ3.swift:118-133: sub-block ib has the 6-bit
 * scale ls = (scales_l nibble ib) | (2 bits ib of scales_h) << 4;
 * dl = d * (ls - 32); w = dl * nl4[nibble], nl4 = the IQ4_NL levels
 * (IQ3Grid.swift:530). */
static void dq_iq4_xs_block(const uint8_t *b, float *out) {
    float d = ldh(b);
    uint16_t sh = ld16(b + 2);
    for (int ib = 0; ib < 8; ib++) {
        uint8_t sl = b[4 + ib / 2];
        int ls = ((sl >> (4 * (ib % 2))) & 0xF) | (((sh >> (2 * ib)) & 3) << 4);
        float dl = d * (float)(ls - 32);
        for (int j = 0; j < 16; j++) {
            uint8_t q = b[8 + ib * 16 + j];
            out[ib * 32 + j] = dl * iq4nl_values[q & 0xF];
            out[ib * 32 + 16 + j] = dl * iq4nl_values[q >> 4];
        }
    }
}

/* IQX.sign, LLM/Quantize/IQ3.swift:9-11: bit j of the sign byte negates */
static inline float iq_sign(uint8_t signs, int j, float v) { return (signs & (1u << j)) ? -v : v; }

/* IQX.iq2XS, LLM/Quantize/IQ3.swift:14-33: { half d; u16 qs[32]; u8 scales[8] } */
static void dq_iq2_xs_block(const uint8_t *b, float *out) {
    float d = ldh(b);
    for (int ib = 0; ib < 8; ib++) {
        uint8_t sc = b[66 + ib];
        float db0 = d * (0.5f + (float)(sc & 0xF)) * 0.25f;
        float db1 = d * (0.5f + (float)(sc >> 4)) * 0.25f;
        for (int l = 0; l < 4; l++) {
            uint16_t q = ld16(b + 2 + (ib * 4 + l) * 2);
            uint64_t entry = okf_ref_iq2xs_grid[q & 511];
            uint8_t signs = okf_ref_ksigns[q >> 9];
            float dl = l / 2 == 0 ? db0 : db1;
            for (int j = 0; j < 8; j++)
                out[ib * 32 + l * 8 + j] = iq_sign(signs, j, dl * (float)((entry >> (8 * j)) & 0xFF));
        }
    }
}

/* IQX.iq2S, LLM/Quantize/IQ3.swift:36-57:
 * { half d; u8 qs[32]; u8 signs[32]; u8 qh[8]; u8 scales[8] } (offsets 2, 34, 66, 74) */
static void dq_iq2_s_block(const uint8_t *b, float *out) {
    float d = ldh(b);
    for (int ib = 0; ib < 8; ib++) {
        uint8_t sc = b[74 + ib];
        float db0 = d * (0.5f + (float)(sc & 0xF)) * 0.25f;
        float db1 = d * (0.5f + (float)(sc >> 4)) * 0.25f;
        uint8_t qh = b[66 + ib];
        for (int l = 0; l < 4; l++) {
            int idx = b[2 + ib * 4 + l] | (((int)qh << (8 - 2 * l)) & 0x300);
            uint64_t entry = okf_ref_iq2s_grid[idx];
            uint8_t signs = b[34 + ib * 4 + l];
            float dl = l / 2 == 0 ? db0 : db1;
            for (int j = 0; j < 8; j++)
                out[ib * 32 + l * 8 + j] = iq_sign(signs, j, dl * (float)((entry >> (8 * j)) & 0xFF));
        }
    }
}

/* IQX.iq3XXS, LLM/Quantize/IQ3.swift:60-82: { half d; u8 qs[64]; u32 scales_and_signs[8] } */
static void dq_iq3_xxs_block(const uint8_t *b, float *out) {
    float d = ldh(b);
    for (int ib = 0; ib < 8; ib++) {
        uint32_t aux = ld32(b + 66 + ib * 4);
        float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
        for (int l = 0; l < 4; l++) {
            uint8_t signs = okf_ref_ksigns[(aux >> (7 * l)) & 127];
            uint32_t g1 = okf_ref_iq3xxs_grid[b[2 + ib * 8 + 2 * l]];
            uint32_t g2 = okf_ref_iq3xxs_grid[b[2 + ib * 8 + 2 * l + 1]];
            int at = ib * 32 + l * 8;
            for (int j = 0; j < 4; j++) {
                out[at + j] = iq_sign(signs, j, db * (float)((g1 >> (8 * j)) & 0xFF));
                out[at + j + 4] = iq_sign(signs, j + 4, db * (float)((g2 >> (8 * j)) & 0xFF));
            }
        }
    }
}

/* IQX.iq3S, LLM/Quantize/IQ3.swift:85-115:
 * { half d; u8 qs[64]; u8 qh[8]; u8 signs[32]; u8 scales[4] } (offsets 2, 66, 74, 106) */
static void dq_iq3_s_block(const uint8_t *b, float *out) {
    float d = ldh(b);
    for (int pair = 0; pair < 4; pair++) {
        uint8_t sc = b[106 + pair];
        float db1 = d * (float)(1 + 2 * (sc & 0xF));
        float db2 = d * (float)(1 + 2 * (sc >> 4));
        for (int half = 0; half < 2; half++) {
            int ib = pair * 2 + half;
            uint8_t qh = b[66 + ib];
            float db = half == 0 ? db1 : db2;
            for (int l = 0; l < 4; l++) {
                int base = 2 + ib * 8 + 2 * l;
                uint32_t g1 = okf_ref_iq3s_grid[b[base] | (((int)qh << (8 - 2 * l)) & 256)];
                uint32_t g2 = okf_ref_iq3s_grid[b[base + 1] | (((int)qh << (7 - 2 * l)) & 256)];
                uint8_t signs = b[74 + ib * 4 + l];
                int at = ib * 32 + l * 8;
                for (int j = 0; j < 4; j++) {
                    out[at + j] = iq_sign(signs, j, db * (float)((g1 >> (8 * j)) & 0xFF));
                    out[at + j + 4] = iq_sign(signs, j + 4, db * (float)((g2 >> (8 * j)) & 0xFF));
                }
            }
        }
    }
}

/* IQ1 grid entry -> the 8 ternary digits n (0, 1, 2), digit j at bit
 * 8 (j % 4) + 4 (j / 4) (IQ1Grid.gpu, LLM/Quantize/IQ1Grid.swift:8) */
static inline int iq1_digit(uint32_t entry, int j) { return (entry >> (8 * (j % 4) + 4 * (j / 4))) & 0xF; }

/* IQ1.dequant, LLM/Quantize/IQ1.swift:44-66: { half d; u8 qs[32]; u16 qh[8] };
 * w = dl * (n - 1 + delta), dl = d * (2 ((h >> 12) & 7) + 1), delta = +-1/8 */
static void dq_iq1_s_block(const uint8_t *b, float *out) {
    float d = ldh(b);
    for (int ib = 0; ib < 8; ib++) {
        uint16_t h = ld16(b + 34 + ib * 2);
        float dl = d * (float)(2 * ((h >> 12) & 7) + 1);
        float delta = (h & 0x8000) ? -0.125f : 0.125f;
        for (int l = 0; l < 4; l++) {
            int idx = b[2 + ib * 4 + l] | (((h >> (3 * l)) & 7) << 8);
            uint32_t entry = okf_ref_iq1s_grid[idx];
            for (int j = 0; j < 8; j++) out[ib * 32 + l * 8 + j] = dl * ((float)iq1_digit(entry, j) - 1 + delta);
        }
    }
}

/* IQ1M.scale + IQ1M.dequant, LLM/Quantize/IQ2XXS.swift:63-98:
 * { u8 qs[32]; u8 qh[16]; u16 scales[4] }, d reassembled from the top
 * nibbles of the four scale shorts */
static void dq_iq1_m_block(const uint8_t *b, float *out) {
    uint16_t sc[4];
    for (int i = 0; i < 4; i++) sc[i] = ld16(b + 48 + i * 2);
    uint16_t bits = (uint16_t)((sc[0] >> 12) | ((sc[1] >> 8) & 0x00f0) | ((sc[2] >> 4) & 0x0f00) | (sc[3] & 0xf000));
    float d = okf_ref_f16_to_f32(bits);
    for (int ib = 0; ib < 8; ib++) {
        uint16_t s = sc[ib / 2];
        int shift = 6 * (ib % 2);
        float dl1 = d * (float)(2 * ((s >> shift) & 7) + 1);
        float dl2 = d * (float)(2 * ((s >> (shift + 3)) & 7) + 1);
        uint8_t h0 = b[32 + ib * 2], h1 = b[33 + ib * 2];
        for (int l = 0; l < 4; l++) {
            uint8_t h = l < 2 ? h0 : h1;
            int hi = (l % 2) == 0 ? ((int)h << 8) : ((int)h << 4);
            int idx = b[ib * 4 + l] | (hi & 0x700);
            int neg = (h & ((l % 2) == 0 ? 0x08 : 0x80)) != 0;
            float delta = neg ? -0.125f : 0.125f;
            float dl = l < 2 ? dl1 : dl2;
            uint32_t entry = okf_ref_iq1s_grid[idx];
            for (int j = 0; j < 8; j++) out[ib * 32 + l * 8 + j] = dl * ((float)iq1_digit(entry, j) - 1 + delta);
        }
    }
}

/* IQ2XXS.dequant, LLM/Quantize/IQ2XXS.swift:34-54 */
static void dq_iq2_xxs_block(const uint8_t *b, float *out) {
    float d = ldh(b);
    for (int ib = 0; ib < 8; ib++) {
        uint32_t a0 = ld32(b + 2 + ib * 8);
        uint32_t a1 = ld32(b + 2 + ib * 8 + 4);
        float db = d * (0.5f + (float)(a1 >> 28)) * 0.25f;
        for (int l = 0; l < 4; l++) {
            uint64_t entry = okf_ref_iq2xxs_grid[(a0 >> (8 * l)) & 0xFF];
            uint8_t signs = okf_ref_ksigns[(a1 >> (7 * l)) & 127];
            for (int j = 0; j < 8; j++) {
                float g = (float)((entry >> (8 * j)) & 0xFF);
                float s = (signs & okf_ref_kmask[j]) ? -1.0f : 1.0f;
                out[ib * 32 + l * 8 + j] = db * g * s;
            }
        }
    }
}

typedef void (*sb_decode_fn)(const uint8_t *, float *);

static sb_decode_fn sb_decoder(int32_t type) {
    switch (type) {
    case OKF_REF_Q4_K: return dq_q4_k_block;
    case OKF_REF_Q5_K: return dq_q5_k_block;
    case OKF_REF_Q6_K: return dq_q6_k_block;
    case OKF_REF_IQ4_XS: return dq_iq4_xs_block;
    case OKF_REF_IQ2_XS: return dq_iq2_xs_block;
    case OKF_REF_IQ2_S: return dq_iq2_s_block;
    case OKF_REF_IQ3_XXS: return dq_iq3_xxs_block;
    case OKF_REF_IQ3_S: return dq_iq3_s_block;
    case OKF_REF_IQ1_S: return dq_iq1_s_block;
    case OKF_REF_IQ1_M: return dq_iq1_m_block;
    case OKF_REF_Q2_K: return dq_q2_k_block;
    case OKF_REF_Q3_K: return dq_q3_k_block;
    case OKF_REF_IQ2_XXS: return dq_iq2_xxs_block;
    default: return NULL;
    }
}

int okf_ref_dequant(int32_t type, const uint8_t *p, uint64_t n, float *out) {
    uint32_t e, bytes;
    if (block_geom(type, &e, &bytes) || n % e) return -1;
    switch (type) {
    case OKF_REF_Q8_0: dq_q8_0(p, n, out); break;
    case OKF_REF_Q2_0: dq_q2_0(p, n, out); break;
    case OKF_REF_Q4_0: dq_q4_0(p, n, out); break;
    case OKF_REF_IQ4_NL: dq_iq4_nl(p, n, out); break;
    case OKF_REF_F32: case OKF_REF_F16: case OKF_REF_BF16:
        for (uint64_t i = 0; i < n; i++) out[i] = dense_element(type, p, i);
        break;
    default: { /* superBlockGather, Gemma4Quant.swift:351-360 */
        sb_decode_fn dec = sb_decoder(type);
        for (uint64_t b = 0; b < n / 256; b++) dec(p + b * bytes, out + b * 256);
    }
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* per-row kernels                                                      */

typedef struct {
    int32_t type;
    const uint8_t *w;
    uint32_t K, M;
    uint64_t row_bytes;
    const float *x; /* matvec: x[K]; blockMatmul: XT[K][N] */
    float *y;
    uint32_t N;
} job_t;

/* GQ.matvec q8_0 arm, Gemma4Quant.swift:115-124, driven by rowParallel
 * :250-279: acc += (sum_j Float(q_j) * x_j) * d, block by block. */
static float row_q8_0(const job_t *j, uint32_t m) {
    const uint8_t *p = j->w + (uint64_t)m * j->row_bytes;
    float acc = 0;
    for (uint32_t k = 0; k < j->K; k += 32, p += 34) {
        float a = 0;
        float d = ldh(p);
        for (int t = 0; t < 32; t++) a += (float)(int8_t)p[2 + t] * j->x[k + t];
        acc += a * d;
    }
    return acc;
}

/* GQ.matvec q4_0 / iq4_nl arms, Gemma4Quant.swift:93-114: per block, for j
 * ascending acc_b += w(lo nibble j) * x[k + j], then += w(hi nibble j) *
 * x[k + j + 16] (w = nibble - 8 or kvalues[nibble]); acc += acc_b * d. */
static float row_nibble32(const job_t *j, uint32_t m) {
    const uint8_t *p = j->w + (uint64_t)m * j->row_bytes;
    const int nl = j->type == OKF_REF_IQ4_NL;
    float acc = 0;
    for (uint32_t k = 0; k < j->K; k += 32, p += 18) {
        float a = 0;
        float d = ldh(p);
        for (int t = 0; t < 16; t++) {
            const uint8_t b = p[2 + t];
            const float lo = nl ? iq4nl_values[b & 0xF] : (float)(b & 0xF) - 8;
            const float hi = nl ? iq4nl_values[b >> 4] : (float)(b >> 4) - 8;
            a += lo * j->x[k + t];
            a += hi * j->x[k + t + 16];
        }
        acc += a * d;
    }
    return acc;
}

/* GQ.denseMatvec, LLM/Gemma/Gemma4Quant.swift:281-300: acc += w_i * x_i over
 * the whole row, in order. */
static float row_dense(const job_t *j, uint32_t m) {
    const uint8_t *p = j->w + (uint64_t)m * j->row_bytes;
    float acc = 0;
    for (uint32_t i = 0; i < j->K; i++) acc += dense_element(j->type, p, i) * j->x[i];
    return acc;
}

/* Q2_0.matvec, LLM/Base/Quant.swift:41-61: acc += d * (lo + 2 * hi - sy). */
static float row_q2_0(const job_t *j, uint32_t m) {
    const uint8_t *p = j->w + (uint64_t)m * j->row_bytes;
    float acc = 0;
    for (uint32_t k = 0; k < j->K; k += 128, p += 34) {
        float d = ldh(p);
        const uint8_t *qs = p + 2;
        float lo = 0, hi = 0, sy = 0;
        for (int t = 0; t < 128; t++) {
            uint8_t code = (qs[t >> 2] >> ((t & 3) << 1)) & 3;
            float xv = j->x[k + t];
            sy += xv;
            if (code & 1) lo += xv;
            if (code & 2) hi += xv;
        }
        acc += d * (lo + 2 * hi - sy);
    }
    return acc;
}

/* GQ.matvec superblock arm, Gemma4Quant.swift:125-136: decode 256 weights,
 * then acc_b = sum_i w_i * x_i; acc += acc_b. */
static float row_superblock(const job_t *j, uint32_t m) {
    const uint8_t *p = j->w + (uint64_t)m * j->row_bytes;
    sb_decode_fn dec = sb_decoder(j->type);
    uint32_t elems, bytes;
    block_geom(j->type, &elems, &bytes);
    float w[256];
    float acc = 0;
    for (uint32_t k = 0; k < j->K; k += 256, p += bytes) {
        dec(p, w);
        float a = 0;
        for (int i = 0; i < 256; i++) a += w[i] * j->x[k + i];
        acc += a;
    }
    return acc;
}

/* GQ.blockMatmul, Gemma4Quant.swift:172-223 (Q8_0, Q4_0): per row, every
 * block is dequantized once and acc[n] += w_j * XT[k + j][n]. */
static void row_block_matmul_q8_0(const job_t *j, uint32_t m, float *acc) {
    const uint8_t *p = j->w + (uint64_t)m * j->row_bytes;
    uint32_t N = j->N;
    const int q4 = j->type == OKF_REF_Q4_0;
    float blk[32];
    for (uint32_t n = 0; n < N; n++) acc[n] = 0;
    for (uint32_t k = 0; k < j->K; k += 32, p += q4 ? 18 : 34) {
        if (q4) dq_q4_0(p, 32, blk);
        else dq_q8_0(p, 32, blk);
        for (int t = 0; t < 32; t++) {
            float wj = blk[t];
            const float *col = j->x + (uint64_t)(k + t) * N;
            for (uint32_t n = 0; n < N; n++) acc[n] += wj * col[n];
        }
    }
    for (uint32_t n = 0; n < N; n++) j->y[(uint64_t)n * j->M + m] = acc[n];
}

/* ------------------------------------------------------------------ */
/* row-parallel driver (DispatchQueue.concurrentPerform over M rows)    */

typedef struct {
    const job_t *job;
    uint32_t m0, m1;
    int matmul;
} slice_t;

static void *run_slice(void *arg) {
    const slice_t *s = (const slice_t *)arg;
    const job_t *j = s->job;
    if (s->matmul) {
        float *acc = (float *)malloc(sizeof(float) * j->N);
        for (uint32_t m = s->m0; m < s->m1; m++) row_block_matmul_q8_0(j, m, acc);
        free(acc);
        return NULL;
    }
    for (uint32_t m = s->m0; m < s->m1; m++) {
        float v;
        switch (j->type) {
        case OKF_REF_Q8_0: v = row_q8_0(j, m); break;
        case OKF_REF_Q2_0: v = row_q2_0(j, m); break;
        case OKF_REF_Q4_0: case OKF_REF_IQ4_NL: v = row_nibble32(j, m); break;
        case OKF_REF_F32: case OKF_REF_F16: case OKF_REF_BF16: v = row_dense(j, m); break;
        default: v = row_superblock(j, m); break;
        }
        j->y[m] = v;
    }
    return NULL;
}

int okf_ref_usable_cores(void) {
    cpu_set_t set;
    if (sched_getaffinity(0, sizeof(set), &set) == 0) {
        int c = CPU_COUNT(&set);
        if (c > 0) return c;
    }
    return 1;
}

static void run_rows(const job_t *job, int threads, int matmul) {
    if (threads <= 0) threads = okf_ref_usable_cores();
    if ((uint32_t)threads > job->M) threads = (int)job->M;
    if (threads < 1) threads = 1;
    pthread_t *tid = (pthread_t *)malloc(sizeof(pthread_t) * threads);
    int *live = (int *)calloc(threads, sizeof(int));
    slice_t *sl = (slice_t *)malloc(sizeof(slice_t) * threads);
    uint32_t per = (job->M + threads - 1) / threads;
    for (int t = 0; t < threads; t++) {
        uint32_t m0 = t * per > job->M ? job->M : t * per;
        uint32_t m1 = m0 + per > job->M ? job->M : m0 + per;
        sl[t] = (slice_t){job, m0, m1, matmul};
    }
    /* slices 1.. on worker threads, slice 0 inline; a failed spawn runs inline */
    for (int t = 1; t < threads; t++)
        live[t] = pthread_create(&tid[t], NULL, run_slice, &sl[t]) == 0;
    run_slice(&sl[0]);
    for (int t = 1; t < threads; t++) {
        if (live[t]) pthread_join(tid[t], NULL);
        else run_slice(&sl[t]);
    }
    free(tid);
    free(live);
    free(sl);
}

static int check(int32_t type, uint32_t K, uint64_t *rb) {
    if (K == 0) return -1;
    return okf_ref_row_bytes(type, K, rb);
}

int okf_ref_matvec(int32_t type, const uint8_t *w, uint32_t K, uint32_t M,
                   const float *x, float *y, int threads) {
    job_t j = {type, w, K, M, 0, x, y, 1};
    if (check(type, K, &j.row_bytes)) return -1;
    run_rows(&j, threads, 0);
    return 0;
}

int okf_ref_matmul(int32_t type, const uint8_t *w, uint32_t K, uint32_t M,
                   const float *X, uint32_t N, float *Y, int threads) {
    uint64_t rb;
    if (check(type, K, &rb)) return -1;
    if (type == OKF_REF_Q8_0 || type == OKF_REF_Q4_0) {
        /* X transposed to [K][N] (Gemma4Quant.swift:181-188) */
        float *XT = (float *)malloc(sizeof(float) * (uint64_t)N * K);
        if (!XT) return -1;
        for (uint32_t n = 0; n < N; n++)
            for (uint32_t k = 0; k < K; k++) XT[(uint64_t)k * N + n] = X[(uint64_t)n * K + k];
        job_t j = {type, w, K, M, rb, XT, Y, N};
        run_rows(&j, threads, 1);
        free(XT);
        return 0;
    }
    /* one column at a time (Gemma4Quant.swift:159-169) */
    for (uint32_t n = 0; n < N; n++) {
        job_t j = {type, w, K, M, rb, X + (uint64_t)n * K, Y + (uint64_t)n * M, 1};
        run_rows(&j, threads, 0);
    }
    return 0;
}

/* Kern.rmsnorm, LLM/Base/Kernels.swift:12-20, after the residual add of
 * add_rmsnorm_batch (LLM/metal/Kernels.metal:2850-2854) */
void okf_ref_add_rmsnorm(float *x, const float *r, const float *w, float *y, uint32_t n, uint32_t rows,
                         float eps) {
    for (uint32_t row = 0; row < rows; row++) {
        float *xr = x + (uint64_t)row * n, *yr = y + (uint64_t)row * n;
        float ss = 0;
        for (uint32_t i = 0; i < n; i++) {
            if (r) xr[i] += r[(uint64_t)row * n + i];
            ss += xr[i] * xr[i];
        }
        const float scale = 1.0f / sqrtf(ss / (float)n + eps);
        for (uint32_t i = 0; i < n; i++) yr[i] = xr[i] * scale * w[i];
    }
}

/* argmax_rows, LLM/metal/Kernels.metal:2766-2772: bv = -inf, bi = 0, take a
 * strictly larger value (so ties keep the lower index and NaN never wins) */
void okf_ref_argmax_rows(const float *x, uint32_t n, uint32_t rows, int32_t *out) {
    for (uint32_t row = 0; row < rows; row++) {
        const float *xr = x + (uint64_t)row * n;
        float bv = -INFINITY;
        int32_t bi = 0;
        for (uint32_t i = 0; i < n; i++)
            if (xr[i] > bv) {
                bv = xr[i];
                bi = (int32_t)i;
            }
        out[row] = bi;
    }
}

/* Swift silu, LLM/Base/Kernels.swift:3: x / (1 + expf(-x)); then times b. */
void okf_ref_silu_mul(const float *a, const float *b, uint32_t n, float *out) {
    for (uint32_t i = 0; i < n; i++) {
        const float x = a[i];
        const float s = x / (1.0f + expf(-x));
        out[i] = s * b[i];
    }
}
