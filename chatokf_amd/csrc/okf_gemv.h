// okf_gemv.h -- decode matvec (N = 1) and narrow matmul (N = 2..5) kernels.
//
// One weight pass serves all NC activation columns (the reference's
// gemv / gemm_nb kernels, LLM/metal/Kernels.metal:1572-1753, :2486-2585).
//
// Layout of the work.  A wavefront is four row slots of L = 16 lanes; each
// slot owns R consecutive rows.  A row is cut into units (Q4_K: one 32-byte
// code group = sub-blocks 2g and 2g+1; IQ2_XXS: two sub-blocks; Q8_0: one
// block; Q2_0: half a block); lane i of a slot walks units i, i + L, ... so
// the lanes of a slot read contiguous bytes of the row with 16-byte loads,
// and the weights of the next D steps are in flight while a step is
// computed.
//
// Arithmetic: exact integer dot products per 32 weights.  Each 32-weight
// group of an activation column is staged once per workgroup as integers
// X_j = rint(x_j 2^(22 - e)), e the binary exponent of the group's largest
// |x| (so |X_j| <= 2^22: 23 significant bits, fp32's precision relative to
// the group, at any fp32 magnitude), each split into three signed bytes
// X = x2 2^16 + x1 2^8 + x0 (balanced digits).  The weights' integer codes
// are laid out as bytes in the same order (nibbles and 2-bit codes are
// masked into bytes; IQ4 levels and IQ2_XXS signed grid values are looked up
// as bytes), and v_dot4_i32_i8 gives each digit's sum of products exactly,
// four weights per instruction.  The three digit sums are combined in fp32
// per group and the group and block scales are applied there, in the
// reference's factored form ((d*sc)*sum(q*x) - (dmin*m)*sum(x) for Q4_K,
// d*sum((code-1)*x) for Q2_0, d*sum(q*x) for Q8_0, db*sum(g*s*x) for
// IQ2_XXS).  The result differs from the reference's fp32 arithmetic only
// by the rounding of x to 23 bits relative to its group and fp32 summation
// order across groups.
#pragma once
#include "okf_common.h"
#include "okf_decode.h"

namespace okf {


// Weights per unit: 64, except Q8_0 whose unit is one 32-weight block (so
// any K that is a whole number of blocks works).
template <int F>
__host__ __device__ constexpr uint32_t unit_weights() {
    return (F == Q8_0 || F == Q4_0 || F == IQ4_NL || gen_fmt(F)) ? 32 : 64;
}
// 32-weight groups per unit, and 16-byte LDS chunks per unit (per group:
// three digit planes of 32 bytes; for the generic formats, whose weights are
// fp32 values, the 32 activations as fp32)
template <int F>
__host__ __device__ constexpr uint32_t unit_groups() {
    return unit_weights<F>() / 32;
}
template <int F>
__host__ __device__ constexpr uint32_t unit_chunks() {
    return unit_groups<F>() * (gen_fmt(F) ? 8 : 6);
}
// bytes of LDS one unit of one column takes: the chunks and one float4 of
// group data per group
template <int F>
__host__ __device__ constexpr uint32_t unit_lds_bytes() {
    return unit_groups<F>() * (unit_chunks<F>() / unit_groups<F>() * 16 + 16);
}

// 16-byte LDS rows of tables gemv_kernel copies per workgroup: IQ2_XXS's
// int8 grid and sign rows, the other grid formats' integer tables (IQ1_S /
// IQ1_M: their grid as it is)
template <int F>
__host__ __device__ constexpr uint32_t gemv_tab_rows() {
    return F == IQ2_XXS ? 384 : itab_rows(F) ? itab_rows(F) : gt_bytes(F) / 16;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// v_perm_b32: byte k of the result is byte sel_k of the 8-byte value {hi, lo}
// (selector 0x0C gives 0x00).
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// four int8 x int8 products summed into c (v_dot4_i32_i8)
__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// ---------------------------------------------------------------- units --
// Raw bytes of one unit for R rows (native vector types keep them in VGPRs).
// The generic formats (gen_fmt) keep only the row: their compute decodes a
// 32-weight sub-block with the bit-exact decoder.
template <int F, int R>
struct Unit {
    const uint8_t *row[R];
};
template <int R>
struct Unit<Q4_K, R> {  // 16-byte header + 32 code bytes of group g
    u32x4 hdr[R], q0[R], q1[R];
};
template <int R>
struct Unit<IQ2_XXS, R> {  // d + two sub-blocks (a0, a1, a0', a1')
    uint32_t d[R];
    u32x4 a[R];
};
template <int R>
struct Unit<IQ3_S, R> {  // d, 16 grid index bytes, their high bits, 8 sign bytes, the scale byte
    uint32_t d[R], qh[R], sc[R];
    u32x4 q[R];
    uint2 sg[R];
};
template <int R>
struct Unit<IQ2_XS, R> {  // d, 8 16-bit index+sign words, 2 scale bytes
    uint32_t d[R], sc[R];
    u32x4 q[R];
};
template <int R>
struct Unit<IQ2_S, R> {  // d, 8 index bytes, 8 sign bytes, 2 high-bit bytes, 2 scale bytes
    uint32_t d[R], qh[R], sc[R];
    uint2 q[R], sg[R];
};
template <int R>
struct Unit<IQ1_S, R> {  // d, 8 index bytes, 2 high-bits words
    uint32_t d[R], qh[R];
    uint2 q[R];
};
template <int R>
struct Unit<IQ1_M, R> {  // 8 index bytes, 4 high-bit bytes, the block's 4 scale words, the unit's one
    uint32_t qh[R], sw[R];
    uint2 q[R], sc[R];
};
template <int R>
struct Unit<Q2_K, R> {  // groups 2g, 2g + 1: their 32 code bytes, four scale bytes, d and dmin
    u32x4 q0[R], q1[R];
    uint32_t sc[R], dd[R];
};
template <int R>
struct Unit<Q3_K, R> {  // groups 2g, 2g + 1: their 32 code bytes, the 32 hmask bytes, the 12 scale bytes, d
    u32x4 q0[R], q1[R], h0[R], h1[R];
    uint2 s8[R];
    uint32_t s4[R], d[R];
};
template <int R>
struct Unit<IQ3_XXS, R> {  // d, the two sub-blocks' 16 grid indices and their two scale-and-sign words
    uint32_t d[R];
    u32x4 q[R];
    uint2 aux[R];
};
template <int R>
struct Unit<Q8_0, R> {  // one block: d + 32 code bytes (2-byte aligned)
    uint32_t d[R];
    u32x4 q0[R], q1[R];
};
template <int R>
struct Unit<Q2_0, R> {  // d + 16 code bytes (64 codes)
    uint32_t d[R];
    u32x4 q[R];
};
template <int R>
struct Unit<Q4_0, R> {  // one block: d + 16 code bytes (32 nibbles)
    uint32_t d[R];
    u32x4 q[R];
};
template <int R>
struct Unit<IQ4_NL, R> {  // as Q4_0
    uint32_t d[R];
    u32x4 q[R];
};

template <int R>
struct Unit<Q5_K, R> {  // header, the 32 qh bytes, 32 code bytes of group g
    u32x4 hdr[R], h0[R], h1[R], q0[R], q1[R];
};
template <int R>
struct Unit<Q6_K, R> {  // d, the half's 8 scales, ql bytes l and l + 32, qh bytes l (l = 16 is ..)
    uint32_t d[R];
    uint2 sc[R];
    u32x4 qa[R], qb[R], qh[R];
};
template <int R>
struct Unit<IQ4_XS, R> {  // d, scales_h, scales_l (8 bytes) + 32 code bytes of sub-blocks 2g, 2g + 1
    uint2 hdr[R];
    u32x4 q0[R], q1[R];
};

template <int F, int R>
__device__ __forceinline__ void load_unit(const uint8_t *const rows[R], uint32_t u, Unit<F, R> &w) {
#pragma unroll
    for (int r = 0; r < R; r++) {
        if constexpr (F == Q4_K) {
            const uint8_t *b = rows[r] + (uint64_t)(u >> 2) * 144;
            const uint32_t g = u & 3;
            w.hdr[r] = *(const u32x4 *)b;
            w.q0[r] = *(const u32x4 *)(b + 16 + g * 32);
            w.q1[r] = *(const u32x4 *)(b + 32 + g * 32);
        } else if constexpr (F == IQ2_XXS) {
            const uint8_t *b = rows[r] + (uint64_t)(u >> 2) * 66;
            w.d[r] = ldu<uint16_t>(b);
            w.a[r] = ldu<u32x4>(b + 2 + (u & 3) * 16);
        } else if constexpr (F == Q8_0) {
            const uint8_t *b = rows[r] + (uint64_t)u * 34;
            w.d[r] = ldu<uint16_t>(b);
            w.q0[r] = ldu<u32x4>(b + 2);
            w.q1[r] = ldu<u32x4>(b + 18);
        } else if constexpr (F == Q5_K) {  // unit = code group g of superblock u >> 2
            const uint8_t *b = rows[r] + (uint64_t)(u >> 2) * 176;
            const uint32_t g = u & 3;
            w.hdr[r] = ldu<u32x4>(b);
            w.h0[r] = ldu<u32x4>(b + 16);
            w.h1[r] = ldu<u32x4>(b + 32);
            w.q0[r] = ldu<u32x4>(b + 48 + g * 32);
            w.q1[r] = ldu<u32x4>(b + 64 + g * 32);
        } else if constexpr (F == Q6_K) {  // unit (n, is) of superblock u >> 2: see Compute<Q6_K>
            const uint8_t *b = rows[r] + (uint64_t)(u >> 2) * 210;
            const uint32_t n = (u >> 1) & 1, is = u & 1;
            w.d[r] = ldu<uint16_t>(b + 208);
            w.sc[r] = ldu<uint2>(b + 192 + n * 8);
            w.qa[r] = ldu<u32x4>(b + n * 64 + is * 16);
            w.qb[r] = ldu<u32x4>(b + n * 64 + 32 + is * 16);
            w.qh[r] = ldu<u32x4>(b + 128 + n * 32 + is * 16);
        } else if constexpr (F == IQ4_XS) {  // unit = sub-blocks 2g, 2g + 1 of superblock u >> 2
            const uint8_t *b = rows[r] + (uint64_t)(u >> 2) * 136;
            const uint32_t g = u & 3;
            w.hdr[r] = ldu<uint2>(b);
            w.q0[r] = ldu<u32x4>(b + 8 + g * 32);
            w.q1[r] = ldu<u32x4>(b + 24 + g * 32);
        } else if constexpr (F == IQ3_XXS) {  // unit = sub-blocks 2g, 2g + 1 of superblock u >> 2
            const uint8_t *b = rows[r] + (uint64_t)(u >> 2) * 98;
            const uint32_t g = u & 3;
            w.d[r] = ldu<uint16_t>(b);
            w.q[r] = ldu<u32x4>(b + 2 + g * 16);
            w.aux[r] = ldu<uint2>(b + 66 + g * 8);
        } else if constexpr (F == IQ3_S) {  // unit = sub-blocks 2g, 2g + 1
            const uint8_t *b = rows[r] + (uint64_t)(u >> 2) * 110;
            const uint32_t g = u & 3;
            w.d[r] = ldu<uint16_t>(b);
            w.q[r] = ldu<u32x4>(b + 2 + g * 16);
            w.qh[r] = ldu<uint16_t>(b + 66 + g * 2);
            w.sg[r] = ldu<uint2>(b + 74 + g * 8);
            w.sc[r] = b[106 + g];
        } else if constexpr (F == IQ2_XS) {
            const uint8_t *b = rows[r] + (uint64_t)(u >> 2) * 74;
            const uint32_t g = u & 3;
            w.d[r] = ldu<uint16_t>(b);
            w.q[r] = ldu<u32x4>(b + 2 + g * 16);
            w.sc[r] = ldu<uint16_t>(b + 66 + g * 2);
        } else if constexpr (F == IQ2_S) {
            const uint8_t *b = rows[r] + (uint64_t)(u >> 2) * 82;
            const uint32_t g = u & 3;
            w.d[r] = ldu<uint16_t>(b);
            w.q[r] = ldu<uint2>(b + 2 + g * 8);
            w.sg[r] = ldu<uint2>(b + 34 + g * 8);
            w.qh[r] = ldu<uint16_t>(b + 66 + g * 2);
            w.sc[r] = ldu<uint16_t>(b + 74 + g * 2);
        } else if constexpr (F == IQ1_S) {
            const uint8_t *b = rows[r] + (uint64_t)(u >> 2) * 50;
            const uint32_t g = u & 3;
            w.d[r] = ldu<uint16_t>(b);
            w.q[r] = ldu<uint2>(b + 2 + g * 8);
            w.qh[r] = ldu<uint32_t>(b + 34 + g * 4);
        } else if constexpr (F == IQ1_M) {
            const uint8_t *b = rows[r] + (uint64_t)(u >> 2) * 56;
            const uint32_t g = u & 3;
            w.q[r] = ldu<uint2>(b + g * 8);
            w.qh[r] = ldu<uint32_t>(b + 32 + g * 4);
            w.sc[r] = ldu<uint2>(b + 48);
            w.sw[r] = ldu<uint16_t>(b + 48 + g * 2);  // sub-blocks 2g, 2g + 1: scale word g
        } else if constexpr (F == Q2_K) {  // unit = groups 2g, 2g + 1 (g = u & 3) of superblock u >> 2
            const uint8_t *b = rows[r] + (uint64_t)(u >> 2) * 84;
            const uint32_t g = u & 3, n = g >> 1;  // (both groups read the same code bytes)
            w.q0[r] = ldu<u32x4>(b + 16 + 32 * n);
            w.q1[r] = ldu<u32x4>(b + 32 + 32 * n);
            w.sc[r] = ldu<uint32_t>(b + 4 * g);
            w.dd[r] = ldu<uint32_t>(b + 80);
        } else if constexpr (F == Q3_K) {
            const uint8_t *b = rows[r] + (uint64_t)(u >> 2) * 110;
            const uint32_t n = (u & 3) >> 1;
            w.q0[r] = ldu<u32x4>(b + 32 + 32 * n);
            w.q1[r] = ldu<u32x4>(b + 48 + 32 * n);
            w.h0[r] = ldu<u32x4>(b);
            w.h1[r] = ldu<u32x4>(b + 16);
            w.s8[r] = ldu<uint2>(b + 96);
            w.s4[r] = ldu<uint32_t>(b + 104);
            w.d[r] = ldu<uint16_t>(b + 108);
        } else if constexpr (gen_fmt(F)) {
            w.row[r] = rows[r];
        } else if constexpr (F == Q4_0 || F == IQ4_NL) {
            const uint8_t *b = rows[r] + (uint64_t)u * 18;
            w.d[r] = ldu<uint16_t>(b);
            w.q[r] = ldu<u32x4>(b + 2);
        } else {
            const uint8_t *b = rows[r] + (uint64_t)(u >> 1) * 34;
            w.d[r] = ldu<uint16_t>(b);
            w.q[r] = ldu<u32x4>(b + 2 + (u & 1) * 16);
        }
    }
}

// -------------------------------------------------------------- staging --
// Byte order of a unit's activations: the order in which the format's
// weight bytes meet them.  A slot is 8 consecutive bytes (4 slots a group);
// its values are read by load_slot.
//  Q2_0: code dword j of the unit holds the 2-bit codes of weights 16j + 4b
//        + k (byte b, field k); (v >> 2k) & 0x03030303 makes bytes of the
//        codes of weights 16j + k + {0, 4, 8, 12}, which is dword 4j + k of
//        the unit's byte order.
//  Q6_K: the unit (half n, is) of superblock u / 4 holds weights 16 is + l +
//        32 grp (l < 16) of its half, 16 per grp in order.
//  every other format: the unit's weights in order.
// Index in x of the first weight of unit u (a row's units in order).
template <int F>
__device__ __forceinline__ uint64_t unit_x_base(uint32_t u) {
    if constexpr (F == Q6_K) return (uint64_t)(u >> 1) * 128 + (u & 1) * 16;
    else return (uint64_t)u * unit_weights<F>();
}

// The 8 activations of slot s of the unit whose x starts at xu.
template <int F>
__device__ __forceinline__ void load_slot(const float *__restrict__ xu, uint32_t s, float (&v)[8]) {
    if constexpr (F == Q2_0) {
        const uint32_t j = s >> 1, k0 = 2 * (s & 1);
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const float2 t = *(const float2 *)(xu + 16 * j + 4 * b + k0);
            v[b] = t.x;
            v[4 + b] = t.y;
        }
    } else {
        const uint32_t base = F == Q6_K ? 32 * (s >> 1) + 8 * (s & 1) : 8 * s;
        const floatx4 a = *(const floatx4 *)(xu + base), b = *(const floatx4 *)(xu + base + 4);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            v[k] = a[k];
            v[4 + k] = b[k];
        }
    }
}

// DPP lane moves (one VALU op, no LDS round trip): quad_perm [1,0,3,2] and
// [2,3,0,1] swap neighbours and pairs within a quad; row_half_mirror (lane
// i <- 7 - i of its 8) and row_mirror (i <- 15 - i of its 16) pair quads
// and half-rows.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                                 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dppi(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
constexpr int DPP_QUAD_XOR1 = 0xB1, DPP_QUAD_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141,
              DPP_MIRROR = 0x140;

// sum / max over the 4 lanes of a quad (every lane gets it)
__device__ __forceinline__ float quad_sum(float v) {
    v += dpp<DPP_QUAD_XOR1>(v);
    return v + dpp<DPP_QUAD_XOR2>(v);
}
__device__ __forceinline__ float quad_max(float v) {
    v = fmaxf(v, dpp<DPP_QUAD_XOR1>(v));
    return fmaxf(v, dpp<DPP_QUAD_XOR2>(v));
}

// Stages one slot v of a 32-weight group; the group's 4 slots are the 4
// lanes of a quad, all of which call this.  Gives the slot's three digit
// planes (8 bytes each) and, in every lane, the group's data
// {sum X over slots 0-1, over slots 2-3, over all, f = 2^(e - 22)}; f is NaN
// when the group holds an inf or NaN, so that it reaches the outputs.
//
// X = rint(x 2^(22 - e)) comes from one fma with 1.5 * 2^23, whose result's
// bits are 0x4B400000 + X; Y = X + 0x808080 then has the unsigned digits
// y_i = x_i + 128, so the signed digits are the bytes of Y ^ 0x808080 (a
// byte xor 0x80 read as int8 is y - 128).  |X| <= 2^22 keeps Y in
// (0, 2^24) and |x2| <= 64.
__device__ __forceinline__ void limb_slot(const float (&v)[8], uint2 (&pl)[3], floatx4 &gd) {
    float m = 0, bad = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        m = fmaxf(m, fabsf(v[k]));
        bad = fmaf(v[k], 0.0f, bad);  // NaN for an inf or NaN value
    }
    m = quad_max(m);
    bad = quad_sum(bad);
    // (frexp gives 0 for inf / NaN; the clamp keeps 2^(22 - e) and f normal)
    const int e = max(min(__builtin_amdgcn_frexp_expf(m), 127), -104);
    const float sc = __builtin_amdgcn_ldexpf(1.0f, 22 - e);
    uint32_t y[8];
    uint32_t sy = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        y[k] = __builtin_bit_cast(uint32_t, fmaf(v[k], sc, 12582912.0f)) - 0x4ABF7F80u;
        sy += y[k];
    }
#pragma unroll
    for (int d = 0; d < 2; d++) {
        const uint32_t *q = y + 4 * d;
        const uint32_t a = perm(q[1], q[0], 0x05010400u), b = perm(q[3], q[2], 0x05010400u);
        const uint32_t c = perm(q[1], q[0], 0x0C0C0602u), e2 = perm(q[3], q[2], 0x0C0C0602u);
        const uint32_t p0 = perm(b, a, 0x05040100u) ^ 0x80808080u;
        const uint32_t p1 = perm(b, a, 0x07060302u) ^ 0x80808080u;
        const uint32_t p2 = perm(e2, c, 0x05040100u) ^ 0x80808080u;
        if (d == 0) {
            pl[0].x = p0;
            pl[1].x = p1;
            pl[2].x = p2;
        } else {
            pl[0].y = p0;
            pl[1].y = p1;
            pl[2].y = p2;
        }
    }
    // sums of X: 8 Y's carry 8 * 0x808080 (< 2^27, so no wrap)
    const int sx = (int)(sy - 8u * 0x808080u);
    const int s16 = sx + dppi<DPP_QUAD_XOR1>(sx), o16 = dppi<DPP_QUAD_XOR2>(s16);
    const bool first = (__lane_id() & 2) == 0;  // lane 0 or 1 of the quad: slots 0-1
    const int a16 = first ? s16 : o16, b16 = first ? o16 : s16;
    gd = floatx4{(float)a16, (float)b16, (float)(a16 + b16), __builtin_amdgcn_ldexpf(1.0f, e - 22) + bad};
}

// LDS layout of the staged activations of one column: units in groups of L
// (one per lane of a row slot); within a group, the unit's 16-byte chunks,
// each [L lanes][16 bytes], so a row slot's lanes read 16 consecutive
// chunks.  Chunk (gi, p, h) is bytes 16 h .. 16 h + 15 of digit plane p of
// the unit's group gi.  Index in uint32.
__host__ __device__ constexpr uint32_t chunk_of(uint32_t gi, uint32_t p, uint32_t h) {
    return (gi * 3 + p) * 2 + h;
}
template <int F, int L>
__device__ __forceinline__ uint32_t xs_index(uint32_t u, uint32_t ch) {
    constexpr uint32_t NCH = unit_chunks<F>();
    const uint32_t t = u / L, i = u % L;
    return ((t * NCH + ch) * L + i) * 4;
}

// Loads slot sidx of unit u (absolute unit uabs in the row) of every column
// (columns K floats apart, with SILU: silu(X) * X2) and stages it: digit
// planes to xs (column stride cs), the group data to gdp (column stride
// gcs) by the quad's first lane.  `store` is false for lanes past the end,
// which still take part in the quad's reductions.
template <int F, int NC, int L, bool SILU>
__device__ __forceinline__ void stage_slot(const float (&v)[NC][8], uint32_t u, uint32_t sidx, bool store,
                                           uint32_t *xs, uint32_t cs, floatx4 *gdp, uint32_t gcs) {
    constexpr uint32_t UG = unit_groups<F>();
    const uint32_t gi = sidx >> 2, k = sidx & 3;
    if constexpr (gen_fmt(F)) {
        // the 8 values as they are: chunks 2k, 2k + 1 of group gi hold
        // values 8k .. 8k + 7 (no group data)
        if (store)
#pragma unroll
            for (int n = 0; n < NC; n++) {
                uint32_t *d = xs + n * cs;
                *(floatx4 *)(d + xs_index<F, L>(u, gi * 8 + 2 * k)) = floatx4{v[n][0], v[n][1], v[n][2], v[n][3]};
                *(floatx4 *)(d + xs_index<F, L>(u, gi * 8 + 2 * k + 1)) = floatx4{v[n][4], v[n][5], v[n][6], v[n][7]};
            }
        (void)gdp;
        (void)gcs;
        return;
    }
#pragma unroll
    for (int n = 0; n < NC; n++) {
        uint2 pl[3];
        floatx4 gd;
        limb_slot(v[n], pl, gd);
        if (store) {
#pragma unroll
            for (int p = 0; p < 3; p++)
                *(uint2 *)(xs + n * cs + xs_index<F, L>(u, chunk_of(gi, p, k >> 1)) + (k & 1) * 2) = pl[p];
            if (k == 0) gdp[n * gcs + u * UG + gi] = gd;
        }
    }
}

// ------------------------------------------------------------- compute --
// acc[r][n] += unit contribution.  The unit's staged activations come
// through an accessor xa: xa.chunk(n, c) is 16-byte chunk c of column n,
// xa.gd(n, gi) the data of group gi of column n (XLds: from LDS, as staged
// per workgroup).
struct XLds {
    const uint32_t *xp;  // this lane's chunk 0 of column 0
    uint32_t ss, cs;     // uint32 stride between chunks, between columns
    const floatx4 *gp;   // the unit's group data of column 0
    uint32_t gcs;        // float4 stride between columns
    __device__ __forceinline__ u32x4 chunk(int n, uint32_t ch) const {
        return *(const u32x4 *)(xp + n * cs + ch * ss);
    }
    __device__ __forceinline__ floatx4 gd(int n, uint32_t gi) const { return gp[n * gcs + gi]; }
};
//
// dot_half: for group gi and chunk half h (plane dwords 4h .. 4h + 3), the
// weight dwords wf(r, k) (int8 bytes in the staged order of plane dword
// 4h + k) dotted with each digit plane into s[digit][r][n].
template <int NC, int R, class XA, class WF>
__device__ __forceinline__ void dot_half(const XA &xa, uint32_t gi, uint32_t h, WF wf, int (&s)[3][R][NC]) {
    u32x4 x[3][NC];
#pragma unroll
    for (int p = 0; p < 3; p++)
#pragma unroll
        for (int n = 0; n < NC; n++) x[p][n] = xa.chunk(n, chunk_of(gi, p, h));
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t wv = wf(r, k);
#pragma unroll
            for (int p = 0; p < 3; p++)
#pragma unroll
                for (int n = 0; n < NC; n++) s[p][r][n] = sdot4(wv, x[p][n][k], s[p][r][n]);
        }
}

template <int NC, int R>
__device__ __forceinline__ void zero3(int (&s)[3][R][NC]) {
#pragma unroll
    for (int p = 0; p < 3; p++)
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int n = 0; n < NC; n++) s[p][r][n] = 0;
}

// sum(q X) of a group from its digit sums: s2 2^16 + s1 2^8 + s0.  (s2 << 8)
// + s1 is exact in int32 (|s2| <= 32 * 128 * 64 = 2^18, so it stays below
// 2^27); its conversion to float is exact below 2^24 (weight bytes within
// +-31: |s2| < 2^16; Q2_0, the 4-bit codes and IQ1's values among them) and
// otherwise rounds once, and the fma rounds once: at most two roundings of
// 2^-24 relative to the group's sum.
template <int NC, int R>
__device__ __forceinline__ float comb(const int (&s)[3][R][NC], int r, int n) {
    return fmaf((float)((s[2][r][n] << 8) + s[1][r][n]), 256.0f, (float)s[0][r][n]);
}

template <int F, int NC, int R, int TS = 1>
struct Compute {
    // The plain f32 / f16 / bf16 weights: the 32 weights of a unit are
    // decoded to fp32 and multiplied in fp32 into the activations, staged as
    // fp32 (chunk c of the unit = values 4c .. 4c + 3): one fma a weight,
    // in order, as the reference's fp32 dot.
    static_assert(gen_fmt(F), "no matvec compute for this format");
    template <class XA>
    __device__ __forceinline__ static void run(const Unit<F, R> &w, const XA &xa, uint32_t u, float (&acc)[R][NC],
                                               const u32x4 *tab) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            float wv[32];
            decode_unit<F>(w.row[r], u, wv, nullptr);
#pragma unroll
            for (int n = 0; n < NC; n++) {
                float a = 0;
#pragma unroll
                for (int c = 0; c < 8; c++) {
                    const floatx4 xv = __builtin_bit_cast(floatx4, xa.chunk(n, c));
#pragma unroll
                    for (int e = 0; e < 4; e++) a = fmaf(wv[4 * c + e], xv[e], a);
                }
                acc[r][n] += a;
            }
        }
    }
};

template <int NC, int R, int TS>
struct Compute<Q4_K, NC, R, TS> {
    // Code dword i (bytes 4i..4i+3 of the unit's 32): low nibbles are weights
    // 4i.. of sub-block 2g (group 0), high nibbles of sub-block 2g + 1.
    template <class XA>
    __device__ __forceinline__ static void run(const Unit<Q4_K, R> &w, const XA &xa, uint32_t u,
                                               float (&acc)[R][NC], const u32x4 *) {
        const uint32_t g = u & 3;
        int s0[3][R][NC], s1[3][R][NC];
        zero3(s0);
        zero3(s1);
        auto code = [&](int r, int i) { return i < 4 ? w.q0[r][i] : w.q1[r][i - 4]; };
#pragma unroll
        for (int h = 0; h < 2; h++) {
            dot_half<NC, R>(xa, 0, h, [&](int r, int k) { return code(r, 4 * h + k) & 0x0F0F0F0Fu; }, s0);
            dot_half<NC, R>(xa, 1, h,
                            [&](int r, int k) { return (code(r, 4 * h + k) >> 4) & 0x0F0F0F0Fu; }, s1);
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            uint32_t sc0, mn0, sc1, mn1;
            const uint4 hv = make_uint4(w.hdr[r][0], w.hdr[r][1], w.hdr[r][2], w.hdr[r][3]);
            q4k_scale_min_pair(hv, g, sc0, mn0, sc1, mn1);
            const float d = h2f(w.hdr[r][0] & 0xFFFF), dmin = h2f(w.hdr[r][0] >> 16);
            const float a0 = d * (float)sc0, a1 = d * (float)sc1;
            const float b0 = dmin * (float)mn0, b1 = dmin * (float)mn1;
#pragma unroll
            for (int n = 0; n < NC; n++) {
                const floatx4 g0 = xa.gd(n, 0), g1 = xa.gd(n, 1);
                acc[r][n] += g0[3] * (a0 * comb(s0, r, n) - b0 * g0[2]) + g1[3] * (a1 * comb(s1, r, n) - b1 * g1[2]);
            }
        }
    }
};

// the IQ2 grid's three values and their negations, as v_perm sources
constexpr uint32_t IQ2_POS = 0x002B1908u, IQ2_NEG = 0x00D5E7F8u;  // {8, 25, 43, 0}, {-8, -25, -43, 0}

template <int NC, int R, int TS>
struct Compute<IQ2_XXS, NC, R, TS> {
    // tab: [0, 256) grid entries {I.x, I.y}: per weight the index 0..2 of
    // its value in {8, 25, 43}; [256, 384) sign entries {S.x, S.y} of
    // selectors, byte j = j % 4 + 4 (weight j negative; the eighth sign from
    // the parity rule).  I + S - {0, 1, 2, 3} selects the signed value from
    // {8, 25, 43 | -8, -25, -43} (no byte carries: each sum is 0..6), so
    // one add and one v_perm make four signed weight bytes, from 8-byte
    // table reads.  Entry e at tab[e * TS] (TS = 16: the
    // replicated, conflict-free layout of gemv_wide_kernel, tab offset by
    // the lane's copy).
    template <class XA>
    __device__ __forceinline__ static void run(const Unit<IQ2_XXS, R> &w, const XA &xa, uint32_t,
                                               float (&acc)[R][NC], const u32x4 *tab) {
#pragma unroll
        for (int sb = 0; sb < 2; sb++) {  // the unit's two sub-blocks = groups
            int s[3][R][NC];
            zero3(s);
#pragma unroll
            for (int h = 0; h < 2; h++) {  // grid entries 2h, 2h + 1 = plane dwords 4h .. 4h + 3
                uint32_t wv[R][4];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const uint32_t a0 = w.a[r][2 * sb], a1 = w.a[r][2 * sb + 1];
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        const int l = 2 * h + e;
                        const uint2 gv = *(const uint2 *)&tab[((a0 >> (8 * l)) & 0xFF) * TS];
                        const uint2 sg = *(const uint2 *)&tab[(256 + ((a1 >> (7 * l)) & 127)) * TS];
                        wv[r][2 * e] = perm(IQ2_NEG, IQ2_POS, gv.x + sg.x - 0x03020100u);
                        wv[r][2 * e + 1] = perm(IQ2_NEG, IQ2_POS, gv.y + sg.y - 0x03020100u);
                    }
                }
                dot_half<NC, R>(xa, sb, h, [&](int r, int k) { return wv[r][k]; }, s);
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t a1 = w.a[r][2 * sb + 1];
                const float db = h2f(w.d[r]) * (0.5f + (float)(a1 >> 28)) * 0.25f;
#pragma unroll
                for (int n = 0; n < NC; n++) acc[r][n] += db * (comb(s, r, n) * xa.gd(n, sb)[3]);
            }
        }
    }
};

template <int NC, int R, int TS>
struct Compute<IQ3_XXS, NC, R, TS> {
    // IQX.iq3XXS (LLM/Quantize/IQ3.swift:60-86) as integer dot products:
    // weight = db * sign * grid byte, db = d (0.5 + aux >> 28) / 2 per
    // 32-weight sub-block, where the grid bytes (4..62) and their signs fit
    // int8.  tab (as 8-byte entries): [0, 256) grid entry e's 4 bytes, then
    // their negations; [256, 384) the v_perm selectors of a 7-bit sign
    // index (byte j selects the positive or the negated byte, eighth sign
    // from the parity rule).
    template <class XA>
    __device__ __forceinline__ static void run(const Unit<IQ3_XXS, R> &w, const XA &xa, uint32_t,
                                               float (&acc)[R][NC], const u32x4 *tab) {
        const uint2 *t2 = (const uint2 *)tab;
#pragma unroll
        for (int sb = 0; sb < 2; sb++) {
            int s[3][R][NC];
            zero3(s);
#pragma unroll
            for (int h = 0; h < 2; h++) {  // index pairs 2h, 2h + 1 = plane dwords 4h .. 4h + 3
                uint32_t wv[R][4];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const uint32_t qd = w.q[r][2 * sb + h], aux = sb ? w.aux[r].y : w.aux[r].x;
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        const int l = 2 * h + e;
                        const uint2 g1 = t2[(qd >> (16 * e)) & 0xFF], g2 = t2[(qd >> (16 * e + 8)) & 0xFF];
                        const uint2 sg = t2[256 + ((aux >> (7 * l)) & 127)];
                        wv[r][2 * e] = perm(g1.y, g1.x, sg.x);
                        wv[r][2 * e + 1] = perm(g2.y, g2.x, sg.y);
                    }
                }
                dot_half<NC, R>(xa, sb, h, [&](int r, int k) { return wv[r][k]; }, s);
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t aux = sb ? w.aux[r].y : w.aux[r].x;
                const float db = h2f(w.d[r]) * (0.5f + (float)(aux >> 28)) * 0.5f;
#pragma unroll
                for (int n = 0; n < NC; n++) acc[r][n] += db * (comb(s, r, n) * xa.gd(n, sb)[3]);
            }
        }
    }
};

template <int NC, int R, int TS>
struct Compute<IQ3_S, NC, R, TS> {
    // IQX.iq3S (LLM/Quantize/IQ3.swift:88-115) as integer dot products:
    // weight = d (1 + 2 sc) * sign * grid byte (1..15) per 32-weight
    // sub-block.  tab (8-byte entries): [0, 512) grid entry e's 4 bytes and
    // their negations; [512, 768) the v_perm selectors of a sign byte.
    template <class XA>
    __device__ __forceinline__ static void run(const Unit<IQ3_S, R> &w, const XA &xa, uint32_t,
                                               float (&acc)[R][NC], const u32x4 *tab) {
        const uint2 *t2 = (const uint2 *)tab;
#pragma unroll
        for (int sb = 0; sb < 2; sb++) {
            int s[3][R][NC];
            zero3(s);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                uint32_t wv[R][4];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const uint32_t qd = w.q[r][2 * sb + h], qh = (w.qh[r] >> (8 * sb)) & 0xFF;
                    const uint32_t sgd = sb ? w.sg[r].y : w.sg[r].x;
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        const int l = 2 * h + e;
                        const uint32_t i1 = ((qd >> (16 * e)) & 0xFF) | ((qh << (8 - 2 * l)) & 256);
                        const uint32_t i2 = ((qd >> (16 * e + 8)) & 0xFF) | ((qh << (7 - 2 * l)) & 256);
                        const uint2 g1 = t2[i1], g2 = t2[i2], sg = t2[512 + ((sgd >> (8 * l)) & 0xFF)];
                        wv[r][2 * e] = perm(g1.y, g1.x, sg.x);
                        wv[r][2 * e + 1] = perm(g2.y, g2.x, sg.y);
                    }
                }
                dot_half<NC, R>(xa, sb, h, [&](int r, int k) { return wv[r][k]; }, s);
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                const float db = h2f(w.d[r]) * (float)(1 + 2 * ((w.sc[r] >> (4 * sb)) & 0xF));
#pragma unroll
                for (int n = 0; n < NC; n++) acc[r][n] += db * (comb(s, r, n) * xa.gd(n, sb)[3]);
            }
        }
    }
};

// IQX.iq2XS / IQX.iq2S (LLM/Quantize/IQ3.swift:14-57) as integer dot
// products: weight = d (0.5 + nibble) / 4 * sign * grid byte (8, 25, 43),
// one scale nibble per 16 weights.  tab (8-byte entries): [0, G) grid entry
// e as its values' indices in {8, 25, 43}, then the selectors of a 7-bit
// sign index (IQ2_XS, eighth sign from the parity rule) or of a sign byte
// (IQ2_S), combined as IQ2_XXS's.
template <int F, int NC, int R, int TS>
struct ComputeIQ2XS {
    static constexpr uint32_t G = F == IQ2_S ? 1024 : 512;
    template <class XA>
    __device__ __forceinline__ static void run(const Unit<F, R> &w, const XA &xa, float (&acc)[R][NC],
                                               const u32x4 *tab) {
        const uint2 *gi = (const uint2 *)tab, *sel = gi + G;
#pragma unroll
        for (int sb = 0; sb < 2; sb++)
#pragma unroll
            for (int h = 0; h < 2; h++) {  // 16 weights, one scale nibble
                int s[3][R][NC];
                zero3(s);
                uint32_t wv[R][4];
#pragma unroll
                for (int r = 0; r < R; r++)
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        const int l = 2 * h + e;
                        uint32_t idx, sv;
                        if constexpr (F == IQ2_S) {
                            const uint32_t qd = sb ? w.q[r].y : w.q[r].x, sgd = sb ? w.sg[r].y : w.sg[r].x;
                            const uint32_t qh = (w.qh[r] >> (8 * sb)) & 0xFF;
                            idx = ((qd >> (8 * l)) & 0xFF) | ((qh << (8 - 2 * l)) & 0x300);
                            sv = (sgd >> (8 * l)) & 0xFF;
                        } else {
                            const uint32_t q16 = (w.q[r][2 * sb + h] >> (16 * e)) & 0xFFFF;
                            idx = q16 & 511;
                            sv = q16 >> 9;
                        }
                        const uint2 gv = gi[idx], sg = sel[sv];
                        wv[r][2 * e] = perm(IQ2_NEG, IQ2_POS, gv.x + sg.x - 0x03020100u);
                        wv[r][2 * e + 1] = perm(IQ2_NEG, IQ2_POS, gv.y + sg.y - 0x03020100u);
                    }
                dot_half<NC, R>(xa, sb, h, [&](int r, int k) { return wv[r][k]; }, s);
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const uint32_t nib = (w.sc[r] >> (8 * sb + 4 * h)) & 0xF;
                    const float db = h2f(w.d[r]) * (0.5f + (float)nib) * 0.25f;
#pragma unroll
                    for (int n = 0; n < NC; n++) acc[r][n] += db * (comb(s, r, n) * xa.gd(n, sb)[3]);
                }
            }
    }
};
template <int NC, int R, int TS>
struct Compute<IQ2_XS, NC, R, TS> {
    template <class XA>
    __device__ __forceinline__ static void run(const Unit<IQ2_XS, R> &w, const XA &xa, uint32_t,
                                               float (&acc)[R][NC], const u32x4 *tab) {
        ComputeIQ2XS<IQ2_XS, NC, R, TS>::run(w, xa, acc, tab);
    }
};
template <int NC, int R, int TS>
struct Compute<IQ2_S, NC, R, TS> {
    template <class XA>
    __device__ __forceinline__ static void run(const Unit<IQ2_S, R> &w, const XA &xa, uint32_t,
                                               float (&acc)[R][NC], const u32x4 *tab) {
        ComputeIQ2XS<IQ2_S, NC, R, TS>::run(w, xa, acc, tab);
    }
};

// IQ1.dequant / IQ1M.dequant (LLM/Quantize/IQ1.swift:44-66,
// LLM/Quantize/IQ2XXS.swift:63-98) as integer dot products: weight =
// dl (n - 1 + delta), delta = +-1/8, n the grid's ternary digit, so 8 w / dl
// = 8 n - 8 +- 1 fits int8; one v_perm picks it per byte from the six
// values {-7, 1, 9 | -9, -1, 7} by n + 4 (delta < 0).  tab: the 2048-entry
// grid (4 bytes an entry: weight j's digit at bit 8 (j % 4) + 4 (j / 4)).
// IQ1_S has one dl and delta per 32 weights; IQ1_M one dl per 16 and a
// delta per 8.
template <int F, int NC, int R, int TS>
struct ComputeIQ1 {
    template <class XA>
    __device__ __forceinline__ static void run(const Unit<F, R> &w, const XA &xa, float (&acc)[R][NC],
                                               const u32x4 *tab) {
        const uint32_t *grid = (const uint32_t *)tab;
        constexpr uint32_t POS = 0x000901F9u, NEG = 0x0007FFF7u;  // {-7, 1, 9, 0}, {-9, -1, 7, 0}
#pragma unroll
        for (int sb = 0; sb < 2; sb++)
#pragma unroll
            for (int h = 0; h < 2; h++) {
                int s[3][R][NC];
                zero3(s);
                uint32_t wv[R][4];
#pragma unroll
                for (int r = 0; r < R; r++)
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        const int l = 2 * h + e;
                        const uint32_t qd = sb ? w.q[r].y : w.q[r].x;
                        uint32_t hb, neg;
                        if constexpr (F == IQ1_S) {
                            const uint32_t qh = (w.qh[r] >> (16 * sb)) & 0xFFFF;
                            hb = (qh >> (3 * l)) & 7;
                            neg = qh >> 15;
                        } else {
                            const uint32_t hq = (w.qh[r] >> (16 * sb + 8 * h)) & 0xFF;
                            hb = (hq >> (4 * e)) & 7;
                            neg = (hq >> (4 * e + 3)) & 1;
                        }
                        const uint32_t gv = grid[((qd >> (8 * l)) & 0xFF) | (hb << 8)];
                        const uint32_t nm = neg ? 0x04040404u : 0u;
                        wv[r][2 * e] = perm(NEG, POS, (gv & 0x0F0F0F0Fu) | nm);
                        wv[r][2 * e + 1] = perm(NEG, POS, ((gv >> 4) & 0x0F0F0F0Fu) | nm);
                    }
                dot_half<NC, R>(xa, sb, h, [&](int r, int k) { return wv[r][k]; }, s);
#pragma unroll
                for (int r = 0; r < R; r++) {
                    float dl;
                    if constexpr (F == IQ1_S) {
                        const uint32_t qh = (w.qh[r] >> (16 * sb)) & 0xFFFF;
                        dl = h2f(w.d[r]) * (float)(2 * ((qh >> 12) & 7) + 1);
                    } else {
                        // d from the tops of the block's four scale words; the
                        // sub-block's 3-bit scales (one per 16 weights) at
                        // bit 6 sb of the unit's word
                        const uint32_t a = w.sc[r].x, b = w.sc[r].y;
                        const uint32_t bits = ((a & 0xFFFF) >> 12) | ((a >> 24) & 0x00f0) |
                                              (((b & 0xFFFF) >> 4) & 0x0f00) | ((b >> 16) & 0xf000);
                        const uint32_t sv = w.sw[r] >> (6 * sb);
                        dl = h2f((uint16_t)bits) * (float)(2 * ((sv >> (3 * h)) & 7) + 1);
                    }
                    const float db = dl * 0.125f;
#pragma unroll
                    for (int n = 0; n < NC; n++) acc[r][n] += db * (comb(s, r, n) * xa.gd(n, sb)[3]);
                }
            }
    }
};
template <int NC, int R, int TS>
struct Compute<IQ1_S, NC, R, TS> {
    template <class XA>
    __device__ __forceinline__ static void run(const Unit<IQ1_S, R> &w, const XA &xa, uint32_t,
                                               float (&acc)[R][NC], const u32x4 *tab) {
        ComputeIQ1<IQ1_S, NC, R, TS>::run(w, xa, acc, tab);
    }
};
template <int NC, int R, int TS>
struct Compute<IQ1_M, NC, R, TS> {
    template <class XA>
    __device__ __forceinline__ static void run(const Unit<IQ1_M, R> &w, const XA &xa, uint32_t,
                                               float (&acc)[R][NC], const u32x4 *tab) {
        ComputeIQ1<IQ1_M, NC, R, TS>::run(w, xa, acc, tab);
    }
};

template <int NC, int R, int TS>
struct Compute<Q2_K, NC, R, TS> {
    // KQuant.q2K (LLM/Quantize/KQuants.swift:9-36) as integer dot products:
    // per 16 weights, w = d (sc & 15) q - dmin (sc >> 4), q = the 2-bit
    // field 2 (j % 4) of group j's code bytes, so sum w x = d (sc & 15)
    // sum q X f - dmin (sc >> 4) sum X f, both sums exact per half group.
    template <class XA>
    __device__ __forceinline__ static void run(const Unit<Q2_K, R> &w, const XA &xa, uint32_t u,
                                               float (&acc)[R][NC], const u32x4 *) {
#pragma unroll
        for (int gi = 0; gi < 2; gi++) {  // group j = 2 (u % 4) + gi
            const uint32_t sh = 2 * ((2 * (u & 3) + gi) & 3);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                int s[3][R][NC];
                zero3(s);
                dot_half<NC, R>(xa, gi, h, [&](int r, int k) {
                    return ((h ? w.q1[r][k] : w.q0[r][k]) >> sh) & 0x03030303u;
                }, s);
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const uint32_t sc = (w.sc[r] >> (16 * gi + 8 * h)) & 0xFF;
                    const float dl = h2f(w.dd[r] & 0xFFFF) * (float)(sc & 0xF);
                    const float ml = h2f(w.dd[r] >> 16) * (float)(sc >> 4);
#pragma unroll
                    for (int n = 0; n < NC; n++) {
                        const floatx4 g = xa.gd(n, gi);
                        acc[r][n] += g[3] * (dl * comb(s, r, n) - ml * g[h]);
                    }
                }
            }
        }
    }
};

template <int NC, int R, int TS>
struct Compute<Q3_K, NC, R, TS> {
    // KQuant.q3K (LLM/Quantize/KQuants.swift:38-83) as integer dot products:
    // w = dl (q + 4 hbit - 4), q + 4 hbit (0..7) a byte, so sum w x =
    // dl (sum (q + 4 hbit) X - 4 sum X) f per 16 weights.
    template <class XA>
    __device__ __forceinline__ static void run(const Unit<Q3_K, R> &w, const XA &xa, uint32_t u,
                                               float (&acc)[R][NC], const u32x4 *) {
#pragma unroll
      for (int gi = 0; gi < 2; gi++) {  // group j = 2 (u % 4) + gi
        const uint32_t j = 2 * (u & 3) + gi, n8 = j >> 2, sh = 2 * (j & 3), hb = 4 * n8 + (j & 3);
#pragma unroll
        for (int h = 0; h < 2; h++) {
            int s[3][R][NC];
            zero3(s);
            dot_half<NC, R>(xa, gi, h, [&](int r, int k) {
                const uint32_t q = ((h ? w.q1[r][k] : w.q0[r][k]) >> sh) & 0x03030303u;
                const uint32_t hm = ((h ? w.h1[r][k] : w.h0[r][k]) >> hb) & 0x01010101u;
                return q | (hm << 2);
            }, s);
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t i = n8 * 8 + (j & 3) * 2 + h;
                const uint32_t lo8 = (i & 7) < 4 ? w.s8[r].x : w.s8[r].y;
                const uint32_t lo = (lo8 >> (8 * (i & 3) + 4 * (i >> 3))) & 0xF;
                const uint32_t hi = (w.s4[r] >> (8 * (i & 3) + 2 * (i >> 2))) & 3;
                const float dl = h2f(w.d[r]) * (float)((int)(lo | (hi << 4)) - 32);
#pragma unroll
                for (int n = 0; n < NC; n++) {
                    const floatx4 g = xa.gd(n, gi);
                    acc[r][n] += g[3] * (dl * (comb(s, r, n) - 4.0f * g[h]));
                }
            }
        }
      }
    }
};

template <int NC, int R, int TS>
struct Compute<Q8_0, NC, R, TS> {
    // the 32 int8 codes are the weight bytes as they are
    template <class XA>
    __device__ __forceinline__ static void run(const Unit<Q8_0, R> &w, const XA &xa, uint32_t,
                                               float (&acc)[R][NC], const u32x4 *) {
        int s[3][R][NC];
        zero3(s);
        dot_half<NC, R>(xa, 0, 0, [&](int r, int k) { return w.q0[r][k]; }, s);
        dot_half<NC, R>(xa, 0, 1, [&](int r, int k) { return w.q1[r][k]; }, s);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float d = h2f(w.d[r]);
#pragma unroll
            for (int n = 0; n < NC; n++) acc[r][n] += d * (comb(s, r, n) * xa.gd(n, 0)[3]);
        }
    }
};

template <int NC, int R, int TS>
struct Compute<Q4_0, NC, R, TS> {
    // Code dword i: low nibbles are weights 4i.., high nibbles 16 + 4i..;
    // sum((q - 8) X) = sum(q X) - 8 sum(X).
    template <class XA>
    __device__ __forceinline__ static void run(const Unit<Q4_0, R> &w, const XA &xa, uint32_t,
                                               float (&acc)[R][NC], const u32x4 *) {
        int s[3][R][NC];
        zero3(s);
        dot_half<NC, R>(xa, 0, 0, [&](int r, int k) { return w.q[r][k] & 0x0F0F0F0Fu; }, s);
        dot_half<NC, R>(xa, 0, 1, [&](int r, int k) { return (w.q[r][k] >> 4) & 0x0F0F0F0Fu; }, s);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float d = h2f(w.d[r]);
#pragma unroll
            for (int n = 0; n < NC; n++) {
                const floatx4 g = xa.gd(n, 0);
                acc[r][n] += d * ((comb(s, r, n) - 8.0f * g[2]) * g[3]);
            }
        }
    }
};

// IQ4_NL's 16 levels as int8 bytes (IQ4_NL.kvalues, Gemma4Quant.swift:8-11):
// a code dword's four low (or high) nibbles index them with two v_perm and a
// per-byte select on bit 3 (v_perm selector 0x0C gives 0x00, 0x0D 0xFF).
__host__ __device__ constexpr uint32_t iq4_lvb(int i) { return (uint32_t)(uint8_t)iq4nl_level(i); }
__host__ __device__ constexpr uint32_t iq4_lv4(int i) {
    return iq4_lvb(i) | iq4_lvb(i + 1) << 8 | iq4_lvb(i + 2) << 16 | iq4_lvb(i + 3) << 24;
}
struct IQ4Levels {
    __device__ __forceinline__ static uint32_t levels(uint32_t nib) {  // 4 nibbles, one per byte
        constexpr uint32_t T0 = iq4_lv4(0), T1 = iq4_lv4(4), T2 = iq4_lv4(8), T3 = iq4_lv4(12);
        const uint32_t sel = nib & 0x07070707u;
        const uint32_t lo = perm(T1, T0, sel), hi = perm(T3, T2, sel);
        const uint32_t m = perm(0, 0, ((nib >> 3) & 0x01010101u) | 0x0C0C0C0Cu);
        return (hi & m) | (lo & ~m);
    }
};

template <int NC, int R, int TS>
struct Compute<IQ4_NL, NC, R, TS> {
    // as Q4_0, each nibble looked up as its signed level
    template <class XA>
    __device__ __forceinline__ static void run(const Unit<IQ4_NL, R> &w, const XA &xa, uint32_t,
                                               float (&acc)[R][NC], const u32x4 *) {
        int s[3][R][NC];
        zero3(s);
        dot_half<NC, R>(xa, 0, 0,
                        [&](int r, int k) { return IQ4Levels::levels(w.q[r][k] & 0x0F0F0F0Fu); }, s);
        dot_half<NC, R>(xa, 0, 1,
                        [&](int r, int k) { return IQ4Levels::levels((w.q[r][k] >> 4) & 0x0F0F0F0Fu); }, s);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float d = h2f(w.d[r]);
#pragma unroll
            for (int n = 0; n < NC; n++) acc[r][n] += d * (comb(s, r, n) * xa.gd(n, 0)[3]);
        }
    }
};

template <int NC, int R, int TS>
struct Compute<Q2_0, NC, R, TS> {
    // code dword j, field k: bytes (v >> 2k) & 0x03030303 = plane dword
    // 4j + k of the staged order (group j >> 1, chunk half j & 1);
    // sum((code - 1) X) = sum(code X) - sum(X) per group.
    template <class XA>
    __device__ __forceinline__ static void run(const Unit<Q2_0, R> &w, const XA &xa, uint32_t,
                                               float (&acc)[R][NC], const u32x4 *) {
        int s0[3][R][NC], s1[3][R][NC];
        zero3(s0);
        zero3(s1);
#pragma unroll
        for (int j = 0; j < 4; j++)
            dot_half<NC, R>(xa, j >> 1, j & 1,
                            [&](int r, int k) { return (w.q[r][j] >> (2 * k)) & 0x03030303u; },
                            j < 2 ? s0 : s1);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float d = h2f(w.d[r]);
#pragma unroll
            for (int n = 0; n < NC; n++) {
                const floatx4 g0 = xa.gd(n, 0), g1 = xa.gd(n, 1);
                acc[r][n] += d * ((comb(s0, r, n) - g0[2]) * g0[3] + (comb(s1, r, n) - g1[2]) * g1[3]);
            }
        }
    }
};

template <int NC, int R, int TS>
struct Compute<Q5_K, NC, R, TS> {
    // As Q4_K, with the fifth bit of weight l from qh byte l: bit 2g for the
    // low nibbles (sub-block 2g), bit 2g + 1 for the high ones.
    template <class XA>
    __device__ __forceinline__ static void run(const Unit<Q5_K, R> &w, const XA &xa, uint32_t u,
                                               float (&acc)[R][NC], const u32x4 *) {
        const uint32_t g = u & 3;
        int s0[3][R][NC], s1[3][R][NC];
        zero3(s0);
        zero3(s1);
        auto code = [&](int r, int i) { return i < 4 ? w.q0[r][i] : w.q1[r][i - 4]; };
        auto high = [&](int r, int i) { return (i < 4 ? w.h0[r][i] : w.h1[r][i - 4]) >> (2 * g); };
#pragma unroll
        for (int h = 0; h < 2; h++) {
            dot_half<NC, R>(xa, 0, h, [&](int r, int k) {
                const int i = 4 * h + k;
                return (code(r, i) & 0x0F0F0F0Fu) | ((high(r, i) & 0x01010101u) << 4);
            }, s0);
            dot_half<NC, R>(xa, 1, h, [&](int r, int k) {
                const int i = 4 * h + k;
                return ((code(r, i) >> 4) & 0x0F0F0F0Fu) | ((high(r, i) & 0x02020202u) << 3);
            }, s1);
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            uint32_t sc0, mn0, sc1, mn1;
            const uint4 hv = make_uint4(w.hdr[r][0], w.hdr[r][1], w.hdr[r][2], w.hdr[r][3]);
            q4k_scale_min_pair(hv, g, sc0, mn0, sc1, mn1);
            const float d = h2f(w.hdr[r][0] & 0xFFFF), dmin = h2f(w.hdr[r][0] >> 16);
            const float a0 = d * (float)sc0, a1 = d * (float)sc1;
            const float b0 = dmin * (float)mn0, b1 = dmin * (float)mn1;
#pragma unroll
            for (int n = 0; n < NC; n++) {
                const floatx4 g0 = xa.gd(n, 0), g1 = xa.gd(n, 1);
                acc[r][n] += g0[3] * (a0 * comb(s0, r, n) - b0 * g0[2]) + g1[3] * (a1 * comb(s1, r, n) - b1 * g1[2]);
            }
        }
    }
};

template <int NC, int R, int TS>
struct Compute<Q6_K, NC, R, TS> {
    // Unit (n, is): weights l, l + 32, l + 64, l + 96 of half n for
    // l = 16 is .. 16 is + 15 (KQuant.q6K's q1..q4).  Group grp of the four
    // (16 weights, staged group grp >> 1, chunk half grp & 1): the low
    // (grp < 2) or high nibble of ql byte l (grp even) or l + 32 (grp odd),
    // with bits 2 grp, 2 grp + 1 of qh byte l on top, a 6-bit q;
    // sum((q - 32) X) = sum(q X) - 32 sum(X) over the 16, scaled by
    // d * scales[8 n + is + 2 grp].  The unit reads exactly its 48 code bytes.
    template <class XA>
    __device__ __forceinline__ static void run(const Unit<Q6_K, R> &w, const XA &xa, uint32_t u, float (&acc)[R][NC],
                                               const u32x4 *) {
        const uint32_t is = u & 1;
        float sg[4][R][NC];
#pragma unroll
        for (int grp = 0; grp < 4; grp++) {
            int s[3][R][NC];
            zero3(s);
            dot_half<NC, R>(xa, grp >> 1, grp & 1, [&](int r, int k) {
                const uint32_t v = (grp & 1) ? w.qb[r][k] : w.qa[r][k];
                return ((v >> (4 * (grp >> 1))) & 0x0F0F0F0Fu) | (((w.qh[r][k] >> (2 * grp)) & 0x03030303u) << 4);
            }, s);
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int n = 0; n < NC; n++) {
                    const floatx4 gd = xa.gd(n, grp >> 1);
                    sg[grp][r][n] = comb(s, r, n) - 32.0f * ((grp & 1) ? gd[1] : gd[0]);
                }
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float d = h2f(w.d[r]);
            // scale bytes is + 2 grp of the half's 8
            const uint32_t s4 = __builtin_amdgcn_perm(w.sc[r].y, w.sc[r].x, is ? 0x07050301u : 0x06040200u);
            float dg[4];
#pragma unroll
            for (int gq = 0; gq < 4; gq++) dg[gq] = d * (float)(int8_t)((s4 >> (8 * gq)) & 0xFF);
#pragma unroll
            for (int n = 0; n < NC; n++)
                acc[r][n] += xa.gd(n, 0)[3] * (dg[0] * sg[0][r][n] + dg[1] * sg[1][r][n]) +
                             xa.gd(n, 1)[3] * (dg[2] * sg[2][r][n] + dg[3] * sg[3][r][n]);
        }
    }
};

template <int NC, int R, int TS>
struct Compute<IQ4_XS, NC, R, TS> {
    // Two IQ4_NL-shaped sub-blocks (16 code bytes each, one group each) with
    // their own 6-bit scales: dl = d (ls - 32), ls = nibble of scales_l byte
    // g | 2 bits of scales_h << 4.
    template <class XA>
    __device__ __forceinline__ static void run(const Unit<IQ4_XS, R> &w, const XA &xa, uint32_t u,
                                               float (&acc)[R][NC], const u32x4 *) {
        const uint32_t g = u & 3;
        int s0[3][R][NC], s1[3][R][NC];
        zero3(s0);
        zero3(s1);
        dot_half<NC, R>(xa, 0, 0,
                        [&](int r, int k) { return IQ4Levels::levels(w.q0[r][k] & 0x0F0F0F0Fu); }, s0);
        dot_half<NC, R>(xa, 0, 1,
                        [&](int r, int k) { return IQ4Levels::levels((w.q0[r][k] >> 4) & 0x0F0F0F0Fu); }, s0);
        dot_half<NC, R>(xa, 1, 0,
                        [&](int r, int k) { return IQ4Levels::levels(w.q1[r][k] & 0x0F0F0F0Fu); }, s1);
        dot_half<NC, R>(xa, 1, 1,
                        [&](int r, int k) { return IQ4Levels::levels((w.q1[r][k] >> 4) & 0x0F0F0F0Fu); }, s1);
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float d = h2f(w.hdr[r].x & 0xFFFF);
            const uint32_t sh = w.hdr[r].x >> 16, sl = byte_of(w.hdr[r].y, g);
            const float dl0 = d * (float)((int)((sl & 0xF) | (((sh >> (4 * g)) & 3) << 4)) - 32);
            const float dl1 = d * (float)((int)((sl >> 4) | (((sh >> (4 * g + 2)) & 3) << 4)) - 32);
#pragma unroll
            for (int n = 0; n < NC; n++)
                acc[r][n] += dl0 * (comb(s0, r, n) * xa.gd(n, 0)[3]) + dl1 * (comb(s1, r, n) * xa.gd(n, 1)[3]);
        }
    }
};

// Sum over the L lanes of a row slot (every lane of the slot gets it).
template <int L>
__device__ __forceinline__ float slot_sum(float v) {
    static_assert(L == 16, "row slots are 16 lanes");
    v = quad_sum(v);
    v += dpp<DPP_HALF_MIRROR>(v);
    return v + dpp<DPP_MIRROR>(v);
}

// ------------------------------------------------------------- kernel --
// A wavefront is four row slots of L = 16 lanes; each slot owns R consecutive
// rows.  The S parts of a workgroup's wavefronts (S = 1, 2 or 4) share the
// same rows and take every S-th step of K, so that short or few rows still
// give many short wavefronts; their partial sums meet in LDS.  D register
// buffers per lane hold the weights of the wavefront's next D steps.
//
// Dynamic LDS: [IQ2 tables (384 x 16 B)], then NC columns of staged digit
// planes for `cunits` units (a multiple of 64), column stride
// cs = cunits * unit_chunks * 4 uint32, then NC columns of group data
// (cunits * unit_groups float4 each), then the S-way partial sums.
constexpr int GV_L = 16;  // lanes per row slot
constexpr int GV_SLOTS = 4;

// silu(g) * u in fp32 (the reference's silu, LLM/Base/Kernels.swift:3 and
// LLM/metal/Kernels.metal:7: x / (1 + exp(-x))), with the hardware exp and
// reciprocal (each about 1 ulp): a handful of instructions per value, which
// matters because every workgroup stages the whole activation vector.
// Large negative g gives exp = inf, rcp = 0 and silu = -0, as the formula.
__device__ __forceinline__ float silu_mul1(float g, float u) {
    return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}
__device__ __forceinline__ floatx4 silu_mul4(floatx4 g, floatx4 u) {
    return floatx4{silu_mul1(g[0], u[0]), silu_mul1(g[1], u[1]), silu_mul1(g[2], u[2]),
                   silu_mul1(g[3], u[3])};
}

// a[i] = silu(a[i]) * b[i], the FFN glue between gate/up and down
// (silu_mul, LLM/metal/Kernels.metal:3280-3285)
static __global__ __launch_bounds__(256) void silu_mul_kernel(float *__restrict__ a,
                                                       const float *__restrict__ b, uint32_t n) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) a[i] = silu_mul1(a[i], b[i]);
}

// Stages activation slots [0, nslots) of chunk c0 (all NC columns) into LDS
// as digit planes and group data.  SP passes per round: every pass's global
// loads are issued before the first is staged.
// With SILU the activations are silu(X) * X2 (the FFN's gate and up
// outputs), computed here in fp32 before they are staged.
// after_loads() runs once, right after the first round's activation loads
// are issued: the caller issues its weight loads there, behind them, so that
// the staging below waits only for the activations (loads complete in issue
// order) while the weights are in flight.
template <int F, int NC, int L, uint32_t SP, bool SILU, typename AfterLoads>
__device__ __forceinline__ void stage_x(const float *__restrict__ X, const float *__restrict__ X2,
                                        uint32_t K, uint32_t c0,
                                        uint32_t nslots, uint32_t tid, uint32_t nthr, uint32_t *xs,
                                        uint32_t cs, floatx4 *gdp, uint32_t gcs, AfterLoads after_loads) {
    constexpr uint32_t UW = unit_weights<F>(), SL = UW / 8;
    for (uint32_t q0 = 0; q0 < nslots; q0 += SP * nthr) {
        float v[SP][NC][8], v2[SILU ? SP : 1][SILU ? NC : 1][8];
#pragma unroll
        for (uint32_t p = 0; p < SP; p++) {
            const uint32_t q = min(q0 + p * nthr + tid, nslots - 1), u = q / SL;
#pragma unroll
            for (int n = 0; n < NC; n++) {
                const uint64_t xo = (uint64_t)n * K + unit_x_base<F>(c0 + u);
                load_slot<F>(X + xo, q % SL, v[p][n]);
                if constexpr (SILU) load_slot<F>(X2 + xo, q % SL, v2[p][n]);
            }
        }
        if (q0 == 0) {
            __builtin_amdgcn_sched_barrier(0);
            after_loads();
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (uint32_t p = 0; p < SP; p++) {
            const uint32_t q = q0 + p * nthr + tid;
            if constexpr (SILU)
#pragma unroll
                for (int n = 0; n < NC; n++)
#pragma unroll
                    for (int k = 0; k < 8; k++) v[p][n][k] = silu_mul1(v[p][n][k], v2[p][n][k]);
            stage_slot<F, NC, L, SILU>(v[p], q / SL, q % SL, q < nslots, xs, cs, gdp, gcs);
        }
    }
}

// Paired mode (W2 != nullptr; one column, S = 1, no SiLU staging): the
// FFN's gate (W) and up (W2) share x, and the workgroup's first half of row
// slots takes rows of W, the second half the same rows of W2.  The outputs
// are Y = silu(W x) * (W2 x) (the reference's in-place siluMul leaves that
// in its gate buffer) and Y2 = W2 x.
template <int F, int NC, int R, int D, int S, bool SILU>
__device__ __forceinline__ void gemv_body(const uint8_t *__restrict__ W, uint64_t row_bytes, uint32_t K,
                                          uint32_t M, const float *__restrict__ X,
                                          const float *__restrict__ X2, float *__restrict__ Y,
                                          const u32x4 *__restrict__ tab_g, uint32_t cunits,
                                          uint32_t blk, const uint8_t *__restrict__ W2 = nullptr,
                                          float *__restrict__ Y2 = nullptr) {
    constexpr int L = GV_L;
    extern __shared__ u32x4 lds[];
    constexpr uint32_t TAB = gemv_tab_rows<F>();
    u32x4 *tab = lds;
    uint32_t *xs = (uint32_t *)(lds + TAB);
    const uint32_t tid = threadIdx.x, nthr = blockDim.x;
    const uint32_t lane = tid & 63, i = lane % L, slot = lane / L;
    const uint32_t wave = tid >> 6, waves = nthr >> 6;
    const uint32_t part = wave % S, group = wave / S, groups = waves / S;
    if constexpr (TAB > 0)
        for (uint32_t e = tid; e < TAB; e += nthr) tab[e] = tab_g[e];

    // row slot q of the workgroup; paired: q < QH takes W, q >= QH W2
    const bool pair = W2 != nullptr;
    const uint32_t q = group * GV_SLOTS + slot, QH = groups * GV_SLOTS / 2;
    const bool second = pair && q >= QH;
    const uint32_t m0 = pair ? (blk * QH + (second ? q - QH : q)) * R : ((blk * groups + group) * GV_SLOTS + slot) * R;
    const uint8_t *Wq = second ? W2 : W;
    const uint8_t *rows[R];
#pragma unroll
    for (int r = 0; r < R; r++) rows[r] = Wq + (uint64_t)min(m0 + r, M - 1) * row_bytes;
    constexpr uint32_t UW = unit_weights<F>();
    constexpr uint32_t UG = unit_groups<F>();
    const uint32_t units = K / UW, cs = cunits * unit_chunks<F>() * 4, gcs = cunits * UG;
    floatx4 *gdp = (floatx4 *)(xs + NC * cs);
    float *red = (float *)(gdp + NC * gcs);  // [groups][slots][R][NC][S]

    float acc[R][NC];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int n = 0; n < NC; n++) acc[r][n] = 0;

    for (uint32_t c0 = 0; c0 < units; c0 += cunits) {
        const uint32_t cn = min(cunits, units - c0);
        // this wavefront's steps: t = part, part + S, ... of the chunk
        const uint32_t steps = ((cn + L - 1) / L + S - 1 - part) / S, last = cn - 1;
        // The first D steps' weights are requested right behind the
        // activation loads of the staging (stage_x's after_loads), so their
        // latency overlaps the staging and the staging waits only for the
        // activations.  Loads are unconditional (past the end they re-read
        // the chunk's last unit, a cache hit) so that no branch hides a load
        // from the compiler's count of outstanding loads, and the wait before
        // a compute covers only the loads of that buffer.
        Unit<F, R> buf[D];
        auto load_first = [&]() {
#pragma unroll
            for (int j = 0; j < D; j++)
                load_unit<F, R>(rows, c0 + min(i + L * (part + S * j), last), buf[j]);
        };

        // stage units [c0, c0 + cn) of every column as fp16 pairs
        __syncthreads();
        // one thread per 8-value slot; 4 consecutive slots (one 32-weight
        // group) sit in 4 consecutive lanes of a wavefront (nthr % 64 == 0)
        constexpr uint32_t SL = UW / 8;
        const uint32_t nslots = cn * SL;
        constexpr uint32_t SP = NC == 1 ? 4 : NC == 2 ? 2 : 1;
        // (a chunk that one or three passes cover takes that copy: no idle passes)
        if (nslots <= nthr)
            stage_x<F, NC, L, 1, SILU>(X, X2, K, c0, nslots, tid, nthr, xs, cs, gdp, gcs, load_first);
        else if (SP == 4 && nslots <= 3 * nthr)
            stage_x<F, NC, L, (SP == 4 ? 3 : 1), SILU>(X, X2, K, c0, nslots, tid, nthr, xs, cs, gdp, gcs,
                                                       load_first);
        else
            stage_x<F, NC, L, SP, SILU>(X, X2, K, c0, nslots, tid, nthr, xs, cs, gdp, gcs, load_first);
        __syncthreads();
        // stream the wavefront's units u = c0 + i + L (part + S t) through
        // the ring
        uint32_t t = 0;
        for (; t + D < steps; t += D) {
#pragma unroll
            for (int j = 0; j < D; j++) {
                const uint32_t u = i + L * (part + S * (t + j));
                if (u < cn)
                    Compute<F, NC, R>::run(buf[j], XLds{xs + xs_index<F, L>(u, 0), 4 * L, cs, gdp + u * UG, gcs},
                                           c0 + u, acc, TAB > 0 ? tab : tab_g);
                load_unit<F, R>(rows, c0 + min(u + L * S * D, last), buf[j]);
            }
        }
#pragma unroll
        for (int j = 0; j < D; j++) {
            const uint32_t u = i + L * (part + S * (t + j));
            if (u < cn)
                Compute<F, NC, R>::run(buf[j], XLds{xs + xs_index<F, L>(u, 0), 4 * L, cs, gdp + u * UG, gcs},
                                       c0 + u, acc, TAB > 0 ? tab : tab_g);
        }
    }
    // reduce: over the slot's lanes, then (S > 1) over the parts in LDS
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int n = 0; n < NC; n++) acc[r][n] = slot_sum<L>(acc[r][n]);
    if constexpr (S > 1) {
        const uint32_t base = ((group * GV_SLOTS + slot) * R) * NC * S;
        if (i == 0)
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int n = 0; n < NC; n++) red[base + (r * NC + n) * S + part] = acc[r][n];
        __syncthreads();
        if (part != 0) return;
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int n = 0; n < NC; n++) {
                float v = red[base + (r * NC + n) * S];
#pragma unroll
                for (int p = 1; p < S; p++) v += red[base + (r * NC + n) * S + p];
                acc[r][n] = v;
            }
    }
    if constexpr (NC == 1 && S == 1 && !SILU) {
        if (pair) {
            // gate and up values of the workgroup's rows meet in LDS
            if (i == 0)
#pragma unroll
                for (int r = 0; r < R; r++) red[q * R + r] = acc[r][0];
            __syncthreads();
            if (tid < QH * R) {
                const uint32_t m = blk * QH * R + tid;
                const float gv = red[tid], uv = red[QH * R + tid];
                if (m < M) {
                    Y[m] = silu_mul1(gv, uv);
                    Y2[m] = uv;
                }
            }
            return;
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int n = 0; n < NC; n++)
            if (i == 0 && m0 + r < M) Y[(uint64_t)n * M + m0 + r] = acc[r][n];
}


// Up to GV_GROUP matrices of one format and one K in one launch (the
// reference's concurrent dispatch group, MetalEnc.parallel): workgroups
// [end[i-1], end[i]) compute y_i = W_i x_i.
constexpr int GV_GROUP = 4;
struct GemvGroup {
    const uint8_t *W[GV_GROUP];
    const float *X[GV_GROUP];
    const float *X2[GV_GROUP];  // with SILU: x = silu(X) * X2
    float *Y[GV_GROUP];
    uint32_t M[GV_GROUP];
    uint32_t end[GV_GROUP];
    uint32_t n;
    uint32_t pair;  // 1: W[0] (gate) and W[1] (up) paired in each workgroup (gemv_body)
};

template <int F, int NC, int R, int D, int S, bool SILU>
__global__ __launch_bounds__(256) void gemv_kernel(GemvGroup g, uint64_t row_bytes, uint32_t K,
                                                   const u32x4 *__restrict__ tab_g, uint32_t cunits) {
    uint32_t i = 0;
#pragma unroll
    for (int k = 0; k + 1 < GV_GROUP; k++)
        if (k + 1 < (int)g.n && blockIdx.x >= g.end[k]) i = k + 1;
    if constexpr (NC == 1 && S == 1 && !SILU)
        if (g.pair) {
            gemv_body<F, NC, R, D, S, SILU>(g.W[0], row_bytes, K, g.M[0], g.X[0], nullptr, g.Y[0], tab_g, cunits,
                                            blockIdx.x, g.W[1], g.Y[1]);
            return;
        }
    const uint32_t blk = blockIdx.x - (i ? g.end[i - 1] : 0);
    gemv_body<F, NC, R, D, S, SILU>(g.W[i], row_bytes, K, g.M[i], g.X[i], g.X2[i], g.Y[i], tab_g, cunits,
                                    blk);
}

}  // namespace okf
