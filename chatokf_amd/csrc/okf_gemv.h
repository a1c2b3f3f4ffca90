// okf_gemv.h -- decode matvec (N = 1) and narrow matmul (N = 2..5) kernels.
//
// One weight pass serves all NC activation columns (the reference's
// gemv / gemm_nb kernels, LLM/metal/Kernels.metal:1572-1753, :2486-2585).
//
// Layout of the work.  A wavefront is 64 / L row slots of L lanes (L = 16 or
// 64); each slot owns R consecutive rows.  A row is cut into units (Q4_K: one 32-byte code
// group = sub-blocks 2g and 2g+1; IQ2_XXS: two sub-blocks; Q8_0: one block;
// Q2_0: half a block); lane i of a slot walks units
// i, i + L, ... so the lanes of a slot read contiguous bytes of the row with
// 16-byte loads, and the weights of the next D steps are in flight while a
// step is computed.
//
// Arithmetic.  The activations are staged once per workgroup into LDS as fp16,
// permuted so that each packed pair of weights meets its pair of activations,
// and every multiply-add is a v_dot2_f32_f16 (two fp16 products, fp32
// accumulate).  Quantized integers become exact fp16 numbers with the
// magic-exponent trick: 0x6400 | q is the fp16 value 1024 + q, and the
// 1024 * sum(x) bias is removed per unit from an fp32 sum of the same fp16
// activations.  Block scales are applied in fp32 per sub-block, in the
// reference's factored form ((d*sc)*sum(q*x) - (dmin*m)*sum(x) for Q4_K,
// d*sum((code-1)*x) for Q2_0, d*sum(q*x) for Q8_0, db*sum(g*s*x) for
// IQ2_XXS).  The fp16 rounding of x is the only approximation beyond fp32
// summation order (relative error ~2e-4 of the output scale).
#pragma once
#include "okf_common.h"
#include "okf_decode.h"

namespace okf {


// Weights per unit: 64, except Q8_0 whose unit is one 32-weight block (so
// any K that is a whole number of blocks works).
template <int F>
__host__ __device__ constexpr uint32_t unit_weights() {
    return (F == Q8_0 || F == Q4_0 || F == IQ4_NL || grid_fmt(F)) ? 32 : 64;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, a), __builtin_bit_cast(half2v, b), c,
                                  false);
}

// v_perm_b32: byte k of the result is byte sel_k of the 8-byte value {hi, lo}.
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// v_bfi_b32: (mask & a) | (~mask & b).  With b = MAGIC2 this drops a's masked
// bits into the mantissa of two fp16 1024.0: bits 0..3 give 1024 + q, bits
// 4..7 give 1024 + 16 q (the factor 16 is folded into the scale).
// (The compiler splits the constant-operand form into v_and + v_or, so the
// single instruction is written out; the mask lives in an SGPR, b in a VGPR.)
__device__ __forceinline__ uint32_t bfi(uint32_t mask, uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "s"(mask), "v"(a), "v"(b));
    return r;
}

constexpr uint32_t MAGIC2 = 0x64006400u;  // two fp16 1024.0
constexpr uint32_t ONES2 = 0x3C003C00u;   // two fp16 1.0

// ---------------------------------------------------------------- units --
// Raw bytes of one unit for R rows (native vector types keep them in VGPRs).
// The grid formats (grid_fmt) keep only the row: their compute decodes a
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
        } else if constexpr (grid_fmt(F)) {
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

// Staging order.  Slot s of a unit holds 4 packed pairs (8 fp16 values) read
// by one 16-byte LDS load; h[0..7] below are those values in memory order,
// built from two float4s A and B of the activations.
//  Q4_K: code dword i (bytes 4i..4i+3) gives low-nibble pairs (4i, 4i+2),
//        (4i+1, 4i+3); so slot s (weights 8s..8s+7 of the unit, the first
//        four slots low nibbles, the last four high nibbles) is
//        A = x[8s..], B = x[8s+4..] as A0 A2 A1 A3 B0 B2 B1 B3.
//  Q2_0: code dword j (16 codes, weights 16j..) gives pairs (c, c + 8); slot
//        s = 2j + h is A = x[16j + 4h..], B = x[16j + 8 + 4h..] as
//        A0 B0 A1 B1 A2 B2 A3 B3.
//  Q4_0: as Q4_K with 16 code bytes: slots 0, 1 are the low nibbles
//        (weights 0..15), slots 2, 3 the high ones (16..31).
//  Q5_K: as Q4_K (32 code bytes of one group: low nibbles, then high).
//  Q6_K: 8 weights 16 is + 32 grp + 8 i2 .. of the half per slot 2 grp + i2,
//        packed as Q4_K's (code dword i gives pairs (4i, 4i+2), (4i+1, 4i+3)).
//  Q8_0, IQ2_XXS, IQ4_NL, IQ4_XS: natural order, A = x[8s..], B = x[8s+4..].
// Index in x of the first weight of unit u (a row's units in order).  The
// Q6_K unit (half n, is) of superblock u / 4 holds weights 16 is + e +
// {0, 32, 64, 96} of its half (e < 16), so its slots start 16 is into the
// half; every other unit is UW contiguous weights.
template <int F>
__device__ __forceinline__ uint64_t unit_x_base(uint32_t u) {
    if constexpr (F == Q6_K) return (uint64_t)(u >> 1) * 128 + (u & 1) * 16;
    else return (uint64_t)u * unit_weights<F>();
}

template <int F>
__device__ __forceinline__ uint32_t slot_first(uint32_t s, uint32_t &second) {
    if constexpr (F == Q6_K) {
        // slot s = 2 grp + i2: weights 32 grp + 8 i2 .. past unit_x_base
        const uint32_t base = 32 * (s >> 1) + 8 * (s & 1);
        second = base + 4;
        return base;
    } else if constexpr (F == Q2_0) {
        const uint32_t base = 16 * (s >> 1) + 4 * (s & 1);
        second = base + 8;
        return base;
    } else {
        second = 8 * s + 4;
        return 8 * s;
    }
}

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    const half2v h = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, h);
}

template <int F>
__device__ __forceinline__ u32x4 slot_pack(floatx4 A, floatx4 B) {
    if constexpr (F == Q4_K || F == Q4_0 || F == Q5_K || F == Q6_K)
        return u32x4{pack_h2(A[0], A[2]), pack_h2(A[1], A[3]), pack_h2(B[0], B[2]),
                     pack_h2(B[1], B[3])};
    else if constexpr (F == Q2_0)
        return u32x4{pack_h2(A[0], B[0]), pack_h2(A[1], B[1]), pack_h2(A[2], B[2]),
                     pack_h2(A[3], B[3])};
    else
        return u32x4{pack_h2(A[0], A[1]), pack_h2(A[2], A[3]), pack_h2(B[0], B[1]),
                     pack_h2(B[2], B[3])};
}

// fp32 sum of the 8 fp16 values of a packed slot
__device__ __forceinline__ float slot_total(u32x4 v) {
    float t = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) t = dot2(v[e], ONES2, t);
    return t;
}

// The per-32 sum staged beside the packed activations: sum(x) for every
// format but Q2_0.  Q2_0 decodes the pair at position c of a code dword
// (codes c and c + 8) as fp16 base_c + code, base_c = 2^(10 - 2c) for
// c <= 4 (the code bits inserted in place by one v_bfi into an fp16 2^(10-2c)
// whose mantissa bit 2c is worth 1) and 1024 for c >= 5 (shifted down
// first); then sum((code - 1) x) = sum((base + code) x) - sum((base + 1) x),
// and the second sum is staged here.  Slot 2j + h holds the pairs at
// positions c = 4h + e.  Every base + 1 (1025, 257, 65, 17, 5) is exact in
// fp16, so each product is exact in fp32 as in slot_total.
template <int F>
__device__ __forceinline__ float slot_bias(u32x4 v, uint32_t sidx) {
    if constexpr (F == Q2_0) {
        constexpr uint32_t B1025 = 0x64016401u, B257 = 0x5C045C04u, B65 = 0x54105410u, B17 = 0x4C404C40u,
                           B5 = 0x45004500u;
        const bool h = sidx & 1;
        float t = dot2(v[0], h ? B5 : B1025, 0.0f);
        t = dot2(v[1], h ? B1025 : B257, t);
        t = dot2(v[2], h ? B1025 : B65, t);
        return dot2(v[3], h ? B1025 : B17, t);
    } else {
        return slot_total(v);
    }
}

// LDS layout of the staged activations of one column: units in groups of L
// (one per lane of a row slot); within a group, the unit's pairs as slots of
// 4 pairs, each slot [L lanes][4 pairs] so a row slot's lanes read contiguous
// bytes.  Index in uint32 (one pair).
template <int F, int L>
__device__ __forceinline__ uint32_t xs_index(uint32_t u, uint32_t p) {
    constexpr uint32_t SL = unit_weights<F>() / 8;  // slots per unit
    const uint32_t t = u / L, i = u % L;
    return ((t * SL + (p >> 2)) * L + i) * 4 + (p & 3);
}

// ------------------------------------------------------------- compute --
// acc[r][n] += unit contribution; xp = this lane's pairs of column 0 in
// LDS (slot s at xp[s * 64]), cs = uint32 stride between columns.
template <int F, int NC, int R, int TS = 1>
struct Compute {
    // The grid formats (IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S, IQ1_M): the
    // 32-weight sub-block is decoded to fp32 with the bit-exact decoder
    // (grid tables from device memory, tab) and multiplied into the staged
    // fp16 activations (natural order) in fp32.
    static_assert(grid_fmt(F), "no matvec compute for this format");
    __device__ __forceinline__ static void run(const Unit<F, R> &w, const uint32_t *xp, uint32_t ss, uint32_t cs,
                                               const float *, uint32_t, uint32_t u, float (&acc)[R][NC],
                                               const u32x4 *tab) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            float wv[32];
            decode_unit<F>(w.row[r], u, wv, nullptr, (const uint8_t *)tab);
#pragma unroll
            for (int s = 0; s < 4; s++) {
#pragma unroll
                for (int n = 0; n < NC; n++) {
                    const u32x4 xv = *(const u32x4 *)(xp + n * cs + s * ss);
                    float a = 0;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        // (the element is copied out first: a bit_cast of a vector
                        // element expression reads the vector's first element)
                        const uint32_t xe = xv[e];
                        a += wv[8 * s + 2 * e] * h2f(xe & 0xFFFF) + wv[8 * s + 2 * e + 1] * h2f(xe >> 16);
                    }
                    acc[r][n] += a;
                }
            }
        }
    }
};

template <int NC, int R, int TS>
struct Compute<Q4_K, NC, R, TS> {
    // xsum: this unit's two 32-weight sums of the staged fp16 x per column
    // (low-nibble half, high-nibble half), columns xcs floats apart.
    __device__ __forceinline__ static void run(const Unit<Q4_K, R> &w, const uint32_t *xp, uint32_t ss, uint32_t cs,
                                               const float *xsum, uint32_t xcs, uint32_t u,
                                               float (&acc)[R][NC], const u32x4 *) {
        const uint32_t g = u & 3;
        float slo[R][NC], shi[R][NC];
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int n = 0; n < NC; n++) slo[r][n] = shi[r][n] = 0;
#pragma unroll
        for (int s = 0; s < 4; s++) {  // code dwords 2s, 2s + 1
            u32x4 xl[NC], xh[NC];
#pragma unroll
            for (int n = 0; n < NC; n++) {
                xl[n] = *(const u32x4 *)(xp + n * cs + s * ss);
                xh[n] = *(const u32x4 *)(xp + n * cs + (4 + s) * ss);
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const uint32_t v = (2 * s + h < 4) ? w.q0[r][2 * s + h] : w.q1[r][2 * s + h - 4];
                    const uint32_t v8 = v >> 8;
                    // low nibbles of bytes (0, 2) and (1, 3): 1024 + q
                    const uint32_t l02 = bfi(0x000F000Fu, v, MAGIC2);
                    const uint32_t l13 = bfi(0x000F000Fu, v8, MAGIC2);
                    // high nibbles: 1024 + 16 q
                    const uint32_t h02 = bfi(0x00F000F0u, v, MAGIC2);
                    const uint32_t h13 = bfi(0x00F000F0u, v8, MAGIC2);
#pragma unroll
                    for (int n = 0; n < NC; n++) {
                        slo[r][n] = dot2(l02, xl[n][2 * h], slo[r][n]);
                        slo[r][n] = dot2(l13, xl[n][2 * h + 1], slo[r][n]);
                        shi[r][n] = dot2(h02, xh[n][2 * h], shi[r][n]);
                        shi[r][n] = dot2(h13, xh[n][2 * h + 1], shi[r][n]);
                    }
                }
            }
        }
        float xlo[NC], xhi[NC];
#pragma unroll
        for (int n = 0; n < NC; n++) {
            const float2 t = *(const float2 *)(xsum + n * xcs);
            xlo[n] = t.x;
            xhi[n] = t.y;
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            uint32_t sc0, mn0, sc1, mn1;
            const uint4 hv = make_uint4(w.hdr[r][0], w.hdr[r][1], w.hdr[r][2], w.hdr[r][3]);
            q4k_scale_min_pair(hv, g, sc0, mn0, sc1, mn1);
            const float d = h2f(w.hdr[r][0] & 0xFFFF), dmin = h2f(w.hdr[r][0] >> 16);
            const float a0 = d * (float)sc0, a1 = d * (float)sc1;
            // bias: sum((1024 + q) x) = sum(q x) + 1024 sum(x); the high
            // nibbles carry an extra factor 16
            const float b0 = 1024.0f * a0 + dmin * (float)mn0;
            const float b1 = 64.0f * a1 + dmin * (float)mn1;
            const float a1s = 0.0625f * a1;
#pragma unroll
            for (int n = 0; n < NC; n++)
                acc[r][n] += (a0 * slo[r][n] + a1s * shi[r][n]) - (b0 * xlo[n] + b1 * xhi[n]);
        }
    }
};

template <int NC, int R, int TS>
struct Compute<IQ2_XXS, NC, R, TS> {
    // tab: [0, 256) fp16 grid entries (8 halves), [256, 384) sign masks
    // (fp16 sign bits of the 8 weights, the eighth from the parity rule);
    // entry e at tab[e * TS] (TS = 16: the replicated, conflict-free layout
    // of gemv_wide_kernel, tab offset by the lane's copy).
    __device__ __forceinline__ static void run(const Unit<IQ2_XXS, R> &w, const uint32_t *xp, uint32_t ss,
                                               uint32_t cs, const float *, uint32_t, uint32_t,
                                               float (&acc)[R][NC], const u32x4 *tab) {
#pragma unroll
        for (int sb = 0; sb < 2; sb++) {  // the unit's two sub-blocks
            float s[R][NC];
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int n = 0; n < NC; n++) s[r][n] = 0;
#pragma unroll
            for (int l = 0; l < 4; l++) {  // 8-weight groups
                u32x4 xv[NC];
#pragma unroll
                for (int n = 0; n < NC; n++) {
                    // pairs 16 sb + 4 l .. +4 = slot 4 sb + l
                    xv[n] = *(const u32x4 *)(xp + n * cs + (4 * sb + l) * ss);
                }
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const uint32_t a0 = w.a[r][2 * sb], a1 = w.a[r][2 * sb + 1];
                    const u32x4 gv = tab[((a0 >> (8 * l)) & 0xFF) * TS];
                    const u32x4 sg = tab[(256 + ((a1 >> (7 * l)) & 127)) * TS];
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const uint32_t wv = gv[e] ^ sg[e];
#pragma unroll
                        for (int n = 0; n < NC; n++) s[r][n] = dot2(wv, xv[n][e], s[r][n]);
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t a1 = w.a[r][2 * sb + 1];
                const float db = h2f(w.d[r]) * (0.5f + (float)(a1 >> 28)) * 0.25f;
#pragma unroll
                for (int n = 0; n < NC; n++) acc[r][n] += db * s[r][n];
            }
        }
    }
};

template <int NC, int R, int TS>
struct Compute<Q8_0, NC, R, TS> {
    // Code byte j is byte j & 3 of code dword j >> 2; XOR 0x80 turns int8 q
    // into q + 128, so the fp16 0x64 | (q + 128) is 1152 + q.
    __device__ __forceinline__ static void run(const Unit<Q8_0, R> &w, const uint32_t *xp, uint32_t ss, uint32_t cs,
                                               const float *xsp, uint32_t xcs, uint32_t,
                                               float (&acc)[R][NC], const u32x4 *) {
        float xsum[NC], s[R][NC];
#pragma unroll
        for (int n = 0; n < NC; n++) xsum[n] = xsp[n * xcs];
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int n = 0; n < NC; n++) s[r][n] = 0;
#pragma unroll
        for (int sl = 0; sl < 4; sl++) {  // pairs 4 sl .. 4 sl + 3 = code dwords 2 sl, 2 sl + 1
            u32x4 xv[NC];
#pragma unroll
            for (int n = 0; n < NC; n++) {
                xv[n] = *(const u32x4 *)(xp + n * cs + sl * ss);
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int dwi = 2 * sl + (e >> 1);
                    const uint32_t dw = (dwi < 4 ? w.q0[r][dwi] : w.q1[r][dwi - 4]) ^ 0x80808080u;
                    // selector bytes 0..3 address dw, 4 addresses 0x64
                    const uint32_t hv = perm(0x64646464u, dw, (e & 1) ? 0x04030402u : 0x04010400u);
#pragma unroll
                    for (int n = 0; n < NC; n++) s[r][n] = dot2(hv, xv[n][e], s[r][n]);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float d = h2f(w.d[r]);
#pragma unroll
            for (int n = 0; n < NC; n++) acc[r][n] += d * (s[r][n] - 1152.0f * xsum[n]);
        }
    }
};

template <int NC, int R, int TS>
struct Compute<Q4_0, NC, R, TS> {
    // Code dword i (bytes 4i..4i+3): low nibbles are weights 4i..4i+3, high
    // nibbles 16 + 4i..; each becomes fp16 1024 + q by v_bfi (the high ones
    // shifted down first), so sum((q - 8) x) = sum((1024 + q) x) - 1032 sum(x).
    __device__ __forceinline__ static void run(const Unit<Q4_0, R> &w, const uint32_t *xp, uint32_t ss, uint32_t cs,
                                               const float *xsp, uint32_t xcs, uint32_t,
                                               float (&acc)[R][NC], const u32x4 *) {
        float xsum[NC], s[R][NC];
#pragma unroll
        for (int n = 0; n < NC; n++) xsum[n] = xsp[n * xcs];
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int n = 0; n < NC; n++) s[r][n] = 0;
#pragma unroll
        for (int sl = 0; sl < 2; sl++) {  // code dwords 2 sl, 2 sl + 1
            u32x4 xl[NC], xh[NC];
#pragma unroll
            for (int n = 0; n < NC; n++) {
                xl[n] = *(const u32x4 *)(xp + n * cs + sl * ss);
                xh[n] = *(const u32x4 *)(xp + n * cs + (2 + sl) * ss);
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const uint32_t v = w.q[r][2 * sl + h], v4 = v >> 4;
                    const uint32_t l02 = bfi(0x000F000Fu, v, MAGIC2);
                    const uint32_t l13 = bfi(0x000F000Fu, v >> 8, MAGIC2);
                    const uint32_t h02 = bfi(0x000F000Fu, v4, MAGIC2);
                    const uint32_t h13 = bfi(0x000F000Fu, v4 >> 8, MAGIC2);
#pragma unroll
                    for (int n = 0; n < NC; n++) {
                        s[r][n] = dot2(l02, xl[n][2 * h], s[r][n]);
                        s[r][n] = dot2(l13, xl[n][2 * h + 1], s[r][n]);
                        s[r][n] = dot2(h02, xh[n][2 * h], s[r][n]);
                        s[r][n] = dot2(h13, xh[n][2 * h + 1], s[r][n]);
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float d = h2f(w.d[r]);
#pragma unroll
            for (int n = 0; n < NC; n++) acc[r][n] += d * (s[r][n] - 1032.0f * xsum[n]);
        }
    }
};

template <int NC, int R, int TS>
struct Compute<IQ4_NL, NC, R, TS> {
    // The 16 levels plus 128 as bytes: entries 0..7 and 8..15.  A code dword's
    // four low (or high) nibbles index them with two v_perm and a per-byte
    // select on bit 3 (v_perm selector 0x0C gives 0x00, 0x0D gives 0xFF);
    // v_perm then puts each byte under 0x64, fp16 1024 + (level + 128), so
    // sum(level x) = sum((1152 + level) x) - 1152 sum(x).
    static constexpr uint32_t lvb(int i) { return (uint32_t)(uint8_t)(iq4nl_level(i) + 128); }
    static constexpr uint32_t T0 = lvb(0) | lvb(1) << 8 | lvb(2) << 16 | lvb(3) << 24;
    static constexpr uint32_t T1 = lvb(4) | lvb(5) << 8 | lvb(6) << 16 | lvb(7) << 24;
    static constexpr uint32_t T2 = lvb(8) | lvb(9) << 8 | lvb(10) << 16 | lvb(11) << 24;
    static constexpr uint32_t T3 = lvb(12) | lvb(13) << 8 | lvb(14) << 16 | lvb(15) << 24;
    __device__ __forceinline__ static uint32_t levels(uint32_t nib) {  // 4 nibbles, one per byte
        const uint32_t sel = nib & 0x07070707u;
        const uint32_t lo = perm(T1, T0, sel), hi = perm(T3, T2, sel);
        const uint32_t m = perm(0, 0, ((nib >> 3) & 0x01010101u) | 0x0C0C0C0Cu);
        return (hi & m) | (lo & ~m);
    }
    __device__ __forceinline__ static void run(const Unit<IQ4_NL, R> &w, const uint32_t *xp, uint32_t ss, uint32_t cs,
                                               const float *xsp, uint32_t xcs, uint32_t,
                                               float (&acc)[R][NC], const u32x4 *) {
        float xsum[NC], s[R][NC];
#pragma unroll
        for (int n = 0; n < NC; n++) xsum[n] = xsp[n * xcs];
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int n = 0; n < NC; n++) s[r][n] = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {  // code dword i: weights 4i.. (low), 16 + 4i.. (high)
            u32x4 xl[NC], xh[NC];
#pragma unroll
            for (int n = 0; n < NC; n++) {
                xl[n] = *(const u32x4 *)(xp + n * cs + (i >> 1) * ss);
                xh[n] = *(const u32x4 *)(xp + n * cs + (2 + (i >> 1)) * ss);
            }
            const int e = 2 * (i & 1);
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t v = w.q[r][i];
                const uint32_t bl = levels(v & 0x0F0F0F0Fu), bh = levels((v >> 4) & 0x0F0F0F0Fu);
                const uint32_t l01 = perm(0x64646464u, bl, 0x04010400u), l23 = perm(0x64646464u, bl, 0x04030402u);
                const uint32_t h01 = perm(0x64646464u, bh, 0x04010400u), h23 = perm(0x64646464u, bh, 0x04030402u);
#pragma unroll
                for (int n = 0; n < NC; n++) {
                    s[r][n] = dot2(l01, xl[n][e], s[r][n]);
                    s[r][n] = dot2(l23, xl[n][e + 1], s[r][n]);
                    s[r][n] = dot2(h01, xh[n][e], s[r][n]);
                    s[r][n] = dot2(h23, xh[n][e + 1], s[r][n]);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float d = h2f(w.d[r]);
#pragma unroll
            for (int n = 0; n < NC; n++) acc[r][n] += d * (s[r][n] - 1152.0f * xsum[n]);
        }
    }
};

template <int NC, int R, int TS>
struct Compute<Q2_0, NC, R, TS> {
    // Pair position c of code dword j (codes c and c + 8, weights
    // 16j + c, 16j + c + 8) becomes fp16 base_c + code: for c <= 4 one v_bfi
    // of the code bits, in place, into 2^(10 - 2c); for c >= 5 a shift, then
    // v_bfi into 1024.  xsp holds the staged sum((base + 1) x) (slot_bias),
    // so sum((code - 1) x) = s - xsp.  Two accumulators (even and odd c)
    // halve the dot2 dependency chain.
    __device__ __forceinline__ static void run(const Unit<Q2_0, R> &w, const uint32_t *xp, uint32_t ss, uint32_t cs,
                                               const float *xsp, uint32_t xcs, uint32_t,
                                               float (&acc)[R][NC], const u32x4 *) {
        constexpr uint32_t MAGIC_C[5] = {0x64006400u, 0x5C005C00u, 0x54005400u, 0x4C004C00u, 0x44004400u};
        float xb[NC], s[R][NC], s2[R][NC];
#pragma unroll
        for (int n = 0; n < NC; n++) {
            const float2 t = *(const float2 *)(xsp + n * xcs);
            xb[n] = t.x + t.y;
        }
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int n = 0; n < NC; n++) s[r][n] = s2[r][n] = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {  // code dword j: pairs 8j .. 8j + 7 = slots 2j, 2j + 1
            u32x4 xa[NC], xc[NC];
#pragma unroll
            for (int n = 0; n < NC; n++) {
                xa[n] = *(const u32x4 *)(xp + n * cs + (2 * j) * ss);
                xc[n] = *(const u32x4 *)(xp + n * cs + (2 * j + 1) * ss);
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t v = w.q[r][j];
#pragma unroll
                for (int c = 0; c < 8; c++) {
                    const uint32_t hv = c <= 4 ? bfi(0x00030003u << (2 * c), v, MAGIC_C[c < 5 ? c : 0])
                                               : bfi(0x00030003u, v >> (2 * c), MAGIC2);
#pragma unroll
                    for (int n = 0; n < NC; n++) {
                        const uint32_t xv = c < 4 ? xa[n][c] : xc[n][c - 4];
                        if (c & 1) s2[r][n] = dot2(hv, xv, s2[r][n]);
                        else s[r][n] = dot2(hv, xv, s[r][n]);
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float d = h2f(w.d[r]);
#pragma unroll
            for (int n = 0; n < NC; n++) acc[r][n] += d * ((s[r][n] + s2[r][n]) - xb[n]);
        }
    }
};

template <int NC, int R, int TS>
struct Compute<Q5_K, NC, R, TS> {
    // As Q4_K, with the fifth bit of weight l from qh byte l: bit 2g for the
    // low nibbles (sub-block 2g), bit 2g + 1 for the high ones.  The 5-bit
    // values become bytes, then fp16 1024 + q by v_bfi, so
    // sum(q x) = sum((1024 + q) x) - 1024 sum(x).
    __device__ __forceinline__ static void run(const Unit<Q5_K, R> &w, const uint32_t *xp, uint32_t ss, uint32_t cs,
                                               const float *xsum, uint32_t xcs, uint32_t u,
                                               float (&acc)[R][NC], const u32x4 *) {
        const uint32_t g = u & 3;
        float slo[R][NC], shi[R][NC];
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int n = 0; n < NC; n++) slo[r][n] = shi[r][n] = 0;
#pragma unroll
        for (int s = 0; s < 4; s++) {  // code dwords 2s, 2s + 1
            u32x4 xl[NC], xh[NC];
#pragma unroll
            for (int n = 0; n < NC; n++) {
                xl[n] = *(const u32x4 *)(xp + n * cs + s * ss);
                xh[n] = *(const u32x4 *)(xp + n * cs + (4 + s) * ss);
            }
#pragma unroll
            for (int r = 0; r < R; r++) {
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const int i = 2 * s + h;
                    const uint32_t v = i < 4 ? w.q0[r][i] : w.q1[r][i - 4];
                    const uint32_t hq = (i < 4 ? w.h0[r][i] : w.h1[r][i - 4]) >> (2 * g);
                    const uint32_t lo = (v & 0x0F0F0F0Fu) | ((hq & 0x01010101u) << 4);
                    const uint32_t hi = ((v >> 4) & 0x0F0F0F0Fu) | ((hq & 0x02020202u) << 3);
                    const uint32_t l02 = bfi(0x001F001Fu, lo, MAGIC2), l13 = bfi(0x001F001Fu, lo >> 8, MAGIC2);
                    const uint32_t h02 = bfi(0x001F001Fu, hi, MAGIC2), h13 = bfi(0x001F001Fu, hi >> 8, MAGIC2);
#pragma unroll
                    for (int n = 0; n < NC; n++) {
                        slo[r][n] = dot2(l02, xl[n][2 * h], slo[r][n]);
                        slo[r][n] = dot2(l13, xl[n][2 * h + 1], slo[r][n]);
                        shi[r][n] = dot2(h02, xh[n][2 * h], shi[r][n]);
                        shi[r][n] = dot2(h13, xh[n][2 * h + 1], shi[r][n]);
                    }
                }
            }
        }
        float xlo[NC], xhi[NC];
#pragma unroll
        for (int n = 0; n < NC; n++) {
            const float2 t = *(const float2 *)(xsum + n * xcs);
            xlo[n] = t.x;
            xhi[n] = t.y;
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            uint32_t sc0, mn0, sc1, mn1;
            const uint4 hv = make_uint4(w.hdr[r][0], w.hdr[r][1], w.hdr[r][2], w.hdr[r][3]);
            q4k_scale_min_pair(hv, g, sc0, mn0, sc1, mn1);
            const float d = h2f(w.hdr[r][0] & 0xFFFF), dmin = h2f(w.hdr[r][0] >> 16);
            const float a0 = d * (float)sc0, a1 = d * (float)sc1;
            const float b0 = 1024.0f * a0 + dmin * (float)mn0, b1 = 1024.0f * a1 + dmin * (float)mn1;
#pragma unroll
            for (int n = 0; n < NC; n++)
                acc[r][n] += (a0 * slo[r][n] + a1 * shi[r][n]) - (b0 * xlo[n] + b1 * xhi[n]);
        }
    }
};

template <int NC, int R, int TS>
struct Compute<Q6_K, NC, R, TS> {
    // Unit (n, is): weights l, l + 32, l + 64, l + 96 of half n for
    // l = 16 is .. 16 is + 15 (KQuant.q6K's q1..q4).  Group grp of the four:
    // the low (grp < 2) or high nibble of ql byte l (grp even) or l + 32
    // (grp odd), with bits 2 grp, 2 grp + 1 of qh byte l on top.  v_bfi
    // makes fp16 1024 + q, one packed fp16 add makes it q - 32 (exact), and
    // each group takes its int8 scale: scales[8 n + is + 2 grp].  The unit
    // reads exactly its 48 code bytes.
    __device__ __forceinline__ static void run(const Unit<Q6_K, R> &w, const uint32_t *xp, uint32_t ss, uint32_t cs,
                                               const float *, uint32_t, uint32_t u, float (&acc)[R][NC],
                                               const u32x4 *) {
        const uint32_t is = u & 1;
        const half2v bias = {(_Float16)-1056.0f, (_Float16)-1056.0f};
        float s[4][R][NC];
#pragma unroll
        for (int g = 0; g < 4; g++)
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int n = 0; n < NC; n++) s[g][r][n] = 0;
#pragma unroll
        for (int sl = 0; sl < 8; sl++) {  // slot 2 grp + i2: code dwords 2 i2, 2 i2 + 1 of group grp
            const int grp = sl >> 1, i2 = sl & 1;
            u32x4 xv[NC];
#pragma unroll
            for (int n = 0; n < NC; n++) xv[n] = *(const u32x4 *)(xp + n * cs + sl * ss);
#pragma unroll
            for (int r = 0; r < R; r++) {
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const int i = 2 * i2 + h;
                    const uint32_t v = (grp & 1) ? w.qb[r][i] : w.qa[r][i];
                    const uint32_t q = ((v >> (4 * (grp >> 1))) & 0x0F0F0F0Fu) |
                                       (((w.qh[r][i] >> (2 * grp)) & 0x03030303u) << 4);
                    const uint32_t p02 = __builtin_bit_cast(
                        uint32_t, __builtin_bit_cast(half2v, bfi(0x003F003Fu, q, MAGIC2)) + bias);
                    const uint32_t p13 = __builtin_bit_cast(
                        uint32_t, __builtin_bit_cast(half2v, bfi(0x003F003Fu, q >> 8, MAGIC2)) + bias);
#pragma unroll
                    for (int n = 0; n < NC; n++) {
                        s[grp][r][n] = dot2(p02, xv[n][2 * h], s[grp][r][n]);
                        s[grp][r][n] = dot2(p13, xv[n][2 * h + 1], s[grp][r][n]);
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float d = h2f(w.d[r]);
            // scale bytes is + 2 grp of the half's 8
            const uint32_t s4 = __builtin_amdgcn_perm(w.sc[r].y, w.sc[r].x, is ? 0x07050301u : 0x06040200u);
            float dg[4];
#pragma unroll
            for (int g = 0; g < 4; g++) dg[g] = d * (float)(int8_t)((s4 >> (8 * g)) & 0xFF);
#pragma unroll
            for (int n = 0; n < NC; n++)
                acc[r][n] += dg[0] * s[0][r][n] + dg[1] * s[1][r][n] + dg[2] * s[2][r][n] + dg[3] * s[3][r][n];
        }
    }
};

template <int NC, int R, int TS>
struct Compute<IQ4_XS, NC, R, TS> {
    // Two IQ4_NL-shaped sub-blocks (16 code bytes each) with their own
    // 6-bit scales: dl = d (ls - 32), ls = nibble of scales_l byte g |
    // 2 bits of scales_h << 4.
    __device__ __forceinline__ static void run(const Unit<IQ4_XS, R> &w, const uint32_t *xp, uint32_t ss, uint32_t cs,
                                               const float *xsp, uint32_t xcs, uint32_t u,
                                               float (&acc)[R][NC], const u32x4 *) {
        const uint32_t g = u & 3;
        float xsum[2][NC], s[2][R][NC];
#pragma unroll
        for (int n = 0; n < NC; n++) {
            const float2 t = *(const float2 *)(xsp + n * xcs);
            xsum[0][n] = t.x;
            xsum[1][n] = t.y;
        }
#pragma unroll
        for (int sb = 0; sb < 2; sb++)
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int n = 0; n < NC; n++) s[sb][r][n] = 0;
#pragma unroll
        for (int sb = 0; sb < 2; sb++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {  // code dword i: weights 4i.. (low), 16 + 4i.. (high)
                u32x4 xl[NC], xh[NC];
#pragma unroll
                for (int n = 0; n < NC; n++) {
                    xl[n] = *(const u32x4 *)(xp + n * cs + (4 * sb + (i >> 1)) * ss);
                    xh[n] = *(const u32x4 *)(xp + n * cs + (4 * sb + 2 + (i >> 1)) * ss);
                }
                const int e = 2 * (i & 1);
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const uint32_t v = sb == 0 ? w.q0[r][i] : w.q1[r][i];
                    const uint32_t bl = Compute<IQ4_NL, NC, R, TS>::levels(v & 0x0F0F0F0Fu);
                    const uint32_t bh = Compute<IQ4_NL, NC, R, TS>::levels((v >> 4) & 0x0F0F0F0Fu);
                    const uint32_t l01 = perm(0x64646464u, bl, 0x04010400u), l23 = perm(0x64646464u, bl, 0x04030402u);
                    const uint32_t h01 = perm(0x64646464u, bh, 0x04010400u), h23 = perm(0x64646464u, bh, 0x04030402u);
#pragma unroll
                    for (int n = 0; n < NC; n++) {
                        s[sb][r][n] = dot2(l01, xl[n][e], s[sb][r][n]);
                        s[sb][r][n] = dot2(l23, xl[n][e + 1], s[sb][r][n]);
                        s[sb][r][n] = dot2(h01, xh[n][e], s[sb][r][n]);
                        s[sb][r][n] = dot2(h23, xh[n][e + 1], s[sb][r][n]);
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float d = h2f(w.hdr[r].x & 0xFFFF);
            const uint32_t sh = w.hdr[r].x >> 16, sl = byte_of(w.hdr[r].y, g);
            const float dl0 = d * (float)((int)((sl & 0xF) | (((sh >> (4 * g)) & 3) << 4)) - 32);
            const float dl1 = d * (float)((int)((sl >> 4) | (((sh >> (4 * g + 2)) & 3) << 4)) - 32);
#pragma unroll
            for (int n = 0; n < NC; n++)
                acc[r][n] += dl0 * (s[0][r][n] - 1152.0f * xsum[0][n]) + dl1 * (s[1][r][n] - 1152.0f * xsum[1][n]);
        }
    }
};

// Sum over the L lanes of a row slot (every lane of the slot gets it).
// DPP lane moves (one VALU op, no LDS round trip): quad_perm [1,0,3,2] and
// [2,3,0,1] swap neighbours and pairs within a quad; row_half_mirror (lane
// i <- 7 - i of its 8) and row_mirror (i <- 15 - i of its 16) pair quads
// and half-rows.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                                 0xF, 0xF, false));
}
constexpr int DPP_QUAD_XOR1 = 0xB1, DPP_QUAD_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141,
              DPP_MIRROR = 0x140;

// sum over the 4 lanes of a quad (every lane gets it)
__device__ __forceinline__ float quad_sum(float v) {
    v += dpp<DPP_QUAD_XOR1>(v);
    return v + dpp<DPP_QUAD_XOR2>(v);
}

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
// Dynamic LDS: [IQ2 tables (384 x 16 B)], then NC columns of staged pairs for
// `cunits` units (a multiple of 64), column stride cs = cunits * UW / 2
// uint32, then NC columns of 32-weight sums of the staged x (cunits * UW / 32
// floats each), then the S-way partial sums.
constexpr int GV_L = 16;  // lanes per row slot
constexpr int GV_SLOTS = 4;

// Stages activation slots [0, nslots) of chunk c0 (all NC columns) into LDS
// as packed fp16 and per-32 sums.  SP passes per round: every pass's global
// loads are issued before the first is packed.
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
__global__ __launch_bounds__(256) void silu_mul_kernel(float *__restrict__ a,
                                                       const float *__restrict__ b, uint32_t n) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) a[i] = silu_mul1(a[i], b[i]);
}

// With SILU the activations are silu(X) * X2 (the FFN's gate and up
// outputs), computed here in fp32 before the fp16 rounding.
// after_loads() runs once, right after the first round's activation loads
// are issued: the caller issues its weight loads there, behind them, so that
// the packing below waits only for the activations (loads complete in issue
// order) while the weights are in flight.
template <int F, int NC, int L, uint32_t SP, bool SILU, typename AfterLoads>
__device__ __forceinline__ void stage_x(const float *__restrict__ X, const float *__restrict__ X2,
                                        uint32_t K, uint32_t c0,
                                        uint32_t nslots, uint32_t tid, uint32_t nthr, uint32_t *xs,
                                        uint32_t cs, float *xsum, uint32_t xcs, AfterLoads after_loads) {
    constexpr uint32_t UW = unit_weights<F>(), SL = UW / 8;
    for (uint32_t q0 = 0; q0 < nslots; q0 += SP * nthr) {
        floatx4 A[SP][NC], B[SP][NC], A2[SILU ? SP : 1][SILU ? NC : 1], B2[SILU ? SP : 1][SILU ? NC : 1];
#pragma unroll
        for (uint32_t p = 0; p < SP; p++) {
            const uint32_t q = min(q0 + p * nthr + tid, nslots - 1), u = q / SL;
            uint32_t kb;
            const uint32_t ka = slot_first<F>(q % SL, kb);
#pragma unroll
            for (int n = 0; n < NC; n++) {
                const uint64_t xo = (uint64_t)n * K + unit_x_base<F>(c0 + u);
                A[p][n] = *(const floatx4 *)(X + xo + ka);
                B[p][n] = *(const floatx4 *)(X + xo + kb);
                if constexpr (SILU) {
                    A2[p][n] = *(const floatx4 *)(X2 + xo + ka);
                    B2[p][n] = *(const floatx4 *)(X2 + xo + kb);
                }
            }
        }
        if (q0 == 0) {
            __builtin_amdgcn_sched_barrier(0);
            after_loads();
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (uint32_t p = 0; p < SP; p++) {
            const uint32_t q = q0 + p * nthr + tid, u = q / SL, sidx = q % SL;
            const bool in = q < nslots;
#pragma unroll
            for (int n = 0; n < NC; n++) {
                if constexpr (SILU) {
                    A[p][n] = silu_mul4(A[p][n], A2[p][n]);
                    B[p][n] = silu_mul4(B[p][n], B2[p][n]);
                }
                const u32x4 v = slot_pack<F>(A[p][n], B[p][n]);
                const float pt = quad_sum(slot_bias<F>(v, sidx));
                if (in) {
                    *(u32x4 *)(xs + n * cs + xs_index<F, L>(u, 4 * sidx)) = v;
                    if ((q & 3) == 0) xsum[n * xcs + q / 4] = pt;
                }
            }
        }
    }
}

template <int F, int NC, int R, int D, int S, bool SILU>
__device__ __forceinline__ void gemv_body(const uint8_t *__restrict__ W, uint64_t row_bytes, uint32_t K,
                                          uint32_t M, const float *__restrict__ X,
                                          const float *__restrict__ X2, float *__restrict__ Y,
                                          const u32x4 *__restrict__ tab_g, uint32_t cunits,
                                          uint32_t blk) {
    constexpr int L = GV_L;
    extern __shared__ u32x4 lds[];
    constexpr uint32_t TAB = F == IQ2_XXS ? 384 : 0;
    u32x4 *tab = lds;
    uint32_t *xs = (uint32_t *)(lds + TAB);
    const uint32_t tid = threadIdx.x, nthr = blockDim.x;
    const uint32_t lane = tid & 63, i = lane % L, slot = lane / L;
    const uint32_t wave = tid >> 6, waves = nthr >> 6;
    const uint32_t part = wave % S, group = wave / S, groups = waves / S;
    if constexpr (F == IQ2_XXS)
        for (uint32_t e = tid; e < TAB; e += nthr) tab[e] = tab_g[e];

    const uint32_t m0 = ((blk * groups + group) * GV_SLOTS + slot) * R;
    const uint8_t *rows[R];
#pragma unroll
    for (int r = 0; r < R; r++) rows[r] = W + (uint64_t)min(m0 + r, M - 1) * row_bytes;
    constexpr uint32_t UW = unit_weights<F>();
    const uint32_t units = K / UW, cs = cunits * (UW / 2), xcs = cunits * (UW / 32);
    float *xsum = (float *)(xs + NC * cs);
    float *red = xsum + NC * xcs;  // [groups][slots][R][NC][S]

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
            stage_x<F, NC, L, 1, SILU>(X, X2, K, c0, nslots, tid, nthr, xs, cs, xsum, xcs, load_first);
        else if (SP == 4 && nslots <= 3 * nthr)
            stage_x<F, NC, L, (SP == 4 ? 3 : 1), SILU>(X, X2, K, c0, nslots, tid, nthr, xs, cs, xsum, xcs,
                                                       load_first);
        else
            stage_x<F, NC, L, SP, SILU>(X, X2, K, c0, nslots, tid, nthr, xs, cs, xsum, xcs, load_first);
        __syncthreads();
        // stream the wavefront's units u = c0 + i + L (part + S t) through
        // the ring
        uint32_t t = 0;
        for (; t + D < steps; t += D) {
#pragma unroll
            for (int j = 0; j < D; j++) {
                const uint32_t u = i + L * (part + S * (t + j));
                if (u < cn)
                    Compute<F, NC, R>::run(buf[j], xs + xs_index<F, L>(u, 0), 4 * L, cs,
                                           xsum + u * (UW / 32), xcs, c0 + u, acc, grid_fmt(F) ? tab_g : tab);
                load_unit<F, R>(rows, c0 + min(u + L * S * D, last), buf[j]);
            }
        }
#pragma unroll
        for (int j = 0; j < D; j++) {
            const uint32_t u = i + L * (part + S * (t + j));
            if (u < cn)
                Compute<F, NC, R>::run(buf[j], xs + xs_index<F, L>(u, 0), 4 * L, cs,
                                       xsum + u * (UW / 32), xcs, c0 + u, acc, grid_fmt(F) ? tab_g : tab);
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
};

template <int F, int NC, int R, int D, int S, bool SILU>
__global__ __launch_bounds__(256) void gemv_kernel(GemvGroup g, uint64_t row_bytes, uint32_t K,
                                                   const u32x4 *__restrict__ tab_g, uint32_t cunits) {
    uint32_t i = 0;
#pragma unroll
    for (int k = 0; k + 1 < GV_GROUP; k++)
        if (k + 1 < (int)g.n && blockIdx.x >= g.end[k]) i = k + 1;
    const uint32_t blk = blockIdx.x - (i ? g.end[i - 1] : 0);
    gemv_body<F, NC, R, D, S, SILU>(g.W[i], row_bytes, K, g.M[i], g.X[i], g.X2[i], g.Y[i], tab_g, cunits,
                                    blk);
}

}  // namespace okf
