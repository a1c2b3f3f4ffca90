// okf_gemm.h -- tile GEMM on CDNA4 matrix cores (N > 5, e.g. pp512 prefill)
// and the row dequantizer.
//
// Y[n][m] = sum_k W[m][k] X[n][k].  A 256-thread workgroup computes a
// 128 (rows m) x 128 (columns n) tile in K steps of 64: each step decodes the
// W tile to fp32 with the bit-exact unit decoders, rounds it to fp16 into LDS,
// converts the X tile to fp16 into LDS, then the four wavefronts (2 x 2, each
// 64 x 64) run v_mfma_f32_16x16x32_f16 with fp32 accumulation.  This is the
// reference's tile (LLM/metal/Kernels.metal:226-294: W dequantized to half in
// threadgroup memory, X float -> half, fp32 accumulate) laid out for 64-wide
// wavefronts and MFMA fragments.
#pragma once
#include "okf_common.h"
#include "okf_decode.h"

namespace okf {

constexpr int GB_M = 128, GB_N = 128, GB_K = 64, G_LDS_STRIDE = GB_K + 8;

// 32 floats -> 32 halves (round to nearest even) stored at dst (16-byte aligned).
__device__ __forceinline__ void store_half32(_Float16 *dst, const float *v) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        half8 h;
#pragma unroll
        for (int e = 0; e < 8; e++) h[e] = (_Float16)v[i * 8 + e];
        *(half8 *)(dst + i * 8) = h;
    }
}

__device__ __forceinline__ void zero_half32(_Float16 *dst) {
#pragma unroll
    for (int i = 0; i < 4; i++) *(half8 *)(dst + i * 8) = half8{};
}

// Q8_0 / Q2_0 units straight to fp16 (halves in weight order, 4 x 8): their
// weights are q d with q a small integer and d an fp16 value, so one fp16
// multiply rounds the exact product once, as decode_unit's fp32 product
// (exact) followed by the fp16 rounding does: the same bits.  q reaches
// fp16 through a byte spread into 0x64xx (1024 + byte) and one packed
// subtraction, exact.
template <int F>
__device__ __forceinline__ void decode_unit_h(const uint8_t *row, uint32_t u, half8 (&h)[4]) {
    uint32_t o[16];
    _Float16 d, off;
    if constexpr (F == Q8_0) {  // Q8_0.dequant (LLM/Gemma/Gemma4Quant.swift:55-68)
        const uint8_t *b = row + (uint64_t)u * 34;
        d = __builtin_bit_cast(_Float16, ldu<uint16_t>(b));
        uint32_t q[8];
        *(uint4 *)&q[0] = ldu<uint4>(b + 2);
        *(uint4 *)&q[4] = ldu<uint4>(b + 18);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t v = q[k] ^ 0x80808080u;  // b + 128
            o[2 * k] = __builtin_amdgcn_perm(0x64646464u, v, 0x04010400u);
            o[2 * k + 1] = __builtin_amdgcn_perm(0x64646464u, v, 0x04030402u);
        }
        off = (_Float16)-1152.0f;
    } else {  // Q2_0.dequant (LLM/Base/Quant.swift:10-25): code j at bits 2 (j % 16) of dword j / 16
        static_assert(F == Q2_0, "fp16 unit decode: Q8_0, Q2_0");
        const uint8_t *b = row + (uint64_t)(u >> 2) * 34;
        d = __builtin_bit_cast(_Float16, ldu<uint16_t>(b));
        const uint2 q = ldu<uint2>(b + 2 + (u & 3) * 8);
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const uint32_t dw = s ? q.y : q.x;
            const uint32_t f0 = dw & 0x03030303u, f1 = (dw >> 2) & 0x03030303u;
            const uint32_t f2 = (dw >> 4) & 0x03030303u, f3 = (dw >> 6) & 0x03030303u;
#pragma unroll
            for (int k = 0; k < 4; k++) {  // weights 16 s + 4 k + {0, 1 | 2, 3}: byte k of f0 f1 | f2 f3
                const uint32_t sel = (uint32_t)k | 0x0C00u | (uint32_t)(4 + k) << 16 | 0x0C000000u;
                o[8 * s + 2 * k] = __builtin_amdgcn_perm(f1, f0, sel) | 0x64006400u;
                o[8 * s + 2 * k + 1] = __builtin_amdgcn_perm(f3, f2, sel) | 0x64006400u;
            }
        }
        off = (_Float16)-1025.0f;
    }
    const half2v d2 = {d, d}, o2 = {off, off};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t r[4];
#pragma unroll
        for (int e = 0; e < 4; e++)
            r[e] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(half2v, o[4 * i + e]) + o2) * d2);
        h[i] = __builtin_bit_cast(half8, uint4{r[0], r[1], r[2], r[3]});
    }
}

// Xh: X in fp16 (converted once per call), else X is rounded here.
// K split: workgroup z of the grid's third dimension takes K range
// [z kper, (z + 1) kper) (kper a multiple of GB_K) and, with part, writes
// its tile to part + z N M (Y's layout) for gemm_ksum_kernel to add.
template <int F>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(const uint8_t *__restrict__ W,
                                                        uint64_t row_bytes, uint32_t K, uint32_t M,
                                                        const float *__restrict__ X, uint32_t N,
                                                        float *__restrict__ Y,
                                                        const uint2 *__restrict__ grid_g,
                                                        const uint8_t *__restrict__ gt, uint32_t kper,
                                                        float *__restrict__ part,
                                                        const _Float16 *__restrict__ Xh) {
    __shared__ __attribute__((aligned(16))) _Float16 As[GB_M * G_LDS_STRIDE];
    __shared__ __attribute__((aligned(16))) _Float16 Bs[GB_N * G_LDS_STRIDE];
    __shared__ uint2 grid[F == IQ2_XXS ? 256 : 1];
    if constexpr (F == IQ2_XXS) grid[threadIdx.x] = grid_g[threadIdx.x];

    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint32_t wm = wave >> 1, wn = wave & 1;
    const uint32_t n0 = blockIdx.x * GB_N, m0 = blockIdx.y * GB_M;
    const uint32_t lr = t >> 1, lh = t & 1;  // loader: tile row, 32-wide half
    const uint32_t units = K / 32;
    const uint8_t *wrow = W + (uint64_t)min(m0 + lr, M - 1) * row_bytes;
    const float *xrow = X + (uint64_t)min(n0 + lr, N - 1) * K;

    floatx4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = floatx4{0, 0, 0, 0};

    const uint32_t kb = blockIdx.z * kper, ke = min(K, kb + kper);
    for (uint32_t k0 = kb; k0 < ke; k0 += GB_K) {
        __syncthreads();  // previous step's fragments are consumed (and grid loaded)
        const uint32_t u = k0 / 32 + lh;
        _Float16 *ad = As + lr * G_LDS_STRIDE + lh * 32;
        _Float16 *bd = Bs + lr * G_LDS_STRIDE + lh * 32;
        if (u < units) {
            if constexpr (F == Q8_0 || F == Q2_0) {
                half8 h[4];
                decode_unit_h<F>(wrow, u, h);
#pragma unroll
                for (int i = 0; i < 4; i++) *(half8 *)(ad + i * 8) = h[i];
            } else {
                float w[32];
                decode_unit<F>(wrow, u, w, grid, gt);
                store_half32(ad, w);
            }
            if (Xh) {  // X already in fp16 (x_to_f16_kernel, the same rounding)
                const half8 *hp = (const half8 *)(Xh + (uint64_t)min(n0 + lr, N - 1) * K + u * 32);
#pragma unroll
                for (int i = 0; i < 4; i++) *(half8 *)(bd + i * 8) = hp[i];
            } else {
                float x[32];
                const float4 *xp = (const float4 *)(xrow + u * 32);
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    float4 v = xp[i];
                    x[4 * i] = v.x;
                    x[4 * i + 1] = v.y;
                    x[4 * i + 2] = v.z;
                    x[4 * i + 3] = v.w;
                }
                store_half32(bd, x);
            }
        } else {
            zero_half32(ad);
            zero_half32(bd);
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < GB_K / 32; kk++) {
            const uint32_t kc = kk * 32 + (lane >> 4) * 8;
            half8 a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; i++)
                a[i] = *(const half8 *)(As + (wm * 64 + i * 16 + (lane & 15)) * G_LDS_STRIDE + kc);
#pragma unroll
            for (int j = 0; j < 4; j++)
                b[j] = *(const half8 *)(Bs + (wn * 64 + j * 16 + (lane & 15)) * G_LDS_STRIDE + kc);
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    }

    // C fragment: lane holds rows 4*(lane>>4) + e of A (weight rows m) for
    // column lane & 15 of B (token n).
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t m = m0 + wm * 64 + i * 16 + 4 * (lane >> 4);
            const uint32_t n = n0 + wn * 64 + j * 16 + (lane & 15);
            if (n >= N) continue;
            float *dst = (part ? part + (uint64_t)blockIdx.z * N * M : Y) + (uint64_t)n * M + m;
            if (m + 3 < M && (M & 3) == 0) {
                *(float4 *)dst = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (m + e < M) dst[e] = acc[i][j][e];
            }
        }
}

// Y = the sum of the ks K-range partials of gemm_mfma_kernel, in K order
// (deterministic): 4 consecutive values of Y's N M per thread, all ks loads
// issued first in groups of 8.  vec: float4 accesses (the host sets it
// only when N M is a multiple of 4 and Y is 16-byte aligned, so that every
// partial and Y are too); else one value at a time.
static __global__ __launch_bounds__(256) void gemm_ksum_kernel(const float *__restrict__ part, float *__restrict__ Y,
                                                        uint64_t nm, uint32_t ks, uint32_t vec) {
    const uint64_t e = ((uint64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (e >= nm) return;
    if (vec && e + 4 <= nm) {
        float4 v = *(const float4 *)(part + e);
        for (uint32_t c0 = 1; c0 < ks; c0 += 8) {
            float4 w[8];
#pragma unroll
            for (uint32_t c = 0; c < 8; c++)
                if (c0 + c < ks) w[c] = *(const float4 *)(part + (uint64_t)(c0 + c) * nm + e);
#pragma unroll
            for (uint32_t c = 0; c < 8; c++)
                if (c0 + c < ks) {
                    v.x += w[c].x;
                    v.y += w[c].y;
                    v.z += w[c].z;
                    v.w += w[c].w;
                }
        }
        *(float4 *)(Y + e) = v;
    } else {
        for (uint64_t i = e; i < nm && i < e + 4; i++) {
            float v = part[i];
            for (uint32_t c = 1; c < ks; c++) v += part[(uint64_t)c * nm + i];
            Y[i] = v;
        }
    }
}

// One thread per 32-weight unit of a row; bit-exact with the CPU decoders.
template <int F>
__global__ __launch_bounds__(256) void dequant_row_kernel(const uint8_t *__restrict__ row,
                                                          uint32_t units, float *__restrict__ out,
                                                          const uint2 *__restrict__ grid_g,
                                                          const uint8_t *__restrict__ gt) {
    __shared__ uint2 grid[F == IQ2_XXS ? 256 : 1];
    if constexpr (F == IQ2_XXS) {
        grid[threadIdx.x] = grid_g[threadIdx.x];
        __syncthreads();
    }
    const uint32_t u = blockIdx.x * 256 + threadIdx.x;
    if (u >= units) return;
    float w[32];
    decode_unit<F>(row, u, w, grid, gt);
    float4 *o = (float4 *)(out + (uint64_t)u * 32);
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = make_float4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
}

// Embedding gather (embedBatch, LLM/Base/MetalEnc.swift:1096-1146): row
// ids[n] of W dequantized into out[n][K], one thread per 32-weight unit;
// bit-exact with dequant_row.  An id outside [0, M) is clamped to the
// nearest row, so a bad id cannot read outside the weights.
template <int F>
__global__ __launch_bounds__(256) void embed_batch_kernel(const uint8_t *__restrict__ W,
                                                          uint64_t row_bytes, uint32_t M,
                                                          const int32_t *__restrict__ ids,
                                                          uint32_t units_per_row, uint32_t units,
                                                          float *__restrict__ out,
                                                          const uint2 *__restrict__ grid_g,
                                                          const uint8_t *__restrict__ gt) {
    __shared__ uint2 grid[F == IQ2_XXS ? 256 : 1];
    if constexpr (F == IQ2_XXS) {
        grid[threadIdx.x] = grid_g[threadIdx.x];
        __syncthreads();
    }
    const uint32_t g = blockIdx.x * 256 + threadIdx.x;
    if (g >= units) return;
    const uint32_t n = g / units_per_row, u = g % units_per_row;
    const int32_t id = ids[n];
    const uint32_t row = id < 0 ? 0u : min((uint32_t)id, M - 1);
    float w[32];
    decode_unit<F>(W + (uint64_t)row * row_bytes, u, w, grid, gt);
    float4 *o = (float4 *)(out + ((uint64_t)n * units_per_row + u) * 32);
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = make_float4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
}

}  // namespace okf

namespace okf {

// ------------------------------------------------------------------------
// Q4_K x fp16 tile GEMM (the pp512 prefill path).
//
// Y[n][m] = sum_k W[m][k] X[n][k] with X already in fp16 (Xh[N][K]).  Tiles
// are 256 weight rows x QG_BN tokens, K steps of QG_BK (one 32-byte code
// group of a superblock); the kernel is gemm_q4k_w8_kernel below.
constexpr int QG_BN = 128, QG_BK = 64;

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

// 8 nibbles of two code dwords (v0, v1: the low nibbles, or the high ones
// shifted down) as one MFMA A operand, fma(q, a, o) per weight in packed
// fp16.  q reaches fp16 exactly through v_cvt_scalef32_pk_f16_fp8: a nibble
// in the low bits of an e4m3 byte is q * 2^-9 (exponent field 0 or 1,
// mantissa the low 3 bits), and the conversion's power-of-two scale 2^9
// restores q.
__device__ __forceinline__ u32x4v q4k_group_a(uint32_t v0, uint32_t v1, half2v a, half2v o) {
    const uint32_t l0 = v0 & 0x0F0F0F0Fu, l1 = v1 & 0x0F0F0F0Fu;
    const half2v q0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(l0, 512.0f, false);
    const half2v q1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(l0, 512.0f, true);
    const half2v q2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(l1, 512.0f, false);
    const half2v q3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(l1, 512.0f, true);
    return u32x4v{__builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q0, a, o)),
                  __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q1, a, o)),
                  __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q2, a, o)),
                  __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q3, a, o))};
}

// Q4_K code group g (64 weights) of one row as the four MFMA A operands of a
// 32x32x16 f16 step: lane half h holds the group's code bytes 16 h .. 16 h + 15
// in qv, and operand kk, element e is weight k = 16 h + 8 (kk & 1) +
// 32 (kk >> 1) + e of the group (low nibbles are k < 32, high nibbles k >= 32).
// The weight is fma(q, fp16(d sc), fp16(-dmin m)) in packed fp16 (q exact,
// q4k_group_a); vf (0 or 1) scales d and dmin, so vf = 0 gives zeros.
__device__ __forceinline__ void q4k_dq_mfma_a(const u32x4v hdr, const u32x4v qv, uint32_t g, float vf,
                                              u32x4v *a) {
    // every loaded dword counts as used here: a dword that a group does
    // not need would otherwise be reused as a temporary while its load
    // is still in flight, and that write has to wait for the load
    asm volatile("" ::"v"(hdr), "v"(qv));
    uint32_t sc0, mn0, sc1, mn1;
    q4k_scale_min_pair(make_uint4(hdr[0], hdr[1], hdr[2], hdr[3]), g, sc0, mn0, sc1, mn1);
    const float d = h2f(hdr[0] & 0xFFFF) * vf, dmin = h2f(hdr[0] >> 16) * vf;
    const half2v a0 = (half2v)(_Float16)(d * (float)sc0), o0 = (half2v)(_Float16)(-dmin * (float)mn0);
    const half2v a1 = (half2v)(_Float16)(d * (float)sc1), o1 = (half2v)(_Float16)(-dmin * (float)mn1);
    // q exact through the fp8 conversion (q4k_group_a), then fma(q, a, o)
    a[0] = q4k_group_a(qv[0], qv[1], a0, o0);
    a[1] = q4k_group_a(qv[2], qv[3], a0, o0);
    a[2] = q4k_group_a(qv[0] >> 4, qv[1] >> 4, a1, o1);
    a[3] = q4k_group_a(qv[2] >> 4, qv[3] >> 4, a1, o1);
}

// X fp32 -> fp16 (round to nearest even), XV float4 per thread with all
// loads issued before the first store; n4 float4 in all.
constexpr uint32_t XV = 4;
static __global__ __launch_bounds__(256) void x_to_f16_kernel(const float *__restrict__ X,
                                                       _Float16 *__restrict__ Xh, uint64_t n4) {
    typedef _Float16 half4 __attribute__((ext_vector_type(4)));
    const uint64_t i0 = (uint64_t)blockIdx.x * (256 * XV) + threadIdx.x;
    floatx4 v[XV];
#pragma unroll
    for (uint32_t j = 0; j < XV; j++)
        if (i0 + j * 256 < n4) v[j] = ((const floatx4 *)X)[i0 + j * 256];
#pragma unroll
    for (uint32_t j = 0; j < XV; j++)
        if (i0 + j * 256 < n4)
            ((half4 *)Xh)[i0 + j * 256] =
                half4{(_Float16)v[j][0], (_Float16)v[j][1], (_Float16)v[j][2], (_Float16)v[j][3]};
}

// Work split.  The first `full` tiles (a multiple of the CU count = one per
// CU per round) are whole tiles; each of the remaining tiles is split over
// `ks` K ranges, so that a grid of 256 + 16 tiles (pp512) costs about 1 + 1/10
// tile times per CU instead of 2.  A split workgroup stores its partial tile to
// `part`; gemm_split_sum_kernel then adds each tile's partials in K order
// (a kernel boundary, not an in-kernel fence: a device-scope fence writes
// back and invalidates the whole L2 of the XCD, which costs the concurrent
// whole tiles their cached operands).
struct GemmSplit {
    uint32_t tiles_n, tiles;
    uint32_t full, full_xcd;        // whole tiles, and per XCD
    uint32_t ks, units, units_xcd;  // K ranges per split tile, split workgroups, per XCD
    float *part;                    // [units][QG_BN][256] partial tiles
    uint32_t ng;                    // wide kernel: N tiles per XCD group (0: plain order)
};

// Y of the split tiles: workgroup b sums float4 (b % per-tile) * 256 + t of
// split tile b / per-tile over its ks partials, in K order (all ks loads
// issued first).  BM is the tile's row count (128 or 256), BN = 128.
template <uint32_t BM>
__global__ __launch_bounds__(256) void gemm_split_sum_kernel(const float *__restrict__ part,
                                                             float *__restrict__ Y, uint32_t M,
                                                             uint32_t N, GemmSplit sp) {
    constexpr uint32_t WG = BM * QG_BN / (4 * 256);  // workgroups per tile
    const uint32_t lt = blockIdx.x / WG, tile = sp.full + lt;
    const uint32_t e = ((blockIdx.x % WG) * 256 + threadIdx.x) * 4;
    const uint32_t nl = e / BM, ml = e % BM;
    const uint32_t m = tile / sp.tiles_n * BM + ml, n = tile % sp.tiles_n * QG_BN + nl;
    if (n >= N || m >= M) return;
    const float *p0 = part + (uint64_t)lt * sp.ks * (BM * QG_BN) + e;
    float4 v = *(const float4 *)p0;
    for (uint32_t c0 = 1; c0 < sp.ks; c0 += 8) {
        float4 w[8];
#pragma unroll
        for (uint32_t c = 0; c < 8; c++)
            if (c0 + c < sp.ks) w[c] = *(const float4 *)(p0 + (uint64_t)(c0 + c) * (BM * QG_BN));
#pragma unroll
        for (uint32_t c = 0; c < 8; c++)
            if (c0 + c < sp.ks) {
                v.x += w[c].x;
                v.y += w[c].y;
                v.z += w[c].z;
                v.w += w[c].w;
            }
    }
    float *dst = Y + (uint64_t)n * M + m;
    if (m + 3 < M && (M & 3) == 0) {
        *(float4 *)dst = v;
    } else {
        const float vv[4] = {v.x, v.y, v.z, v.w};
        for (int k = 0; k < 4; k++)
            if (m + k < M) dst[k] = vv[k];
    }
}

constexpr int QW_BM = 256;

// Tile and K range of workgroup blockIdx.x of a wide-tile launch (whole tiles
// first, one per CU, then the split units; each XCD's whole tiles share one
// N tile when 8 is a multiple of the N tiles).  K range [sb0, sb1) in
// superblocks.  False when the workgroup has nothing to do.
__device__ __forceinline__ bool wide_tile_of(const GemmSplit &sp, uint32_t sbs, uint32_t &tile, uint32_t &unit,
                                             uint32_t &sb0, uint32_t &sb1, bool &split) {
    const uint32_t xcd = blockIdx.x % 8, slot = blockIdx.x / 8;
    split = slot >= sp.full_xcd;
    sb0 = 0;
    sb1 = sbs;
    unit = 0;
    if (!split) {
        // groups of ng N tiles; XCD x takes N-tile group x % groups and, in
        // its slots, ng consecutive N tiles of each of its row blocks
        const uint32_t ng = sp.ng, groups = sp.tiles_n / ng;
        if (ng && sp.tiles_n % ng == 0 && 8 % groups == 0 && sp.full_xcd % ng == 0) {
            const uint32_t nt = (xcd % groups) * ng + slot % ng;
            const uint32_t mt = (xcd / groups) * (sp.full_xcd / ng) + slot / ng;
            tile = mt * sp.tiles_n + nt;
        } else {
            tile = xcd * sp.full_xcd + slot;
        }
    } else {
        unit = xcd * sp.units_xcd + (slot - sp.full_xcd);
        if (unit >= sp.units) return false;
        tile = sp.full + unit / sp.ks;
        const uint32_t c = unit % sp.ks;
        sb0 = c * sbs / sp.ks;
        sb1 = (c + 1) * sbs / sp.ks;
    }
    return tile < sp.tiles;
}

// ------------------------------------------------------------------------
// The same 256 x 128 tile with eight wavefronts (two per SIMD): wavefronts
// 0-3 take the even superblocks of the K range and 4-7 the odd ones, each
// with a 64-row x 128-token slice.  While one
// wavefront of a SIMD waits (on its loads, the barrier or LDS), the other
// issues.  At the end the odd half's accumulators are added to the even
// half's through LDS (even + odd, a fixed order).  When the range has an odd
// number of superblocks the odd half runs its last superblock with zero
// scales (every weight 0), so both halves meet at every barrier.
//
// The activations go from memory straight to LDS (global_load_lds_dwordx4,
// XD steps ahead, XD + 2 stages per half): a stage is 128 tokens x 64 k
// fp16 without padding, token t's 16-byte chunk c (k = 8 c .. 8 c + 7) at
// t * 128 + 16 * (c ^ ((t >> 1) & 7)), so that the 16 lanes of each
// ds_read_b128 quarter hit 16 different 16-byte bank groups.  The weight
// bytes come D steps ahead in registers.
//
// The LDS reads are written out in asm with explicit waits: the compiler
// cannot tell the stage being filled by the direct loads from the one being
// read, and would otherwise wait for every outstanding load before each read.
template <int D, int XD>
__global__ __launch_bounds__(512, 1) void gemm_q4k_w8_kernel(const uint8_t *__restrict__ W, uint64_t row_bytes,
                                                          uint32_t K, uint32_t M,
                                                          const _Float16 *__restrict__ Xh, uint32_t N,
                                                          float *__restrict__ Y, GemmSplit sp) {
    constexpr uint32_t NST = XD + 2, STAGE_B = QG_BN * QG_BK * 2;  // bytes per stage
    static_assert(2 * NST * STAGE_B >= 4 * 64 * 64 * 4, "the reduction reuses the stages");
    __shared__ __attribute__((aligned(1024))) uint8_t Bs[2][NST][STAGE_B];  // [K half][stage]
    const uint32_t sbs = K / 256;
    uint32_t tile, unit, sb0, sb1;
    bool split;
    if (!wide_tile_of(sp, sbs, tile, unit, sb0, sb1, split)) return;
    const uint32_t nt = tile % sp.tiles_n, mt = tile / sp.tiles_n;
    const uint32_t m0 = mt * QW_BM, n0 = nt * QG_BN;

    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6, h = lane >> 5;
    // (read through the first lane: the compiler then knows they are uniform)
    const uint32_t wu = __builtin_amdgcn_readfirstlane(wave), kh = wu >> 2, wr = wu & 3;
    const uint32_t rm = m0 + wr * 64 + (lane & 31);
    const uint8_t *w0 = W + (uint64_t)min(rm, M - 1) * row_bytes;
    const uint8_t *w1 = W + (uint64_t)min(rm + 32, M - 1) * row_bytes;
    // direct loads: instruction i of wavefront wr fills chunk
    // (4 wr + i) * 64 + lane of the stage = token xt, position xp
    const uint32_t xt0 = (wr * 4) * 8 + (lane >> 3), xp = lane & 7;
    uint32_t xsrc[4];  // element offsets into Xh (N * K < 2^32)
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t tok = xt0 + i * 8, c = xp ^ ((tok >> 1) & 7);
        xsrc[i] = min(n0 + tok, N - 1) * K + 8 * c;
    }
    typedef __attribute__((address_space(3))) void lds_void;
    lds_void *const xdst = (lds_void *)(&Bs[kh][0][0] + (wr * 4) * 1024);

    struct WRegs {
        u32x4v q0, q1;
    };
    // local step l of this half: superblock sb0 + 2 (l / 4) + kh (clamped
    // to the row, so every load is unconditional), code group l % 4
    auto lsb = [&](uint32_t l) { return min(sb0 + 2 * (l >> 2) + kh, sbs - 1); };
    // (written out, like every load of the loop: the compiler's own count
    // of outstanding loads is lost once a direct-to-LDS load is in flight,
    // and it would wait for all of them; the waits below are explicit)
    // the code bytes of step l, rows r and r + 32
    auto fetch_w = [&](uint32_t l, WRegs &r) {
        const uint64_t qo = (uint64_t)lsb(l) * 144 + 16 + (l & 3) * 32 + 16 * h;
        asm volatile("global_load_dwordx4 %0, %2, off\n\t"
                     "global_load_dwordx4 %1, %3, off"
                     : "=&v"(r.q0), "=&v"(r.q1)
                     : "v"(w0 + qo), "v"(w1 + qo));
    };
    // the 16-byte header (d, dmin, packed scales) of step l's superblock:
    // loaded once per superblock, it serves the superblock's four steps
    auto fetch_h = [&](uint32_t l, u32x4v &h0, u32x4v &h1) {
        const uint64_t sbo = (uint64_t)lsb(l) * 144;
        asm volatile("global_load_dwordx4 %0, %2, off\n\t"
                     "global_load_dwordx4 %1, %3, off"
                     : "=&v"(h0), "=&v"(h1)
                     : "v"(w0 + sbo), "v"(w1 + sbo));
    };
    // stage l % NST <- activations of local step l (4 direct loads per lane)
    auto fetch_x = [&](uint32_t l, uint32_t st) {
        const uint32_t ko = lsb(l) * 256 + (l & 3) * QG_BK;
#pragma unroll
        for (int i = 0; i < 4; i++)
            __builtin_amdgcn_global_load_lds((const void *)(Xh + xsrc[i] + ko),
                                             (lds_void *)((__attribute__((address_space(3))) uint8_t *)xdst +
                                                          st * STAGE_B + i * 1024),
                                             16, 0, 0);
    };
    auto dq_row = [&](const u32x4v hdr, const u32x4v qv, uint32_t g, float vf, u32x4v *a) {
        q4k_dq_mfma_a(hdr, qv, g, vf, a);
    };
    // B reads: MFMA kk takes chunk 2 h + (kk & 1) + 4 (kk >> 1) of token
    // 32 jn + lane % 32; jn and the stage are immediate offsets
    const uint32_t swz = ((lane & 31) >> 1) & 7;
    const uint32_t bbase =
        (uint32_t)(uintptr_t)((__attribute__((address_space(3))) uint8_t *)&Bs[kh][0][0]) + (lane & 31) * 128;
    uint32_t baddr[4];
#pragma unroll
    for (int kk = 0; kk < 4; kk++) baddr[kk] = bbase + 16 * ((2 * h + (kk & 1) + 4 * (kk >> 1)) ^ swz);
    auto read_b = [&](uint32_t addr, u32x4v *b) {
        asm volatile("ds_read_b128 %0, %4\n\t"
                     "ds_read_b128 %1, %4 offset:4096\n\t"
                     "ds_read_b128 %2, %4 offset:8192\n\t"
                     "ds_read_b128 %3, %4 offset:12288"
                     : "=&v"(b[0]), "=&v"(b[1]), "=&v"(b[2]), "=&v"(b[3])
                     : "v"(addr));
    };

    auto read_b1 = [&](uint32_t addr, u32x4v &b) { asm volatile("ds_read_b128 %0, %1" : "+v"(b) : "v"(addr)); };

    typedef float floatx16 __attribute__((ext_vector_type(16)));
    floatx16 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = floatx16{};

    // Two halves in ping-pong.  Every wavefront runs the same steps (issue
    // the activations of step t + XD, dequantize step t and issue its
    // weights of step t + D, MFMAs of step t), but the even half meets the
    // step's barrier before its dequant and the odd half after it.  Between
    // two barriers the even half dequantizes while the odd half runs its
    // MFMAs, and then the other way round, so each SIMD always has one
    // wavefront in a VALU phase and one in an MFMA + LDS phase.  (Only the
    // waits and the barrier sit in the branches: a branch holding loads or
    // MFMAs would make the compiler copy their registers at the join.)
    //
    // The odd half issues step t + XD's activations before the barrier, while
    // its partners may still read stage t - 1: hence XD + 2 stages.
    static_assert(NST == XD + 2 && D == 2 && XD == 2, "stages and the wait counts below");
    // Loads issued at step s: step s + 2's activations (4 direct loads) and
    // code bytes (2), and at s % 4 == 2, after those, the next superblock's
    // headers (2).  The prologue issues steps 0 and 1 and the first headers
    // in the same order.  Counting the loads issued later, with s % 4 = jj
    // static in the loop:
    //   even half's barrier, step s's activations: 8, + 2 where headers
    //     were issued at step s - 1 or s - 2 (jj 3, 0);
    //   odd half's barrier: that + 6, + 2 more at jj 2;
    //   the dequant's wait, step s's code bytes: 10, + 2 at jj 3, 0;
    //   a superblock's end (jj 3), the headers and code bytes issued at jj 2:
    //     6.
    constexpr int WAIT_E[4] = {10, 8, 8, 10}, WAIT_O[4] = {16, 14, 16, 16}, WAIT_W[4] = {12, 10, 10, 12};
    constexpr int WAIT_N = 6;
    WRegs r[D];
    u32x4v hcur0, hcur1, hnext0, hnext1;  // superblock headers, rows r and r + 32
    fetch_x(0, 0);
    __builtin_amdgcn_sched_barrier(0);
    fetch_w(0, r[0]);
    __builtin_amdgcn_sched_barrier(0);
    fetch_h(0, hcur0, hcur1);
    __builtin_amdgcn_sched_barrier(0);
    fetch_x(1, 1);
    __builtin_amdgcn_sched_barrier(0);
    fetch_w(1, r[1]);
    __builtin_amdgcn_sched_barrier(0);
    // (step 0's dequant waits for its code bytes only)
    asm volatile("s_waitcnt vmcnt(6)" : "+v"(hcur0), "+v"(hcur1));
    const uint32_t nit = (sb1 - sb0 + 1) / 2;
    // one loop trip is a superblock: the code group and every ring slot are static
    static_assert(4 % D == 0 && 4 % NST == 0, "ring sizes divide the 4 steps of a superblock");
    for (uint32_t l0 = 0; l0 < 4 * nit; l0 += 4) {
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
            const uint32_t l = l0 + jj;
            WRegs &rj = r[jj % D];
            // (a bare barrier: __syncthreads' release fence would wait for
            // every outstanding direct load, the prefetched ones included)
            if (kh == 0) {
                asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(WAIT_E[jj]));
            }
            __builtin_amdgcn_sched_barrier(0);
            fetch_x(l + XD, (jj + XD) % NST);
            __builtin_amdgcn_sched_barrier(0);
            const float vf = sb0 + 2 * (l >> 2) + kh < sb1 ? 1.0f : 0.0f;
            asm volatile("s_waitcnt vmcnt(%4)"
                         : "+v"(rj.q0), "+v"(rj.q1), "+v"(hcur0), "+v"(hcur1)
                         : "n"(WAIT_W[jj]));
            u32x4v a[2][4];
            dq_row(hcur0, rj.q0, jj, vf, a[0]);
            dq_row(hcur1, rj.q1, jj, vf, a[1]);
            __builtin_amdgcn_sched_barrier(0);
            fetch_w(l + D, rj);
            if (jj == 2) fetch_h(l + 2, hnext0, hnext1);
            __builtin_amdgcn_sched_barrier(0);
            if (kh != 0) {
                asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(WAIT_O[jj]));
            }
            __builtin_amdgcn_sched_barrier(0);
            const uint32_t so = (jj % NST) * STAGE_B;
            u32x4v b[4];
            read_b(baddr[0] + so, b);
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
#pragma unroll
                for (int jn = 0; jn < 4; jn++) {
                    // fragment jn of group kk: the reads issued after it are
                    // group kk's jn + 1.. and group kk + 1's ..jn - 1
                    asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(b[jn]) : "n"(kk < 3 ? 3 : 3 - jn));
#pragma unroll
                    for (int i = 0; i < 2; i++)
                        acc[i][jn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                            __builtin_bit_cast(half8, a[i][kk]), __builtin_bit_cast(half8, b[jn]), acc[i][jn], 0,
                            0, 0);
                    __builtin_amdgcn_sched_barrier(0);
                    // group kk + 1's fragment jn, into the same registers
                    // (the MFMAs above have read them once issued), so the
                    // LDS latency hides behind the MFMAs
                    if (kk < 3) read_b1(baddr[kk + 1] + so + 4096 * jn, b[jn]);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            if (jj == 3) {
                // the next superblock's headers, issued a step ago, into
                // the registers the next trip reads: a copy the compiler
                // makes at the loop's back edge then moves landed data
                asm volatile("s_waitcnt vmcnt(%4)"
                             : "+v"(hnext0), "+v"(hnext1), "+v"(r[0].q0), "+v"(r[0].q1)
                             : "n"(WAIT_N));
                hcur0 = hnext0;
                hcur1 = hnext1;
            }
        }
    }
    // The loads issued past the end are still in flight: the direct ones
    // write the stages, and the weight registers must stay allocated until
    // their data has landed (an asm output whose value is never read could
    // otherwise be handed to another value while the load still writes it).
#pragma unroll
    for (int j = 0; j < D; j++) asm volatile("s_waitcnt vmcnt(0)" : "+v"(r[j].q0), "+v"(r[j].q1)::"memory");
    asm volatile("" : "+v"(hnext0), "+v"(hnext1));

    // odd half -> even half, one row tile (i) at a time through LDS:
    // red[(wr * 64 + e) * 64 + lane], e = 16 jn + register
    float *red = (float *)&Bs[0][0][0];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        __syncthreads();
        if (kh == 1) {
#pragma unroll
            for (int jn = 0; jn < 4; jn++)
#pragma unroll
                for (int e = 0; e < 16; e++) red[(wr * 64 + jn * 16 + e) * 64 + lane] = acc[i][jn][e];
        }
        __syncthreads();
        if (kh == 0) {
#pragma unroll
            for (int jn = 0; jn < 4; jn++)
#pragma unroll
                for (int e = 0; e < 16; e++) acc[i][jn][e] += red[(wr * 64 + jn * 16 + e) * 64 + lane];
        }
    }
    if (kh == 1) return;

    if (split) {
        float *pt = sp.part + (uint64_t)unit * (QW_BM * QG_BN);  // [n_local][m_local]
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int jn = 0; jn < 4; jn++) {
                const uint32_t nl = jn * 32 + (lane & 31);
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const uint32_t ml = wr * 64 + i * 32 + 8 * q + 4 * h;
                    const floatx16 &c = acc[i][jn];
                    *(float4 *)(pt + nl * QW_BM + ml) =
                        make_float4(c[4 * q], c[4 * q + 1], c[4 * q + 2], c[4 * q + 3]);
                }
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int jn = 0; jn < 4; jn++) {
            const uint32_t n = n0 + jn * 32 + (lane & 31);
            if (n >= N) continue;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint32_t m = m0 + wr * 64 + i * 32 + 8 * q + 4 * h;
                float *dst = Y + (uint64_t)n * M + m;
                const floatx16 &c = acc[i][jn];
                if (m + 3 < M && (M & 3) == 0) {
                    *(float4 *)dst = make_float4(c[4 * q], c[4 * q + 1], c[4 * q + 2], c[4 * q + 3]);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        if (m + e < M) dst[e] = c[4 * q + e];
                }
            }
        }
}

// ------------------------------------------------------------------------
// Leftover tiles of the wide-tile launch (the tiles past the last whole
// round of one tile per CU, 16 of them at pp512).  Each 256 x 128 tile is
// cut into 16 pieces of 64 rows x 32 tokens over the whole K, one 512-thread
// workgroup per piece: wavefront w takes the 64-weight code-group steps
// w, w + 8, ... of K (weights and activations straight into registers, two
// steps in flight), with two 32x32x16 f16 MFMAs per step, and the eight
// partial tiles are added through LDS in wavefront order.  Every output is
// written once, with no partial tiles in memory and no second kernel, and
// 16 x the leftover count of small workgroups spread over all the CUs.
constexpr uint32_t QT_BM = 64, QT_BN = 32;

template <int NW, int D>
__global__ __launch_bounds__(NW * 64) void gemm_q4k_thin_kernel(const uint8_t *__restrict__ W,
                                                              uint64_t row_bytes, uint32_t K, uint32_t M,
                                                              const _Float16 *__restrict__ Xh, uint32_t N,
                                                              float *__restrict__ Y, uint32_t tile0,
                                                              uint32_t tiles_n, uint32_t pieces) {
    __shared__ float red[NW][32][64];  // [wavefront][accumulator][lane]
    // (pieces in plain order: a contiguous piece range per XCD measured
    // the same)
    const uint32_t pc = blockIdx.x;
    if (pc >= pieces) return;
    const uint32_t tile = tile0 + pc / 16;
    const uint32_t m0 = tile / tiles_n * QW_BM + (pc % 16) / 4 * QT_BM;
    const uint32_t n0 = tile % tiles_n * QG_BN + (pc % 4) * QT_BN;
    if (m0 >= M || n0 >= N) return;  // (uniform over the workgroup)
    const uint32_t t = threadIdx.x, lane = t & 63, h = lane >> 5;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t rm = m0 + (lane & 31);
    const uint8_t *w0 = W + (uint64_t)min(rm, M - 1) * row_bytes;
    const uint8_t *w1 = W + (uint64_t)min(rm + 32, M - 1) * row_bytes;
    const _Float16 *xr = Xh + (uint64_t)min(n0 + (lane & 31), N - 1) * K;
    const uint32_t steps = K / QG_BK;

    struct Regs {
        u32x4v h0, h1, q0, q1, x[4];
    };
    // step s: code group s % 4 of superblock s / 4; activation operand kk
    // is chunk 2 h + (kk & 1) + 4 (kk >> 1) of the step's 64 k (the order
    // q4k_dq_mfma_a gives the weights).  Past the end a load re-reads the
    // last step (a cache hit), so every load is unconditional.
    auto load = [&](uint32_t s, Regs &r) {
        s = min(s, steps - 1);
        const uint64_t sbo = (uint64_t)(s >> 2) * 144, qo = sbo + 16 + (s & 3) * 32 + 16 * h;
        r.h0 = *(const u32x4v *)(w0 + sbo);
        r.h1 = *(const u32x4v *)(w1 + sbo);
        r.q0 = *(const u32x4v *)(w0 + qo);
        r.q1 = *(const u32x4v *)(w1 + qo);
#pragma unroll
        for (int kk = 0; kk < 4; kk++)
            r.x[kk] = *(const u32x4v *)(xr + (uint64_t)s * QG_BK + 8 * (2 * h + (kk & 1) + 4 * (kk >> 1)));
    };
    typedef float floatx16 __attribute__((ext_vector_type(16)));
    floatx16 acc[2] = {floatx16{}, floatx16{}};
    auto compute = [&](uint32_t s, const Regs &r) {
        u32x4v a[2][4];
        q4k_dq_mfma_a(r.h0, r.q0, s & 3, 1.0f, a[0]);
        q4k_dq_mfma_a(r.h1, r.q1, s & 3, 1.0f, a[1]);
#pragma unroll
        for (int kk = 0; kk < 4; kk++)
#pragma unroll
            for (int i = 0; i < 2; i++)
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a[i][kk]),
                                                                __builtin_bit_cast(half8, r.x[kk]), acc[i], 0, 0,
                                                                0);
    };
    // wavefront w takes steps w, w + NW, ...; D of them in flight
    Regs r[D];
#pragma unroll
    for (int j = 0; j < D; j++) load(wave + j * NW, r[j]);
    for (uint32_t s = wave; s < steps; s += D * NW) {
#pragma unroll
        for (int j = 0; j < D; j++) {
            if (s + j * NW < steps) compute(s + j * NW, r[j]);
            load(s + (j + D) * NW, r[j]);
        }
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) red[wave][16 * i + e][lane] = acc[i][e];
    __syncthreads();
    // the 2048 outputs as 512 groups of 4 rows: group q = t + 64 NW c holds
    // accumulators 4 (q / 64) .. + 3 of lane q % 64, added over the
    // wavefronts in order; rows 32 (g / 4) + 8 (g % 4) + 4 h + j, g = q / 64
    for (uint32_t q = t; q < 512; q += NW * 64) {
        const uint32_t g = q >> 6;
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float a = red[0][4 * g + j][lane];
#pragma unroll
            for (int w = 1; w < NW; w++) a += red[w][4 * g + j][lane];
            v[j] = a;
        }
        const uint32_t n = n0 + (lane & 31), m = m0 + 32 * (g / 4) + 8 * (g % 4) + 4 * h;
        if (n >= N) continue;
        float *dst = Y + (uint64_t)n * M + m;
        if (m + 3 < M && (M & 3) == 0) {
            *(float4 *)dst = make_float4(v[0], v[1], v[2], v[3]);
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (m + j < M) dst[j] = v[j];
        }
    }
}

}  // namespace okf
