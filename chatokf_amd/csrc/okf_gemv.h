// okf_gemv.h -- decode matvec (N = 1) and narrow matmul (N = 2..5) kernels.
//
// One weight pass serves all NC activation columns (the reference's
// gemv / gemm_nb kernels, LLM/metal/Kernels.metal:1572-1753, :2486-2585).
//
// Work split: a 256-thread workgroup is 4 wavefronts; each wavefront owns R
// consecutive output rows.  Lane l walks the row's 32-weight units
// u = l, l + 64, ... so that, per load instruction, consecutive lanes read
// consecutive bytes of every row (coalesced 16-byte loads for Q4_K, 8/16-byte
// loads for the 2-byte-aligned formats).  The lane's activation slice is
// loaded once per unit and reused for all R rows, then the row sums are
// reduced across the wavefront.  Scales are factored out of the inner sums:
// Q4_K uses (d*sc)*sum(q*x) - (dmin*m)*sum(x) per 32 weights, Q2_0 uses
// d*(sum(code*x) - sum(x)), Q8_0 and IQ2_XXS use d * sum(q*x) per unit.
#pragma once
#include "okf_common.h"
#include "okf_decode.h"

namespace okf {

template <int NC>
struct XSlice {
    float v[NC][16];
};

// 16 consecutive activations of each column, starting at k.
template <int NC>
__device__ __forceinline__ void load_x16(const float *X, uint32_t K, uint32_t k, XSlice<NC> &xs) {
#pragma unroll
    for (int n = 0; n < NC; n++) {
        const float4 *p = (const float4 *)(X + (uint64_t)n * K + k);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float4 t = p[i];
            xs.v[n][4 * i + 0] = t.x;
            xs.v[n][4 * i + 1] = t.y;
            xs.v[n][4 * i + 2] = t.z;
            xs.v[n][4 * i + 3] = t.w;
        }
    }
}

template <int NC>
__device__ __forceinline__ void sum_x16(const XSlice<NC> &xs, float *s) {
#pragma unroll
    for (int n = 0; n < NC; n++) {
        float a = 0;
#pragma unroll
        for (int i = 0; i < 16; i++) a += xs.v[n][i];
        s[n] = a;
    }
}

// sum_i byte_i(q) * x_i over the 16 bytes of q (unsigned bytes).
template <int NC>
__device__ __forceinline__ void dot_u8x16(const uint32_t q[4], const XSlice<NC> &xs, float *s) {
#pragma unroll
    for (int n = 0; n < NC; n++) s[n] = 0;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        float w = (float)byte_of(q[i >> 2], i & 3);
#pragma unroll
        for (int n = 0; n < NC; n++) s[n] += w * xs.v[n][i];
    }
}

// ---------------------------------------------------------------- Q8_0 --
template <int NC, int R>
__device__ __forceinline__ void unit_q8_0(const uint8_t *const rows[R], uint32_t u, const float *X,
                                          uint32_t K, float (&acc)[R][NC]) {
    uint32_t q[R][8];
    float d[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint8_t *b = rows[r] + (uint64_t)u * 34;
        d[r] = h2f(ldu<uint16_t>(b));
        *(uint4 *)&q[r][0] = ldu<uint4>(b + 2);
        *(uint4 *)&q[r][4] = ldu<uint4>(b + 18);
    }
    float s[R][NC];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int n = 0; n < NC; n++) s[r][n] = 0;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        XSlice<NC> xs;
        load_x16<NC>(X, K, u * 32 + h * 16, xs);
#pragma unroll
        for (int r = 0; r < R; r++) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                float w = (float)(int)(int8_t)byte_of(q[r][h * 4 + (i >> 2)], i & 3);
#pragma unroll
                for (int n = 0; n < NC; n++) s[r][n] += w * xs.v[n][i];
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int n = 0; n < NC; n++) acc[r][n] += d[r] * s[r][n];
}

// ---------------------------------------------------------------- Q2_0 --
template <int NC, int R>
__device__ __forceinline__ void unit_q2_0(const uint8_t *const rows[R], uint32_t u, const float *X,
                                          uint32_t K, float (&acc)[R][NC]) {
    uint2 q[R];
    float d[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint8_t *b = rows[r] + (uint64_t)(u >> 2) * 34;
        d[r] = h2f(ldu<uint16_t>(b));
        q[r] = ldu<uint2>(b + 2 + (u & 3) * 8);
    }
    float s[R][NC], sx[NC];
#pragma unroll
    for (int n = 0; n < NC; n++) sx[n] = 0;
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int n = 0; n < NC; n++) s[r][n] = 0;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        XSlice<NC> xs;
        load_x16<NC>(X, K, u * 32 + h * 16, xs);
        float t[NC];
        sum_x16<NC>(xs, t);
#pragma unroll
        for (int n = 0; n < NC; n++) sx[n] += t[n];
#pragma unroll
        for (int r = 0; r < R; r++) {
            uint32_t dw = h ? q[r].y : q[r].x;
            // codes 2i of the 4 bytes land at byte positions: expand by masks
            uint32_t c0 = dw & 0x03030303u, c1 = (dw >> 2) & 0x03030303u;
            uint32_t c2 = (dw >> 4) & 0x03030303u, c3 = (dw >> 6) & 0x03030303u;
            uint32_t cs[4] = {c0, c1, c2, c3};
#pragma unroll
            for (int i = 0; i < 16; i++) {
                // weight i: byte i>>2, code position i&3
                float w = (float)byte_of(cs[i & 3], i >> 2);
#pragma unroll
                for (int n = 0; n < NC; n++) s[r][n] += w * xs.v[n][i];
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int n = 0; n < NC; n++) acc[r][n] += d[r] * (s[r][n] - sx[n]);
}

// ---------------------------------------------------------------- Q4_K --
// Unit u = 16-byte code chunk c = u & 7 of superblock u >> 3: its low nibbles
// are weights 64g + 16h + i of sub-block 2g, its high nibbles weights
// 64g + 32 + 16h + i of sub-block 2g + 1 (g = c >> 1, h = c & 1).
template <int NC, int R>
__device__ __forceinline__ void unit_q4_k(const uint8_t *const rows[R], uint32_t u, const float *X,
                                          uint32_t K, float (&acc)[R][NC]) {
    uint32_t sb = u >> 3, c = u & 7, g = c >> 1, h = c & 1;
    uint4 hdr[R], qv[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint8_t *b = rows[r] + (uint64_t)sb * 144;
        hdr[r] = *(const uint4 *)b;
        qv[r] = *(const uint4 *)(b + 16 + c * 16);
    }
    uint32_t k0 = sb * 256 + g * 64 + h * 16;
    float slo[R][NC], shi[R][NC], xlo[NC], xhi[NC];
    {
        XSlice<NC> xs;
        load_x16<NC>(X, K, k0, xs);
        sum_x16<NC>(xs, xlo);
#pragma unroll
        for (int r = 0; r < R; r++) {
            uint32_t q[4] = {qv[r].x & 0x0F0F0F0Fu, qv[r].y & 0x0F0F0F0Fu, qv[r].z & 0x0F0F0F0Fu,
                             qv[r].w & 0x0F0F0F0Fu};
            dot_u8x16<NC>(q, xs, slo[r]);
        }
    }
    {
        XSlice<NC> xs;
        load_x16<NC>(X, K, k0 + 32, xs);
        sum_x16<NC>(xs, xhi);
#pragma unroll
        for (int r = 0; r < R; r++) {
            uint32_t q[4] = {(qv[r].x >> 4) & 0x0F0F0F0Fu, (qv[r].y >> 4) & 0x0F0F0F0Fu,
                             (qv[r].z >> 4) & 0x0F0F0F0Fu, (qv[r].w >> 4) & 0x0F0F0F0Fu};
            dot_u8x16<NC>(q, xs, shi[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        uint32_t sc0, mn0, sc1, mn1;
        q4k_scale_min_pair(hdr[r], g, sc0, mn0, sc1, mn1);
        float d = h2f(hdr[r].x & 0xFFFF), dmin = h2f(hdr[r].x >> 16);
        float a0 = d * (float)sc0, a1 = d * (float)sc1;
        float b0 = dmin * (float)mn0, b1 = dmin * (float)mn1;
#pragma unroll
        for (int n = 0; n < NC; n++)
            acc[r][n] += (a0 * slo[r][n] + a1 * shi[r][n]) - (b0 * xlo[n] + b1 * xhi[n]);
    }
}

// ------------------------------------------------------------- IQ2_XXS --
template <int NC, int R>
__device__ __forceinline__ void unit_iq2_xxs(const uint8_t *const rows[R], uint32_t u,
                                             const float *X, uint32_t K, float (&acc)[R][NC],
                                             const uint2 *grid) {
    uint2 a[R];
    float d[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint8_t *b = rows[r] + (uint64_t)(u >> 3) * 66;
        d[r] = h2f(ldu<uint16_t>(b));
        a[r] = ldu<uint2>(b + 2 + (u & 7) * 8);
    }
    float s[R][NC];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int n = 0; n < NC; n++) s[r][n] = 0;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        XSlice<NC> xs;
        load_x16<NC>(X, K, u * 32 + h * 16, xs);
#pragma unroll
        for (int r = 0; r < R; r++) {
#pragma unroll
            for (int ll = 0; ll < 2; ll++) {
                int l = 2 * h + ll;
                uint2 e = grid[byte_of(a[r].x, l)];
                uint32_t sg = iq2_signs((a[r].y >> (7 * l)) & 127);
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    float gv = (float)byte_of(j < 4 ? e.x : e.y, j & 3);
                    // the sign goes into the weight's sign bit
                    gv = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, gv) ^ (((sg >> j) & 1u) << 31));
#pragma unroll
                    for (int n = 0; n < NC; n++) s[r][n] += gv * xs.v[n][ll * 8 + j];
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        float db = d[r] * (0.5f + (float)(a[r].y >> 28)) * 0.25f;
#pragma unroll
        for (int n = 0; n < NC; n++) acc[r][n] += db * s[r][n];
    }
}

// ------------------------------------------------------------- kernel --
template <int F, int NC, int R>
__global__ __launch_bounds__(256) void gemv_kernel(const uint8_t *__restrict__ W, uint64_t row_bytes,
                                                   uint32_t K, uint32_t M,
                                                   const float *__restrict__ X,
                                                   float *__restrict__ Y,
                                                   const uint2 *__restrict__ grid_g) {
    __shared__ uint2 grid[F == IQ2_XXS ? 256 : 1];
    if constexpr (F == IQ2_XXS) {
        grid[threadIdx.x] = grid_g[threadIdx.x];
        __syncthreads();
    }
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t m0 = (blockIdx.x * 4 + wave) * R;
    if (m0 >= M) return;
    const uint8_t *rows[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        uint32_t m = m0 + r < M ? m0 + r : M - 1;  // clamp: result discarded
        rows[r] = W + (uint64_t)m * row_bytes;
    }
    float acc[R][NC];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int n = 0; n < NC; n++) acc[r][n] = 0;
    const uint32_t units = K / 32;
    for (uint32_t u = lane; u < units; u += 64) {
        if constexpr (F == Q8_0) unit_q8_0<NC, R>(rows, u, X, K, acc);
        else if constexpr (F == Q2_0) unit_q2_0<NC, R>(rows, u, X, K, acc);
        else if constexpr (F == Q4_K) unit_q4_k<NC, R>(rows, u, X, K, acc);
        else unit_iq2_xxs<NC, R>(rows, u, X, K, acc, grid);
    }
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int n = 0; n < NC; n++) {
            float v = wave_sum(acc[r][n]);
            if (lane == 0 && m0 + r < M) Y[(uint64_t)n * M + m0 + r] = v;
        }
}

}  // namespace okf
