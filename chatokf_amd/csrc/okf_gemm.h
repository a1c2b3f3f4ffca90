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

template <int F>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(const uint8_t *__restrict__ W,
                                                        uint64_t row_bytes, uint32_t K, uint32_t M,
                                                        const float *__restrict__ X, uint32_t N,
                                                        float *__restrict__ Y,
                                                        const uint2 *__restrict__ grid_g) {
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

    for (uint32_t k0 = 0; k0 < K; k0 += GB_K) {
        __syncthreads();  // previous step's fragments are consumed (and grid loaded)
        const uint32_t u = k0 / 32 + lh;
        _Float16 *ad = As + lr * G_LDS_STRIDE + lh * 32;
        _Float16 *bd = Bs + lr * G_LDS_STRIDE + lh * 32;
        if (u < units) {
            float w[32];
            decode_unit<F>(wrow, u, w, grid);
            store_half32(ad, w);
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
            float *dst = Y + (uint64_t)n * M + m;
            if (m + 3 < M && (M & 3) == 0) {
                *(float4 *)dst = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (m + e < M) dst[e] = acc[i][j][e];
            }
        }
}

// One thread per 32-weight unit of a row; bit-exact with the CPU decoders.
template <int F>
__global__ __launch_bounds__(256) void dequant_row_kernel(const uint8_t *__restrict__ row,
                                                          uint32_t units, float *__restrict__ out,
                                                          const uint2 *__restrict__ grid_g) {
    __shared__ uint2 grid[F == IQ2_XXS ? 256 : 1];
    if constexpr (F == IQ2_XXS) {
        grid[threadIdx.x] = grid_g[threadIdx.x];
        __syncthreads();
    }
    const uint32_t u = blockIdx.x * 256 + threadIdx.x;
    if (u >= units) return;
    float w[32];
    decode_unit<F>(row, u, w, grid);
    float4 *o = (float4 *)(out + (uint64_t)u * 32);
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = make_float4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
}

}  // namespace okf
