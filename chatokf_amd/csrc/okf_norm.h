// okf_norm.h -- the FFN path's two non-matvec neighbours: the residual add +
// RMSNorm in front of the projections and the argmax over the lm_head output
// behind them.  Both are HBM-streaming row reductions.
#pragma once
#include "okf_common.h"

namespace okf {

constexpr int NORM_THREADS = 256;

// Sum over a workgroup of NORM_THREADS threads (every thread gets it):
// the wavefront's 64 lanes with cross-lane adds, then the 4 wavefront sums
// through LDS in wavefront order.
__device__ __forceinline__ float block_sum(float v, float *red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    const uint32_t w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    const float s = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();  // red is reused by the next call
    return s;
}

// add_rmsnorm_batch (LLM/metal/Kernels.metal:2839-2862) and, with R null,
// rmsnorm_batch (:2818-2836): per row, x += r (stored back), then
// y = x * (1 / sqrt(mean(x^2) + eps)) * w, with w fp32 (llama.cpp's
// build_norm: the stored weight multiplies directly).  One workgroup per
// row; a row is read once into registers when it fits (n <= 4 * 256 * 8),
// else read twice.
template <bool ADD>
__global__ __launch_bounds__(NORM_THREADS) void add_rmsnorm_kernel(float *X,
                                                                   const float *__restrict__ R,
                                                                   const float *__restrict__ Wn,
                                                                   float *Y, uint32_t n,
                                                                   float eps) {
    __shared__ float red[4];
    const uint64_t row = blockIdx.x;
    float *x = X + row * n;
    const float *r = R + (ADD ? row * n : 0);
    float *y = Y + row * n;
    const uint32_t tid = threadIdx.x;
    constexpr uint32_t V = 8;  // float4 per thread kept in registers
    const uint32_t n4 = n / 4;
    floatx4 v[V];
    float ss = 0;
    const bool vec = (n % 4) == 0 && n4 <= V * NORM_THREADS &&
                     (((uintptr_t)X | (uintptr_t)R | (uintptr_t)Wn | (uintptr_t)Y) & 15) == 0;
    if (vec) {
#pragma unroll
        for (uint32_t k = 0; k < V; k++) {
            const uint32_t i = tid + k * NORM_THREADS;
            if (i < n4) {
                floatx4 a = ((const floatx4 *)x)[i];
                if constexpr (ADD) {
                    a += ((const floatx4 *)r)[i];
                    ((floatx4 *)x)[i] = a;
                }
                v[k] = a;
                ss += a[0] * a[0] + a[1] * a[1] + a[2] * a[2] + a[3] * a[3];
            }
        }
    } else {
        for (uint32_t i = tid; i < n; i += NORM_THREADS) {
            float a = x[i];
            if constexpr (ADD) {
                a += r[i];
                x[i] = a;
            }
            ss += a * a;
        }
    }
    const float scale = 1.0f / sqrtf(block_sum(ss, red) / (float)n + eps);
    if (vec) {
#pragma unroll
        for (uint32_t k = 0; k < V; k++) {
            const uint32_t i = tid + k * NORM_THREADS;
            if (i < n4) ((floatx4 *)y)[i] = v[k] * scale * ((const floatx4 *)Wn)[i];
        }
    } else {
        // (each thread re-reads only the elements it wrote itself)
        for (uint32_t i = tid; i < n; i += NORM_THREADS) y[i] = x[i] * scale * Wn[i];
    }
}

// argmax_rows (LLM/metal/Kernels.metal:2756-2795): per row the index of the
// largest value, ties to the lower index; NaN never wins, and a row with no
// value above -inf gives 0 (the kernel's start, bv = -inf, bi = 0).
//
// A 248320-wide vocabulary row is 1 MB, so one row is split over many
// workgroups, in one launch: each reduces ARGMAX_CHUNK values to a
// (value, index) pair, and the last workgroup of a row to finish (counted
// in cnt[row]) reduces the row's pairs in chunk order and sets cnt[row]
// back to 0 for the next call.
// two float4 per thread: ~120 workgroups for a 248320-wide row (measured
// on MI355X: 7.2 us with one float4, 6.2 with two, 6.5 with four)
constexpr uint32_t ARGMAX_CHUNK = NORM_THREADS * 8;

struct ArgPair {
    float v;
    int32_t i;
};

__device__ __forceinline__ void arg_take(float &bv, int32_t &bi, float ov, int32_t oi) {
    if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
    }
}

__device__ __forceinline__ void block_argmax(float &bv, int32_t &bi, ArgPair *red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) arg_take(bv, bi, __shfl_xor(bv, o), __shfl_xor(bi, o));
    const uint32_t w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = ArgPair{bv, bi};
    __syncthreads();
    bv = red[0].v;
    bi = red[0].i;
    for (int k = 1; k < NORM_THREADS / 64; k++) arg_take(bv, bi, red[k].v, red[k].i);
}

// grid (chunks, rows): pairs[row * chunks + chunk]; cnt[rows] are 0 on entry
// and on exit.
__global__ __launch_bounds__(NORM_THREADS) void argmax_kernel(const float *__restrict__ X, uint32_t n,
                                                              ArgPair *__restrict__ pairs, uint32_t *cnt,
                                                              int32_t *__restrict__ out) {
    __shared__ ArgPair red[NORM_THREADS / 64];
    __shared__ uint32_t last;
    const uint32_t c = blockIdx.x, chunks = gridDim.x, row = blockIdx.y;
    const float *x = X + (uint64_t)row * n;
    const uint32_t b = c * ARGMAX_CHUNK, e = min(b + ARGMAX_CHUNK, n);
    float bv = -__builtin_inff();
    int32_t bi = 0;
    if ((n & 3) == 0 && ((uintptr_t)X & 15) == 0) {
        // float4 loads: thread t takes quads t, t + 256, ... of the chunk
        for (uint32_t i = b + 4 * threadIdx.x; i < e; i += 4 * NORM_THREADS) {
            const floatx4 q = *(const floatx4 *)(x + i);
#pragma unroll
            for (int k = 0; k < 4; k++)
                if (q[k] > bv) {  // (in index order: a tie keeps the first)
                    bv = q[k];
                    bi = (int32_t)(i + k);
                }
        }
    } else {
        for (uint32_t i = b + threadIdx.x; i < e; i += NORM_THREADS)
            if (x[i] > bv) {
                bv = x[i];
                bi = (int32_t)i;
            }
    }
    block_argmax(bv, bi, red);
    ArgPair *p = pairs + (uint64_t)row * chunks;
    // Cross-workgroup hand-off without fences.  The pair is stored and the
    // row's counter incremented as agent-scope relaxed atomics (on gfx950
    // these are issued with the sc1 bit: coherent across the XCDs' L2s);
    // s_waitcnt vmcnt(0) between them makes the pair's store complete at
    // the coherence point before the count that announces it is issued.
    // The last workgroup reads the pairs with agent-scope atomic loads.
    // (An acquire-release counter costs an L2 write-back and invalidate per
    // workgroup: measured 9.7 us for a 248320-wide row, against 5.6 us with
    // this scheme.)
    if (threadIdx.x == 0) {
        const uint64_t pk = (uint64_t)__float_as_uint(bv) | ((uint64_t)(uint32_t)bi << 32);
        __hip_atomic_store((uint64_t *)(p + c), pk, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
        const uint32_t prev = __hip_atomic_fetch_add(cnt + row, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = prev == chunks - 1;
    }
    __syncthreads();
    if (!last) return;
    bv = -__builtin_inff();
    bi = 0;
    for (uint32_t k = threadIdx.x; k < chunks; k += NORM_THREADS) {
        const uint64_t q = __hip_atomic_load((const uint64_t *)(p + k), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        arg_take(bv, bi, __uint_as_float((uint32_t)q), (int32_t)(q >> 32));
    }
    __syncthreads();  // (red is reused)
    block_argmax(bv, bi, red);
    if (threadIdx.x == 0) {
        out[row] = bi;
        __hip_atomic_store(cnt + row, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

}  // namespace okf

namespace okf {

// Streaming read of a byte range: the attainable single-launch HBM read rate
// that the matvec rows are compared with (no reference counterpart; it is a
// measurement of the machine).  1024-thread workgroups, one to four per CU
// (the launch picks by size); each owns a contiguous range of 16-byte chunks and keeps four loads per thread
// in flight.  The xor of every dword is folded into *out (one atomic per
// wavefront), so the read cannot be elided and its result can be checked.
constexpr int SR_THREADS = 1024, SR_U = 4;
static __global__ __launch_bounds__(SR_THREADS) void stream_read_kernel(const u32x4 *__restrict__ p, uint64_t n16,
                                                                      uint64_t per_wg, uint32_t *out) {
    const uint64_t b = (uint64_t)blockIdx.x * per_wg, e = min(b + per_wg, n16);
    uint32_t acc = 0;
    uint64_t i = b + threadIdx.x;
    for (; i + (SR_U - 1) * SR_THREADS < e; i += SR_U * SR_THREADS) {
        u32x4 v[SR_U];
#pragma unroll
        for (int u = 0; u < SR_U; u++) v[u] = p[i + u * SR_THREADS];
#pragma unroll
        for (int u = 0; u < SR_U; u++) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
    for (; i < e; i += SR_THREADS) {
        const u32x4 v = p[i];
        acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc ^= __shfl_xor(acc, o);
    if ((threadIdx.x & 63) == 0 && acc) atomicXor(out, acc);
}

}  // namespace okf
