// okf_common.h -- shared device helpers for the gfx950 quantized kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace okf {

enum Fmt : int {
    Q4_0 = 2, Q8_0 = 8, Q4_K = 12, Q5_K = 13, Q6_K = 14, IQ2_XXS = 16, IQ2_XS = 17, IQ3_XXS = 18, IQ1_S = 19,
    IQ4_NL = 20, IQ3_S = 21, IQ2_S = 22, IQ4_XS = 23, IQ1_M = 29, Q2_0 = 42,
    F32 = 0, F16 = 1, BF16 = 30, Q2_K = 10, Q3_K = 11
};

// The grid formats past IQ2_XXS (decoded through tables in device memory:
// one buffer, byte offsets below), the small K-quants Q2_K / Q3_K and the
// plain f32 / f16 / bf16 weights take a generic matvec: the bit-exact
// decoder, then fp32 products.
__host__ __device__ constexpr bool grid_fmt(int f) {
    return f == IQ2_XS || f == IQ2_S || f == IQ3_XXS || f == IQ3_S || f == IQ1_S || f == IQ1_M || f == Q2_K ||
           f == Q3_K || f == F32 || f == F16 || f == BF16;
}
// The formats the matvec takes through that generic compute: the plain
// weights (the grid formats and Q2_K / Q3_K have integer computes of their
// own)
__host__ __device__ constexpr bool gen_fmt(int f) {
    return f == F32 || f == F16 || f == BF16;
}
// 16-byte rows of those computes' tables, and where they start in the
// context's table buffer (after IQ2_XXS's 384 rows)
__host__ __device__ constexpr uint32_t itab_rows(int f) {
    return f == IQ3_XXS ? 192 : f == IQ3_S ? 384 : f == IQ2_XS ? 320 : f == IQ2_S ? 640 : 0;
}
__host__ __device__ constexpr uint32_t itab_at(int f) {
    return f == IQ3_XXS ? 384 : f == IQ3_S ? 576 : f == IQ2_XS ? 960 : f == IQ2_S ? 1280 : 0;
}
constexpr uint32_t ITAB_ROWS = 1920;
constexpr uint32_t GT_IQ2XS = 0, GT_IQ2S = 4096, GT_IQ3XXS = 12288, GT_IQ3S = 13312, GT_IQ1S = 15360,
                   GT_BYTES = 23552;
// a grid format's own grid: its offset in that buffer and its size (IQ1_M
// shares IQ1_S's); 0, 0 for the other formats
__host__ __device__ constexpr uint32_t gt_off(int f) {
    return f == IQ2_S ? GT_IQ2S : f == IQ3_XXS ? GT_IQ3XXS : f == IQ3_S ? GT_IQ3S : (f == IQ1_S || f == IQ1_M) ? GT_IQ1S : 0;
}
__host__ __device__ constexpr uint32_t gt_bytes(int f) {
    return f == IQ2_XS ? GT_IQ2S - GT_IQ2XS : f == IQ2_S ? GT_IQ3XXS - GT_IQ2S : f == IQ3_XXS ? GT_IQ3S - GT_IQ3XXS
         : f == IQ3_S ? GT_IQ1S - GT_IQ3S : (f == IQ1_S || f == IQ1_M) ? GT_BYTES - GT_IQ1S : 0;
}

// Bytes of one 256-weight span (Q8_0: 8 blocks, Q2_0: 2 blocks), matching the
// reference's IQArgs.blk (LLM/Base/MetalEnc.swift:162-167).
__host__ __device__ constexpr uint32_t block_bytes(int f) {
    return f == Q8_0 ? 34 : f == Q2_0 ? 34 : f == Q4_K ? 144 : (f == Q4_0 || f == IQ4_NL) ? 18
         : f == Q5_K ? 176 : f == Q6_K ? 210 : f == IQ4_XS ? 136 : f == IQ2_XS ? 74 : f == IQ2_S ? 82
         : f == IQ3_XXS ? 98 : f == IQ3_S ? 110 : f == IQ1_S ? 50 : f == IQ1_M ? 56 : f == Q2_K ? 84
         : f == Q3_K ? 110 : f == F32 ? 128 : (f == F16 || f == BF16) ? 64 : 66;
}
__host__ __device__ constexpr uint32_t block_elems(int f) {
    return (f == Q8_0 || f == Q4_0 || f == IQ4_NL || f == F32 || f == F16 || f == BF16) ? 32 : f == Q2_0 ? 128 : 256;
}

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// Unaligned load: gfx950 runs with unaligned global access enabled, so this
// compiles to one global_load_dword{,x2,x4} at any byte address.
template <class T>
__device__ __forceinline__ T ldu(const uint8_t *p) {
    T v;
    __builtin_memcpy(&v, p, sizeof(T));
    return v;
}

// Exact binary16 -> binary32 (v_cvt_f32_f16).
__device__ __forceinline__ float h2f(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

__device__ __forceinline__ uint32_t byte_of(uint32_t v, uint32_t i) {
    return __builtin_amdgcn_ubfe(v, i * 8, 8);
}

// Sum over the 64 lanes of a wavefront; every lane gets the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// ksigns (LLM/Quantize/IQ2Grid.swift:73): the 7 stored sign bits plus an
// eighth that makes the count of set bits even.
__device__ __forceinline__ uint32_t iq2_signs(uint32_t s7) {
    return s7 | ((__builtin_popcount(s7) & 1u) << 7);
}

// IQ4_NL's 16 levels (IQ4_NL.kvalues, LLM/Gemma/Gemma4Quant.swift:8-11)
__host__ __device__ constexpr int8_t iq4nl_level(int i) {
    constexpr int8_t v[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
    return v[i];
}

}  // namespace okf
