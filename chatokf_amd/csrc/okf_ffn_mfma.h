// okf_ffn_mfma.h -- the one-launch Q2_0 FFN (gate, up, SiLU, down) with the
// dot products on the integer matrix cores (v_mfma_i32_16x16x64_i8), for the
// Bonsai FFN shapes (LLM/Qwen/QwenMetalEngine.swift:918-929, Q2_0 blocks of
// LLM/metal/Kernels.metal's gemv).  Same grid, barrier and outputs as
// ffn_fused_kernel (okf_ffn.h); only the arithmetic of the two phases and
// the activations' staging differ.
//
// Arithmetic, per Q2_0 block of 128 weights (code c in {0, 1, 2}, weight
// d (c - 1)): the block's 128 activations are staged as integers
// X = rint(x 2^(22 - e)), e the binary exponent of the block's largest |x|,
// in three signed byte digits (X = x2 2^16 + x1 2^8 + x0, as in okf_gemv.h),
// plus sum(X) and f = 2^(e - 22).  One MFMA takes 64 weights of 16 rows:
// A = the three digit planes as rows 0-2 (rows 3-15 zero), B = the codes of
// the 16 rows as int8 columns, so C[p][n] = sum(c X_p) of row n exactly, and
// a lane of the first 16 holds the three digit sums of its row in its first
// three accumulators.  Two MFMAs make a block; then, in that lane,
//   T = (s2 << 16) + (s1 << 8) + s0 - sum(X)   (exact: |T| < 2^31)
//   acc += float(T) (d f)
// so the only roundings are T's conversion and the fp32 accumulation over
// blocks.
//
// Byte order (K inside a block): code dword dd (bytes 4 dd .. 4 dd + 3,
// weights 16 dd .. 16 dd + 15, weight 4 b + k of them in field k of byte b)
// gives the B bytes (v >> 2k) & 0x03030303, k = 0..3, byte b of dword k =
// weight 16 dd + 4 b + k; the digit planes are staged in that order (the
// staged order of okf_gemv.h's Q2_0 units), so lane group q's 16 A bytes of
// MFMA t are plane bytes 16 (2 q + t) .. + 15 of the block, and its B bytes
// come from code dword 2 q + t (one 12-byte load per block and lane, which
// for q = 0 holds the block scale too).
//
// Work: workgroup b takes gate / up rows b RA .. b RA + RA - 1 (RA <= 24:
// 2 RA columns in three 16-column tiles) and down rows b RB .. (RB <= 16, one
// tile); wavefront w takes K blocks w NB .. w NB + NB - 1 of every tile, and
// the eight partial sums of a row are added through LDS in wavefront order,
// so results are deterministic.
#pragma once
#include "okf_ffn.h"

namespace okf {

typedef int int32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t FM_RA = 24, FM_RB = 16, FM_T = 512, FM_W = FM_T / 64;

// LDS of ffn_mfma_kernel for K (the larger of gate / up K and down K): the
// three digit planes (K bytes each), 32 zero bytes, one int2 {sum X, f bits}
// a block, the partial sums.
__host__ __device__ constexpr size_t fm_lds_bytes(uint32_t K) {
    return 3 * (size_t)K + 32 + (size_t)(K / 128) * 8 + FM_W * 48 * 4;
}

// Staging of n values (n / 8 slots of 8, slot s of block s / 16 in the staged
// order of load_slot<Q2_0>) as digit planes with per-block scales.  v: the
// slot's values; the 16 slots of a block are 16 consecutive lanes (a DPP
// row).  Every lane of the wavefront calls this (lanes past the end with
// valid = false: they take part in the row's reductions with zeros).
__device__ __forceinline__ void fm_stage_slot(const float (&v)[8], uint32_t s, bool valid, uint8_t *planes,
                                              uint32_t K, int2 *gd) {
    float m = 0, bad = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        m = fmaxf(m, fabsf(v[k]));
        bad = fmaf(v[k], 0.0f, bad);  // NaN for an inf or NaN value
    }
    m = quad_max(m);
    m = fmaxf(m, dpp<DPP_HALF_MIRROR>(m));
    m = fmaxf(m, dpp<DPP_MIRROR>(m));
    bad = quad_sum(bad);
    bad += dpp<DPP_HALF_MIRROR>(bad);
    bad += dpp<DPP_MIRROR>(bad);
    const int e = max(min(__builtin_amdgcn_frexp_expf(m), 127), -104);
    const float sc = __builtin_amdgcn_ldexpf(1.0f, 22 - e);
    uint32_t y[8];
    uint32_t sy = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        // X + 0x808080 (unsigned digits) from one fma with 1.5 * 2^23
        y[k] = __builtin_bit_cast(uint32_t, fmaf(v[k], sc, 12582912.0f)) - 0x4ABF7F80u;
        sy += y[k];
    }
    uint2 pl[3];
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
    int sx = valid ? (int)(sy - 8u * 0x808080u) : 0;
    sx += dppi<DPP_QUAD_XOR1>(sx);
    sx += dppi<DPP_QUAD_XOR2>(sx);
    sx += dppi<DPP_HALF_MIRROR>(sx);
    sx += dppi<DPP_MIRROR>(sx);
    if (valid) {
#pragma unroll
        for (int p = 0; p < 3; p++) *(uint2 *)(planes + p * K + 8 * s) = pl[p];
        if ((s & 15) == 0)
            gd[s >> 4] = make_int2(sx, (int)__builtin_bit_cast(uint32_t, __builtin_amdgcn_ldexpf(1.0f, e - 22) + bad));
    }
}

// A lane's bytes of one block: 12 bytes from byte 8 q of the block (8 q - 2
// for q = 3, so that no load passes the block's end): its two code dwords
// (block bytes 2 + 8 q .. 9 + 8 q) at byte 2 of them (byte 4, dwords 1 and
// 2, for q = 3), and for q = 0 the block scale d in the first two.
__device__ __forceinline__ uint32_t fm_off(uint32_t q) { return 8 * q - (q == 3 ? 2 : 0); }

// One 16-column tile over NB blocks: acc (lanes 0-15: column lane) +=
// sum over the blocks of d (sum (c - 1) x).  raw[i]: this lane's 12 bytes of
// block i, q3: lane group 3 (fm_off); abase: this lane's A bytes of block 0
// (its plane, or the zero bytes), ablk: bytes a block in LDS (128 for a
// plane, 0 for the zeros).  KS (the K-split tile of q2m_gemv_kernel):
// lanes 16-31 hold sums too (A rows 4-6, the planes of the other K half),
// and take d from lane - 16, which loaded the block's first bytes.
template <int NB, bool KS = false>
__device__ __forceinline__ void fm_tile(const uint3 (&raw)[NB], bool q3, const uint8_t *abase, uint32_t ablk,
                                        const int2 *gd, float &acc) {
#pragma unroll
    for (int i = 0; i < NB; i++) {
        int32x4 c = {0, 0, 0, 0};
#pragma unroll
        for (int t = 0; t < 2; t++) {
            // code dword 2 q + t (v_alignbyte takes the byte shift mod 4)
            const uint32_t v = t ? (q3 ? raw[i].z : __builtin_amdgcn_alignbyte(raw[i].z, raw[i].y, 2))
                                 : (q3 ? raw[i].y : __builtin_amdgcn_alignbyte(raw[i].y, raw[i].x, 2));
            const int32x4 b = {(int)(v & 0x03030303u), (int)((v >> 2) & 0x03030303u), (int)((v >> 4) & 0x03030303u),
                               (int)((v >> 6) & 0x03030303u)};
            const int32x4 a = *(const int32x4 *)(abase + i * ablk + 16 * t);
            c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
        }
        const int2 g = gd[i];
        const int T = (c[2] << 16) + (c[1] << 8) + c[0] - g.x;
        uint32_t dw = raw[i].x;
        if constexpr (KS) dw = (uint32_t)__builtin_amdgcn_ds_bpermute((int)((threadIdx.x & 15) << 2), (int)dw);
        acc = fmaf((float)T, h2f((uint16_t)dw) * __builtin_bit_cast(float, g.y), acc);
    }
}

// NBA / NBB: K blocks a wavefront of gate / up (K = 1024 NBA) and of down
// (K = 1024 NBB).
template <int NBA, int NBB>
__global__ __launch_bounds__(FM_T) void ffn_mfma_kernel(FfnArgs a) {
    constexpr uint32_t KA = 1024 * NBA, KB = 1024 * NBB;
    static_assert(KA / 8 <= FM_T, "one x slot a thread");
    extern __shared__ u32x4 lds[];
    uint8_t *planes = (uint8_t *)lds;
    constexpr uint32_t KM = KA > KB ? KA : KB;
    int2 *gd = (int2 *)(planes + 3 * KM + 32);
    float *red = (float *)(gd + KM / 128);  // [wavefront][48]
    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6, col = lane & 15, q = lane >> 4;
    const uint32_t RA = (a.ma + gridDim.x - 1) / gridDim.x, RB = (a.mb + gridDim.x - 1) / gridDim.x;
#ifdef OKF_TRACE
    uint64_t ftr[FF_TRACE_N] = {}, fep = 0;
#endif
    FF_MARK(0);

    // x's loads first (slot tid of KA / 8), then gate / up's weight loads,
    // unconditional (columns past the rows re-read the last row)
    float xv[8];
    {
        const uint32_t s = min(tid, KA / 8 - 1), u = s >> 3;
        load_slot<Q2_0>(a.x + (uint64_t)u * 64, s & 7, xv);
    }
    __builtin_amdgcn_sched_barrier(0);
    // one 12-byte load a block (fm_off)
    uint3 ca[3][NBA], cb[NBB];
    const uint32_t lo = fm_off(q);
#pragma unroll
    for (int t = 0; t < 3; t++) {
        // column n = 16 t + col: gate row n, up row n - RA.  (Written with
        // the clamp outside the select: hipcc 7.2 folded the form
        // gate ? n : min(n - RA, RA - 1) to its second arm and never read a
        // gate row.)
        const uint32_t n = 16 * t + col;
        const bool gate = n < RA;
        const uint32_t k = gate ? n : n - RA;
        const uint32_t r = min(blockIdx.x * RA + min(k, RA - 1), a.ma - 1);
        const uint8_t *row = (gate ? a.wg : a.wu) + (uint64_t)r * a.rba;
#pragma unroll
        for (int i = 0; i < NBA; i++) {
            ca[t][i] = ldu<uint3>(row + (uint64_t)(w * NBA + i) * 34 + lo);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    FF_MARK(1);

    // A bytes: lanes of rows 0-2 read their digit plane, the others zeros
    const bool arow = col < 3;
    if (tid < 8) ((uint32_t *)(planes + 3 * KM))[tid] = 0;
    fm_stage_slot(xv, tid, tid < KA / 8, planes, KA, gd);
    __syncthreads();
    FF_MARK(2);
    // the down projection's weights only now: issued at the start they
    // shared the first microseconds' stream with gate / up's, which phase A
    // waits for (launch span 8.6 -> 8.1 us); they arrive during phase A and
    // the barrier
    {
        const uint32_t r = min(blockIdx.x * RB + min(col, RB - 1), a.mb - 1);
        const uint8_t *row = a.wd + (uint64_t)r * a.rbb;
#pragma unroll
        for (int i = 0; i < NBB; i++) cb[i] = ldu<uint3>(row + (uint64_t)(w * NBB + i) * 34 + lo);
    }
    __builtin_amdgcn_sched_barrier(0);

    // phase A: three tiles of gate / up columns
    {
        const uint8_t *ab = arow ? planes + col * KA + (w * NBA) * 128 + 32 * q : planes + 3 * KM;
        const uint32_t ablk = arow ? 128 : 0;
        float acc[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < 3; t++) fm_tile<NBA>(ca[t], q == 3, ab, ablk, gd + w * NBA, acc[t]);
        if (lane < 16)
#pragma unroll
            for (int t = 0; t < 3; t++) red[w * 48 + 16 * t + lane] = acc[t];
        __syncthreads();
        if (tid < RA) {
            const uint32_t r = blockIdx.x * RA + tid;
            float gs = 0.0f, us = 0.0f;
#pragma unroll
            for (int v = 0; v < (int)FM_W; v++) {
                gs += red[v * 48 + tid];
                us += red[v * 48 + RA + tid];
            }
            if (r < a.ma) {
                ff_put(a.g + r, silu_mul1(gs, us));
                a.u[r] = us;
            }
        }
    }
    FF_SYNC_MARK(3);
#ifdef OKF_TRACE
    const bool synced = ff_grid_sync(a.bar, a.spin, a.stall, a.status, &fep);
#else
    const bool synced = ff_grid_sync(a.bar, a.spin, a.stall, a.status);
#endif
    FF_MARK(4);

    // phase B: g (written by every workgroup before the barrier) staged the
    // same way, read with device-scope loads, all issued before the staging
    {
        constexpr uint32_t SR = (KB / 8 + FM_T - 1) / FM_T;
        float gv[SR][8];
#pragma unroll
        for (uint32_t k = 0; k < SR; k++) {
            const uint32_t s = min(k * FM_T + tid, KB / 8 - 1), u = s >> 3, su = s & 7;
            const uint64_t *xu = (const uint64_t *)(a.g + (uint64_t)u * 64 + 16 * (su >> 1) + 2 * (su & 1));
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const float2 t = __builtin_bit_cast(
                    float2, __hip_atomic_load(xu + 2 * b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
                gv[k][b] = t.x;
                gv[k][4 + b] = t.y;
            }
        }
        __syncthreads();  // every wavefront is past phase A's reads of the planes
#pragma unroll
        for (uint32_t k = 0; k < SR; k++)
            if (k * FM_T < KB / 8)  // (the whole workgroup)
                fm_stage_slot(gv[k], k * FM_T + tid, k * FM_T + tid < KB / 8, planes, KB, gd);
    }
    __syncthreads();
    FF_MARK(5);
    {
        const uint8_t *ab = arow ? planes + col * KB + (w * NBB) * 128 + 32 * q : planes + 3 * KM;
        const uint32_t ablk = arow ? 128 : 0;
        float acc = 0.0f;
        fm_tile<NBB>(cb, q == 3, ab, ablk, gd + w * NBB, acc);
        if (lane < 16) red[w * 48 + lane] = acc;
        __syncthreads();
        if (tid < RB) {
            const uint32_t r = blockIdx.x * RB + tid;
            float ys = 0.0f;
#pragma unroll
            for (int v = 0; v < (int)FM_W; v++) ys += red[v * 48 + tid];
            // a failed barrier leaves NaN in every row of the workgroup
            if (r < a.mb) a.y[r] = synced ? ys : __builtin_nanf("");
        }
    }
    FF_SYNC_MARK(6);
#ifdef OKF_TRACE
    if (threadIdx.x == 0 && blockIdx.x < FF_TRACE_WG) {
        uint64_t *o = ff_trace + ((fep % FF_TRACE_L) * FF_TRACE_WG + blockIdx.x) * FF_TRACE_N;
        ftr[7] = fep;
#pragma unroll
        for (uint32_t k = 0; k < FF_TRACE_N; k++) o[k] = ftr[k];
    }
#endif
}

// ------------------------------------------------------------------------
// The same arithmetic for one Q2_0 matvec (or gate and up paired), the
// reference's gemv (LLM/metal/Kernels.metal:1572-1617) on the Bonsai
// shapes: y = W x, K = 1024 NB, one workgroup per CU taking rows
// b R .. b R + R - 1 (R = ceil(M / grid)) as up to three 16-column tiles;
// x staged per workgroup (with SILU: silu(x) * x2, okf_gemv_silu); with
// PAIR, W0 = gate and W1 = up share x: columns 0 .. R - 1 gate rows, R ..
// 2 R - 1 up rows, and the outputs y0 = silu(gate x) * (up x), y1 = up x
// (okf_gemv_gate_up).  The wavefronts split K as in ffn_mfma_kernel.
struct Q2mArgs {
    const uint8_t *w0, *w1;
    uint64_t rb;
    uint32_t K, M;
    const float *x, *x2;
    float *y0, *y1;
};

// LDS of q2m_gemv_kernel with NW wavefronts: the planes, zeros, block data
// as fm_lds_bytes, the partial sums NW x 48 floats
__host__ __device__ constexpr size_t q2m_lds_bytes(uint32_t K, uint32_t NW) {
    return 3 * (size_t)K + 32 + (size_t)(K / 128) * 8 + (size_t)NW * 48 * 4;
}

// NW wavefronts, each NB K blocks (K = 128 NB NW); NT: the workgroup's
// 16-column tiles, ceil(R / 16) (PAIR: ceil(2 R / 16)), host-checked.
// KS (one tile, R <= 8, not PAIR): columns 8 + r take row r over the second
// half of the wavefront's blocks, whose planes are A rows 4-6, so no column
// repeats a row and a wavefront runs NB / 2 block steps.
template <int NB, int NT, bool PAIR, bool SILU, int NW, bool KS = false>
__global__ __launch_bounds__(NW * 64) void q2m_gemv_kernel(Q2mArgs a) {
    static_assert(!KS || (NT == 1 && !PAIR && NB % 2 == 0), "K split: one tile of one matrix");
    constexpr int NL = KS ? NB / 2 : NB;  // blocks a lane loads
    // WL (with KS): each wavefront stages the x slots of its own K blocks (WS
    // = 16 a block, in rounds of 64) and reads no other wavefront's planes,
    // so no workgroup barrier sits between staging and compute (down 3.67
    // -> 3.64 us, the SiLU down 4.45 -> 4.17; gate / up measured 4.14
    // against 4.10 with it and gate alone 3.62 against 3.58, so they stage as
    // one workgroup, rounds of T)
    constexpr bool WL = KS;
    constexpr uint32_t T = NW * 64, K = 128 * NB * NW, WS = 16 * NB, SN = WL ? 64 : T, SS = WL ? WS : K / 8,
                       SR = (SS + SN - 1) / SN;
    const uint32_t s0 = WL ? (threadIdx.x >> 6) * WS : 0, sl = WL ? (threadIdx.x & 63) : threadIdx.x;
    extern __shared__ u32x4 lds[];
    uint8_t *planes = (uint8_t *)lds;
    int2 *gd = (int2 *)(planes + 3 * K + 32);
    float *red = (float *)(gd + K / 128);  // [wavefront][48]
    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6, col = lane & 15, q = lane >> 4;
    const uint32_t R = (a.M + gridDim.x - 1) / gridDim.x;

    // x's loads (with SILU x2's too), then every weight load
    float xv[SR][8], x2v[SR][8];
#pragma unroll
    for (uint32_t k = 0; k < SR; k++) {
        const uint32_t s = s0 + min(k * SN + sl, SS - 1);
        load_slot<Q2_0>(a.x + (uint64_t)(s >> 3) * 64, s & 7, xv[k]);
        if constexpr (SILU) load_slot<Q2_0>(a.x2 + (uint64_t)(s >> 3) * 64, s & 7, x2v[k]);
    }
    __builtin_amdgcn_sched_barrier(0);
    uint3 cw[NT][NL];
    const uint32_t lo = fm_off(q);
#pragma unroll
    for (int t = 0; t < NT; t++) {
        // column n = 16 t + col: with PAIR gate row n, up row n - R (the
        // clamp outside the select, as in ffn_mfma_kernel); with KS row n % 8
        // of K half n / 8
        const uint32_t n = 16 * t + col;
        const bool first = !PAIR || n < R;
        const uint32_t kk = KS ? (n & 7) : first ? n : n - R;
        const uint32_t r = min(blockIdx.x * R + min(kk, R - 1), a.M - 1);
        const uint8_t *row = (first ? a.w0 : a.w1) + (uint64_t)r * a.rb;
        const uint32_t b0 = w * NB + (KS ? (n >> 3) * NL : 0);
#pragma unroll
        for (int i = 0; i < NL; i++) cw[t][i] = ldu<uint3>(row + (uint64_t)(b0 + i) * 34 + lo);
    }
    __builtin_amdgcn_sched_barrier(0);

    // the 32 zero bytes of the A rows past the planes (with WL every
    // wavefront writes them, the same values)
    if ((WL ? lane : tid) < 8) ((uint32_t *)(planes + 3 * K))[WL ? lane : tid] = 0;
#pragma unroll
    for (uint32_t k = 0; k < SR; k++)
        if (k * SN < SS) {  // (the whole wavefront / workgroup: a block's 16 lanes reduce together)
            if constexpr (SILU)
#pragma unroll
                for (int j = 0; j < 8; j++) xv[k][j] = silu_mul1(xv[k][j], x2v[k][j]);
            fm_stage_slot(xv[k], s0 + k * SN + sl, k * SN + sl < SS, planes, K, gd);
        }
    if constexpr (WL) {
        // the planes are this wavefront's own, and its LDS accesses
        // complete in order
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
    } else {
        __syncthreads();
    }

    // A row ar: plane ar of the first K half (rows 0-2), with KS plane ar - 4
    // of the second (rows 4-6); the other rows read the zeros
    const uint32_t ar = col, ah = KS ? ar >> 2 : 0, ap = ar - 4 * ah;
    // (zero rows as an LDS read like the planes': from registers, a
    // divergent select, they measured 0.04-0.08 us slower)
    const bool arow = ap < 3 && ah < 2;
    const uint8_t *ab = arow ? planes + ap * K + (w * NB + ah * NL) * 128 + 32 * q : planes + 3 * K;
    const uint32_t ablk = arow ? 128 : 0;
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        acc[t] = 0.0f;
        // (KS: lanes 16-31 sum the second half, whose block data follow)
        fm_tile<NL, KS>(cw[t], q == 3, ab, ablk, gd + w * NB + (KS && q == 1 ? NL : 0), acc[t]);
    }
    // KS: row r's halves in lanes r and 24 + r, kept at red[r], red[8 + r]
    if (KS ? (lane < 8 || (lane >= 24 && lane < 32)) : lane < 16)
#pragma unroll
        for (int t = 0; t < NT; t++) red[w * 48 + 16 * t + (KS ? lane & 15 : lane)] = acc[t];
    __syncthreads();
    if (tid < R) {
        const uint32_t r = blockIdx.x * R + tid;
        float v0 = 0.0f, v1 = 0.0f;
#pragma unroll
        for (int v = 0; v < NW; v++) {
            v0 += red[v * 48 + tid];
            if constexpr (KS) v0 += red[v * 48 + 8 + tid];
            if constexpr (PAIR) v1 += red[v * 48 + R + tid];
        }
        if (r < a.M) {
            if constexpr (PAIR) {
                a.y0[r] = silu_mul1(v0, v1);
                a.y1[r] = v1;
            } else {
                a.y0[r] = v0;
            }
        }
    }
}

}  // namespace okf
