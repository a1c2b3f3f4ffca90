// okf_gemv_wide.h -- matvec / narrow matmul for matrices large enough to
// give every CU many rows: one 1024-thread workgroup per CU.
//
// Workgroup b owns the contiguous rows [b M / G, (b + 1) M / G).  Its 64 row
// slots (16 wavefronts x 4 slots of 16 lanes) split those rows' steps (a step
// = 16 consecutive units of one row, one unit per lane) into 64 contiguous
// ranges, so every slot does the same work whatever M and K are.  A range
// may start or end inside a row: at each row boundary the slot reduces its
// partial sum over its 16 lanes and parks it in LDS, and after one barrier
// each row adds the partials of the slots that cover it, in slot order (a
// fixed order, so the result does not depend on timing).
//
// All of a lane's weight loads for its first D steps are issued before the
// activations are staged, and each slot runs only ~M K / (16 * 64 * G * UW)
// steps, so at the configurations of this path (17408 x 5120) every weight
// byte of the kernel is requested in the first microsecond.
//
// IQ2_XXS: the grid and sign tables (384 rows of 16 bytes) are replicated
// 16 times in LDS as [row][copy], so that lane i of a slot reads copy i: the
// 16 lanes of a slot then always hit 16 different 16-byte bank groups, where
// a single copy read at random rows conflicts.  Measured on MI355X with
// random rows: 11.5 clocks per wavefront-wide 16-byte read and CU with one
// copy, 4.7 (the conflict-free rate) with 16.
#pragma once
#include "okf_gemv.h"

namespace okf {

constexpr int GW_THREADS = 1024;
constexpr uint32_t GW_SLOTS = GW_THREADS / GV_L;  // row slots per workgroup
constexpr uint32_t GW_TAB = 384 * GV_L;           // replicated IQ2_XXS table rows (u32x4)

// Step s of the workgroup -> first step of slot z: floor(z T / 64).
__device__ __forceinline__ uint32_t gw_start(uint32_t z, uint32_t T) {
    return (uint32_t)((uint64_t)z * T / GW_SLOTS);
}

// Dynamic LDS: [replicated IQ2_XXS tables], NC columns of staged digit
// planes (cs uint32 each), NC columns of group data (gcs float4 each), then
// the parked partials [64 slots][kmax rows][NC].
template <int F, int NC, int D, uint32_t SP>
__global__ __launch_bounds__(GW_THREADS) void gemv_wide_kernel(const uint8_t *__restrict__ W,
                                                               uint64_t row_bytes, uint32_t K, uint32_t M,
                                                               const float *__restrict__ X,
                                                               float *__restrict__ Y,
                                                               const u32x4 *__restrict__ tab_g,
                                                               uint32_t kmax) {
    constexpr int L = GV_L;
    constexpr uint32_t UW = unit_weights<F>(), SL = UW / 8;
    constexpr uint32_t TAB = F == IQ2_XXS ? GW_TAB : 0;
    extern __shared__ u32x4 lds[];
    const uint32_t tid = threadIdx.x, i = tid % L, z = tid / L;
    const uint32_t r0 = (uint32_t)((uint64_t)blockIdx.x * M / gridDim.x);
    const uint32_t r1 = (uint32_t)((uint64_t)(blockIdx.x + 1) * M / gridDim.x);
    if (r0 == r1) return;  // whole workgroup: no rows (M < grid)
    const uint32_t units = K / UW, P = (units + L - 1) / L;  // steps per row
    const uint32_t T = (r1 - r0) * P, s0 = gw_start(z, T), s1 = gw_start(z + 1, T);
    constexpr uint32_t UG = unit_groups<F>();
    const uint32_t cunits = P * L, cs = cunits * unit_chunks<F>() * 4, gcs = cunits * UG;
    u32x4 *tab = lds;
    uint32_t *xs = (uint32_t *)(lds + TAB);
    floatx4 *gdp = (floatx4 *)(xs + NC * cs);
    float *part = (float *)(gdp + NC * gcs);

    // Weight loads walk the slot's steps in order: step ls is unit
    // lsu L + i of row lrow.  The cursor stops at the range's last step, so
    // the loads past it (and those of an empty range) re-read that unit and
    // stay in bounds (s0 < T for every slot).
    const uint8_t *lrow = W + (uint64_t)(r0 + s0 / P) * row_bytes;
    uint32_t ls = s0, lsu = s0 % P;
    auto load_next = [&](Unit<F, 1> &w) {
        const uint8_t *rows[1] = {lrow};
        load_unit<F, 1>(rows, min(lsu * L + i, units - 1), w);
        if (ls + 1 < s1) {
            ls++;
            if (++lsu == P) {
                lsu = 0;
                lrow += row_bytes;
            }
        }
    };
    // Loads in this order: the table row and the activations this thread
    // stages, then the weight ring.  Loads complete in issue order, so the
    // staging then waits for its own loads only, while the weights stream.
    // (every thread loads and writes TAB / 1024 = 6 table entries, no branch,
    // so the compiler keeps the loads here)
    constexpr uint32_t TPT = TAB / GW_THREADS;
    static_assert(TAB % GW_THREADS == 0, "table entries per thread");
    u32x4 trow[TPT ? TPT : 1];
#pragma unroll
    for (uint32_t k = 0; k < TPT; k++) trow[k] = tab_g[(tid + k * GW_THREADS) / L];
    const uint32_t nslots = units * SL;  // <= SP * GW_THREADS (host-checked)
    float v[SP][NC][8];
#pragma unroll
    for (uint32_t p = 0; p < SP; p++) {
        const uint32_t q = min(p * GW_THREADS + tid, nslots - 1), u = q / SL;
#pragma unroll
        for (int n = 0; n < NC; n++) load_slot<F>(X + (uint64_t)n * K + unit_x_base<F>(u), q % SL, v[p][n]);
    }
    __builtin_amdgcn_sched_barrier(0);  // (keep the order of the loads)
    Unit<F, 1> buf[D];
#pragma unroll
    for (int j = 0; j < D; j++) load_next(buf[j]);
    __builtin_amdgcn_sched_barrier(0);

#pragma unroll
    for (uint32_t k = 0; k < TPT; k++) tab[tid + k * GW_THREADS] = trow[k];
    // x as digit planes and group data (as stage_x)
#pragma unroll
    for (uint32_t p = 0; p < SP; p++) {
        const uint32_t q = p * GW_THREADS + tid;
        stage_slot<F, NC, L, false>(v[p], q / SL, q % SL, q < nslots, xs, cs, gdp, gcs);
    }
    __syncthreads();

    // walk the slot's steps; (rl, su) = (row, step within row) of step s
    float acc[1][NC];
#pragma unroll
    for (int n = 0; n < NC; n++) acc[0][n] = 0;
    uint32_t rl = s0 / P, su = s0 - rl * P, k = 0;
    auto flush = [&]() {
#pragma unroll
        for (int n = 0; n < NC; n++) {
            const float v = slot_sum<L>(acc[0][n]);
            if (i == 0) part[(z * kmax + k) * NC + n] = v;
            acc[0][n] = 0;
        }
    };
    for (uint32_t t = s0; t < s1; t += D) {
#pragma unroll
        for (int j = 0; j < D; j++) {
            if (t + j < s1) {
                const uint32_t u = su * L + i;
                if (u < units)
                    Compute<F, NC, 1, (F == IQ2_XXS ? L : 1)>::run(
                        buf[j], XLds{xs + xs_index<F, L>(u, 0), 4 * L, cs, gdp + u * UG, gcs}, u, acc,
                        tab + i);
                if (++su == P && t + j + 1 < s1) {  // next step starts a row
                    flush();
                    su = 0;
                    rl++;
                    k++;
                }
            }
            load_next(buf[j]);
        }
    }
    if (s0 < s1) flush();
    __syncthreads();

    // each row: the partials of slots zA..zB (those whose range meets it)
    const uint32_t n_rows = r1 - r0;
    for (uint32_t e = tid; e < n_rows * NC; e += GW_THREADS) {
        const uint32_t rho = e / NC, n = e % NC;
        const uint32_t sa = rho * P, sb = sa + P - 1;
        // (T * 64 < 2^32, host-checked)
        const uint32_t za = ((sa + 1) * GW_SLOTS - 1) / T, zb = ((sb + 1) * GW_SLOTS - 1) / T;
        float v = 0;
        for (uint32_t zz = za; zz <= zb; zz++) {
            const uint32_t st = gw_start(zz, T);
            if (st < gw_start(zz + 1, T)) v += part[(zz * kmax + (rho - st / P)) * NC + n];
        }
        Y[(uint64_t)n * M + r0 + rho] = v;
    }
    (void)rl;
}

// ------------------------------------------------------------------------
// IQ2_XXS with 2..4 activation columns on the matrix cores.
//
// v_mfma_f32_4x4x4_16b_f16 computes 16 independent 4x4x4 products; in block
// b (lanes 4b..4b+3) lane t supplies row t of A and column t of B and
// receives column t of D (one VGPR per row of D).  Here A = 4 activation
// columns x 4 consecutive k (zero for columns past NC) and B = 4 k of 4
// weight rows, so a wavefront is one row quad (lane t: row t of the quad)
// times 16 units (block b: unit b of the step), and lane t's D is row t's
// dot product with each of the 4 columns for its unit: sub-block scales
// are applied lane-locally, and the 16 blocks are summed over lanes once
// per row quad.  Each lane's 4 weights x 4 columns take one MFMA where the
// dot2 kernel takes 2 v_dot2 per column, so the weight decode (table reads
// + sign XOR) is what remains, shared by the columns.  Measured at
// 17408 x 5120: N = 2 18.6 -> 16.2 us, N = 4 22.7 -> 17.3 us.
//
// Activations in LDS, per unit u: 8 k-slots s of 8 halves for each of the 4
// columns c, hi at 16-byte slot u * 68 + s * 4 + c and lo 32 slots further
// (the 4 slots of padding per unit put the 16 lanes of a read on 16
// distinct 16-byte bank groups); after them the per-32 scales, one float4
// (the 4 columns) per (unit, sub-block).  The tables are replicated 8 times
// (lane i reads copy i % 8), which leaves room for the hi / lo activations
// of 4 columns at K = 5120.
constexpr uint32_t GM_WAVES = GW_THREADS / 64;
constexpr uint32_t GM_UNIT = 68;  // 16-byte x slots per unit
constexpr uint32_t GM_COPIES = 8;
constexpr uint32_t GM_TAB = 384 * GM_COPIES;

typedef _Float16 half4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    const half2v h = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, h);
}
// 8 values in order as 4 packed fp16 pairs
__device__ __forceinline__ u32x4 pack_h8(floatx4 A, floatx4 B) {
    return u32x4{pack_h2(A[0], A[1]), pack_h2(A[2], A[3]), pack_h2(B[0], B[1]), pack_h2(B[2], B[3])};
}

__device__ __forceinline__ uint32_t gm_start(uint32_t z, uint32_t T) {
    return (uint32_t)((uint64_t)z * T / GM_WAVES);
}

// int8 bytes b (4) -> two dwords of fp16 pairs of 1152 + b (exact); the
// caller subtracts 1152 (or folds it into an fma)
__device__ __forceinline__ void i8_h2(uint32_t b4, uint32_t &lo, uint32_t &hi) {
    const uint32_t u = b4 ^ 0x80808080u;  // b + 128, 0..255
    lo = perm(0x64646464u, u, 0x04010400u);
    hi = perm(0x64646464u, u, 0x04030402u);
}

// Q8_0's unit here: blocks 2u, 2u + 1 (64 weights)
struct Q8Pair {
    uint32_t d[2];
    u32x4 q[2][2];
};
template <int F>
struct MMUnit {
    using type = Unit<F, 1>;
};
template <>
struct MMUnit<Q8_0> {
    using type = Q8Pair;
};

// The body of the 2..4-column matrix-core kernels, per 64-weight unit (two
// 32-weight sub-blocks): F = IQ2_XXS (weights from the replicated fp16
// tables), Q4_K / Q5_K (weights sc * q, exact in fp16, from the nibbles and
// the fifth bit; the mins through the per-32 activation sums staged beside
// the scales), IQ4_XS (the levels, scale per sub-block), Q8_0 (the int8
// codes, scale per block), the grid formats (their signed int8 grid values
// from the matvec's tables, copied once to LDS; a scale per 32 or per 16
// weights) or Q2_K / Q3_K (the small codes, a scale per 16 weights and the
// per-16 activation sums for their offsets).
template <int F, int NC, int D, uint32_t SP>
__device__ __forceinline__ void wide_mm_body(const uint8_t *__restrict__ W, uint64_t row_bytes, uint32_t K,
                                             uint32_t M, const float *__restrict__ X, float *__restrict__ Y,
                                             const u32x4 *__restrict__ tab_g, uint32_t kmax) {
    static_assert(F == IQ2_XXS || F == Q4_K || F == Q5_K || F == IQ4_XS || F == Q8_0 || F == IQ3_XXS ||
                      F == IQ3_S || F == IQ2_XS || F == IQ2_S || F == IQ1_S || F == IQ1_M || F == Q2_K || F == Q3_K,
                  "matrix-core narrow formats");
    constexpr bool MINS = F == Q4_K || F == Q5_K;
    // (IQ2_XS, IQ2_S, IQ1_M, Q2_K, Q3_K: a scale per 16 weights, one per
    // pair of 8-weight steps l) the activations' per-16 sums where the
    // format subtracts a multiple of them
    constexpr bool HSUM = F == Q2_K || F == Q3_K;
    // tables: IQ2_XXS's fp16 rows replicated GM_COPIES times; the other grid
    // formats' integer tables (the matvec's) once
    constexpr uint32_t TREP = F == IQ2_XXS ? GM_COPIES : 1;
    constexpr uint32_t TABR = F == IQ2_XXS ? GM_TAB : (F == IQ1_S || F == IQ1_M) ? 512 : itab_rows(F);
    constexpr int L = GV_L;
    constexpr uint32_t UW = 64;
    extern __shared__ u32x4 lds[];
    const uint32_t tid = threadIdx.x, lane = tid & 63, z = tid >> 6;
    const uint32_t t = lane & 3, q = lane >> 2;  // row in the quad, unit in the step
    const uint32_t r0 = (uint32_t)((uint64_t)blockIdx.x * M / gridDim.x);
    const uint32_t r1 = (uint32_t)((uint64_t)(blockIdx.x + 1) * M / gridDim.x);
    if (r0 == r1) return;
    const uint32_t units = K / UW, P = (units + L - 1) / L;
    const uint32_t nq = (r1 - r0 + 3) / 4, T = nq * P, s0 = gm_start(z, T), s1 = gm_start(z + 1, T);
    u32x4 *tab = lds;
    u32x4 *xs = lds + TABR;
    floatx4 *xf = (floatx4 *)(xs + (size_t)P * L * GM_UNIT);
    floatx4 *xsum = xf + (size_t)P * L * 2;  // per-32 (Q4_K, Q5_K) or per-16 (Q2_K, Q3_K) sums of x
    float *part = (float *)(xsum + (MINS ? (size_t)P * L * 2 : HSUM ? (size_t)P * L * 4 : 0));

    // loads: table entries, then activations, then the weight ring
    constexpr uint32_t TPT = (TABR + GW_THREADS - 1) / GW_THREADS;
    u32x4 trow[TPT > 0 ? TPT : 1];
#pragma unroll
    for (uint32_t k = 0; k < TPT; k++) trow[k] = tab_g[min(tid + k * GW_THREADS, TABR - 1) / TREP];
    const uint32_t nx = units * 8 * 4;  // (unit, k-slot, column) entries, <= SP * 1024
    floatx4 A[SP], B[SP];
#pragma unroll
    for (uint32_t p = 0; p < SP; p++) {
        const uint32_t e = min(p * GW_THREADS + tid, nx - 1), c = e & 3;
        const uint64_t xo = (uint64_t)min(c, (uint32_t)NC - 1) * K + (e >> 2) * 8;
        A[p] = *(const floatx4 *)(X + xo);
        B[p] = *(const floatx4 *)(X + xo + 4);
    }
    __builtin_amdgcn_sched_barrier(0);
    // weight cursor: step ls = unit lsu * 16 + q of row 4 quad + t
    const uint32_t lrow0 = r0 + (s0 / P) * 4 + t;
    const uint8_t *lrow = W + (uint64_t)min(lrow0, r1 - 1) * row_bytes;
    uint32_t ls = s0, lsu = s0 % P, lr = lrow0;
    using UnitT = typename MMUnit<F>::type;
    auto load_next = [&](UnitT &w) {
        const uint32_t uu = min(lsu * L + q, units - 1);
        if constexpr (F == Q8_0) {
#pragma unroll
            for (int b = 0; b < 2; b++) {
                const uint8_t *bp = lrow + (uint64_t)(2 * uu + b) * 34;
                w.d[b] = ldu<uint16_t>(bp);
                w.q[b][0] = ldu<u32x4>(bp + 2);
                w.q[b][1] = ldu<u32x4>(bp + 18);
            }
        } else {
            const uint8_t *rows[1] = {lrow};
            load_unit<F, 1>(rows, uu, w);
        }
        if (ls + 1 < s1) {
            ls++;
            if (++lsu == P) {
                lsu = 0;
                lr += 4;
                lrow = W + (uint64_t)min(lr, r1 - 1) * row_bytes;
            }
        }
    };
    UnitT buf[D];
#pragma unroll
    for (int j = 0; j < D; j++) load_next(buf[j]);
    __builtin_amdgcn_sched_barrier(0);

#pragma unroll
    for (uint32_t k = 0; k < TPT; k++)
        if (tid + k * GW_THREADS < TABR) tab[tid + k * GW_THREADS] = trow[k];
#pragma unroll
    for (uint32_t p = 0; p < SP; p++) {
        // (c, sl, u) = lane bits 0-1, 2-4, 5-: a 32-weight group of column c
        // is k-slots 0-3 or 4-7, the lanes that differ in bits 2 and 3; its
        // scale and hi / lo split as split_slot's
        const uint32_t e = p * GW_THREADS + tid;
        const uint32_t c = e & 3, sl = (e >> 2) & 7, u = e >> 5;
        float m = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) m = fmaxf(m, fmaxf(fabsf(A[p][k]), fabsf(B[p][k])));
        m = fmaxf(m, __shfl_xor(m, 4, 64));
        m = fmaxf(m, __shfl_xor(m, 8, 64));
        const int ex = min(__builtin_amdgcn_frexp_expf(m), 127);
        float sx = 0;  // (MINS, HSUM) the group's (half group's) sum of x
        if constexpr (MINS || HSUM) {
#pragma unroll
            for (int k = 0; k < 4; k++) sx += A[p][k];
#pragma unroll
            for (int k = 0; k < 4; k++) sx += B[p][k];
            sx += __shfl_xor(sx, 4, 64);
            if constexpr (MINS) sx += __shfl_xor(sx, 8, 64);
        }
        floatx4 Ah, Al, Bh, Bl;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float a = __builtin_amdgcn_ldexpf(A[p][k], -ex), b = __builtin_amdgcn_ldexpf(B[p][k], -ex);
            Ah[k] = (float)(_Float16)a;
            Bh[k] = (float)(_Float16)b;
            Al[k] = a - Ah[k];
            Bl[k] = b - Bh[k];
        }
        u32x4 hi = pack_h8(Ah, Bh), lo = pack_h8(Al, Bl);
        float f = __builtin_amdgcn_ldexpf(1.0f, ex);
        if (c >= (uint32_t)NC) {
            hi = lo = u32x4{0, 0, 0, 0};
            f = 0;
            sx = 0;
        }
        if (e < nx) {
            xs[u * GM_UNIT + sl * 4 + c] = hi;
            xs[u * GM_UNIT + 32 + sl * 4 + c] = lo;
            if ((sl & 3) == 0) {
                ((float *)xf)[(u * 2 + (sl >> 2)) * 4 + c] = f;
                if constexpr (MINS) ((float *)xsum)[(u * 2 + (sl >> 2)) * 4 + c] = sx;
            }
            if constexpr (HSUM)
                if ((sl & 1) == 0) ((float *)xsum)[(u * 4 + (sl >> 1)) * 4 + c] = sx;
        }
    }
    __syncthreads();

    floatx4 tot = {0, 0, 0, 0};
    uint32_t su = s0 % P, k = 0;
    const u32x4 *tl = tab + (lane & (GM_COPIES - 1));  // this lane's table copy
    auto flush = [&]() {
#pragma unroll
        for (int c = 0; c < 4; c++) {
            float v = tot[c];
            v += __shfl_xor(v, 4);
            v += __shfl_xor(v, 8);
            v += __shfl_xor(v, 16);
            v += __shfl_xor(v, 32);
            tot[c] = v;
        }
        if (q == 0)
#pragma unroll
            for (int c = 0; c < NC; c++) part[((z * kmax + k) * 4 + t) * NC + c] = tot[c];
        tot = floatx4{0, 0, 0, 0};
    };
    for (uint32_t st = s0; st < s1; st += D) {
#pragma unroll
        for (int j = 0; j < D; j++) {
            if (st + j < s1) {
                const uint32_t u = su * L + q;
                const UnitT &w = buf[j];
                const bool live = u < units;
                const u32x4 *xp = xs + min(u, units - 1) * GM_UNIT + t;
                [[maybe_unused]] uint32_t sc[2], mn[2];
                if constexpr (MINS)
                    q4k_scale_min_pair(make_uint4(w.hdr[0][0], w.hdr[0][1], w.hdr[0][2], w.hdr[0][3]),
                                       (u & 3), sc[0], mn[0], sc[1], mn[1]);
#pragma unroll
                for (int sb = 0; sb < 2; sb++) {
                    floatx4 acc2[2] = {{0, 0, 0, 0}, {0, 0, 0, 0}};  // steps l = 0, 1 and 2, 3
#pragma unroll
                    for (int l = 0; l < 4; l++) {
                        floatx4 &acc = acc2[l >> 1];
                        const u32x4 xv = xp[(4 * sb + l) * 4], xl = xp[32 + (4 * sb + l) * 4];
                        u32x4 wv;
                        if constexpr (F == IQ2_XXS) {
                            const uint32_t a0 = w.a[0][2 * sb], a1 = w.a[0][2 * sb + 1];
                            const u32x4 gv = tl[((a0 >> (8 * l)) & 0xFF) * GM_COPIES];
                            const u32x4 sg = tl[(256 + ((a1 >> (7 * l)) & 127)) * GM_COPIES];
                            wv = gv ^ sg;
                        } else if constexpr (MINS) {
                            // weights 8 l .. 8 l + 7 of sub-block sb: code
                            // bytes 8 l .. 8 l + 7, low (sb 0) or high nibbles
                            // (Q5_K: with bit 2 g + sb of qh bytes 8 l .. as
                            // the fifth), as 1024 + q in fp16, then
                            // sc (1024 + q) - 1024 sc = sc q, exact (<= 945,
                            // Q5_K 1953), in one fma
                            const uint32_t c0 = l < 2 ? w.q0[0][2 * l] : w.q1[0][2 * l - 4];
                            const uint32_t c1 = l < 2 ? w.q0[0][2 * l + 1] : w.q1[0][2 * l - 3];
                            uint32_t n0 = (c0 >> (4 * sb)) & 0x0F0F0F0Fu, n1 = (c1 >> (4 * sb)) & 0x0F0F0F0Fu;
                            if constexpr (F == Q5_K) {
                                const uint32_t hb = 2 * (u & 3) + sb;
                                const uint32_t q0h = l < 2 ? w.h0[0][2 * l] : w.h1[0][2 * l - 4];
                                const uint32_t q1h = l < 2 ? w.h0[0][2 * l + 1] : w.h1[0][2 * l - 3];
                                n0 |= ((q0h >> hb) & 0x01010101u) << 4;
                                n1 |= ((q1h >> hb) & 0x01010101u) << 4;
                            }
                            const _Float16 s = (_Float16)(float)sc[sb], o = (_Float16)(-1024.0f * (float)sc[sb]);
                            const half2v s2 = {s, s}, o2 = {o, o};
                            const uint32_t e4[4] = {perm(0x64646464u, n0, 0x04010400u), perm(0x64646464u, n0, 0x04030402u),
                                                    perm(0x64646464u, n1, 0x04010400u), perm(0x64646464u, n1, 0x04030402u)};
#pragma unroll
                            for (int i = 0; i < 4; i++)
                                wv[i] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(
                                                                         __builtin_bit_cast(half2v, e4[i]), s2, o2));
                        } else {
                            // int8 weights as fp16: IQ4_XS the levels of the
                            // nibbles (weight j of a sub-block in byte j % 16's
                            // low (j < 16) or high nibble), Q8_0 the codes, the
                            // grid formats their signed grid values (the
                            // matvec's tables and v_perm selection), Q2_K the
                            // 2-bit fields, Q3_K q + 4 hbit
                            uint32_t b0, b1;
                            const uint2 *t2 = (const uint2 *)tab;
                            const int e = l & 1;
                            if constexpr (F == IQ4_XS) {
                                const u32x4 &cq = sb ? w.q1[0] : w.q0[0];
                                const uint32_t sh = 4 * (l >> 1), i0 = 2 * (l & 1);
                                b0 = IQ4Levels::levels((cq[i0] >> sh) & 0x0F0F0F0Fu);
                                b1 = IQ4Levels::levels((cq[i0 + 1] >> sh) & 0x0F0F0F0Fu);
                            } else if constexpr (F == Q8_0) {
                                b0 = w.q[sb][l >> 1][2 * (l & 1)];
                                b1 = w.q[sb][l >> 1][2 * (l & 1) + 1];
                            } else if constexpr (F == IQ3_XXS || F == IQ3_S) {
                                const uint32_t qd = w.q[0][2 * sb + (l >> 1)];
                                uint32_t i1 = (qd >> (16 * e)) & 0xFF, i2 = (qd >> (16 * e + 8)) & 0xFF, sv;
                                if constexpr (F == IQ3_S) {
                                    const uint32_t qh = (w.qh[0] >> (8 * sb)) & 0xFF;
                                    i1 |= (qh << (8 - 2 * l)) & 256;
                                    i2 |= (qh << (7 - 2 * l)) & 256;
                                    sv = 512 + (((sb ? w.sg[0].y : w.sg[0].x) >> (8 * l)) & 0xFF);
                                } else {
                                    sv = 256 + (((sb ? w.aux[0].y : w.aux[0].x) >> (7 * l)) & 127);
                                }
                                const uint2 g1 = t2[i1], g2 = t2[i2], sg = t2[sv];
                                b0 = perm(g1.y, g1.x, sg.x);
                                b1 = perm(g2.y, g2.x, sg.y);
                            } else if constexpr (F == IQ2_XS || F == IQ2_S) {
                                uint32_t idx, sv;
                                if constexpr (F == IQ2_S) {
                                    const uint32_t qd = sb ? w.q[0].y : w.q[0].x, qh = (w.qh[0] >> (8 * sb)) & 0xFF;
                                    idx = ((qd >> (8 * l)) & 0xFF) | ((qh << (8 - 2 * l)) & 0x300);
                                    sv = 1024 + (((sb ? w.sg[0].y : w.sg[0].x) >> (8 * l)) & 0xFF);
                                } else {
                                    const uint32_t q16 = (w.q[0][2 * sb + (l >> 1)] >> (16 * e)) & 0xFFFF;
                                    idx = q16 & 511;
                                    sv = 512 + (q16 >> 9);
                                }
                                const uint2 gv = t2[idx], sg = t2[sv];
                                b0 = perm(IQ2_NEG, IQ2_POS, gv.x + sg.x - 0x03020100u);
                                b1 = perm(IQ2_NEG, IQ2_POS, gv.y + sg.y - 0x03020100u);
                            } else if constexpr (F == IQ1_S || F == IQ1_M) {
                                const uint32_t qd = sb ? w.q[0].y : w.q[0].x;
                                uint32_t hb, neg;
                                if constexpr (F == IQ1_S) {
                                    const uint32_t qh = (w.qh[0] >> (16 * sb)) & 0xFFFF;
                                    hb = (qh >> (3 * l)) & 7;
                                    neg = qh >> 15;
                                } else {
                                    const uint32_t hq = (w.qh[0] >> (16 * sb + 8 * (l >> 1))) & 0xFF;
                                    hb = (hq >> (4 * e)) & 7;
                                    neg = (hq >> (4 * e + 3)) & 1;
                                }
                                const uint32_t gv = ((const uint32_t *)tab)[((qd >> (8 * l)) & 0xFF) | (hb << 8)];
                                const uint32_t nm = neg ? 0x04040404u : 0u;
                                b0 = perm(0x0007FFF7u, 0x000901F9u, (gv & 0x0F0F0F0Fu) | nm);
                                b1 = perm(0x0007FFF7u, 0x000901F9u, ((gv >> 4) & 0x0F0F0F0Fu) | nm);
                            } else {  // Q2_K, Q3_K: group j = 2 (u % 4) + sb, half l / 2
                                const uint32_t jg = 2 * (u & 3) + sb, sh = 2 * (jg & 3);
                                const u32x4 &cq = (l >> 1) ? w.q1[0] : w.q0[0];
                                b0 = (cq[2 * e] >> sh) & 0x03030303u;
                                b1 = (cq[2 * e + 1] >> sh) & 0x03030303u;
                                if constexpr (F == Q3_K) {
                                    const uint32_t hbit = 4 * (jg >> 2) + (jg & 3);
                                    const u32x4 &hq = (l >> 1) ? w.h1[0] : w.h0[0];
                                    b0 |= ((hq[2 * e] >> hbit) & 0x01010101u) << 2;
                                    b1 |= ((hq[2 * e + 1] >> hbit) & 0x01010101u) << 2;
                                }
                            }
                            const half2v m2 = {(_Float16)-1152.0f, (_Float16)-1152.0f};
                            uint32_t e4[4];
                            i8_h2(b0, e4[0], e4[1]);
                            i8_h2(b1, e4[2], e4[3]);
#pragma unroll
                            for (int i = 0; i < 4; i++)
                                wv[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, e4[i]) + m2);
                        }
#pragma unroll
                        for (int h = 0; h < 2; h++) {
                            const half4v wh = __builtin_bit_cast(half4v, uint2{wv[2 * h], wv[2 * h + 1]});
                            acc = __builtin_amdgcn_mfma_f32_4x4x4f16(
                                __builtin_bit_cast(half4v, uint2{xv[2 * h], xv[2 * h + 1]}), wh, acc, 0, 0, 0);
                            acc = __builtin_amdgcn_mfma_f32_4x4x4f16(
                                __builtin_bit_cast(half4v, uint2{xl[2 * h], xl[2 * h + 1]}), wh, acc, 0, 0, 0);
                        }
                    }
                    const uint32_t uc = min(u, units - 1);
                    const floatx4 acc = acc2[0] + acc2[1];
                    if constexpr (F == IQ2_XXS) {
                        const float db = live ? h2f(w.d[0]) * (0.5f + (float)(w.a[0][2 * sb + 1] >> 28)) * 0.25f : 0.0f;
                        tot += db * (acc * xf[uc * 2 + sb]);
                    } else if constexpr (MINS) {
                        const float d = live ? h2f(w.hdr[0][0] & 0xFFFF) : 0.0f;
                        const float dm = live ? h2f(w.hdr[0][0] >> 16) * (float)mn[sb] : 0.0f;
                        tot += d * (acc * xf[uc * 2 + sb]) - dm * xsum[uc * 2 + sb];
                    } else if constexpr (F == IQ4_XS) {
                        const uint32_t g = u & 3, shi = w.hdr[0].x >> 16, slo = byte_of(w.hdr[0].y, g);
                        const uint32_t ls = ((slo >> (4 * sb)) & 0xF) | (((shi >> (4 * g + 2 * sb)) & 3) << 4);
                        const float dl = live ? h2f(w.hdr[0].x & 0xFFFF) * (float)((int)ls - 32) : 0.0f;
                        tot += dl * (acc * xf[uc * 2 + sb]);
                    } else if constexpr (F == Q8_0) {
                        const float d = live ? h2f(w.d[sb]) : 0.0f;
                        tot += d * (acc * xf[uc * 2 + sb]);
                    } else if constexpr (F == IQ3_XXS) {
                        const uint32_t aux = sb ? w.aux[0].y : w.aux[0].x;
                        const float db = live ? h2f(w.d[0]) * (0.5f + (float)(aux >> 28)) * 0.5f : 0.0f;
                        tot += db * (acc * xf[uc * 2 + sb]);
                    } else if constexpr (F == IQ3_S) {
                        const float db = live ? h2f(w.d[0]) * (float)(1 + 2 * ((w.sc[0] >> (4 * sb)) & 0xF)) : 0.0f;
                        tot += db * (acc * xf[uc * 2 + sb]);
                    } else if constexpr (F == IQ1_S) {
                        const uint32_t qh = (w.qh[0] >> (16 * sb)) & 0xFFFF;
                        const float db = live ? h2f(w.d[0]) * (float)(2 * ((qh >> 12) & 7) + 1) * 0.125f : 0.0f;
                        tot += db * (acc * xf[uc * 2 + sb]);
                    } else {
                        // HALF: a scale per 16 weights (acc2[0]: weights 0-15)
                        const floatx4 f = xf[uc * 2 + sb];
#pragma unroll
                        for (int h = 0; h < 2; h++) {
                            float dl = 0, ml = 0;
                            if constexpr (F == IQ2_XS || F == IQ2_S) {
                                dl = h2f(w.d[0]) * (0.5f + (float)((w.sc[0] >> (8 * sb + 4 * h)) & 0xF)) * 0.25f;
                            } else if constexpr (F == IQ1_M) {
                                const uint32_t a = w.sc[0].x, b = w.sc[0].y;
                                const uint32_t bits = ((a & 0xFFFF) >> 12) | ((a >> 24) & 0x00f0) |
                                                      (((b & 0xFFFF) >> 4) & 0x0f00) | ((b >> 16) & 0xf000);
                                const uint32_t sv = w.sw[0] >> (6 * sb);
                                dl = h2f((uint16_t)bits) * (float)(2 * ((sv >> (3 * h)) & 7) + 1) * 0.125f;
                            } else if constexpr (F == Q2_K) {
                                const uint32_t scb = (w.sc[0] >> (16 * sb + 8 * h)) & 0xFF;
                                dl = h2f(w.dd[0] & 0xFFFF) * (float)(scb & 0xF);
                                ml = h2f(w.dd[0] >> 16) * (float)(scb >> 4);
                            } else {  // Q3_K: scale i of the superblock, dl (sum (q + 4 hbit) x - 4 sum x)
                                const uint32_t jg = 2 * (u & 3) + sb, i = (jg >> 2) * 8 + (jg & 3) * 2 + h;
                                const uint32_t lo8 = (i & 7) < 4 ? w.s8[0].x : w.s8[0].y;
                                const uint32_t lo = (lo8 >> (8 * (i & 3) + 4 * (i >> 3))) & 0xF;
                                const uint32_t hi = (w.s4[0] >> (8 * (i & 3) + 2 * (i >> 2))) & 3;
                                dl = h2f(w.d[0]) * (float)((int)(lo | (hi << 4)) - 32);
                                ml = 4.0f * dl;
                            }
                            if (!live) dl = ml = 0.0f;
                            tot += dl * (acc2[h] * f);
                            if constexpr (HSUM) tot -= ml * xsum[uc * 4 + sb * 2 + h];
                        }
                    }
                }
                if (++su == P && st + j + 1 < s1) {  // next step starts a row quad
                    flush();
                    su = 0;
                    k++;
                }
            }
            load_next(buf[j]);
        }
    }
    // every lane of the wavefront takes part in the shuffles
    if (s0 < s1) flush();
    __syncthreads();

    const uint32_t n_rows = r1 - r0;
    for (uint32_t e = tid; e < n_rows * NC; e += GW_THREADS) {
        const uint32_t rho = e / NC, n = e % NC, qd = rho / 4;
        const uint32_t sa = qd * P, sb = sa + P - 1;
        const uint32_t za = ((sa + 1) * GM_WAVES - 1) / T, zb = ((sb + 1) * GM_WAVES - 1) / T;
        float v = 0;
        for (uint32_t zz = za; zz <= zb; zz++) {
            const uint32_t st = gm_start(zz, T);
            if (st < gm_start(zz + 1, T)) v += part[((zz * kmax + (qd - st / P)) * 4 + rho % 4) * NC + n];
        }
        Y[(uint64_t)n * M + r0 + rho] = v;
    }
}

template <int NC, int D, uint32_t SP>
__global__ __launch_bounds__(GW_THREADS) void gemv_wide_iq2mm_kernel(const uint8_t *__restrict__ W,
                                                                     uint64_t row_bytes, uint32_t K,
                                                                     uint32_t M, const float *__restrict__ X,
                                                                     float *__restrict__ Y,
                                                                     const u32x4 *__restrict__ tab_g,
                                                                     uint32_t kmax) {
    wide_mm_body<IQ2_XXS, NC, D, SP>(W, row_bytes, K, M, X, Y, tab_g, kmax);
}

template <int F, int NC, int D, uint32_t SP>
__global__ __launch_bounds__(GW_THREADS) void gemv_wide_mm_kernel(const uint8_t *__restrict__ W,
                                                                  uint64_t row_bytes, uint32_t K, uint32_t M,
                                                                  const float *__restrict__ X,
                                                                  float *__restrict__ Y,
                                                                  const u32x4 *__restrict__ tab_g, uint32_t kmax) {
    wide_mm_body<F, NC, D, SP>(W, row_bytes, K, M, X, Y, tab_g, kmax);
}

}  // namespace okf
