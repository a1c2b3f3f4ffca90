// okf_gemv_sb.h -- matvec with one superblock per lane (Q4_K, IQ2_XXS).
//
// Work items are (row, superblock) pairs.  A workgroup owns RW consecutive
// rows, i.e. RW * nsb items that lie back to back in memory (GGUF rows are
// contiguous), and its T lanes take items lane, lane + T, ...  A lane reads
// its superblock as nine 16-byte loads (header, then the eight 16-byte code
// chunks), so one load instruction of a wavefront touches 64 consecutive
// superblocks at a 144-byte stride and the nine together consume every byte
// of a 9 KB span: each instruction moves 16 bytes per lane, and the header,
// decoded once per lane, serves all 256 weights.  Measured on MI355X, this
// pattern reads a 50 MB Q4_K matrix as fast as a plain contiguous stream.
// An IQ2_XXS superblock (66 bytes) is d plus four 16-byte loads from byte 2.
//
// Arithmetic is the exact per-group scheme of okf_gemv.h: each 32-weight
// group of x is staged once per workgroup as three signed byte planes of a
// 23-bit integer (group exponent e, f = 2^(e-22)); a group's dot product
// sum(q X) is exact in int32 (|sum| < 2^31), and the superblock is
//   d * sum_j sc_j (f_j sum(q X)_j) - dmin * sum_j m_j sum(x)_j,
// the reference's factored form of q4K (LLM/Quantize/KQuants.swift:104-125,
// matvec GQ.matvec, LLM/Gemma/Gemma4Quant.swift:89-120) in fp32.
// Each item's partial sum goes to LDS; each row then adds its nsb partials
// in a fixed order, so results are deterministic.
#pragma once
#include "okf_gemv.h"

namespace okf {

// LDS record of one superblock of one column: 16-byte chunks; chunk
// (j * 6 + p * 2 + h) holds bytes 16h..16h+15 of digit plane p of group j,
// chunk 48 + j the group data {sum x (fp32), f, 0, 0}; one chunk of padding
// makes the stride 57 chunks, so the superblocks that neighbouring lanes
// read start in different bank groups.
constexpr uint32_t SB_CHUNKS = 57;

template <int F>
__host__ __device__ constexpr bool sb_fmt() {
    return F == Q4_K || F == IQ2_XXS;
}
// 16-byte loads a superblock takes, its bytes, and the LDS table rows its
// compute reads (IQ2_XXS: the grid and sign rows of Compute<IQ2_XXS>)
template <int F>
__host__ __device__ constexpr int sb_loads() {
    return F == Q4_K ? 9 : 5;
}
template <int F>
__host__ __device__ constexpr uint32_t sb_bytes() {
    return F == Q4_K ? 144 : 66;
}
template <int F>
__host__ __device__ constexpr uint32_t sb_tab_rows() {
    return F == IQ2_XXS ? 384 : 0;
}

// Stages slots [0, K/8) of the NC columns into the superblock records, in
// SR rounds of nthr slots (SR * nthr >= K/8).  A quad of lanes holds one
// 32-weight group (limb_slot).  Every round's activation loads are issued
// first, then after_loads() (the caller's weight loads): loads complete in
// issue order, so the staging waits for the activations only while the
// weights are in flight.
template <int NC, int SR, bool SILU, typename AfterLoads>
__device__ __forceinline__ void sb_stage_x(const float *__restrict__ X, const float *__restrict__ X2, uint32_t K,
                                           uint32_t tid, uint32_t nthr, u32x4 *xs, uint32_t cs,
                                           AfterLoads after_loads) {
    const uint32_t nslots = K / 8;
    float v[SR][NC][8], v2[SILU ? SR : 1][SILU ? NC : 1][8];
#pragma unroll
    for (int r = 0; r < SR; r++) {
        const uint32_t q = min(r * nthr + tid, nslots - 1);
#pragma unroll
        for (int n = 0; n < NC; n++) {
            const float *xp = X + (uint64_t)n * K + 8 * q;
            const floatx4 a = *(const floatx4 *)xp, b = *(const floatx4 *)(xp + 4);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                v[r][n][k] = a[k];
                v[r][n][4 + k] = b[k];
            }
            if constexpr (SILU) {
                const float *up = X2 + (uint64_t)n * K + 8 * q;
                const floatx4 c = *(const floatx4 *)up, d = *(const floatx4 *)(up + 4);
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    v2[r][n][k] = c[k];
                    v2[r][n][4 + k] = d[k];
                }
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    after_loads();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int r = 0; r < SR; r++) {
        const uint32_t q = min(r * nthr + tid, nslots - 1);
        const bool store = r * nthr + tid < nslots;
        const uint32_t s = q >> 5, j = (q >> 2) & 7, k = q & 3;
#pragma unroll
        for (int n = 0; n < NC; n++) {
            if constexpr (SILU)
#pragma unroll
                for (int i = 0; i < 8; i++) v[r][n][i] = silu_mul1(v[r][n][i], v2[r][n][i]);
            uint2 pl[3];
            floatx4 gd;
            limb_slot(v[r][n], pl, gd);
            if (store) {
                u32x4 *rec = xs + n * cs + s * SB_CHUNKS;
#pragma unroll
                for (int p = 0; p < 3; p++)
                    *(uint2 *)((uint32_t *)(rec + j * 6 + p * 2 + (k >> 1)) + (k & 1) * 2) = pl[p];
                if (k == 0) *(floatx4 *)&rec[48 + j] = floatx4{gd[2] * gd[3], gd[3], 0.0f, 0.0f};
            }
        }
    }
}

// The 6-bit scales and mins of a Q4_K header, one byte per sub-block:
// sc[0] = sub-blocks 0-3, sc[1] = 4-7 (KQuant.scaleMin,
// LLM/Quantize/KQuants.swift:90-102).
struct Q4KScales {
    uint32_t sc[2], mn[2];
    float d, dmin;
    __device__ __forceinline__ explicit Q4KScales(const u32x4 &h) {
        d = h2f(h[0] & 0xFFFF);
        dmin = h2f(h[0] >> 16);
        sc[0] = h[1] & 0x3F3F3F3Fu;
        mn[0] = h[2] & 0x3F3F3F3Fu;
        sc[1] = (h[3] & 0x0F0F0F0Fu) | ((h[1] >> 2) & 0x30303030u);
        mn[1] = ((h[3] >> 4) & 0x0F0F0F0Fu) | ((h[2] >> 2) & 0x30303030u);
    }
};

// R Q4_K superblocks at the same K position (c[r][0] header, c[r][1..8]
// codes) against the staged record of NC columns: out[r][n] = their
// contributions.  Each activation chunk read from LDS serves the R rows.
template <int NC, int R>
__device__ __forceinline__ void sb_q4k(const u32x4 (&c)[R][9], const u32x4 *rec, uint32_t cs, float (&out)[R][NC]) {
    float accA[R][NC], accB[R][NC];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int n = 0; n < NC; n++) accA[r][n] = accB[r][n] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        int s[R][NC][3];
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int n = 0; n < NC; n++) s[r][n][0] = s[r][n][1] = s[r][n][2] = 0;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            uint32_t w[R][4];
#pragma unroll
            for (int r = 0; r < R; r++) {
                const u32x4 cc = c[r][1 + 2 * (j >> 1) + h];
#pragma unroll
                for (int k = 0; k < 4; k++) w[r][k] = (j & 1) ? (cc[k] >> 4) & 0x0F0F0F0Fu : cc[k] & 0x0F0F0F0Fu;
            }
#pragma unroll
            for (int n = 0; n < NC; n++)
#pragma unroll
                for (int p = 0; p < 3; p++) {
                    const u32x4 xv = rec[n * cs + j * 6 + p * 2 + h];
#pragma unroll
                    for (int r = 0; r < R; r++)
#pragma unroll
                        for (int k = 0; k < 4; k++) s[r][n][p] = sdot4(w[r][k], xv[k], s[r][n][p]);
                }
        }
#pragma unroll
        for (int n = 0; n < NC; n++) {
            const floatx4 gd = *(const floatx4 *)&rec[n * cs + 48 + j];
#pragma unroll
            for (int r = 0; r < R; r++) {
                const Q4KScales q(c[r][0]);
                const float sc = (float)byte_of(q.sc[j >> 2], j & 3), mn = (float)byte_of(q.mn[j >> 2], j & 3);
                // sum(q X) of the group, exact: |sum| < 2^31
                const int S = (s[r][n][2] << 16) + (s[r][n][1] << 8) + s[r][n][0];
                accA[r][n] = fmaf(sc, gd[1] * (float)S, accA[r][n]);
                accB[r][n] = fmaf(mn, gd[0], accB[r][n]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
        const Q4KScales q(c[r][0]);
#pragma unroll
        for (int n = 0; n < NC; n++) out[r][n] = q.d * accA[r][n] - q.dmin * accB[r][n];
    }
}

// R IQ2_XXS superblocks (IQ2XXS.dot, LLM/Quantize/IQ2XXS.swift:34-54, as
// the integer form of Compute<IQ2_XXS>): c[r][0].x low half d, c[r][1..4]
// the 16 qs dwords (loaded from byte 2); sub-block j = qs dwords 2j (four
// grid indices, 8 weights each) and 2j + 1 (four 7-bit sign indices, the
// 4-bit scale on top) = staged group j.  Per 8 weights: two 8-byte table
// reads, one add and one v_perm per 4 weights make the signed grid bytes
// (tab layout as Compute<IQ2_XXS>), dotted with the three digit planes;
// per sub-block db (f sum(g s X)), db = d (0.5 + scale) / 4.
template <int NC, int R>
__device__ __forceinline__ void sb_iq2(const u32x4 (&c)[R][5], const u32x4 *rec, uint32_t cs, const u32x4 *tab,
                                       float (&out)[R][NC]) {
    float acc[R][NC];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int n = 0; n < NC; n++) acc[r][n] = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        int s[3][R][NC];
#pragma unroll
        for (int p = 0; p < 3; p++)
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int n = 0; n < NC; n++) s[p][r][n] = 0;
#pragma unroll
        for (int h = 0; h < 2; h++) {  // grid entries 2h, 2h + 1 = plane chunk h of the group
            uint32_t w[R][4];
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t a0 = c[r][1 + (j >> 1)][2 * (j & 1)], a1 = c[r][1 + (j >> 1)][2 * (j & 1) + 1];
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const int l = 2 * h + e;
                    const uint2 gv = *(const uint2 *)&tab[(a0 >> (8 * l)) & 0xFF];
                    const uint2 sg = *(const uint2 *)&tab[256 + ((a1 >> (7 * l)) & 127)];
                    w[r][2 * e] = perm(IQ2_NEG, IQ2_POS, gv.x + sg.x - 0x03020100u);
                    w[r][2 * e + 1] = perm(IQ2_NEG, IQ2_POS, gv.y + sg.y - 0x03020100u);
                }
            }
#pragma unroll
            for (int n = 0; n < NC; n++)
#pragma unroll
                for (int p = 0; p < 3; p++) {
                    const u32x4 xv = rec[n * cs + j * 6 + p * 2 + h];
#pragma unroll
                    for (int r = 0; r < R; r++)
#pragma unroll
                        for (int k = 0; k < 4; k++) s[p][r][n] = sdot4(w[r][k], xv[k], s[p][r][n]);
                }
        }
#pragma unroll
        for (int n = 0; n < NC; n++) {
            const floatx4 gd = *(const floatx4 *)&rec[n * cs + 48 + j];
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t a1 = c[r][1 + (j >> 1)][2 * (j & 1) + 1];
                const float db = h2f(c[r][0][0] & 0xFFFF) * (0.5f + (float)(a1 >> 28)) * 0.25f;
                acc[r][n] += db * (comb(s, r, n) * gd[1]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int n = 0; n < NC; n++) out[r][n] = acc[r][n];
}

// Grid: one workgroup per RW rows of a matrix of the group (GemvGroup as
// gemv_kernel).  Items are (row pair-set, superblock): item i covers
// superblock i % nsb of rows i / nsb + k RW / R, k < R (RW a multiple of R).
// Dynamic LDS: the format's table rows (copied from tab_g), NC columns of
// nsb records (column stride cs = nsb * SB_CHUNKS chunks), then the
// partials [row][superblock][NC].
template <int F, int NC, int R, int T, int SR, bool SILU>
__global__ __launch_bounds__(T) void gemv_sb_kernel(GemvGroup g, uint64_t row_bytes, uint32_t K, uint32_t RW,
                                                    const u32x4 *__restrict__ tab_g) {
    static_assert(sb_fmt<F>(), "no superblock-per-lane matvec for this format");
    uint32_t mi = 0;
#pragma unroll
    for (int k = 0; k + 1 < GV_GROUP; k++)
        if (k + 1 < (int)g.n && blockIdx.x >= g.end[k]) mi = k + 1;
    const uint32_t blk = blockIdx.x - (mi ? g.end[mi - 1] : 0);
    const uint32_t M = g.M[mi];
    const float *__restrict__ X = g.X[mi];
    const float *__restrict__ X2 = g.X2[mi];
    float *__restrict__ Y = g.Y[mi];
    extern __shared__ u32x4 lds[];
    const uint32_t tid = threadIdx.x, nsb = K / 256, cs = nsb * SB_CHUNKS;
    constexpr uint32_t TABR = sb_tab_rows<F>(), NL = sb_loads<F>();
    u32x4 *tab = lds;
    if constexpr (TABR > 0)
        for (uint32_t e = tid; e < TABR; e += T) tab[e] = tab_g[e];
    u32x4 *xs = lds + TABR;
    float *part = (float *)(xs + NC * cs);
    const uint32_t r0 = blk * RW, rows = min(RW, M - r0), rs = RW / R;
    const uint32_t items = rs * nsb;
    const uint8_t *base = g.W[mi] + (uint64_t)r0 * row_bytes;

    u32x4 c[R][NL];
    auto load = [&](uint32_t it) {
        const uint32_t i = min(it, items - 1), row = i / nsb, sb = i - row * nsb;
#pragma unroll
        for (int r = 0; r < R; r++) {
            // rows past the matrix re-read the last row (their results are dropped)
            const uint32_t rr = min(row + r * rs, rows - 1);
            const uint8_t *p = base + (uint64_t)rr * row_bytes + (uint64_t)sb * sb_bytes<F>();
            if constexpr (F == IQ2_XXS) {
                c[r][0] = u32x4{ldu<uint16_t>(p), 0u, 0u, 0u};
#pragma unroll
                for (int k = 0; k < 4; k++) c[r][1 + k] = ldu<u32x4>(p + 2 + 16 * k);
            } else {
#pragma unroll
                for (int k = 0; k < 9; k++) c[r][k] = ((const u32x4 *)p)[k];
            }
        }
    };
    // the first item's loads go right behind the staging's activation loads
    sb_stage_x<NC, SR, SILU>(X, X2, K, tid, T, xs, cs, [&]() { load(tid); });
    __syncthreads();
    // a lane's next item is requested right after its current one is
    // consumed (one register buffer; other wavefronts cover the latency)
    for (uint32_t it = tid; it < items; it += T) {
        float o[R][NC];
        const uint32_t row = it / nsb, sb = it - row * nsb;
        if constexpr (F == IQ2_XXS) sb_iq2<NC, R>(c, xs + sb * SB_CHUNKS, cs, tab, o);
        else sb_q4k<NC, R>(c, xs + sb * SB_CHUNKS, cs, o);
        if (it + T < items) load(it + T);
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int n = 0; n < NC; n++) part[((row + r * rs) * nsb + sb) * NC + n] = o[r][n];
    }
    __syncthreads();
    // row sums: four lanes per (row, column) add every fourth partial in
    // order, then the quad adds its four sums (fixed order: deterministic);
    // the four lanes of a quad share q, so a quad is active as a whole.
    // Long rows: sixteen lanes per row, every sixteenth partial, then a
    // fixed butterfly over the sixteen (a shorter chain of dependent reads)
    const uint32_t pairs = rows * NC;
    if (nsb > 32 && pairs <= T / 16) {
        const uint32_t l16 = tid & 15, q = tid >> 4;
        if (q < pairs) {  // (whole groups of sixteen)
            const uint32_t r = q / NC, n = q % NC;
            float v = 0.0f;
            for (uint32_t sb = l16; sb < nsb; sb += 16) v += part[(r * nsb + sb) * NC + n];
#pragma unroll
            for (int m = 1; m < 16; m <<= 1) v += __shfl_xor(v, m, 16);
            if (l16 == 0) Y[(uint64_t)n * M + r0 + r] = v;
        }
    } else {
        const uint32_t lane4 = tid & 3;
        for (uint32_t q = tid >> 2; q < pairs; q += T >> 2) {
            const uint32_t r = q / NC, n = q % NC;
            float v = 0.0f;
            for (uint32_t sb = lane4; sb < nsb; sb += 4) v += part[(r * nsb + sb) * NC + n];
            v = quad_sum(v);
            if (lane4 == 0) Y[(uint64_t)n * M + r0 + r] = v;
        }
    }
}

}  // namespace okf
