// okf_impl.h -- host-side internals shared by the translation units of
// libokf_quant.so: the context, argument checks, scratch management and the
// per-format launchers.  The launchers are templates instantiated once per
// format in okf_fmt_*.hip (so the formats compile in parallel) and declared
// extern here for okf_quant.hip, which holds the C ABI.
#pragma once
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <new>
#include <type_traits>
#include <vector>

#include "../../include/okf_quant.h"
#include "okf_common.h"
#include "okf_decode.h"
#include "okf_gemm.h"
#include "okf_gemv.h"
#include "okf_gemv_wide.h"
#include "okf_gemv_sb.h"
#include "okf_ffn.h"
#include "okf_ffn_mfma.h"

// one matvec y = W x of a launch group (with X2: x = silu(X) * X2)
struct GemvCall {
    const uint8_t *W;
    const float *X;
    float *Y;
    uint32_t M;
    const float *X2 = nullptr;
};

struct okf_ctx {
    int device = -1;
    hipStream_t stream = nullptr;
    uint2 *grid = nullptr;  // 256 IQ2_XXS grid entries in device memory
    uint8_t *grids = nullptr;  // the grids of IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S / IQ1_M (GT_* offsets)
    okf::u32x4 *tab = nullptr;   // IQ2_XXS fp16 grid (256 x 8 halves) + sign masks (128): MFMA kernel
    okf::u32x4 *tab8 = nullptr;  // IQ2_XXS int8 grid (256) + sign byte masks (128): dot4 kernels
    size_t max_lds = 65536;  // dynamic LDS a workgroup may use
    // matvec tuning (defaults chosen per shape; OKF_GEMV_* environment
    // variables override them for measurements)
    int gemv_s = 0;      // K split across a workgroup's wavefronts (0 = auto)
    int gemv_wide = -1;  // one-workgroup-per-CU matvec: -1 auto, 0 never, 1 where it fits
    int gemv_sb = -1;    // superblock-per-lane matvec: -1 auto, 0 never, 1 where it fits
    int gemv_sb_rw = 0;  // its rows per workgroup (0 = auto)
    int gemv_sb_t = 0;   // its threads per workgroup (0 = auto)
    int gemv_sb_r = 2;   // its rows per lane for IQ2_XXS (2: each x record read serves two rows; or 1)
    int gemm_ks = 0;     // wide-tile GEMM: K ranges per remainder tile (0 = auto)
    int q4k_mm = 0xFFF;  // 2..4 columns on the matrix cores, bits mm_bit(F) (0: the dot4 kernels)
    int gemm_split = 1;  // tile GEMM of the other formats: K split when the grid is small (0 never, > 1 ways)
    int gemm_xh = 1;     // tile GEMM of the other formats: fp16 X converted once from N = 256 (0: never)
    int gemm_thin = 0;   // leftover-tile kernel variant (A/B switch)
    int gemm_ng = 4;     // wide-tile GEMM: N tiles that share an XCD's row blocks
    uint32_t cus = 256;  // compute units of the device
    double fault_rate = 0;
    uint64_t fault_state = 0;
    int last_hip = 0;
    _Float16 *xh = nullptr;  // fp16 copy of the GEMM activations (grown on demand)
    size_t xh_bytes = 0;
    // okf_parallel_begin .. okf_parallel_end: recorded matvecs
    struct Pending {
        int32_t type;
        uint32_t K;
        uint64_t rb;
        GemvCall call;
    };
    bool grouping = false;
    std::vector<Pending> pending;
    float *part = nullptr;   // split-tile partial sums of the Q4_K GEMM, argmax pairs
    size_t part_bytes = 0;
    uint32_t *cnt = nullptr;  // argmax per-row counters (zero between calls)
    size_t cnt_n = 0;
    bool reserved = false;    // okf_ctx_reserve fixed the scratch sizes: no growth
    uint8_t *scratch = nullptr;  // this device's copy of the static scratch array
    uint32_t *ffn_bar = nullptr;  // the one-launch FFN's grid barrier (zeroed at creation)
    uint32_t *ffn_status = nullptr;  // pinned host word: 1 once a launch's barrier gave up (GPUGate verdict)
    int ffn_fused = 1;            // okf_ffn as one launch with a grid barrier: 1 where it fits and is the faster
                                  // form, 2 wherever it fits, 0 never (two launches)
    int ffn_wg = 1;               // its workgroups per CU, at most
    int ffn_coop = 0;             // launched with hipLaunchCooperativeKernel (1) or as a plain grid
    int q2_mfma = 1;              // Q2_0 Bonsai matvecs on the integer matrix cores (q2m_gemv_kernel; 0: off)
    int q2_ks = 1;                // ... down (R <= 8 rows a workgroup) as the K-split tile (0: rows repeated)
    int ffn_mfma = 1;             // the Bonsai shape on the integer matrix cores (ffn_mfma_kernel; 0: off)
    int ffn_nb[4] = {0, 0, 0, 0}; // its kernels' resident workgroups per CU (0: not yet queried)
    int ffn_spin = 0;             // its barrier's poll limit (0: FF_SPIN)
    int ffn_stall = 0;            // its next launches whose barrier must time out (failure tests)
    int ffn_t = 0;                // its exact-fit variant: threads a workgroup (0: the default, 512)
};

namespace okf_impl {

using namespace okf;


inline bool supported(int32_t t) {
    return t == Q8_0 || t == Q4_K || t == IQ2_XXS || t == Q2_0 || t == Q4_0 || t == IQ4_NL || t == Q5_K ||
           t == Q6_K || t == IQ4_XS || grid_fmt(t);
}

inline int hip_fail(okf_ctx *c, hipError_t e) {
    c->last_hip = (int)e;
    return OKF_E_HIP;
}

// splitmix64 -> uniform [0, 1); deterministic per seed.
inline double next_uniform(uint64_t &s) {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (double)(z >> 11) * (1.0 / 9007199254740992.0);
}

// Shared prologue of every launch call: arguments, fault injection, device.
inline int begin(okf_ctx *c) {
    if (!c) return OKF_E_ARG;
    if (c->fault_rate > 0 && next_uniform(c->fault_state) < c->fault_rate) return OKF_E_INJECTED;
    if (c->device < 0) return OKF_E_NODEV;
    hipError_t e = hipSetDevice(c->device);
    return e == hipSuccess ? OKF_OK : hip_fail(c, e);
}

inline int check_weight(const okf_weight *w, uint64_t *row_bytes) {
    if (!w || !w->base) return OKF_E_ARG;
    if (!supported(w->ggml_type)) return OKF_E_TYPE;
    if (w->K == 0 || w->M == 0 || w->K % block_elems(w->ggml_type)) return OKF_E_SHAPE;
    *row_bytes = (uint64_t)w->K / block_elems(w->ggml_type) * block_bytes(w->ggml_type);
    const uintptr_t a = (uintptr_t)w->base + w->off;
    // Q4_K kernels read 16-byte header/code chunks; others need 2-byte alignment.
    if (w->ggml_type == Q4_K ? (a & 15) : (a & 1)) return OKF_E_SHAPE;
    return OKF_OK;
}

// The one-launch FFN's failure word (written by the kernel, read by the
// host without a copy): OKF_E_TIMEOUT once, and cleared, after a launch whose
// grid barrier gave up (GPUGate.verdict, LLM/Base/MetalGates.swift:130-142).
inline int take_timeout(okf_ctx *c) {
    volatile uint32_t *w = c->ffn_status;
    if (!w || *w == 0) return OKF_OK;
    *w = 0;
    return OKF_E_TIMEOUT;
}

inline bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// Raises a kernel's dynamic LDS limit once per device (done: one bit per
// device, shared by every context and thread; a repeated call is harmless).
// The limit is the workgroup's LDS less the kernel's static LDS; a failure
// (which leaves the launch at the default limit) is cleared so that it is
// not reported as the launch's error.
inline void set_lds_attr(const okf_ctx *c, const void *fn, std::atomic<uint64_t> &done) {
    const uint64_t bit = 1ull << (c->device & 63);
    if (done.load(std::memory_order_acquire) & bit) return;
    hipFuncAttributes fa{};
    size_t stat = 0;
    if (hipFuncGetAttributes(&fa, fn) == hipSuccess) stat = fa.sharedSizeBytes;
    if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)(c->max_lds - stat)) !=
        hipSuccess)
        (void)hipGetLastError();
    done.fetch_or(bit, std::memory_order_acq_rel);
}

inline int finish(okf_ctx *c) {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? OKF_OK : hip_fail(c, e);
}

template <int F, int NC, int S, bool SILU, int DX = 0>
void launch_gemv_s(okf_ctx *c, const GemvCall *calls, int n, uint64_t rb, uint32_t K,
                   uint32_t cunits, size_t lds, bool pair = false) {
    // Q2_0 and Q8_0 at N = 1: a three-deep ring when a wavefront runs three
    // or more steps (the down projection), so that no step waits for a load
    // issued after the first compute; two otherwise (a third buffer would
    // only re-read).  Measured: Q2_0 2048x6144 4.95 -> 4.75 us.
    if constexpr (DX == 0 && NC == 1 && (F == Q2_0 || F == Q8_0)) {
        const uint32_t steps = (K / unit_weights<F>() + GV_L * S - 1) / (GV_L * S);
        if (steps >= 3) return launch_gemv_s<F, NC, S, SILU, 3>(c, calls, n, rb, K, cunits, lds, pair);
    }
    // two rows per slot (each staged activation read serves both) where
    // measured faster: IQ2_XXS with 1..5 columns (16.9 -> 16.4 us at one), the
    // generic formats with 2..5 (17408 x 5120, N = 4: 15-18 % faster; at one
    // column 10-25 % slower), Q4_K and Q2_0 with 5.  (A
    // three-deep ring for the Q4_K matvec measured 3-4 % slower than two
    // once the weight loads were issued behind the staging's.)
    constexpr int R = ((F == IQ2_XXS && NC >= 1) || (grid_fmt(F) && NC >= 2) ||
                       (NC == 5 && F != Q8_0 && F != Q5_K && F != Q6_K && F != IQ4_XS)) ? 2 : 1,
                  D = DX ? DX : 2, WAVES = 4;
    const void *fn = (const void *)gemv_kernel<F, NC, R, D, S, SILU>;
    static std::atomic<uint64_t> attr{0};  // devices that have the attribute set
    set_lds_attr(c, fn, attr);
    const uint32_t rows_per_wg = (WAVES / S) * GV_SLOTS * R;
    GemvGroup g{};
    uint32_t total = 0;
    for (int i = 0; i < n; i++) {
        g.W[i] = calls[i].W;
        g.X[i] = calls[i].X;
        g.X2[i] = calls[i].X2;
        g.Y[i] = calls[i].Y;
        g.M[i] = calls[i].M;
        total += (calls[i].M + rows_per_wg - 1) / rows_per_wg;
        g.end[i] = total;
    }
    g.n = (uint32_t)n;
    if (pair) {  // gate and up rows in the same workgroups: half the row slots each
        g.pair = 1;
        total = (calls[0].M + rows_per_wg / 2 - 1) / (rows_per_wg / 2);
    }
    // the tables the compute reads: IQ2_XXS's LDS rows (copied from c->tab),
    // or the grid formats' device-memory grids
    const u32x4 *tabs = itab_rows(F) ? c->tab8 + itab_at(F) : grid_fmt(F) ? (const u32x4 *)(c->grids + gt_off(F)) : c->tab8;
    hipLaunchKernelGGL((gemv_kernel<F, NC, R, D, S, SILU>), dim3(total), dim3(64 * WAVES), lds, c->stream,
                       g, rb, K, tabs, cunits);
}

// Launch geometry: 256-thread workgroups of four wavefronts, each four row
// slots of 16 lanes.  For one column with fewer than ~3072 wavefronts' worth
// of rows, K is split two ways across the wavefronts of a workgroup (more,
// shorter wavefronts); measured on MI355X, a four-way split loses to the
// extra activation staging it needs.
template <int F, int NC, uint32_t SP>
void launch_wide_sp(okf_ctx *c, const GemvCall &call, uint64_t rb, uint32_t K, uint32_t G, size_t lds,
                    uint32_t kmax) {
    // weight ring depth: as deep as the registers allow without spills
    constexpr int D = (F == Q4_K || F == Q8_0) ? (NC == 1 ? 3 : 2)
                      : F == Q2_0                ? (NC == 1 ? 6 : 2)
                                                 : (NC <= 2 ? 6 : NC == 3 ? 4 : 3);
    const void *fn = (const void *)gemv_wide_kernel<F, NC, D, SP>;
    static std::atomic<uint64_t> attr{0};  // devices that have the attribute set
    set_lds_attr(c, fn, attr);
    hipLaunchKernelGGL((gemv_wide_kernel<F, NC, D, SP>), dim3(G), dim3(GW_THREADS), lds, c->stream, call.W,
                       rb, K, call.M, call.X, call.Y, c->tab8, kmax);
}

// Where the one-workgroup-per-CU kernel measured faster on MI355X than the
// many-workgroup one (A/B in one process, configuration shapes): IQ2_XXS
// with 2..5 columns (conflict-free tables; 28.2 -> 22.5 us at N = 4),
// Q4_0 / IQ4_NL and long-K Q2_0 with 4..5 columns, and the long-K Q4_K
// matvec (5120 x 17408: 16.0 -> 15.4 us).
template <int F, int NC>
bool wide_auto(const okf_ctx *c, uint32_t M, uint32_t K) {
    if (M < 8 * c->cus) return F == Q2_0 && NC >= 4 && K >= 4096;
    if (F == IQ2_XXS) return NC >= 2;
    if (F == Q4_0 || F == IQ4_NL) return NC >= 4;
    if (F == Q2_0) return NC >= 4 && K >= 4096;
    if (F == Q4_K) return NC == 1 && K >= 8192;
    return false;
}

// IQ2_XXS with 2..4 columns on the matrix cores (gemv_wide_iq2mm_kernel):
// true when launched.
template <int NC>
bool launch_iq2mm(okf_ctx *c, const GemvCall &call, uint64_t rb, uint32_t K) {
    const uint32_t G = std::min(c->cus, call.M), units = K / 64, P = (units + GV_L - 1) / GV_L;
    const uint64_t nq = ((call.M + G - 1) / G + 3) / 4, lmax = (nq * P + GM_WAVES - 1) / GM_WAVES;
    const uint32_t kmax = (uint32_t)((lmax + P - 1) / P + 1);
    const size_t lds = GM_TAB * 16 + (size_t)P * GV_L * (GM_UNIT + 2) * 16 + (size_t)GM_WAVES * kmax * 4 * NC * 4;
    const uint32_t sp = (units * 32 + GW_THREADS - 1) / GW_THREADS;
    if (lds > c->max_lds || sp > 3 || nq * P * GM_WAVES >= (1ull << 32)) return false;
    constexpr int D = 2;  // weight ring depth (17408 x 5120, N = 4: 1 19.4, 2 19.5, 3 20.2, 4 20.9, 6 21.2, 8 22.9 us)
    auto go = [&](auto spc) {
        constexpr uint32_t SP = decltype(spc)::value;
        const void *fn = (const void *)gemv_wide_iq2mm_kernel<NC, D, SP>;
        static std::atomic<uint64_t> attr{0};  // devices that have the attribute set
        set_lds_attr(c, fn, attr);
        hipLaunchKernelGGL((gemv_wide_iq2mm_kernel<NC, D, SP>), dim3(G), dim3(GW_THREADS), lds, c->stream,
                           call.W, rb, K, call.M, call.X, call.Y, c->tab, kmax);
    };
    if (sp <= 1) go(std::integral_constant<uint32_t, 1>{});
    else if (sp == 2) go(std::integral_constant<uint32_t, 2>{});
    else go(std::integral_constant<uint32_t, 3>{});
    return true;
}

// The formats with a matrix-core 2..4-column kernel, and their bit in
// okf_ctx::q4k_mm.
constexpr int mm_bit(int f) {
    return f == Q4_K ? 0 : f == Q5_K ? 1 : f == IQ4_XS ? 2 : f == Q8_0 ? 3 : f == IQ3_XXS ? 4 : f == IQ3_S ? 5
         : f == IQ2_XS ? 6 : f == IQ2_S ? 7 : f == IQ1_S ? 8 : f == IQ1_M ? 9 : f == Q2_K ? 10 : f == Q3_K ? 11 : -1;
}

// Q4_K, Q5_K, IQ4_XS, Q8_0, the grid formats, Q2_K and Q3_K with 2..4
// columns on the matrix cores (gemv_wide_mm_kernel): true when launched.
template <int F, int NC>
bool launch_widemm(okf_ctx *c, const GemvCall &call, uint64_t rb, uint32_t K) {
    // (measured on MI355X: at M = 2048 the many-workgroup dot4 kernels are
    // faster, e.g. Q8_0 2048 x 2048 N = 2 5.6 against 14.6 us; Q8_0 at N = 2
    // also at 17408 x 5120, 29.6 against 35.4)
    static_assert(mm_bit(F) >= 0, "matrix-core narrow format");
    if (!(c->q4k_mm & (1 << mm_bit(F))) || K % 64 || call.M < 4096 || (F == Q8_0 && NC < 3)) return false;
    constexpr bool MINS = F == Q4_K || F == Q5_K, HSUM = F == Q2_K || F == Q3_K;
    constexpr uint32_t TABR = (F == IQ1_S || F == IQ1_M) ? 512 : itab_rows(F);
    const uint32_t G = std::min(c->cus, call.M), units = K / 64, P = (units + GV_L - 1) / GV_L;
    const uint64_t nq = ((call.M + G - 1) / G + 3) / 4, lmax = (nq * P + GM_WAVES - 1) / GM_WAVES;
    const uint32_t kmax = (uint32_t)((lmax + P - 1) / P + 1);
    const size_t lds = (size_t)TABR * 16 + (size_t)P * GV_L * (GM_UNIT + (MINS ? 4 : HSUM ? 6 : 2)) * 16 +
                       (size_t)GM_WAVES * kmax * 4 * NC * 4;
    const uint32_t sp = (units * 32 + GW_THREADS - 1) / GW_THREADS;
    if (lds > c->max_lds || sp > 3 || nq * P * GM_WAVES >= (1ull << 32)) return false;
    const u32x4 *tab = itab_rows(F) ? c->tab8 + itab_at(F)
                     : TABR ? (const u32x4 *)(c->grids + gt_off(F)) : nullptr;
    constexpr int D = 2;
    auto go = [&](auto spc) {
        constexpr uint32_t SP = decltype(spc)::value;
        const void *fn = (const void *)gemv_wide_mm_kernel<F, NC, D, SP>;
        static std::atomic<uint64_t> attr{0};  // devices that have the attribute set
        set_lds_attr(c, fn, attr);
        hipLaunchKernelGGL((gemv_wide_mm_kernel<F, NC, D, SP>), dim3(G), dim3(GW_THREADS), lds, c->stream,
                           call.W, rb, K, call.M, call.X, call.Y, tab, kmax);
    };
    if (sp <= 1) go(std::integral_constant<uint32_t, 1>{});
    else if (sp == 2) go(std::integral_constant<uint32_t, 2>{});
    else go(std::integral_constant<uint32_t, 3>{});
    return true;
}

// One workgroup per CU (gemv_wide_kernel) for a single matrix: true when
// launched.
template <int F, int NC>
bool launch_gemv_wide(okf_ctx *c, const GemvCall &call, uint64_t rb, uint32_t K) {
    const int mode = c->gemv_wide;
    if (mode == 0 || (mode < 0 && !wide_auto<F, NC>(c, call.M, K))) return false;
    if constexpr (F == IQ2_XXS && NC >= 2 && NC <= 4)  // (mode 2: the dot2 kernel)
        if (mode != 2 && launch_iq2mm<NC>(c, call, rb, K)) return true;
    constexpr uint32_t UW = unit_weights<F>();
    const uint32_t G = std::min(c->cus, call.M), units = K / UW, P = (units + GV_L - 1) / GV_L;
    const uint64_t nmax = (call.M + G - 1) / G, lmax = (nmax * P + GW_SLOTS - 1) / GW_SLOTS;
    const uint32_t kmax = (uint32_t)((lmax + P - 1) / P + 1);
    const uint64_t cunits = (uint64_t)P * GV_L;
    const size_t lds = (F == IQ2_XXS ? GW_TAB * 16 : 0) + (size_t)NC * cunits * unit_lds_bytes<F>() +
                       (size_t)GW_SLOTS * kmax * NC * sizeof(float);
    // one staging round (x slots per thread <= SP), step indices in 32 bits
    const uint32_t nslots = K / 8, sp = (nslots + GW_THREADS - 1) / GW_THREADS;
    if (lds > c->max_lds || sp > (NC == 1 ? 3u : 1u) || nmax * P * GW_SLOTS >= (1ull << 32)) return false;
    if constexpr (NC == 1)
        if (sp > 1) {
            launch_wide_sp<F, NC, 3>(c, call, rb, K, G, lds, kmax);
            return true;
        }
    launch_wide_sp<F, NC, 1>(c, call, rb, K, G, lds, kmax);
    return true;
}

template <int F, int NC, int T, bool SILU, int R = 1>
void launch_sb_t(okf_ctx *c, const GemvGroup &g, uint32_t total, uint64_t rb, uint32_t K, uint32_t RW, size_t lds,
                 uint32_t sr) {
    auto go = [&](auto src) {
        constexpr int SR = decltype(src)::value;
        const void *fn = (const void *)gemv_sb_kernel<F, NC, R, T, SR, SILU>;
        static std::atomic<uint64_t> attr{0};  // devices that have the attribute set
        set_lds_attr(c, fn, attr);
        hipLaunchKernelGGL((gemv_sb_kernel<F, NC, R, T, SR, SILU>), dim3(total), dim3(T), lds, c->stream, g, rb, K,
                           RW, (const u32x4 *)c->tab8);
    };
    // (one register buffer: a two-deep ring measured slower at every
    // workgroup size tried, 15.5 against 13.6 us at 17408 x 5120)
    switch (sr) {
        case 1: go(std::integral_constant<int, 1>{}); break;
        case 2: go(std::integral_constant<int, 2>{}); break;
        case 3: go(std::integral_constant<int, 3>{}); break;
        case 4:
        case 5: go(std::integral_constant<int, 5>{}); break;
        default: go(std::integral_constant<int, 9>{}); break;
    }
}

// Superblock-per-lane matvec (gemv_sb_kernel): true when launched.  Short
// rows (<= 32 superblocks): T = 256 lanes and RW = T / nsb rows, one
// superblock per lane (IQ2_XXS: two rows per lane, RW = 2 T / nsb; 17408 x
// 5120 in 15.5 us against 16.1 for one row per lane and for gemv_kernel).  Long rows: T = 512 and RW = M / CUs (one workgroup
// per CU, each lane a few superblocks), so that the per-workgroup staging of
// x is shared by more rows.  Measured on MI355X (A/B in one process):
// Q4_K 17408 x 5120 from 15.7 us (gemv_kernel) to 13.6 us; 5120 x 17408
// from 17.6 us (gemv_wide_kernel) to 16.4 us.
template <int F, int NC, bool SILU>
bool launch_gemv_sb(okf_ctx *c, const GemvCall *calls, int n, uint64_t rb, uint32_t K) {
    if constexpr (!sb_fmt<F>() || NC > 1) {
        return false;
    } else {
        const uint32_t nsb = K / 256;
        if (c->gemv_sb == 0) return false;
        const bool lng = nsb > 32;
        if (F == IQ2_XXS && lng) return false;  // (long rows: gemv_kernel, not measured here)
        uint32_t T = c->gemv_sb_t ? (uint32_t)c->gemv_sb_t : lng ? 512 : 256;
        if (T != 256 && T != 512) T = 256;
        const uint32_t sr = (K / 8 + T - 1) / T;  // staging rounds
        if (sr > 9) return false;
        uint32_t M = 0;
        for (int i = 0; i < n; i++) M += calls[i].M;
        const uint32_t RW = c->gemv_sb_rw ? (uint32_t)c->gemv_sb_rw
                            : lng       ? std::min(32u, std::max(4u, (M + c->cus - 1) / c->cus))
                                        : std::max(1u, T / nsb) * (F == IQ2_XXS && c->gemv_sb_r == 2 ? 2 : 1);
        const size_t lds = (size_t)sb_tab_rows<F>() * 16 + ((size_t)NC * nsb * SB_CHUNKS * 16) +
                           (size_t)RW * nsb * NC * sizeof(float);
        if (lds > c->max_lds) return false;
        GemvGroup g{};
        uint32_t total = 0;
        for (int i = 0; i < n; i++) {
            g.W[i] = calls[i].W;
            g.X[i] = calls[i].X;
            g.X2[i] = calls[i].X2;
            g.Y[i] = calls[i].Y;
            g.M[i] = calls[i].M;
            total += (calls[i].M + RW - 1) / RW;
            g.end[i] = total;
        }
        g.n = (uint32_t)n;
        if (F == IQ2_XXS && c->gemv_sb_r == 2 && T == 256 && RW % 2 == 0)
            launch_sb_t<F, NC, 256, SILU, 2>(c, g, total, rb, K, RW, lds, sr);
        else if (T == 256) launch_sb_t<F, NC, 256, SILU>(c, g, total, rb, K, RW, lds, sr);
        else launch_sb_t<F, NC, 512, SILU>(c, g, total, rb, K, RW, lds, sr);
        return true;
    }
}

template <int F, int NC, bool SILU = false>
void launch_gemv_nc(okf_ctx *c, const GemvCall *calls, int n, uint64_t rb, uint32_t K) {
    if (launch_gemv_sb<F, NC, SILU>(c, calls, n, rb, K)) return;
    if constexpr (mm_bit(F) >= 0 && !SILU && NC >= 2 && NC <= 4)
        if (n == 1 && launch_widemm<F, NC>(c, calls[0], rb, K)) return;
    // (Q4_K and Q8_0 units are too large for a deep ring at N > 1; the
    // formats added after the measurements take the many-workgroup kernel)
    if constexpr (!SILU && !((F == Q4_K || F == Q8_0) && NC > 1) && F != Q5_K && F != Q6_K && F != IQ4_XS &&
                  !grid_fmt(F))  // (IQ3_XXS included: the wide kernel has no tables for it)
        if (n == 1 && launch_gemv_wide<F, NC>(c, calls[0], rb, K)) return;
    constexpr uint32_t UW = unit_weights<F>();
    const size_t tab = gemv_tab_rows<F>() * 16;
    const uint32_t units = K / UW;
    // stage all of x when it fits, else in chunks of 64-unit groups (per
    // 32 weights: three 32-byte digit planes and a float4 of group data)
    const size_t per_unit = (size_t)NC * unit_lds_bytes<F>();
    const size_t red = 4 * GV_SLOTS * NC * 4 * sizeof(float);
    uint32_t cunits = (units + 63) / 64 * 64;
    const size_t budget = c->max_lds - tab - red;
    if (cunits * per_unit > budget) cunits = (uint32_t)(budget / per_unit) / 64 * 64;
    const size_t lds = tab + cunits * per_unit + red;
    uint32_t rows = 0;
    for (int i = 0; i < n; i++) rows += calls[i].M;
    const uint32_t waves1 = (rows + GV_SLOTS - 1) / GV_SLOTS;  // wavefronts without a split
    uint32_t S = c->gemv_s ? (uint32_t)c->gemv_s : (NC == 1 && waves1 < 3072 ? 2 : 1);
    if (S >= 4) launch_gemv_s<F, NC, 4, SILU>(c, calls, n, rb, K, cunits, lds);
    else if (S == 2) launch_gemv_s<F, NC, 2, SILU>(c, calls, n, rb, K, cunits, lds);
    else launch_gemv_s<F, NC, 1, SILU>(c, calls, n, rb, K, cunits, lds);
}

// Q2_0 matvecs of the Bonsai shapes on the integer matrix cores
// (q2m_gemv_kernel, okf_ffn_mfma.h): K = 2048 (gate / up, alone or paired
// with the SiLU) or 6144 (down, with or without the SiLU formed in the
// staging), one workgroup per CU; true when launched.
inline bool launch_q2m(okf_ctx *c, const GemvCall &g0, const GemvCall *g1, uint64_t rb, uint32_t K) {
    if (!c->q2_mfma || !c->cus || (K != 2048 && K != 6144) || (g1 && (K != 2048 || g1->M != g0.M))) return false;
    const uint32_t G = c->cus, R = (g0.M + G - 1) / G, nt = ((g1 ? 2 : 1) * R + 15) / 16;
    // Eight wavefronts (with sixteen, each a half of the K blocks, gate / up
    // took 4.89 against 4.09 us and down 4.33 against 4.25; with four, gate /
    // up 4.40 against 4.14); twelve for the K-split down, so that every
    // thread stages one slot of its 6144 values (3.67 against 3.76 us).
    constexpr uint32_t nw = 8, nwk = 12;
    const bool ks = K == 6144 && !g1 && nt == 1 && R <= 8 && c->q2_ks;
    const size_t lds = q2m_lds_bytes(K, ks ? nwk : nw);
    if (lds > c->max_lds || nt > 3) return false;
    const Q2mArgs a{g0.W, g1 ? g1->W : nullptr, rb, K, g0.M, g0.X, g0.X2, g0.Y, g1 ? g1->Y : nullptr};
    const void *fn = nullptr;
    if (K == 2048 && g1 && !g0.X2) fn = nt == 3 ? (const void *)q2m_gemv_kernel<2, 3, true, false, nw> : nullptr;
    else if (K == 2048 && !g0.X2) fn = nt == 2 ? (const void *)q2m_gemv_kernel<2, 2, false, false, nw> : nullptr;
    else if (ks)
        fn = g0.X2 ? (const void *)q2m_gemv_kernel<4, 1, false, true, nwk, true>
                   : (const void *)q2m_gemv_kernel<4, 1, false, false, nwk, true>;
    else if (K == 6144 && !g1 && nt == 1)
        fn = g0.X2 ? (const void *)q2m_gemv_kernel<6, 1, false, true, nw>
                   : (const void *)q2m_gemv_kernel<6, 1, false, false, nw>;
    if (!fn) return false;
    void *args[] = {(void *)&a};
    if (hipLaunchKernel(fn, dim3(G), dim3((ks ? nwk : nw) * 64), args, lds, c->stream) == hipSuccess) return true;
    (void)hipGetLastError();  // (the caller's fallback launch is the call's result)
    return false;
}

// okf_ffn's two launches both on q2m_gemv_kernel (gate / up K 2048, down K
// 6144): then they are faster than the one launch with its grid barrier
// (8.6 against 9.5 us a step), so okf_ffn takes them unless told otherwise.
inline bool q2m_ffn_fits(const okf_ctx *c, uint32_t ka, uint32_t ma, uint32_t mb) {
    if (!c->q2_mfma || !c->cus || ka != 2048 || ma != 6144) return false;
    const uint32_t G = c->cus, ra = (ma + G - 1) / G, rb = (mb + G - 1) / G;
    return (2 * ra + 15) / 16 == 3 && (rb + 15) / 16 == 1 && q2m_lds_bytes(6144, 12) <= c->max_lds;
}

template <int F>
void launch_gemv(okf_ctx *c, const GemvCall *calls, int n, uint64_t rb, uint32_t K, uint32_t N) {
    if constexpr (F == Q2_0)
        if (n == 1 && N == 1 && launch_q2m(c, calls[0], nullptr, rb, K)) return;
    if (calls[0].X2) {  // SiLU-gated activations: one column
        launch_gemv_nc<F, 1, true>(c, calls, n, rb, K);
        return;
    }
    switch (N) {
    case 1: launch_gemv_nc<F, 1>(c, calls, n, rb, K); break;
    case 2: launch_gemv_nc<F, 2>(c, calls, n, rb, K); break;
    case 3: launch_gemv_nc<F, 3>(c, calls, n, rb, K); break;
    case 4: launch_gemv_nc<F, 4>(c, calls, n, rb, K); break;
    default: launch_gemv_nc<F, 5>(c, calls, n, rb, K); break;
    }
}

// The FFN's gate and up (one format, same shape, shared x) in one grid
// whose workgroups each take the same rows of both: gate <- silu(gate x) *
// (up x), up <- up x.  The down projection then reads one activation vector
// with no SiLU in its staging.
template <int F>
void launch_gemv_pair(okf_ctx *c, const GemvCall *calls, uint64_t rb, uint32_t K) {
    if constexpr (F == Q2_0)
        if (launch_q2m(c, calls[0], &calls[1], rb, K)) return;
    constexpr uint32_t UW = unit_weights<F>();
    const size_t tab = gemv_tab_rows<F>() * 16;
    const uint32_t units = K / UW;
    const size_t per_unit = unit_lds_bytes<F>();
    const size_t red = 4 * GV_SLOTS * 4 * sizeof(float);
    uint32_t cunits = (units + 63) / 64 * 64;
    const size_t budget = c->max_lds - tab - red;
    if (cunits * per_unit > budget) cunits = (uint32_t)(budget / per_unit) / 64 * 64;
    launch_gemv_s<F, 1, 1, false>(c, calls, 2, rb, K, cunits, tab + cunits * per_unit + red, true);
}

// The FFN block of Q2_0 gate / up / down in one launch (grid barrier)
// (okf_fmt_q2_0.hip): false, with nothing launched, where its shape or the
// device does not fit it.
bool launch_ffn_fused(okf_ctx *c, const FfnArgs &a);

// Whether the context's scratch may grow now: not after okf_ctx_reserve, and
// not while the stream is being captured into a graph (a synchronisation or
// hipMalloc would invalidate the capture).
inline bool can_grow(okf_ctx *c) {
    if (c->reserved) return false;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(c->stream, &cs) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return cs == hipStreamCaptureStatusNone;
}

// Grows one scratch buffer to at least `need` bytes (the stream is drained
// before an old buffer is freed).  Where it may not grow (can_grow) a call
// that needs more is an OKF_E_SHAPE, so nothing on a reserved or captured
// hot path allocates or synchronises.  `optional`: a failure leaves the
// buffer as it was and records no HIP error (the caller runs without it).
inline int grow_buf(okf_ctx *c, void **buf, size_t &bytes, size_t need, bool zero, bool optional) {
    if (need <= bytes) return OKF_OK;
    if (!can_grow(c)) return OKF_E_SHAPE;
    hipError_t e = hipSuccess;
    if (*buf) {
        e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) return optional ? ((void)hipGetLastError(), OKF_E_HIP) : hip_fail(c, e);
        (void)hipFree(*buf);
        *buf = nullptr;
        bytes = 0;
    }
    e = hipMalloc(buf, need);
    if (e == hipSuccess && zero) e = hipMemset(*buf, 0, need);
    if (e != hipSuccess) {
        if (*buf) (void)hipFree(*buf);
        *buf = nullptr;
        return optional ? ((void)hipGetLastError(), OKF_E_HIP) : hip_fail(c, e);
    }
    bytes = need;
    return OKF_OK;
}

// split-tile partial sums and argmax pairs
inline int grow_part(okf_ctx *c, size_t need, bool optional = false) {
    return grow_buf(c, (void **)&c->part, c->part_bytes, need, false, optional);
}

// argmax row counters, zeroed when allocated (the kernel leaves them zero)
inline int grow_cnt(okf_ctx *c, size_t rows) {
    size_t bytes = c->cnt_n * sizeof(uint32_t);
    const int st = grow_buf(c, (void **)&c->cnt, bytes, rows * sizeof(uint32_t), true, false);
    c->cnt_n = bytes / sizeof(uint32_t);
    return st;
}

// the fp16 copy of a GEMM's activations: N K values
inline int grow_xh(okf_ctx *c, size_t need, bool optional = false) {
    return grow_buf(c, (void **)&c->xh, c->xh_bytes, need, false, optional);
}

// The wide-tile Q4_K GEMM (gemm_q4k_w8_kernel): one 256 x 128 tile per CU.
// Whole rounds of `cus` tiles stay whole; each remaining tile is split over
// 16 thin pieces of 64 rows x 32 tokens (gemm_q4k_thin_kernel), or, with
// OKF_GEMM_KS set, over ks K ranges of whole superblocks
// (ks * remaining <= cus), whose partial tiles gemm_split_sum_kernel adds in
// K order.
inline int launch_gemm_q4k_w(okf_ctx *c, const uint8_t *W, uint64_t rb, uint32_t K, uint32_t M, uint32_t N,
                      float *Y) {
    const uint32_t tm = (M + QW_BM - 1) / QW_BM, tn = (N + QG_BN - 1) / QG_BN, sbs = K / 256;
    GemmSplit sp{};
    sp.tiles_n = tn;
    sp.tiles = tm * tn;
    sp.ng = (uint32_t)c->gemm_ng;
    const uint32_t round = c->cus ? c->cus : 256, rem = sp.tiles % round;
    sp.full = sp.tiles - rem;
    sp.ks = rem ? std::min(c->gemm_ks > 0 ? (uint32_t)c->gemm_ks : round / rem, sbs) : 1;
    if (sp.ks < 2) {
        sp.full = sp.tiles + 7 & ~7u;  // no split: every tile whole
        sp.ks = 1;
    } else if (c->gemm_ks == 0) {
        // the leftover tiles as 16 thin pieces each (gemm_q4k_thin_kernel)
        if (sp.full) {
            sp.ks = 1;
            sp.full_xcd = sp.full / 8;
            hipLaunchKernelGGL((gemm_q4k_w8_kernel<2, 2>), dim3(sp.full), dim3(512), 0, c->stream, W, rb, K, M,
                               (const _Float16 *)c->xh, N, Y, sp);
        }
        auto thin = [&](auto kern, uint32_t nw) {
            hipLaunchKernelGGL(kern, dim3((rem * 16 + 7) & ~7u), dim3(nw * 64), 0, c->stream, W, rb, K, M,
                               (const _Float16 *)c->xh, N, Y, sp.full, tn, rem * 16);
        };
        switch (c->gemm_thin) {
            case 1: thin(gemm_q4k_thin_kernel<8, 2>, 8); break;
            case 2: thin(gemm_q4k_thin_kernel<8, 4>, 8); break;
            case 3: thin(gemm_q4k_thin_kernel<4, 2>, 4); break;
            case 5: thin(gemm_q4k_thin_kernel<4, 6>, 4); break;
            default: thin(gemm_q4k_thin_kernel<4, 4>, 4); break;
        }
        return OKF_OK;
    }
    sp.full_xcd = sp.full / 8;
    sp.units = sp.ks > 1 ? rem * sp.ks : 0;
    sp.units_xcd = (sp.units + 7) / 8;
    if (sp.units) {
        const int st = grow_part(c, (size_t)sp.units * QW_BM * QG_BN * sizeof(float));
        if (st) return st;
        sp.part = c->part;
    }
    const uint32_t grid = 8 * (sp.full_xcd + sp.units_xcd);
    hipLaunchKernelGGL((gemm_q4k_w8_kernel<2, 2>), dim3(grid), dim3(512), 0, c->stream, W, rb, K, M,
                       (const _Float16 *)c->xh, N, Y, sp);
    if (sp.units)
        hipLaunchKernelGGL(gemm_split_sum_kernel<QW_BM>, dim3((sp.tiles - sp.full) * (QW_BM * QG_BN / 1024)),
                           dim3(256), 0, c->stream, (const float *)c->part, Y, M, N, sp);
    return OKF_OK;
}

template <int F>
int launch_gemm(okf_ctx *c, const uint8_t *W, uint64_t rb, uint32_t K, uint32_t M, const float *X,
                uint32_t N, float *Y) {
    if constexpr (F == Q4_K) {
        // fp16 activations, converted once per call into the context's buffer
        const int st = grow_xh(c, (size_t)N * K * sizeof(_Float16));
        if (st) return st;
        const uint64_t n4 = (uint64_t)N * K / 4;
        hipLaunchKernelGGL(x_to_f16_kernel, dim3((uint32_t)((n4 + 256 * XV - 1) / (256 * XV))), dim3(256), 0,
                           c->stream, X, c->xh, n4);
        return launch_gemm_q4k_w(c, W, rb, K, M, N, Y);
    }
    // a grid of fewer than two tiles a CU (small M or N) takes K in ks
    // ranges of whole 64-steps, partial tiles added by gemm_ksum_kernel
    // (measured on MI355X, N = 512: Q2_0 2048 x 6144 178 us, Q8_0 2048 x 2048
    // 72.6 us as one K range); without room for the partials (a reserved
    // context), one range
    const uint32_t tiles = ((N + GB_N - 1) / GB_N) * ((M + GB_M - 1) / GB_M), steps = (K + GB_K - 1) / GB_K;
    uint32_t ks = 1;
    if (c->gemm_split != 0 && tiles < 2 * c->cus) {
        ks = c->gemm_split > 1 ? (uint32_t)c->gemm_split : (2 * c->cus + tiles - 1) / tiles;
        ks = std::max(1u, std::min(ks, steps / 4));
    }
    const uint32_t kper = (steps + ks - 1) / ks * GB_K;
    ks = (K + kper - 1) / kper;
    float *part = nullptr;
    if (ks > 1) {
        if (grow_part(c, (size_t)ks * N * M * sizeof(float), true) == OKF_OK) part = c->part;
        else ks = 1;
    }
    // from N = 256 X is converted to fp16 once (every row tile would round
    // the same columns again), when the buffer can hold it (measured, us,
    // N = 512: Q2_0 6144 x 2048 58.9 -> 46.0, 2048 x 6144 52.0 -> 41.8; at
    // N = 64..128 the extra launch costs about what it saves)
    const _Float16 *xh = nullptr;
    if (c->gemm_xh && N >= 256 && K % 32 == 0 && grow_xh(c, (size_t)N * K * sizeof(_Float16), true) == OKF_OK) {
        const uint64_t n4 = (uint64_t)N * K / 4;
        hipLaunchKernelGGL(x_to_f16_kernel, dim3((uint32_t)((n4 + 256 * XV - 1) / (256 * XV))), dim3(256), 0,
                           c->stream, X, c->xh, n4);
        xh = c->xh;
    }
    dim3 grid((N + GB_N - 1) / GB_N, (M + GB_M - 1) / GB_M, ks);
    hipLaunchKernelGGL((gemm_mfma_kernel<F>), grid, dim3(256), 0, c->stream, W, rb, K, M, X, N, Y,
                       c->grid, c->grids, ks > 1 ? kper : (steps * GB_K), part, xh);
    if (part) {
        const uint64_t nm = (uint64_t)N * M;
        hipLaunchKernelGGL(gemm_ksum_kernel, dim3((uint32_t)((nm + 1023) / 1024)), dim3(256), 0, c->stream,
                           (const float *)part, Y, nm, ks, (uint32_t)(nm % 4 == 0 && aligned16(Y)));
    }
    return OKF_OK;
}

template <int F>
void launch_dequant(okf_ctx *c, const uint8_t *row, uint32_t n, float *out) {
    const uint32_t units = n / 32;
    hipLaunchKernelGGL((dequant_row_kernel<F>), dim3((units + 255) / 256), dim3(256), 0, c->stream,
                       row, units, out, c->grid, c->grids);
}

template <int F>
void launch_embed(okf_ctx *c, const uint8_t *W, uint64_t rb, uint32_t K, uint32_t M,
                  const int32_t *ids, uint32_t N, float *out) {
    const uint32_t upr = K / 32, units = N * upr;
    hipLaunchKernelGGL((embed_batch_kernel<F>), dim3((units + 255) / 256), dim3(256), 0, c->stream, W,
                       rb, M, ids, upr, units, out, c->grid, c->grids);
}

// Every format with kernels here, for the per-format instantiations.
#define OKF_FOR_EACH_FORMAT(X)                                                                           \
    X(Q8_0) X(Q2_0) X(Q4_K) X(Q4_0) X(IQ4_NL) X(Q5_K) X(Q6_K) X(IQ4_XS) X(IQ2_XS) X(IQ2_S) X(IQ3_XXS)     \
    X(IQ3_S) X(IQ1_S) X(IQ1_M) X(Q2_K) X(Q3_K) X(F32) X(F16) X(BF16) X(IQ2_XXS)

#define OKF_LAUNCHERS(EXT, F)                                                                            \
    EXT template void launch_gemv<F>(okf_ctx *, const GemvCall *, int, uint64_t, uint32_t, uint32_t);    \
    EXT template void launch_gemv_pair<F>(okf_ctx *, const GemvCall *, uint64_t, uint32_t);               \
    EXT template int launch_gemm<F>(okf_ctx *, const uint8_t *, uint64_t, uint32_t, uint32_t, const float *, \
                                    uint32_t, float *);                                                  \
    EXT template void launch_dequant<F>(okf_ctx *, const uint8_t *, uint32_t, float *);                  \
    EXT template void launch_embed<F>(okf_ctx *, const uint8_t *, uint64_t, uint32_t, uint32_t,          \
                                      const int32_t *, uint32_t, float *);
#define OKF_EXTERN(F) OKF_LAUNCHERS(extern, F)
#define OKF_INSTANTIATE(F) OKF_LAUNCHERS(, F)

}  // namespace okf_impl
