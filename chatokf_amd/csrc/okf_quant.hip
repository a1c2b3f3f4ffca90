// okf_quant.hip -- the C ABI (include/okf_quant.h) over the gfx950 kernels.
//
// Host-side dispatch mirrors the reference's MetalEnc (LLM/Base/MetalEnc.swift):
// gemv picks the per-format kernel (:84-153), gemm applies the
// N == 1 / 2..5 / > 5 policy (:241-289), dequantRow unpacks one row (:402-459).
// Validation failures return a status instead of the reference's
// fatalError / precondition.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <new>

#include "../../include/okf_quant.h"
#include "okf_common.h"
#include "okf_decode.h"
#include "okf_gemm.h"
#include <algorithm>
#include <type_traits>
#include <vector>
#include "okf_gemv.h"
#include "okf_gemv_wide.h"
#include "okf_gguf.h"
#include "okf_norm.h"

#include "iq2xxs_grid.inc"
#include "iq_grids.inc"

// one matvec y = W x of a launch group (with X2: x = silu(X) * X2)
struct GemvCall {
    const uint8_t *W;
    const float *X;
    float *Y;
    uint32_t M;
    const float *X2 = nullptr;
};

struct okf_gguf {
    okf_gguf_impl::File f;
};

// The scratch of okf_argmax_rows_noalloc: OKF_NOALLOC_ARGMAX_PAIRS
// (value, index) pairs, then OKF_NOALLOC_ARGMAX_ROWS row counters (zero
// between calls: zero at load, and each call's last workgroup per row sets
// its counter back).  Each GPU holds its own copy until the process ends;
// host code uses the device address hipGetSymbolAddress gives, never the
// name (which is a host-side stand-in).
constexpr size_t SCRATCH_CNT_OFF = (size_t)OKF_NOALLOC_ARGMAX_PAIRS * 8;
static __device__ __align__(256) uint8_t scratch[SCRATCH_CNT_OFF + (size_t)OKF_NOALLOC_ARGMAX_ROWS * 4];

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
    int gemm_ks = 0;     // wide-tile GEMM: K ranges per remainder tile (0 = auto)
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
};

namespace {

using namespace okf;

bool supported(int32_t t) {
    return t == Q8_0 || t == Q4_K || t == IQ2_XXS || t == Q2_0 || t == Q4_0 || t == IQ4_NL || t == Q5_K ||
           t == Q6_K || t == IQ4_XS || grid_fmt(t);
}

int hip_fail(okf_ctx *c, hipError_t e) {
    c->last_hip = (int)e;
    return OKF_E_HIP;
}

// splitmix64 -> uniform [0, 1); deterministic per seed.
double next_uniform(uint64_t &s) {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (double)(z >> 11) * (1.0 / 9007199254740992.0);
}

// Shared prologue of every launch call: arguments, fault injection, device.
int begin(okf_ctx *c) {
    if (!c) return OKF_E_ARG;
    if (c->fault_rate > 0 && next_uniform(c->fault_state) < c->fault_rate) return OKF_E_INJECTED;
    if (c->device < 0) return OKF_E_NODEV;
    hipError_t e = hipSetDevice(c->device);
    return e == hipSuccess ? OKF_OK : hip_fail(c, e);
}

int check_weight(const okf_weight *w, uint64_t *row_bytes) {
    if (!w || !w->base) return OKF_E_ARG;
    if (!supported(w->ggml_type)) return OKF_E_TYPE;
    if (w->K == 0 || w->M == 0 || w->K % block_elems(w->ggml_type)) return OKF_E_SHAPE;
    *row_bytes = (uint64_t)w->K / block_elems(w->ggml_type) * block_bytes(w->ggml_type);
    const uintptr_t a = (uintptr_t)w->base + w->off;
    // Q4_K kernels read 16-byte header/code chunks; others need 2-byte alignment.
    if (w->ggml_type == Q4_K ? (a & 15) : (a & 1)) return OKF_E_SHAPE;
    return OKF_OK;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// Raises a kernel's dynamic LDS limit once per device (done: one bit per
// device, shared by every context and thread; a repeated call is harmless).
void set_lds_attr(const okf_ctx *c, const void *fn, std::atomic<uint64_t> &done) {
    const uint64_t bit = 1ull << (c->device & 63);
    if (done.load(std::memory_order_acquire) & bit) return;
    (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)c->max_lds);
    done.fetch_or(bit, std::memory_order_acq_rel);
}

int finish(okf_ctx *c) {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? OKF_OK : hip_fail(c, e);
}

// IQ2_XXS tables the matvec keeps in LDS: the grid as fp16 (entry e = 8
// halves, two per dword) and, per 7-bit sign index, the fp16 sign bits of the
// eight weights (the eighth from the even-parity rule of ksigns,
// LLM/Quantize/IQ2Grid.swift:73).
void build_iq2_tables(uint32_t *t) {
    for (int e = 0; e < 256; e++) {
        const uint64_t g = okf_iq2xxs_grid_host[e];
        for (int j = 0; j < 4; j++) {
            const _Float16 a = (_Float16)(float)((g >> (16 * j)) & 0xFF);
            const _Float16 b = (_Float16)(float)((g >> (16 * j + 8)) & 0xFF);
            t[e * 4 + j] = (uint32_t)__builtin_bit_cast(uint16_t, a) |
                           ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
        }
    }
    for (int s7 = 0; s7 < 128; s7++) {
        const uint32_t s = s7 | ((__builtin_popcount(s7) & 1u) << 7);
        for (int j = 0; j < 4; j++)
            t[(256 + s7) * 4 + j] = (((s >> (2 * j)) & 1u) << 15) | (((s >> (2 * j + 1)) & 1u) << 31);
    }
}

// The same tables for the integer dot-product kernels: grid entry e as its 8
// unsigned bytes {lo, hi, 0, 0}; sign entry s7 as the byte mask M (0xFF per
// negative weight) and M & 0x01010101, {M.lo, M.hi, M1.lo, M1.hi}, so that a
// signed weight byte is (g ^ M) + M1.
void build_iq2_tables8(uint32_t *t) {
    for (int e = 0; e < 256; e++) {
        const uint64_t g = okf_iq2xxs_grid_host[e];
        t[e * 4 + 0] = (uint32_t)g;
        t[e * 4 + 1] = (uint32_t)(g >> 32);
        t[e * 4 + 2] = t[e * 4 + 3] = 0;
    }
    for (int s7 = 0; s7 < 128; s7++) {
        const uint32_t s = s7 | ((__builtin_popcount(s7) & 1u) << 7);
        uint32_t m[2] = {0, 0};
        for (int j = 0; j < 8; j++)
            if ((s >> j) & 1) m[j >> 2] |= 0xFFu << (8 * (j & 3));
        t[(256 + s7) * 4 + 0] = m[0];
        t[(256 + s7) * 4 + 1] = m[1];
        t[(256 + s7) * 4 + 2] = m[0] & 0x01010101u;
        t[(256 + s7) * 4 + 3] = m[1] & 0x01010101u;
    }
}

template <int F, int NC, int S, bool SILU, int DX = 0>
void launch_gemv_s(okf_ctx *c, const GemvCall *calls, int n, uint64_t rb, uint32_t K,
                   uint32_t cunits, size_t lds) {
    // Q2_0 and Q8_0 at N = 1: a three-deep ring when a wavefront runs three
    // or more steps (the down projection), so that no step waits for a load
    // issued after the first compute; two otherwise (a third buffer would
    // only re-read).  Measured: Q2_0 2048x6144 4.95 -> 4.75 us.
    if constexpr (DX == 0 && NC == 1 && (F == Q2_0 || F == Q8_0)) {
        const uint32_t steps = (K / unit_weights<F>() + GV_L * S - 1) / (GV_L * S);
        if (steps >= 3) return launch_gemv_s<F, NC, S, SILU, 3>(c, calls, n, rb, K, cunits, lds);
    }
    // two rows per slot (each staged activation read serves both) where
    // measured faster: IQ2_XXS with 2..5 columns, Q4_K and Q2_0 with 5.  (A
    // three-deep ring for the Q4_K matvec measured 3-4 % slower than two
    // once the weight loads were issued behind the staging's.)
    constexpr int R = ((F == IQ2_XXS && NC >= 2) || (NC == 5 && F != Q8_0 && F != Q5_K && F != Q6_K && F != IQ4_XS && !grid_fmt(F))) ? 2 : 1,
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
    // the tables the compute reads: IQ2_XXS's LDS rows (copied from c->tab),
    // or the grid formats' device-memory grids
    const u32x4 *tabs = grid_fmt(F) ? (const u32x4 *)c->grids : c->tab8;
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
    constexpr int D = 4;
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

template <int F, int NC, bool SILU = false>
void launch_gemv_nc(okf_ctx *c, const GemvCall *calls, int n, uint64_t rb, uint32_t K) {
    // (Q4_K and Q8_0 units are too large for a deep ring at N > 1; the
    // formats added after the measurements take the many-workgroup kernel)
    if constexpr (!SILU && !((F == Q4_K || F == Q8_0) && NC > 1) && F != Q5_K && F != Q6_K && F != IQ4_XS &&
                  !grid_fmt(F))
        if (n == 1 && launch_gemv_wide<F, NC>(c, calls[0], rb, K)) return;
    constexpr uint32_t UW = unit_weights<F>();
    const size_t tab = F == IQ2_XXS ? 384 * 16 : 0;
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

template <int F>
void launch_gemv(okf_ctx *c, const GemvCall *calls, int n, uint64_t rb, uint32_t K, uint32_t N) {
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

// The context's scratch (split-tile partial sums, argmax pairs), grown to at
// least `need` bytes; the stream is drained before an old buffer is freed.
// After okf_ctx_reserve the sizes are fixed: a call that needs more is an
// OKF_E_SHAPE, so nothing on the hot path allocates or synchronises.
int grow_part(okf_ctx *c, size_t need) {
    if (need <= c->part_bytes) return OKF_OK;
    if (c->reserved) return OKF_E_SHAPE;
    hipError_t e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) return hip_fail(c, e);
    if (c->part) (void)hipFree(c->part);
    c->part = nullptr;
    c->part_bytes = 0;
    e = hipMalloc((void **)&c->part, need);
    if (e != hipSuccess) return hip_fail(c, e);
    c->part_bytes = need;
    return OKF_OK;
}

// argmax row counters, zeroed when allocated (the kernel leaves them zero)
int grow_cnt(okf_ctx *c, size_t rows) {
    if (rows <= c->cnt_n) return OKF_OK;
    if (c->reserved) return OKF_E_SHAPE;
    hipError_t e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) return hip_fail(c, e);
    if (c->cnt) (void)hipFree(c->cnt);
    c->cnt = nullptr;
    c->cnt_n = 0;
    e = hipMalloc((void **)&c->cnt, rows * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMemset(c->cnt, 0, rows * sizeof(uint32_t));
    if (e != hipSuccess) return hip_fail(c, e);
    c->cnt_n = rows;
    return OKF_OK;
}

// the fp16 copy of a Q4_K GEMM's activations: N K values
int grow_xh(okf_ctx *c, size_t need) {
    if (need <= c->xh_bytes) return OKF_OK;
    if (c->reserved) return OKF_E_SHAPE;
    if (c->xh) {
        hipError_t e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) return hip_fail(c, e);
        (void)hipFree(c->xh);
        c->xh = nullptr;
        c->xh_bytes = 0;
    }
    hipError_t e = hipMalloc((void **)&c->xh, need);
    if (e != hipSuccess) return hip_fail(c, e);
    c->xh_bytes = need;
    return OKF_OK;
}

// The wide-tile Q4_K GEMM (gemm_q4k_w8_kernel): one 256 x 128 tile per CU.
// Whole rounds of `cus` tiles stay whole; each remaining tile is split over
// 16 thin pieces of 64 rows x 32 tokens (gemm_q4k_thin_kernel), or, with
// OKF_GEMM_KS set, over ks K ranges of whole superblocks
// (ks * remaining <= cus), whose partial tiles gemm_split_sum_kernel adds in
// K order.
int launch_gemm_q4k_w(okf_ctx *c, const uint8_t *W, uint64_t rb, uint32_t K, uint32_t M, uint32_t N,
                      float *Y) {
    const uint32_t tm = (M + QW_BM - 1) / QW_BM, tn = (N + QG_BN - 1) / QG_BN, sbs = K / 256;
    GemmSplit sp{};
    sp.tiles_n = tn;
    sp.tiles = tm * tn;
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
    sp.ng = (uint32_t)c->gemm_ng;
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
    dim3 grid((N + GB_N - 1) / GB_N, (M + GB_M - 1) / GB_M);
    hipLaunchKernelGGL((gemm_mfma_kernel<F>), grid, dim3(256), 0, c->stream, W, rb, K, M, X, N, Y,
                       c->grid, c->grids);
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

#define OKF_DISPATCH(type, fn, ...)                         \
    switch (type) {                                         \
    case Q8_0: fn<Q8_0>(__VA_ARGS__); break;                \
    case Q2_0: fn<Q2_0>(__VA_ARGS__); break;                \
    case Q4_K: fn<Q4_K>(__VA_ARGS__); break;                \
    case Q4_0: fn<Q4_0>(__VA_ARGS__); break;                \
    case IQ4_NL: fn<IQ4_NL>(__VA_ARGS__); break;            \
    case Q5_K: fn<Q5_K>(__VA_ARGS__); break;                \
    case Q6_K: fn<Q6_K>(__VA_ARGS__); break;                \
    case IQ4_XS: fn<IQ4_XS>(__VA_ARGS__); break;            \
    case IQ2_XS: fn<IQ2_XS>(__VA_ARGS__); break;            \
    case IQ2_S: fn<IQ2_S>(__VA_ARGS__); break;              \
    case IQ3_XXS: fn<IQ3_XXS>(__VA_ARGS__); break;          \
    case IQ3_S: fn<IQ3_S>(__VA_ARGS__); break;              \
    case IQ1_S: fn<IQ1_S>(__VA_ARGS__); break;              \
    case IQ1_M: fn<IQ1_M>(__VA_ARGS__); break;              \
    case Q2_K: fn<Q2_K>(__VA_ARGS__); break;                \
    case Q3_K: fn<Q3_K>(__VA_ARGS__); break;                \
    case F32: fn<F32>(__VA_ARGS__); break;                  \
    case F16: fn<F16>(__VA_ARGS__); break;                  \
    case BF16: fn<BF16>(__VA_ARGS__); break;                \
    default: fn<IQ2_XXS>(__VA_ARGS__); break;               \
    }

enum class Path { Auto, Tile };

int run_gemm(okf_ctx *c, const okf_weight *w, const float *X, uint32_t N, float *Y, Path path,
             const float *X2 = nullptr) {
    uint64_t rb = 0;
    int st = check_weight(w, &rb);
    if (st) return st;
    if (!X || !Y) return OKF_E_ARG;
    if (N == 0) return OKF_E_SHAPE;
    if (!aligned16(X) || (X2 && !aligned16(X2))) return OKF_E_SHAPE;
    if ((st = begin(c))) return st;
    const uint8_t *W = (const uint8_t *)w->base + w->off;
    if (path == Path::Auto && N <= 5) {
        const GemvCall call{W, X, Y, w->M, X2};
        if (c->grouping && N == 1) {
            // inside a parallel group: launched together at okf_parallel_end
            // (capacity for a whole launch group is reserved at
            // okf_parallel_begin; past it a failed allocation is a status)
            try {
                c->pending.push_back({w->ggml_type, w->K, rb, call});
            } catch (const std::bad_alloc &) {
                return OKF_E_ARG;
            }
            return OKF_OK;
        }
        OKF_DISPATCH(w->ggml_type, launch_gemv, c, &call, 1, rb, w->K, N);
    } else {
        switch (w->ggml_type) {
        case Q8_0: st = launch_gemm<Q8_0>(c, W, rb, w->K, w->M, X, N, Y); break;
        case Q2_0: st = launch_gemm<Q2_0>(c, W, rb, w->K, w->M, X, N, Y); break;
        case Q4_K: st = launch_gemm<Q4_K>(c, W, rb, w->K, w->M, X, N, Y); break;
        case Q4_0: st = launch_gemm<Q4_0>(c, W, rb, w->K, w->M, X, N, Y); break;
        case IQ4_NL: st = launch_gemm<IQ4_NL>(c, W, rb, w->K, w->M, X, N, Y); break;
        case Q5_K: st = launch_gemm<Q5_K>(c, W, rb, w->K, w->M, X, N, Y); break;
        case Q6_K: st = launch_gemm<Q6_K>(c, W, rb, w->K, w->M, X, N, Y); break;
        case IQ4_XS: st = launch_gemm<IQ4_XS>(c, W, rb, w->K, w->M, X, N, Y); break;
        case IQ2_XS: st = launch_gemm<IQ2_XS>(c, W, rb, w->K, w->M, X, N, Y); break;
        case IQ2_S: st = launch_gemm<IQ2_S>(c, W, rb, w->K, w->M, X, N, Y); break;
        case IQ3_XXS: st = launch_gemm<IQ3_XXS>(c, W, rb, w->K, w->M, X, N, Y); break;
        case IQ3_S: st = launch_gemm<IQ3_S>(c, W, rb, w->K, w->M, X, N, Y); break;
        case IQ1_S: st = launch_gemm<IQ1_S>(c, W, rb, w->K, w->M, X, N, Y); break;
        case IQ1_M: st = launch_gemm<IQ1_M>(c, W, rb, w->K, w->M, X, N, Y); break;
        case Q2_K: st = launch_gemm<Q2_K>(c, W, rb, w->K, w->M, X, N, Y); break;
        case Q3_K: st = launch_gemm<Q3_K>(c, W, rb, w->K, w->M, X, N, Y); break;
        case F32: st = launch_gemm<F32>(c, W, rb, w->K, w->M, X, N, Y); break;
        case F16: st = launch_gemm<F16>(c, W, rb, w->K, w->M, X, N, Y); break;
        case BF16: st = launch_gemm<BF16>(c, W, rb, w->K, w->M, X, N, Y); break;
        default: st = launch_gemm<IQ2_XXS>(c, W, rb, w->K, w->M, X, N, Y); break;
        }
        if (st) return st;
    }
    return finish(c);
}

// Launches the recorded matvecs: those of one format and one K together,
// GV_GROUP at a time, in recording order otherwise.
int flush_group(okf_ctx *c) {
    std::vector<okf_ctx::Pending> p;
    p.swap(c->pending);
    std::vector<bool> done(p.size(), false);
    for (size_t i = 0; i < p.size(); i++) {
        if (done[i]) continue;
        GemvCall calls[GV_GROUP];
        int n = 0;
        for (size_t j = i; j < p.size() && n < GV_GROUP; j++)
            if (!done[j] && p[j].type == p[i].type && p[j].K == p[i].K &&
                (p[j].call.X2 != nullptr) == (p[i].call.X2 != nullptr)) {
                calls[n++] = p[j].call;
                done[j] = true;
            }
        OKF_DISPATCH(p[i].type, launch_gemv, c, calls, n, p[i].rb, p[i].K, 1u);
    }
    return p.empty() ? OKF_OK : finish(c);
}

}  // namespace

extern "C" {

int okf_ctx_create(int device, okf_ctx **out) {
    if (!out) return OKF_E_ARG;
    *out = nullptr;
    okf_ctx *c = new (std::nothrow) okf_ctx();
    if (!c) return OKF_E_ARG;
    c->device = device;
    if (device >= 0) {
        hipError_t e = hipSetDevice(device);
        // A blocking stream: it orders with the legacy default stream, so buffers
        // filled there (e.g. by a framework) are complete before our kernels run.
        if (e == hipSuccess) e = hipStreamCreate(&c->stream);
        if (e == hipSuccess) e = hipMalloc((void **)&c->grid, sizeof(okf_iq2xxs_grid_host));
        if (e == hipSuccess)
            e = hipMemcpy(c->grid, okf_iq2xxs_grid_host, sizeof(okf_iq2xxs_grid_host),
                          hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMalloc((void **)&c->grids, GT_BYTES);
        if (e == hipSuccess) {
            static_assert(sizeof(okf_host_iq2xs_grid) == GT_IQ2S - GT_IQ2XS &&
                              sizeof(okf_host_iq2s_grid) == GT_IQ3XXS - GT_IQ2S &&
                              sizeof(okf_host_iq3xxs_grid) == GT_IQ3S - GT_IQ3XXS &&
                              sizeof(okf_host_iq3s_grid) == GT_IQ1S - GT_IQ3S &&
                              sizeof(okf_host_iq1s_grid) == GT_BYTES - GT_IQ1S,
                          "grid table layout");
            const struct { const void *p; size_t n, off; } parts[] = {
                {okf_host_iq2xs_grid, sizeof(okf_host_iq2xs_grid), GT_IQ2XS},
                {okf_host_iq2s_grid, sizeof(okf_host_iq2s_grid), GT_IQ2S},
                {okf_host_iq3xxs_grid, sizeof(okf_host_iq3xxs_grid), GT_IQ3XXS},
                {okf_host_iq3s_grid, sizeof(okf_host_iq3s_grid), GT_IQ3S},
                {okf_host_iq1s_grid, sizeof(okf_host_iq1s_grid), GT_IQ1S}};
            for (const auto &q : parts)
                if (e == hipSuccess) e = hipMemcpy(c->grids + q.off, q.p, q.n, hipMemcpyHostToDevice);
        }
        uint32_t tabh[384 * 4];
        build_iq2_tables(tabh);
        if (e == hipSuccess) e = hipMalloc((void **)&c->tab, sizeof(tabh));
        if (e == hipSuccess) e = hipMemcpy(c->tab, tabh, sizeof(tabh), hipMemcpyHostToDevice);
        build_iq2_tables8(tabh);
        if (e == hipSuccess) e = hipMalloc((void **)&c->tab8, sizeof(tabh));
        if (e == hipSuccess) e = hipMemcpy(c->tab8, tabh, sizeof(tabh), hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            if (c->grid) (void)hipFree(c->grid);
            if (c->grids) (void)hipFree(c->grids);
            if (c->tab) (void)hipFree(c->tab);
            if (c->tab8) (void)hipFree(c->tab8);
            if (c->stream) (void)hipStreamDestroy(c->stream);
            delete c;
            return OKF_E_HIP;
        }
        if (e == hipSuccess) e = hipGetSymbolAddress((void **)&c->scratch, HIP_SYMBOL(scratch));
        if (e != hipSuccess) {
            if (c->grid) (void)hipFree(c->grid);
            if (c->grids) (void)hipFree(c->grids);
            if (c->tab) (void)hipFree(c->tab);
            if (c->tab8) (void)hipFree(c->tab8);
            if (c->stream) (void)hipStreamDestroy(c->stream);
            delete c;
            return OKF_E_HIP;
        }
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, device) ==
                hipSuccess && v > 0)
            c->max_lds = (size_t)v;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess &&
            v > 0)
            c->cus = (uint32_t)v;
        if (const char *e = getenv("OKF_GEMV_S")) c->gemv_s = atoi(e);
        if (const char *e = getenv("OKF_GEMV_WIDE")) c->gemv_wide = atoi(e);
        if (const char *e = getenv("OKF_GEMM_KS")) c->gemm_ks = atoi(e);
        if (const char *e = getenv("OKF_GEMM_NG")) c->gemm_ng = atoi(e);
        if (const char *e = getenv("OKF_GEMM_THIN")) c->gemm_thin = atoi(e);
    } else if (device != -1) {
        delete c;
        return OKF_E_ARG;
    }
    *out = c;
    return OKF_OK;
}

int okf_ctx_destroy(okf_ctx *c) {
    if (!c) return OKF_E_ARG;
    int st = OKF_OK;
    if (c->device >= 0) {
        (void)hipSetDevice(c->device);
        if (hipStreamSynchronize(c->stream) != hipSuccess) st = OKF_E_HIP;
        (void)hipFree(c->grid);
        (void)hipFree(c->grids);
        (void)hipFree(c->tab);
        (void)hipFree(c->tab8);
        if (c->xh) (void)hipFree(c->xh);
        if (c->part) (void)hipFree(c->part);
        if (c->cnt) (void)hipFree(c->cnt);
        (void)hipStreamDestroy(c->stream);
    }
    delete c;
    return st;
}

int okf_ctx_stream(okf_ctx *c, void **stream) {
    if (!c || !stream) return OKF_E_ARG;
    if (c->device < 0) return OKF_E_NODEV;
    *stream = (void *)c->stream;
    return OKF_OK;
}

int okf_row_bytes(int32_t type, uint64_t n, uint64_t *out) {
    if (!out) return OKF_E_ARG;
    if (!supported(type)) return OKF_E_TYPE;
    if (type == F32 || type == F16 || type == BF16) {  // any n, as GGUF.rowByteCount
        *out = n * (type == F32 ? 4 : 2);
        return OKF_OK;
    }
    if (n % block_elems(type)) return OKF_E_SHAPE;
    *out = n / block_elems(type) * block_bytes(type);
    return OKF_OK;
}

int okf_gemv(okf_ctx *c, const okf_weight *w, const float *x, float *y) {
    return run_gemm(c, w, x, 1, y, Path::Auto);
}

int okf_gemm(okf_ctx *c, const okf_weight *w, const float *X, uint32_t N, float *Y) {
    return run_gemm(c, w, X, N, Y, Path::Auto);
}

int okf_gemm_tile(okf_ctx *c, const okf_weight *w, const float *X, uint32_t N, float *Y) {
    return run_gemm(c, w, X, N, Y, Path::Tile);
}

int okf_dequant_row(okf_ctx *c, const okf_weight *row, uint32_t n, float *out) {
    if (!row || !row->base || !out) return OKF_E_ARG;
    if (!supported(row->ggml_type)) return OKF_E_TYPE;
    if (n == 0 || n % block_elems(row->ggml_type)) return OKF_E_SHAPE;
    if (!aligned16(out)) return OKF_E_SHAPE;
    int st = begin(c);
    if (st) return st;
    const uint8_t *p = (const uint8_t *)row->base + row->off;
    OKF_DISPATCH(row->ggml_type, launch_dequant, c, p, n, out);
    return finish(c);
}

int okf_gemv_silu(okf_ctx *c, const okf_weight *w, const float *gate, const float *up, float *y) {
    if (!gate || !up) return OKF_E_ARG;
    return run_gemm(c, w, gate, 1, y, Path::Auto, up);
}

int okf_silu_mul(okf_ctx *c, float *a, const float *b, uint32_t n) {
    if (!a || !b) return OKF_E_ARG;
    if (n == 0) return OKF_E_SHAPE;
    int st = begin(c);
    if (st) return st;
    hipLaunchKernelGGL(silu_mul_kernel, dim3((n + 255) / 256), dim3(256), 0, c->stream, a, b, n);
    return finish(c);
}

int okf_add_rmsnorm_batch(okf_ctx *c, float *x, const float *r, const float *w, float *y, uint32_t n,
                          uint32_t rows, float eps) {
    if (!x || !w || !y) return OKF_E_ARG;
    if (n == 0 || rows == 0) return OKF_E_SHAPE;
    int st = begin(c);
    if (st) return st;
    if (r)
        hipLaunchKernelGGL(add_rmsnorm_kernel<true>, dim3(rows), dim3(NORM_THREADS), 0, c->stream, x, r, w, y,
                           n, eps);
    else
        hipLaunchKernelGGL(add_rmsnorm_kernel<false>, dim3(rows), dim3(NORM_THREADS), 0, c->stream, x, r, w,
                           y, n, eps);
    return finish(c);
}

int okf_argmax_rows(okf_ctx *c, const float *x, uint32_t n, uint32_t rows, int32_t *out) {
    if (!x || !out) return OKF_E_ARG;
    if (n == 0 || rows == 0 || n > 0x7FFFFFFFu || rows > 65535) return OKF_E_SHAPE;
    int st = begin(c);
    if (st) return st;
    const uint32_t chunks = (n + ARGMAX_CHUNK - 1) / ARGMAX_CHUNK;
    if ((st = grow_part(c, (size_t)chunks * rows * sizeof(ArgPair)))) return st;
    if ((st = grow_cnt(c, rows))) return st;
    hipLaunchKernelGGL(argmax_kernel, dim3(chunks, rows), dim3(NORM_THREADS), 0, c->stream, x, n,
                       (ArgPair *)c->part, c->cnt, out);
    return finish(c);
}

int okf_argmax_rows_noalloc(okf_ctx *c, const float *x, uint32_t n, uint32_t rows, int32_t *out) {
    if (!x || !out) return OKF_E_ARG;
    if (n == 0 || rows == 0 || n > 0x7FFFFFFFu || rows > OKF_NOALLOC_ARGMAX_ROWS) return OKF_E_SHAPE;
    const uint32_t chunks = (n + ARGMAX_CHUNK - 1) / ARGMAX_CHUNK;
    if ((uint64_t)chunks * rows > OKF_NOALLOC_ARGMAX_PAIRS) return OKF_E_SHAPE;
    int st = begin(c);
    if (st) return st;
    // the device's scratch array through its device address (c->scratch,
    // from hipGetSymbolAddress at okf_ctx_create): pairs, then row counters
    ArgPair *pairs = (ArgPair *)c->scratch;
    uint32_t *cnt = (uint32_t *)(c->scratch + SCRATCH_CNT_OFF);
    hipLaunchKernelGGL(argmax_kernel, dim3(chunks, rows), dim3(NORM_THREADS), 0, c->stream, x, n, pairs, cnt,
                       out);
    return finish(c);
}

int okf_ctx_reserve(okf_ctx *c, uint64_t gemm_nk, uint32_t argmax_n, uint32_t argmax_rows) {
    if (!c) return OKF_E_ARG;
    if (c->device < 0) return OKF_E_NODEV;
    if (argmax_rows > 65535 || argmax_n > 0x7FFFFFFFu) return OKF_E_SHAPE;
    (void)hipSetDevice(c->device);
    c->reserved = false;  // (grow up to the reservation)
    int st = grow_xh(c, (size_t)gemm_nk * sizeof(_Float16));
    const uint32_t chunks = (argmax_n + ARGMAX_CHUNK - 1) / ARGMAX_CHUNK;
    if (!st) st = grow_part(c, std::max<size_t>((size_t)chunks * argmax_rows * sizeof(ArgPair), 1));
    if (!st) st = grow_cnt(c, std::max<uint32_t>(argmax_rows, 1));
    if (st) return st;
    hipError_t e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) return hip_fail(c, e);
    c->reserved = true;
    return OKF_OK;
}

int okf_parallel_begin(okf_ctx *c) {
    if (!c) return OKF_E_ARG;
    if (c->grouping) return OKF_E_ARG;
    try {
        c->pending.reserve(4 * GV_GROUP);
    } catch (const std::bad_alloc &) {
        return OKF_E_ARG;
    }
    c->grouping = true;
    return OKF_OK;
}

int okf_parallel_end(okf_ctx *c) {
    if (!c) return OKF_E_ARG;
    if (!c->grouping) return OKF_E_ARG;
    c->grouping = false;
    if (c->pending.empty()) return OKF_OK;
    if (c->device < 0) return OKF_E_NODEV;
    (void)hipSetDevice(c->device);
    try {
        return flush_group(c);
    } catch (const std::bad_alloc &) {
        c->pending.clear();
        return OKF_E_ARG;
    }
}

int okf_embed_batch(okf_ctx *c, const okf_weight *w, const int32_t *ids, uint32_t N, float *out) {
    uint64_t rb = 0;
    int st = check_weight(w, &rb);
    if (st) return st;
    if (!ids || !out) return OKF_E_ARG;
    if (N == 0 || (uint64_t)N * (w->K / 32) > 0xFFFFFFFFull) return OKF_E_SHAPE;
    if (!aligned16(out)) return OKF_E_SHAPE;
    if ((st = begin(c))) return st;
    const uint8_t *W = (const uint8_t *)w->base + w->off;
    OKF_DISPATCH(w->ggml_type, launch_embed, c, W, rb, w->K, w->M, ids, N, out);
    return finish(c);
}

int okf_sync(okf_ctx *c) {
    if (!c) return OKF_E_ARG;
    if (c->device < 0) return OKF_E_NODEV;
    (void)hipSetDevice(c->device);
    if (!c->pending.empty()) {
        c->grouping = false;
        int st;
        try {
            st = flush_group(c);
        } catch (const std::bad_alloc &) {
            c->pending.clear();
            st = OKF_E_ARG;
        }
        if (st) return st;
    }
    hipError_t e = hipStreamSynchronize(c->stream);
    return e == hipSuccess ? OKF_OK : hip_fail(c, e);
}

int okf_set_fault_rate(okf_ctx *c, double rate, uint64_t seed) {
    if (!c || !(rate >= 0.0 && rate <= 1.0)) return OKF_E_ARG;
    c->fault_rate = rate;
    c->fault_state = seed;
    return OKF_OK;
}

int okf_last_hip_error(okf_ctx *c) { return c ? c->last_hip : 0; }

int okf_gguf_open(const char *path, okf_gguf **out) {
    if (!path || !out) return OKF_E_ARG;
    *out = nullptr;
    okf_gguf *g = new (std::nothrow) okf_gguf();
    if (!g) return OKF_E_ARG;
    okf_gguf_impl::File &f = g->f;
    f.fd = open(path, O_RDONLY);
    struct stat st;
    if (f.fd < 0 || fstat(f.fd, &st) != 0 || st.st_size <= 0) {
        delete g;
        return OKF_E_IO;
    }
    f.size = (uint64_t)st.st_size;
    void *m = mmap(nullptr, f.size, PROT_READ, MAP_PRIVATE, f.fd, 0);
    if (m == MAP_FAILED) {
        delete g;
        return OKF_E_IO;
    }
    f.map = (const uint8_t *)m;
    int st2;
    try {  // (the directory's strings and maps allocate)
        st2 = okf_gguf_impl::parse(f);
    } catch (const std::bad_alloc &) {
        st2 = OKF_E_FORMAT;
    }
    if (st2) {
        delete g;
        return st2;
    }
    *out = g;
    return OKF_OK;
}

int okf_gguf_close(okf_gguf *g) {
    if (!g) return OKF_E_ARG;
    delete g;
    return OKF_OK;
}

int okf_gguf_tensor_count(const okf_gguf *g, uint64_t *n) {
    if (!g || !n) return OKF_E_ARG;
    *n = g->f.tensors.size();
    return OKF_OK;
}

int okf_gguf_tensor_at(const okf_gguf *g, uint64_t i, okf_gguf_tensor *t) {
    if (!g || !t) return OKF_E_ARG;
    if (i >= g->f.tensors.size()) return OKF_E_NOTFOUND;
    const okf_gguf_impl::Tensor &x = g->f.tensors[i];
    t->name = x.name.c_str();
    t->n_dims = x.n_dims;
    for (int d = 0; d < 4; d++) t->dims[d] = x.dims[d];
    t->ggml_type = x.type;
    t->offset = x.offset;
    t->bytes = x.bytes;
    return OKF_OK;
}

int okf_gguf_find(const okf_gguf *g, const char *name, okf_gguf_tensor *t) {
    if (!g || !name || !t) return OKF_E_ARG;
    auto it = g->f.by_name.find(name);
    if (it == g->f.by_name.end()) return OKF_E_NOTFOUND;
    return okf_gguf_tensor_at(g, it->second, t);
}

int okf_gguf_kv_int(const okf_gguf *g, const char *key, int64_t *v) {
    if (!g || !key || !v) return OKF_E_ARG;
    auto it = g->f.meta.find(key);
    if (it == g->f.meta.end()) return OKF_E_NOTFOUND;
    const auto &x = it->second;
    if (x.kind != okf_gguf_impl::Value::Int && x.kind != okf_gguf_impl::Value::Bool) return OKF_E_NOTFOUND;
    *v = x.i;
    return OKF_OK;
}

int okf_gguf_kv_double(const okf_gguf *g, const char *key, double *v) {
    if (!g || !key || !v) return OKF_E_ARG;
    auto it = g->f.meta.find(key);
    if (it == g->f.meta.end()) return OKF_E_NOTFOUND;
    const auto &x = it->second;
    if (x.kind == okf_gguf_impl::Value::Double) *v = x.d;
    else if (x.kind == okf_gguf_impl::Value::Int) *v = (double)x.i;
    else return OKF_E_NOTFOUND;
    return OKF_OK;
}

int okf_gguf_kv_string(const okf_gguf *g, const char *key, const char **s, uint64_t *len) {
    if (!g || !key || !s || !len) return OKF_E_ARG;
    auto it = g->f.meta.find(key);
    if (it == g->f.meta.end() || it->second.kind != okf_gguf_impl::Value::String) return OKF_E_NOTFOUND;
    *s = it->second.s.c_str();
    *len = it->second.s.size();
    return OKF_OK;
}

int okf_gguf_data(const okf_gguf *g, const void **host, uint64_t *bytes) {
    if (!g || !host || !bytes) return OKF_E_ARG;
    *host = g->f.map + g->f.data_start;
    *bytes = g->f.size - g->f.data_start;
    return OKF_OK;
}

int okf_gguf_upload(okf_ctx *c, const okf_gguf *g, void **device) {
    if (!g || !device) return OKF_E_ARG;
    *device = nullptr;
    int st = begin(c);
    if (st) return st;
    const uint64_t n = g->f.size - g->f.data_start;
    void *d = nullptr;
    hipError_t e = hipMalloc(&d, n ? n : 1);
    if (e == hipSuccess && n) e = hipMemcpy(d, g->f.map + g->f.data_start, n, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        if (d) (void)hipFree(d);
        return hip_fail(c, e);
    }
    *device = d;
    return OKF_OK;
}

int okf_gguf_free_device(okf_ctx *c, void *device) {
    if (!c || !device) return OKF_E_ARG;
    if (c->device < 0) return OKF_E_NODEV;
    (void)hipSetDevice(c->device);
    hipError_t e = hipFree(device);
    return e == hipSuccess ? OKF_OK : hip_fail(c, e);
}

const char *okf_strerror(int s) {
    switch (s) {
    case OKF_OK: return "ok";
    case OKF_E_TYPE: return "unsupported ggml type";
    case OKF_E_SHAPE: return "bad shape or alignment";
    case OKF_E_HIP: return "HIP runtime error";
    case OKF_E_INJECTED: return "injected fault";
    case OKF_E_ARG: return "bad argument";
    case OKF_E_NODEV: return "detached context has no device";
    case OKF_E_IO: return "cannot open or map the file";
    case OKF_E_FORMAT: return "malformed GGUF file";
    case OKF_E_NOTFOUND: return "no such tensor or key";
    default: return "unknown status";
    }
}

}  // extern "C"
