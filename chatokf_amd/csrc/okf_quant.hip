// okf_quant.hip -- the C ABI (include/okf_quant.h) over the gfx950 kernels.
//
// Host-side dispatch mirrors the reference's MetalEnc (LLM/Base/MetalEnc.swift):
// gemv picks the per-format kernel (:84-153), gemm applies the
// N == 1 / 2..5 / > 5 policy (:241-289), dequantRow unpacks one row (:402-459).
// Validation failures return a status instead of the reference's
// fatalError / precondition.
#include "okf_impl.h"
#include "okf_gguf.h"
#include "okf_norm.h"

#include "iq2xxs_grid.inc"
#include "iq_grids.inc"

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

namespace okf_impl {
OKF_FOR_EACH_FORMAT(OKF_EXTERN)
}

namespace {

using namespace okf;
using namespace okf_impl;

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
    // grid entry e: per weight the index of its value in {8, 25, 43} (the
    // grid's only bytes), 8 bytes; the dot4 kernels add 4 for a negative
    // weight and pick the signed byte with one v_perm
    for (int e = 0; e < 256; e++) {
        const uint64_t g = okf_iq2xxs_grid_host[e];
        uint64_t ix = 0;
        for (int j = 0; j < 8; j++) {
            const uint32_t v = (uint32_t)((g >> (8 * j)) & 0xFF);
            ix |= (uint64_t)(v == 8 ? 0 : v == 25 ? 1 : 2) << (8 * j);
        }
        t[e * 4 + 0] = (uint32_t)ix;
        t[e * 4 + 1] = (uint32_t)(ix >> 32);
        t[e * 4 + 2] = t[e * 4 + 3] = 0;
    }
    // sign entry s7: v_perm selectors, byte j of weight dword k is j (the
    // positive value) or j + 4 (the negated one) for the eighth sign from the
    // parity rule (ksigns, LLM/Quantize/IQ2Grid.swift:73)
    for (int s7 = 0; s7 < 128; s7++) {
        const uint32_t s = s7 | ((__builtin_popcount(s7) & 1u) << 7);
        uint32_t m[2] = {0, 0};
        for (int j = 0; j < 8; j++) m[j >> 2] |= (uint32_t)((j & 3) + 4 * ((s >> j) & 1)) << (8 * (j & 3));
        t[(256 + s7) * 4 + 0] = m[0];
        t[(256 + s7) * 4 + 1] = m[1];
        t[(256 + s7) * 4 + 2] = t[(256 + s7) * 4 + 3] = 0;
    }
}

// IQ3_XXS's tables for its integer matvec, 8-byte entries: [0, 256) grid
// entry e's 4 bytes (LLM/Quantize/IQ3Grid.swift), then their negations;
// [256, 384) the first 8 bytes of IQ2_XXS's sign selector rows (sel8, 16
// bytes a row): a 7-bit sign index gives the same 8 signs.
void build_iq3_xxs_tables8(uint32_t *t, const uint32_t *sel8) {
    for (int e = 0; e < 256; e++) {
        const uint32_t g = okf_host_iq3xxs_grid[e];
        uint32_t ng = 0;
        for (int j = 0; j < 4; j++) ng |= (uint32_t)(uint8_t)(-(int)((g >> (8 * j)) & 0xFF)) << (8 * j);
        t[2 * e] = g;
        t[2 * e + 1] = ng;
    }
    for (int s7 = 0; s7 < 128; s7++) {
        t[2 * (256 + s7)] = sel8[4 * s7];
        t[2 * (256 + s7) + 1] = sel8[4 * s7 + 1];
    }
}

// v_perm selectors of an 8-bit sign byte (bit j negates weight j): byte j of
// dword j / 4 is j % 4 or j % 4 + 4
static void sign_byte_selectors(uint32_t s, uint32_t *m) {
    m[0] = m[1] = 0;
    for (int j = 0; j < 8; j++) m[j >> 2] |= (uint32_t)((j & 3) + 4 * ((s >> j) & 1)) << (8 * (j & 3));
}

// IQ3_S's tables, 8-byte entries: [0, 512) grid entry e's 4 bytes
// (LLM/Quantize/IQ3Grid.swift), then their negations; [512, 768) the
// selectors of a sign byte.
void build_iq3_s_tables8(uint32_t *t) {
    for (int e = 0; e < 512; e++) {
        const uint32_t g = okf_host_iq3s_grid[e];
        uint32_t ng = 0;
        for (int j = 0; j < 4; j++) ng |= (uint32_t)(uint8_t)(-(int)((g >> (8 * j)) & 0xFF)) << (8 * j);
        t[2 * e] = g;
        t[2 * e + 1] = ng;
    }
    for (int s = 0; s < 256; s++) sign_byte_selectors((uint32_t)s, t + 2 * (512 + s));
}

// IQ2_XS's / IQ2_S's tables, 8-byte entries: [0, n) grid entry e as the
// indices 0..2 of its 8 values in {8, 25, 43} (as IQ2_XXS's); then the
// selectors (byte j = j % 4 + 4 for a negative weight): of a 7-bit sign
// index (the first 8 bytes of IQ2_XXS's selector rows, sel7, 16 bytes a
// row) or, with sel7 null, of a sign byte.
void build_iq2_xs_s_tables8(uint32_t *t, const uint64_t *grid, int n, const uint32_t *sel7) {
    for (int e = 0; e < n; e++) {
        const uint64_t g = grid[e];
        uint64_t ix = 0;
        for (int j = 0; j < 8; j++) {
            const uint32_t v = (uint32_t)((g >> (8 * j)) & 0xFF);
            ix |= (uint64_t)(v == 8 ? 0 : v == 25 ? 1 : 2) << (8 * j);
        }
        t[e * 2] = (uint32_t)ix;
        t[e * 2 + 1] = (uint32_t)(ix >> 32);
    }
    uint32_t *s2 = t + n * 2;
    if (sel7)
        for (int s = 0; s < 128; s++) {
            s2[2 * s] = sel7[4 * s];
            s2[2 * s + 1] = sel7[4 * s + 1];
        }
    else
        for (int s = 0; s < 256; s++) sign_byte_selectors((uint32_t)s, s2 + 2 * s);
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

// N > 5 as consecutive narrow launches of up to narrow_cols columns, while N
// <= narrow_max, where that is faster than the tile kernels.  Measured on
// MI355X against the tile kernels with their K split (us, N = 6 / 8 / 12 /
// 16): 2048 x 2048 Q8_0 chunks 11.3 / 12.4 / 18.2 / 24.6, tile 11.5 / 11.4 /
// 11.6 / 11.6; Q6_K 11.1 / 12.5 against 12.3 / 12.6; IQ4_XS 11.2 / 12.0 /
// 18.2 against 14.0 / 14.1 / 14.4; Q4_0, Q4_K, IQ2_XXS, IQ3_XXS, Q2_K and
// Q2_0 (2048 x 6144) tile from N = 6.  17408 x 5120: IQ2_XXS 35.4 / 36.8 /
// 54.8 / 72.5 against 56.7 / 56.5 / 56.8 / 57.3, IQ3_XXS 40.5 / 43.2 / 64.9
// / 84.1 against 75.2-76.9, Q3_K 69.2 / 68.6 / 101.6 against 80.2-80.7,
// Q4_0 48.3 / 57.1 against 57.2 / 57.4, Q8_0 84.7 against 66.2, Q4_K 36.1
// / 36.9 / 57.1 / 80.7 against 78.8 / 81.1 / 86.6 / 91.7.
// The formats whose 2..4-column matrix-core kernel runs (K <= 6144, M >=
// 4096), Q8_0 aside: 4-column chunks, each about as long as one column
// (17408 x 5120: Q4_K 19.8, Q5_K 22.8, IQ4_XS 21.9 us against 56.9, 67.0
// and 61.7 us for 5 columns at once; the grid formats 17.4-21.4 against
// 48-53 for 4 columns on the dot4 kernel, Q2_K 17.9 / 43.2, Q3_K 32.0 /
// 53.5).
bool mm_fits(int32_t t, uint32_t M, uint32_t K) {
    return mm_bit(t) >= 0 && t != Q8_0 && K <= 6144 && K % 64 == 0 && M >= 4096;
}
uint32_t narrow_cols(int32_t t, uint32_t M, uint32_t K) {
    return t == IQ2_XXS || t == Q4_0 || t == IQ4_NL || mm_fits(t, M, K) ? 4 : 5;
}
// the first N taken in chunks: 5 where a 4-column kernel is much faster
// than the 5-column one (IQ2_XXS 19.4 + 16.3 against 52.6 us, Q4_K 19.8 +
// 14.2 against 56.9)
uint32_t narrow_from(int32_t t, uint32_t M, uint32_t K) { return t == IQ2_XXS || mm_fits(t, M, K) ? 5 : 6; }
uint32_t narrow_max(int32_t t, uint32_t M, uint32_t K) {
    if (M < 4096) {  // (a small grid: the K-split tile fills the GPU)
        switch (t) {
        case Q8_0: case Q5_K: return 6;
        case Q6_K: case IQ4_XS: return 8;
        default: return 5;
        }
    }
    if (mm_fits(t, M, K)) return t == Q4_K ? 16 : t == Q3_K ? 8 : 12;
    switch (t) {
    case Q4_K: return 7;
    case IQ2_XXS: return 12;
    case Q4_0: case IQ4_NL: return 8;
    case Q8_0: case Q6_K: case Q2_0: case F32: case F16: case BF16: return 5;
    default: return 12;  // the other grid formats and K-quants with K > 6144
    }
}

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
    const uint32_t nmax = narrow_max(w->ggml_type, w->M, w->K);
    if (path == Path::Auto && N >= narrow_from(w->ggml_type, w->M, w->K) && N <= nmax && !X2) {
        const uint32_t nc = narrow_cols(w->ggml_type, w->M, w->K);
        for (uint32_t c0 = 0; c0 < N; c0 += nc) {
            const GemvCall call{W, X + (uint64_t)c0 * w->K, Y + (uint64_t)c0 * w->M, w->M, nullptr};
            OKF_DISPATCH(w->ggml_type, launch_gemv, c, &call, 1, rb, w->K, std::min(nc, N - c0));
        }
    } else if (path == Path::Auto && N <= 5) {
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
        std::vector<uint32_t> tab8v(ITAB_ROWS * 4);
        uint32_t *tab8h = tab8v.data();
        build_iq2_tables8(tab8h);
        build_iq3_xxs_tables8(tab8h + itab_at(IQ3_XXS) * 4, tab8h + 256 * 4);
        build_iq3_s_tables8(tab8h + itab_at(IQ3_S) * 4);
        build_iq2_xs_s_tables8(tab8h + itab_at(IQ2_XS) * 4, okf_host_iq2xs_grid, 512, tab8h + 256 * 4);
        build_iq2_xs_s_tables8(tab8h + itab_at(IQ2_S) * 4, okf_host_iq2s_grid, 1024, nullptr);
        if (e == hipSuccess) e = hipMalloc((void **)&c->tab8, tab8v.size() * 4);
        if (e == hipSuccess) e = hipMemcpy(c->tab8, tab8h, tab8v.size() * 4, hipMemcpyHostToDevice);
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
        if (e == hipSuccess) e = hipMalloc((void **)&c->ffn_bar, FF_BAR_BYTES);
        if (e == hipSuccess) e = hipMemset(c->ffn_bar, 0, FF_BAR_BYTES);
        if (e == hipSuccess) e = hipHostMalloc((void **)&c->ffn_status, sizeof(uint32_t), hipHostMallocMapped);
        if (e == hipSuccess) *(volatile uint32_t *)c->ffn_status = 0;
        if (e != hipSuccess) {
            if (c->ffn_status) (void)hipHostFree(c->ffn_status);
            if (c->ffn_bar) (void)hipFree(c->ffn_bar);
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
        if (const char *e = getenv("OKF_GEMV_SB")) c->gemv_sb = atoi(e);
        if (const char *e = getenv("OKF_GEMV_SB_RW")) c->gemv_sb_rw = atoi(e);
        if (const char *e = getenv("OKF_GEMV_SB_T")) c->gemv_sb_t = atoi(e);
        if (const char *e = getenv("OKF_GEMV_SB_R")) c->gemv_sb_r = atoi(e);
        if (const char *e = getenv("OKF_GEMM_KS")) c->gemm_ks = atoi(e);
        if (const char *e = getenv("OKF_GEMM_NG")) c->gemm_ng = atoi(e);
        if (const char *e = getenv("OKF_GEMM_THIN")) c->gemm_thin = atoi(e);
        if (const char *e = getenv("OKF_GEMM_SPLIT")) c->gemm_split = atoi(e);
        if (const char *e = getenv("OKF_GEMM_XH")) c->gemm_xh = atoi(e);
        if (const char *e = getenv("OKF_Q4K_MM")) c->q4k_mm = atoi(e);
        if (const char *e = getenv("OKF_FFN_FUSED")) c->ffn_fused = atoi(e);
        if (const char *e = getenv("OKF_FFN_MFMA")) c->ffn_mfma = atoi(e);
        if (const char *e = getenv("OKF_Q2_MFMA")) c->q2_mfma = atoi(e);
        if (const char *e = getenv("OKF_Q2_KS")) c->q2_ks = atoi(e);
        if (const char *e = getenv("OKF_FFN_WG")) c->ffn_wg = atoi(e);
        if (const char *e = getenv("OKF_FFN_COOP")) c->ffn_coop = atoi(e);
        if (const char *e = getenv("OKF_FFN_T")) c->ffn_t = atoi(e);
        if (const char *e = getenv("OKF_FFN_SPIN")) c->ffn_spin = atoi(e);
        if (const char *e = getenv("OKF_FFN_STALL")) c->ffn_stall = atoi(e);
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
        if (c->ffn_bar) (void)hipFree(c->ffn_bar);
        if (c->ffn_status) (void)hipHostFree(c->ffn_status);
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

// The FFN of the reference's engines (QwenMetalEngine.swift:918-929): gate
// and up on x as one launch group where their format and K match, then
// down on silu(gate) * up with the SiLU folded into its activation staging.
int okf_gemv_gate_up(okf_ctx *c, const okf_weight *gate, const okf_weight *up, const float *x, float *g,
                     float *u) {
    uint64_t rb0 = 0, rb0u = 0;
    int st = check_weight(gate, &rb0);
    if (!st) st = check_weight(up, &rb0u);
    if (st) return st;
    if (!x || !g || !u) return OKF_E_ARG;
    if (gate->K != up->K || gate->M != up->M) return OKF_E_SHAPE;
    if (!aligned16(x) || !aligned16(g) || !aligned16(u)) return OKF_E_SHAPE;
    if (c && c->grouping) return OKF_E_ARG;
    if ((st = begin(c))) return st;
    const GemvCall gu[2] = {{(const uint8_t *)gate->base + gate->off, x, g, gate->M},
                            {(const uint8_t *)up->base + up->off, x, u, up->M}};
    if (gate->ggml_type == up->ggml_type) {
        // one grid, each workgroup the same rows of gate and up: g <- silu(g) * u
        OKF_DISPATCH(gate->ggml_type, launch_gemv_pair, c, gu, rb0, gate->K);
    } else {
        OKF_DISPATCH(gate->ggml_type, launch_gemv, c, &gu[0], 1, rb0, gate->K, 1u);
        OKF_DISPATCH(up->ggml_type, launch_gemv, c, &gu[1], 1, rb0u, up->K, 1u);
        hipLaunchKernelGGL(silu_mul_kernel, dim3((gate->M + 255) / 256), dim3(256), 0, c->stream, g, u, gate->M);
    }
    return finish(c);
}

int okf_ffn(okf_ctx *c, const okf_weight *gate, const okf_weight *up, const okf_weight *down, const float *x,
            float *g, float *u, float *y) {
    uint64_t rb1 = 0;
    int st = check_weight(down, &rb1);
    if (st) return st;
    if (!gate || !y) return OKF_E_ARG;
    if (down->K != gate->M) return OKF_E_SHAPE;
    if (gate->ggml_type == Q2_0 && up && up->ggml_type == Q2_0 && down->ggml_type == Q2_0 && c && !c->grouping) {
        // the ternary FFN in one launch where it fits
        uint64_t rb0 = 0, rb0u = 0;
        if ((st = check_weight(gate, &rb0)) || (st = check_weight(up, &rb0u))) return st;
        if (!x || !g || !u) return OKF_E_ARG;
        if (gate->K != up->K || gate->M != up->M) return OKF_E_SHAPE;
        if (!aligned16(x) || !aligned16(g) || !aligned16(u)) return OKF_E_SHAPE;
        if ((st = begin(c))) return st;
        // an earlier launch's barrier that gave up is this call's failure (nothing is launched)
        if ((st = take_timeout(c))) return st;
        const FfnArgs a{(const uint8_t *)gate->base + gate->off, (const uint8_t *)up->base + up->off,
                        (const uint8_t *)down->base + down->off, rb0, rb1, gate->K, gate->M, down->M,
                        x, g, u, y, nullptr};
        // (at the Bonsai shape the two matrix-core launches are the faster form)
        if ((c->ffn_fused == 2 || !q2m_ffn_fits(c, gate->K, gate->M, down->M)) && launch_ffn_fused(c, a))
            return finish(c);
    }
    if ((st = okf_gemv_gate_up(c, gate, up, x, g, u))) return st;
    const GemvCall dn{(const uint8_t *)down->base + down->off, g, y, down->M};
    OKF_DISPATCH(down->ggml_type, launch_gemv, c, &dn, 1, rb1, down->K, 1u);
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
    // the documented limit counts 1024-value chunks (the kernel's chunks are
    // larger, so it uses at most that many pairs)
    static_assert(ARGMAX_CHUNK % 1024 == 0, "argmax chunks are whole 1024-value pieces");
    if ((uint64_t)((n + 1023) / 1024) * rows > OKF_NOALLOC_ARGMAX_PAIRS) return OKF_E_SHAPE;
    const uint32_t chunks = (n + ARGMAX_CHUNK - 1) / ARGMAX_CHUNK;
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

int okf_stream_read(okf_ctx *c, const void *p, uint64_t bytes, uint32_t *out) {
    if (!p || !out) return OKF_E_ARG;
    if (bytes == 0 || bytes % 16 || !aligned16(p)) return OKF_E_SHAPE;
    int st = begin(c);
    if (st) return st;
    const uint64_t n16 = bytes / 16;
    // one workgroup per 48 KB, between one and four per CU (measured best
    // on MI355X for 3 MB and 50 MB reads)
    const uint32_t wgs = (uint32_t)std::min<uint64_t>(4 * c->cus, std::max<uint64_t>(c->cus, bytes / (48 << 10)));
    const uint64_t per = (n16 + wgs - 1) / wgs;
    hipLaunchKernelGGL(stream_read_kernel, dim3(wgs), dim3(SR_THREADS), 0, c->stream, (const u32x4 *)p, n16, per,
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
    if (e != hipSuccess) return hip_fail(c, e);
    return take_timeout(c);
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
    case OKF_E_TIMEOUT: return "grid barrier timed out (outputs are NaN)";
    default: return "unknown status";
    }
}

}  // extern "C"
