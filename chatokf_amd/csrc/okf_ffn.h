// okf_ffn.h -- the FFN block of one token (gate, up, SiLU, down) in one
// launch, for the ternary Q2_0 blocks of the Bonsai FFN
// (LLM/Qwen/QwenMetalEngine.swift:918-929: MetalEnc.parallel { gemv(gate);
// gemv(up) }, siluMul, gemv(down)).
//
// The three weight matrices of this FFN are small (3.3 MB each at 6144 x
// 2048), so as separate launches every kernel pays its own start-up: the
// first weight bytes arrive a full HBM latency after the launch, and the
// down projection cannot even request its weights before gate and up are
// done.  Here every lane requests all of its weights of both phases at the
// kernel's start (a few units per lane: the whole FFN fits in the
// registers of a co-resident grid), then
//   phase A: x staged as digit planes; each wavefront takes row pairs (gate
//            row r on lanes 0-31, up row r on lanes 32-63) and writes
//            g[r] = silu(gate x) * (up x), u[r] = up x;
//   a grid-wide barrier (all workgroups are resident: one per CU, a grid
//            the occupancy query allows);
//   phase B: g staged as digit planes; each wavefront takes down rows
//            (units lane, lane + 64, ...) and writes y.
// The arithmetic per unit is the exact digit-plane scheme of okf_gemv.h;
// each row's lanes add their partial sums in a fixed shuffle order, so the
// results are deterministic.
#pragma once
#include "okf_gemv.h"

namespace okf {

// Phase timestamps (a diagnostic build only, compiled with OKF_TRACE): each
// workgroup takes s_memrealtime (a 100 MHz counter common to the device) at
// FF_TRACE_N points and thread 0 writes them at the end into slot
// epoch % FF_TRACE_L of a ring of launches (the barrier's epoch numbers the
// launches), so that a run of back-to-back launches can be read afterwards
// with okf_ffn_trace_read (okf_fmt_q2_0.hip, same build).  Points 3 and 6
// add a workgroup barrier so that they mark the last wavefront.
#ifdef OKF_TRACE
constexpr uint32_t FF_TRACE_N = 8, FF_TRACE_WG = 256, FF_TRACE_L = 64;
static __device__ uint64_t ff_trace[FF_TRACE_L * FF_TRACE_WG * FF_TRACE_N];
#define FF_MARK(k) ftr[k] = __builtin_amdgcn_s_memrealtime()
#define FF_SYNC_MARK(k) \
    do {                \
        __syncthreads(); \
        FF_MARK(k);     \
    } while (0)
#else
#define FF_MARK(k) ((void)0)
#define FF_SYNC_MARK(k) ((void)0)
#endif

constexpr uint32_t FF_SPIN = 1u << 20;  // default barrier polls before giving up (~0.3 s)
// the barrier's words, each on its own 256-byte line (FF_LINE uint32):
// FF_SUB 64-bit arrival counters, FF_SUB 64-bit release flags, the
// time-out flag
constexpr uint32_t FF_SUB = 8, FF_LINE = 64;
constexpr uint32_t FF_FLAG = FF_SUB * FF_LINE, FF_TIMEOUT = 2 * FF_SUB * FF_LINE;
constexpr size_t FF_BAR_BYTES = (FF_TIMEOUT + FF_LINE) * 4;

struct FfnArgs {
    const uint8_t *wg, *wu, *wd;
    uint64_t rba, rbb;    // row bytes of gate / up, of down
    uint32_t ka, ma, mb;  // gate / up K and M (= down K), down M
    const float *x;
    float *g, *u, *y;
    uint32_t *bar;  // FF_BAR_BYTES, zero before the first launch
    uint32_t *status;  // host-visible failure word (pinned host memory): set to 1 by a failed barrier
    uint32_t spin;  // polls before a waiting workgroup gives up
    uint32_t stall;  // 1: the barrier waits for one arrival more than the grid has (time-out tests)
};

// Grid-wide barrier for a grid whose workgroups are all resident.  The
// grid is split into FF_SUB subgroups (workgroup b in b % FF_SUB), each with
// a 64-bit arrival counter and a 64-bit release flag, every word on its own
// 256-byte line.  The counters only ever grow (every launch adds each
// subgroup's size: every launch on them has the same grid), and the flags
// hold the epoch, the number of barriers passed.  A workgroup reads its
// subgroup's flag (the epoch e) and then, once that read is back, adds one
// to its counter without waiting for the result.  Workgroup 0's first
// wavefront polls the counters (lane k counter k) until each reaches
// (e + 1) times its subgroup's size, then sets every flag to e + 1; the
// other workgroups poll their flag.  So the atomics meet no polling on
// their lines, and only one wavefront polls them.
//
// Time-out: the polls are bounded.  A master that gives up writes the
// barrier's time-out word = e + 1 (low 32 bits) and waits for that store's
// acknowledgement before it releases the flags, so the counters and flags
// still agree for the next launch.  Every workgroup reads the time-out word
// after its release, so a barrier the master gave up on fails in every
// workgroup of the launch (the word names the epoch, so later launches are
// not affected); a workgroup whose own poll gave up fails too.  A failed
// workgroup writes NaN to all of its outputs and sets the host-visible
// status word (`status`, pinned host memory) that okf_sync / okf_ffn turn
// into OKF_E_TIMEOUT.  `stall` (a test of that path) makes the master wait
// for one arrival too many.
//
// Memory: the data exchanged across the barrier (g) is written with
// agent-scope stores and read with agent-scope loads (issued with the sc1
// bit, so they miss any stale line in this XCD's L2), and every wave waits
// for its stores to be acknowledged (s_waitcnt vmcnt(0), which
// __syncthreads does not do for global memory) before the workgroup
// arrives.  The counter add and the flag accesses are relaxed atomics: no
// release or acquire fence orders them, because on gfx950 an agent-scope
// release writes back and an acquire invalidates the whole L2 of the XCD
// (device-scope fences here, one per wave, made the kernel take 60 us).
// The ordering rests on the ISA instead: stores are acknowledged in the
// s_waitcnt before the arrival is issued, the flag load that ends a poll
// has returned before any later load is issued (the loop exit depends on
// its value), and the asm waits carry a memory clobber so that the compiler
// moves no memory access across them.
__device__ __forceinline__ bool ff_grid_sync(uint32_t *bar, uint32_t spin, uint32_t stall, uint32_t *status,
                                             uint64_t *epoch_out = nullptr) {
    __shared__ uint64_t epoch;
    __shared__ uint32_t ok;
    uint64_t *cnt = (uint64_t *)bar;             // counter k at cnt[k * FF_LINE / 2]
    uint64_t *flag = (uint64_t *)(bar + FF_FLAG);  // flag k at flag[k * FF_LINE / 2]
    const uint32_t nb = gridDim.x, s = blockIdx.x % FF_SUB;
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");  // this wave's stores of g acknowledged
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint64_t e = __hip_atomic_load(flag + s * (FF_LINE / 2), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        epoch = e;
        ok = 1;
        // the added value depends on e (e < 2^63: it is 1), so the add is
        // issued only once the read is back
        __hip_atomic_fetch_add(cnt + s * (FF_LINE / 2), 1 + (e >> 63), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    const uint64_t e = epoch;
    if (epoch_out) *epoch_out = e;
    if (blockIdx.x == 0 && threadIdx.x < 64) {
        const uint32_t k = threadIdx.x, mk = k < FF_SUB ? (nb - k + FF_SUB - 1) / FF_SUB : 0;
        const uint64_t target = (e + 1) * mk + (k == 0 ? stall : 0);
        bool done = k >= FF_SUB || mk == 0;
        for (uint32_t it = 0;; it++) {
            if (!done)
                done = __hip_atomic_load(cnt + k * (FF_LINE / 2), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >=
                       target;
            if (__all(done)) break;
            if (it == spin) {
                if (k == 0) ok = 0;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (__any(k == 0 && !ok)) {
            // the time-out word names this epoch; acknowledged before the release
            if (k == 0)
                __hip_atomic_store(bar + FF_TIMEOUT, (uint32_t)(e + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        if (k < FF_SUB)
            __hip_atomic_store(flag + k * (FF_LINE / 2), e + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else if (threadIdx.x == 0) {
        for (uint32_t it = 0;
             __hip_atomic_load(flag + s * (FF_LINE / 2), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == e; it++) {
            if (it == spin) {
                ok = 0;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        // released: did the master give up on this epoch?
        asm volatile("" ::: "memory");
        if (ok && __hip_atomic_load(bar + FF_TIMEOUT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(e + 1))
            ok = 0;
    }
    if (threadIdx.x == 0 && !ok) __hip_atomic_store(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __syncthreads();
    return ok != 0;
}

// a device-scope store of one float (see ff_grid_sync)
__device__ __forceinline__ void ff_put(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Staging of n values v (n / UW units) as digit planes and group data for
// Compute<F, 1, 1>, in the layout of xs_index<F, GV_L>, in rounds of one
// 8-value slot per thread.  Every thread of the workgroup takes part (a quad
// of lanes shares each 32-value group; nslots and the round bases are
// multiples of 4, so quads are whole).  ff_load_x / ff_stage_x split it so
// that the loads can go first: loads complete in issue order, so the
// staging must not sit behind the weight loads.
template <int F, int T, int XR>
__device__ __forceinline__ void ff_load_x(const float *v, uint32_t n, float (&s)[XR][1][8]) {
    constexpr uint32_t SL = unit_weights<F>() / 8;
    const uint32_t nslots = n / unit_weights<F>() * SL;
#pragma unroll
    for (int k = 0; k < XR; k++) {
        const uint32_t q = min(k * T + threadIdx.x, nslots - 1), uu = q / SL;
        load_slot<F>(v + unit_x_base<F>(uu), q % SL, s[k][0]);
    }
}
template <int F, int T, int XR>
__device__ __forceinline__ void ff_stage_x(const float (&s)[XR][1][8], uint32_t n, uint32_t *xs, floatx4 *&gdp) {
    constexpr int L = GV_L;
    constexpr uint32_t UW = unit_weights<F>(), SL = UW / 8, UG = unit_groups<F>();
    const uint32_t units = n / UW, cu = (units + L - 1) / L * L, cs = cu * unit_chunks<F>() * 4;
    gdp = (floatx4 *)(xs + cs);
    const uint32_t nslots = units * SL;
#pragma unroll
    for (int k = 0; k < XR; k++) {
        const uint32_t q0 = k * T + threadIdx.x, q = min(q0, nslots - 1);
        if (k * T < nslots)  // (the whole workgroup)
            stage_slot<F, 1, L, false>(s[k], q / SL, q % SL, q0 < nslots, xs, cs, gdp, cu * UG);
    }
}
// g (written by other workgroups behind the grid barrier) staged the same
// way, read with device-scope loads, 8 bytes each, all issued before the
// staging: the 8 values of a slot are those load_slot<Q2_0> reads,
// x[16 j + 4 b + k0] and x[16 j + 4 b + k0 + 1] (b < 4).
template <int F, int T, int XR>
__device__ __forceinline__ void ff_stage_g(const float *v, uint32_t n, uint32_t *xs, floatx4 *&gdp) {
    static_assert(F == Q2_0, "the slot order of load_slot<Q2_0>");
    constexpr uint32_t SL = unit_weights<F>() / 8;
    const uint32_t nslots = n / unit_weights<F>() * SL;
    float s[XR][1][8];
#pragma unroll
    for (int k = 0; k < XR; k++) {
        const uint32_t q = min(k * T + threadIdx.x, nslots - 1), uu = q / SL;
        const uint64_t *xu = (const uint64_t *)(v + unit_x_base<F>(uu) + 16 * ((q % SL) >> 1) + 2 * (q & 1));
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const float2 t = __builtin_bit_cast(
                float2, __hip_atomic_load(xu + 2 * b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
            s[k][0][b] = t.x;
            s[k][0][4 + b] = t.y;
        }
    }
    ff_stage_x<F, T, XR>(s, n, xs, gdp);
}

template <int F>
__device__ __forceinline__ uint32_t ff_cs(uint32_t n) {
    const uint32_t units = n / unit_weights<F>(), cu = (units + GV_L - 1) / GV_L * GV_L;
    return cu * unit_chunks<F>() * 4;
}

// T threads a workgroup; UA: units per lane of a gate / up row (32 lanes a
// row), UB: of a down row (64 lanes a row).  Wavefront w takes row pairs
// w + p W (p < RA) and down rows w + p W (p < RB), W = the grid's
// wavefronts (host-checked).
template <int F, int T, int UA, int UB, int RA, int RB>
__global__ __launch_bounds__(T) void ffn_fused_kernel(FfnArgs a) {
    constexpr uint32_t FF_WAVES = T / 64;
    constexpr int L = GV_L;
    constexpr uint32_t UW = unit_weights<F>(), UG = unit_groups<F>();
    extern __shared__ u32x4 lds[];
    uint32_t *xs = (uint32_t *)lds;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t W = gridDim.x * FF_WAVES, w0 = blockIdx.x * FF_WAVES + (tid >> 6);
    const uint32_t una = a.ka / UW, unb = a.ma / UW;
    const uint32_t half = lane >> 5, lh = lane & 31;
#ifdef OKF_TRACE
    uint64_t ftr[FF_TRACE_N] = {}, fep = 0;
#endif
    FF_MARK(0);  // start

    // x's loads, then every weight load of both phases; x of gate / up is at
    // most UA * 32 units, UA rounds of slots.  The loads are unconditional
    // (rows past the end re-read the last row): loads under a branch make
    // the compiler wait for all of them before the staging.
    constexpr int XR = (UA * 32 * unit_weights<F>() / 8 + T - 1) / T;
    float xv[XR][1][8];
    ff_load_x<F, T, XR>(a.x, a.ka, xv);
    __builtin_amdgcn_sched_barrier(0);
    // (a lane's RA gate / up rows in one Unit: their units meet the same
    // activations, read from LDS once for all of them)
    Unit<F, RA> wa[UA];
    Unit<F, 1> wb[RB][UB];
    {
        const uint8_t *rows[RA];
#pragma unroll
        for (int p = 0; p < RA; p++) rows[p] = (half ? a.wu : a.wg) + (uint64_t)min(w0 + p * W, a.ma - 1) * a.rba;
#pragma unroll
        for (int j = 0; j < UA; j++) load_unit<F, RA>(rows, min(lh + 32 * j, una - 1), wa[j]);
    }
#pragma unroll
    for (int p = 0; p < RB; p++) {
        const uint32_t r = min(w0 + p * W, a.mb - 1);
        const uint8_t *rows[1] = {a.wd + (uint64_t)r * a.rbb};
#pragma unroll
        for (int j = 0; j < UB; j++) load_unit<F, 1>(rows, min(lane + 64 * j, unb - 1), wb[p][j]);
    }
    __builtin_amdgcn_sched_barrier(0);
    FF_MARK(1);  // every load issued (wavefront 0)

    // phase A: gate and up
    floatx4 *gdp;
    ff_stage_x<F, T, XR>(xv, a.ka, xs, gdp);
    __syncthreads();
    FF_MARK(2);  // x in, staged
    {
        const uint32_t cs = ff_cs<F>(a.ka), gcs = cs / (unit_chunks<F>() * 4) * UG;
        float acc[RA][1] = {};
#pragma unroll
        for (int j = 0; j < UA; j++) {
            const uint32_t uu = lh + 32 * j;
            if (uu < una)
                Compute<F, 1, RA>::run(wa[j], XLds{xs + xs_index<F, L>(uu, 0), 4 * L, cs, gdp + uu * UG, gcs}, uu,
                                       acc, nullptr);
        }
#pragma unroll
        for (int p = 0; p < RA; p++) {
            const uint32_t r = w0 + p * W;
            if (r < a.ma) {  // (the whole wavefront)
                float v = acc[p][0];
#pragma unroll
                for (int m = 16; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
                const float up = __shfl(v, 32, 64);
                if (lane == 0) {
                    ff_put(a.g + r, silu_mul1(v, up));
                    a.u[r] = up;
                }
            }
        }
    }
    FF_SYNC_MARK(3);  // phase A done
#ifdef OKF_TRACE
    const bool synced = ff_grid_sync(a.bar, a.spin, a.stall, a.status, &fep);
#else
    const bool synced = ff_grid_sync(a.bar, a.spin, a.stall, a.status);
#endif
    FF_MARK(4);  // released

    // phase B: down on g (staged after the barrier, so every row of it is in)
    constexpr int XB = (UB * 64 * unit_weights<F>() / 8 + T - 1) / T;
    ff_stage_g<F, T, XB>(a.g, a.ma, xs, gdp);
    __syncthreads();
    FF_MARK(5);  // g in, staged
    {
        const uint32_t cs = ff_cs<F>(a.ma), gcs = cs / (unit_chunks<F>() * 4) * UG;
#pragma unroll
        for (int p = 0; p < RB; p++) {
            const uint32_t r = w0 + p * W;
            if (r < a.mb) {
                float acc[1][1] = {{0.0f}};
#pragma unroll
                for (int j = 0; j < UB; j++) {
                    const uint32_t uu = lane + 64 * j;
                    if (uu < unb)
                        Compute<F, 1, 1>::run(wb[p][j], XLds{xs + xs_index<F, L>(uu, 0), 4 * L, cs, gdp + uu * UG, gcs},
                                              uu, acc, nullptr);
                }
                float v = acc[0][0];
#pragma unroll
                for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
                // a failed barrier (this workgroup's poll or the master's
                // gave up) leaves NaN in every row of the workgroup
                if (lane == 0) a.y[r] = synced ? v : __builtin_nanf("");
            }
        }
    }
    FF_SYNC_MARK(6);  // phase B done
#ifdef OKF_TRACE
    if (threadIdx.x == 0 && blockIdx.x < FF_TRACE_WG) {
        uint64_t *o = ff_trace + ((fep % FF_TRACE_L) * FF_TRACE_WG + blockIdx.x) * FF_TRACE_N;
        ftr[7] = fep;
#pragma unroll
        for (uint32_t k = 0; k < FF_TRACE_N; k++) o[k] = ftr[k];
    }
#endif
}

}  // namespace okf
