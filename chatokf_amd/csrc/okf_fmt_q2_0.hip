// okf_fmt_q2_0.hip -- the launchers (and with them the kernels) of Q2_0.
#include "okf_impl.h"
#include "okf_ffn_mfma.h"

namespace okf_impl {
OKF_INSTANTIATE(Q2_0)

// ffn_fused_kernel on one workgroup per CU (okf_ctx::ffn_wg, the same for
// every launch of a context), all resident (the occupancy query must allow
// it; the barrier's polls are bounded all the same): the exact fits of the
// Bonsai FFN (gate / up 6144 x 2048, down 2048 x 6144 on 256 CUs; with 512
// threads a workgroup 3 row pairs and 1 down row per wavefront, with 256
// threads 6 and 2; no load re-reads a row), or the general instance for
// gate / up rows of up to 64 units (K <= 4096), down rows of up to 128
// (gate M <= 8192), and up to 4 row pairs and 2 down rows per wavefront.
bool launch_ffn_fused(okf_ctx *c, const FfnArgs &a0) {
    constexpr uint32_t UW = unit_weights<Q2_0>();
    if (!c->ffn_fused || !c->ffn_bar || !c->ffn_status || a0.ka % UW || a0.ma % UW) return false;
    const uint32_t una = a0.ka / UW, unb = a0.ma / UW;
    if (una > 64 || unb > 128) return false;
    auto stage_bytes = [](uint32_t units) {
        const size_t cu = (units + GV_L - 1) / GV_L * GV_L;
        return cu * unit_lds_bytes<Q2_0>();
    };
    const size_t lds = std::max(stage_bytes(una), stage_bytes(unb));
    if (lds > c->max_lds) return false;
    // the Bonsai shape on the integer matrix cores (okf_ffn_mfma.h): gate /
    // up 6144 x 2048, down 2048 x 6144, at most 24 gate / up rows and 16
    // down rows a workgroup
    if (c->ffn_mfma && a0.ka == 2048 && a0.ma == 6144 && c->cus) {
        const void *fn = (const void *)ffn_mfma_kernel<2, 6>;
        const size_t lb = fm_lds_bytes(6144);
        int &nb = c->ffn_nb[3];
        if (nb == 0) {
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, fn, (int)FM_T, lb) != hipSuccess || nb < 1) {
                (void)hipGetLastError();
                nb = -1;
            }
        }
        const int wg = std::max(c->ffn_wg, 1);
        const uint32_t G = (uint32_t)wg * c->cus;
        if (nb >= wg && lb <= c->max_lds && (a0.ma + G - 1) / G <= FM_RA && (a0.mb + G - 1) / G <= FM_RB) {
            FfnArgs a = a0;
            a.bar = c->ffn_bar;
            a.status = c->ffn_status;
            a.spin = c->ffn_spin > 0 ? (uint32_t)c->ffn_spin : FF_SPIN;
            a.stall = c->ffn_stall > 0 ? 1u : 0u;
            void *args[] = {&a};
            const hipError_t e =
                c->ffn_coop ? hipLaunchCooperativeKernel(fn, dim3(G), dim3(FM_T), args, (unsigned)lb, c->stream)
                            : hipLaunchKernel(fn, dim3(G), dim3(FM_T), args, lb, c->stream);
            if (e != hipSuccess) {
                (void)hipGetLastError();
                return false;
            }
            if (c->ffn_stall > 0) c->ffn_stall--;
            return true;
        }
    }
    struct Var {
        const void *fn;
        uint32_t threads, ra, rb;  // ra = rb = 0: the general instance
    };
    const Var vars[3] = {{(const void *)ffn_fused_kernel<Q2_0, 512, 1, 2, 3, 1>, 512, 3, 1},
                         {(const void *)ffn_fused_kernel<Q2_0, 256, 1, 2, 6, 2>, 256, 6, 2},
                         {(const void *)ffn_fused_kernel<Q2_0, 512, 2, 2, 4, 2>, 512, 0, 0}};
    for (int v = 0; v < 3; v++) {
        const Var &k = vars[v];
        if (v < 2 && (c->ffn_t ? (uint32_t)c->ffn_t != k.threads : v != 0)) continue;
        // resident workgroups per CU, queried once per context and kernel (at
        // the largest LDS any call uses: FF stages at most 128 units)
        int &nb = c->ffn_nb[v];
        if (nb == 0) {
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k.fn, (int)k.threads, stage_bytes(128)) !=
                    hipSuccess ||
                nb < 1) {
                (void)hipGetLastError();
                nb = -1;
            }
        }
        // every launch on the context's barrier counters has the same grid
        // (ff_grid_sync derives its epoch from it): ffn_wg workgroups a CU
        const int wg = std::max(c->ffn_wg, 1);
        if (nb < wg) return false;
        const uint32_t G = (uint32_t)wg * c->cus, W = G * (k.threads / 64);
        const uint32_t ra = (a0.ma + W - 1) / W, rb = (a0.mb + W - 1) / W;
        if (k.ra ? (una > 32 || unb <= 64 || ra != k.ra || rb != k.rb) : (ra > 4 || rb > 2)) continue;
        FfnArgs a = a0;
        a.bar = c->ffn_bar;
        a.status = c->ffn_status;
        a.spin = c->ffn_spin > 0 ? (uint32_t)c->ffn_spin : FF_SPIN;
        a.stall = c->ffn_stall > 0 ? 1u : 0u;
        void *args[] = {&a};
        const hipError_t e =
            c->ffn_coop ? hipLaunchCooperativeKernel(k.fn, dim3(G), dim3(k.threads), args, (unsigned)lds, c->stream)
                        : hipLaunchKernel(k.fn, dim3(G), dim3(k.threads), args, lds, c->stream);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            return false;
        }
        if (c->ffn_stall > 0) c->ffn_stall--;
        return true;
    }
    return false;
}
}  // namespace okf_impl

#ifdef OKF_TRACE
// the phase timestamps of the last FF_TRACE_L ffn_fused_kernel launches
// (okf_ffn.h): n values, [slot][workgroup][point], point 7 the epoch
extern "C" int okf_ffn_trace_read(uint64_t *host, uint32_t n) {
    if (n > okf::FF_TRACE_L * okf::FF_TRACE_WG * okf::FF_TRACE_N) return OKF_E_SHAPE;
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(okf::ff_trace), (size_t)n * sizeof(uint64_t), 0,
                               hipMemcpyDeviceToHost) == hipSuccess ? OKF_OK : OKF_E_HIP;
}
#endif
