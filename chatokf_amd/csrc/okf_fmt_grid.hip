// okf_fmt_grid.hip -- the launchers (and with them the kernels) of IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S, IQ1_M.
#include "okf_impl.h"

namespace okf_impl {
OKF_INSTANTIATE(IQ2_XS)
OKF_INSTANTIATE(IQ2_S)
OKF_INSTANTIATE(IQ3_XXS)
OKF_INSTANTIATE(IQ3_S)
OKF_INSTANTIATE(IQ1_S)
OKF_INSTANTIATE(IQ1_M)
}  // namespace okf_impl
