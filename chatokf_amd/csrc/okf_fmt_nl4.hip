// okf_fmt_nl4.hip -- the launchers (and with them the kernels) of Q4_0, IQ4_NL, IQ4_XS.
#include "okf_impl.h"

namespace okf_impl {
OKF_INSTANTIATE(Q4_0)
OKF_INSTANTIATE(IQ4_NL)
OKF_INSTANTIATE(IQ4_XS)
}  // namespace okf_impl
