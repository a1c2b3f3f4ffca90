// okf_fmt_q2_0.hip -- the launchers (and with them the kernels) of Q2_0.
#include "okf_impl.h"

namespace okf_impl {
OKF_INSTANTIATE(Q2_0)
}  // namespace okf_impl
