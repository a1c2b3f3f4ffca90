// okf_fmt_q8_0.hip -- the launchers (and with them the kernels) of Q8_0.
#include "okf_impl.h"

namespace okf_impl {
OKF_INSTANTIATE(Q8_0)
}  // namespace okf_impl
