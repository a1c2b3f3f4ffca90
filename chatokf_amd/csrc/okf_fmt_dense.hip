// okf_fmt_dense.hip -- the launchers (and with them the kernels) of F32, F16, BF16.
#include "okf_impl.h"

namespace okf_impl {
OKF_INSTANTIATE(F32)
OKF_INSTANTIATE(F16)
OKF_INSTANTIATE(BF16)
}  // namespace okf_impl
