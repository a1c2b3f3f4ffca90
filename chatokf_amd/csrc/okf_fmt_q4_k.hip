// okf_fmt_q4_k.hip -- the launchers (and with them the kernels) of Q4_K.
#include "okf_impl.h"

namespace okf_impl {
OKF_INSTANTIATE(Q4_K)
}  // namespace okf_impl
