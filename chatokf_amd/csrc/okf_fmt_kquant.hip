// okf_fmt_kquant.hip -- the launchers (and with them the kernels) of Q5_K, Q6_K, Q2_K, Q3_K.
#include "okf_impl.h"

namespace okf_impl {
OKF_INSTANTIATE(Q5_K)
OKF_INSTANTIATE(Q6_K)
OKF_INSTANTIATE(Q2_K)
OKF_INSTANTIATE(Q3_K)
}  // namespace okf_impl
