// okf_fmt_iq2_xxs.hip -- the launchers (and with them the kernels) of IQ2_XXS.
#include "okf_impl.h"

namespace okf_impl {
OKF_INSTANTIATE(IQ2_XXS)
}  // namespace okf_impl
