// qmm mode DENSE: one instantiation unit of qmm_impl.hpp.
#include "qmm_impl.hpp"

namespace sx::qmm::detail {
template hipError_t launch_mode<DENSE>(int, int, int, const Params &, dim3, hipStream_t);
}
