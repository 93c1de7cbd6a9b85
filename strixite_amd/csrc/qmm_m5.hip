// qmm mode SLOT_SWIGLU: one instantiation unit of qmm_impl.hpp.
#include "qmm_impl.hpp"

namespace sx::qmm::detail {
template hipError_t launch_mode<SLOT_SWIGLU>(int, int, int, const Params &, dim3, hipStream_t);
}
