// qmm mode SLOT_GATHER: one instantiation unit of qmm_impl.hpp.
#include "qmm_impl.hpp"

namespace sx::qmm::detail {
template hipError_t launch_mode<SLOT_GATHER>(int, int, int, const Params &, dim3, hipStream_t);
}
