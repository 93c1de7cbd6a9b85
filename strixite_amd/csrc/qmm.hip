// qmm launch dispatch over the per-mode instantiation units (qmm_m0.hip .. qmm_m6.hip).
#include "qmm.hpp"

namespace sx::qmm {
namespace detail {
template <int MODE>
hipError_t launch_mode(int bits, int ax, int ay, const Params &p, dim3 grid, hipStream_t s);
extern template hipError_t launch_mode<DENSE>(int, int, int, const Params &, dim3, hipStream_t);
extern template hipError_t launch_mode<GATHER>(int, int, int, const Params &, dim3, hipStream_t);
extern template hipError_t launch_mode<SWIGLU>(int, int, int, const Params &, dim3, hipStream_t);
extern template hipError_t launch_mode<COMBINE>(int, int, int, const Params &, dim3, hipStream_t);
extern template hipError_t launch_mode<SLOT_GATHER>(int, int, int, const Params &, dim3, hipStream_t);
extern template hipError_t launch_mode<SLOT_SWIGLU>(int, int, int, const Params &, dim3, hipStream_t);
extern template hipError_t launch_mode<SLOT_COMBINE>(int, int, int, const Params &, dim3, hipStream_t);
}  // namespace detail

hipError_t launch(int mode, int bits, int act_x, int act_y, const Params &p, dim3 grid, hipStream_t stream) {
    using namespace detail;
    switch (mode) {
        case DENSE: return launch_mode<DENSE>(bits, act_x, act_y, p, grid, stream);
        case GATHER: return launch_mode<GATHER>(bits, act_x, act_y, p, grid, stream);
        case SWIGLU: return launch_mode<SWIGLU>(bits, act_x, act_y, p, grid, stream);
        case COMBINE: return launch_mode<COMBINE>(bits, act_x, act_y, p, grid, stream);
        case SLOT_GATHER: return launch_mode<SLOT_GATHER>(bits, act_x, act_y, p, grid, stream);
        case SLOT_SWIGLU: return launch_mode<SLOT_SWIGLU>(bits, act_x, act_y, p, grid, stream);
        default: return launch_mode<SLOT_COMBINE>(bits, act_x, act_y, p, grid, stream);
    }
}

}  // namespace sx::qmm
