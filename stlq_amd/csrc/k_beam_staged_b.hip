// Beam layers on the staged kernel (LayerKernelStaged): the instantiations of layers 14..19
// (beam_kernels.hpp), compiled apart from the other layers so the build runs them in parallel.
#include "beam_kernels.hpp"

namespace stlq_mi355 {

hipError_t LaunchStagedLayerB(int L, bool large_root, const LayerArgs& a, hipStream_t s) {
    switch (L) {
        case 14: return LaunchL<14>(large_root, a, s);
        case 15: return LaunchL<15>(large_root, a, s);
        case 16: return LaunchL<16>(large_root, a, s);
        case 17: return LaunchL<17>(large_root, a, s);
        case 18: return LaunchL<18>(large_root, a, s);
        case 19: return LaunchL<19>(large_root, a, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace stlq_mi355
