// Beam layers on the staged kernel (LayerKernelStaged): the instantiations of layers 9..13
// (beam_kernels.hpp), compiled apart from the other layers so the build runs them in parallel.
#include "beam_kernels.hpp"

namespace stlq_mi355 {

hipError_t LaunchStagedLayerA(int L, bool large_root, const LayerArgs& a, hipStream_t s) {
    switch (L) {
        case 9: return LaunchL<9>(large_root, a, s);
        case 10: return LaunchL<10>(large_root, a, s);
        case 11: return LaunchL<11>(large_root, a, s);
        case 12: return LaunchL<12>(large_root, a, s);
        case 13: return LaunchL<13>(large_root, a, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace stlq_mi355
