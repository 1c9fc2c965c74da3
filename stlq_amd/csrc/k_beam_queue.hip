// Beam layers on the survivor-queue kernel (LayerKernel): the instantiations of layers 1..8
// (beam_kernels.hpp), compiled apart from the other layers so the build runs them in parallel.
#include "beam_kernels.hpp"

namespace stlq_mi355 {

hipError_t LaunchQueueLayer(int L, bool large_root, const LayerArgs& a, hipStream_t s) {
    switch (L) {
        case 1: return LaunchL<1>(large_root, a, s);
        case 2: return LaunchL<2>(large_root, a, s);
        case 3: return LaunchL<3>(large_root, a, s);
        case 4: return LaunchL<4>(large_root, a, s);
        case 5: return LaunchL<5>(large_root, a, s);
        case 6: return LaunchL<6>(large_root, a, s);
        case 7: return LaunchL<7>(large_root, a, s);
        case 8: return LaunchL<8>(large_root, a, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace stlq_mi355
