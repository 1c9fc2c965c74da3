"""stlq_amd — MI355X-native (gfx950) STLQ multi-codebook beam-search encoder.

The encoder runs in libstlq_mi355.so (hand-written HIP kernels behind a C ABI,
include/stlq_mi355.h). This package holds the build script, the ctypes binding and a Python
mirror of the reference's encoder interface (stlq::BuildPrecomp, BeamSearchPrefixLS,
SolveLeastSquaresAll, ComputeCosts, DynamicIcmWithIls*, EncodeBase, EncodeBaseStreamingF32).
"""
from .encoder import (  # noqa: F401
    BaseEncoding,
    BeamSearchPrefixLS,
    BeamSearchPrefixLSLargeRoot,
    BuildPrecomp,
    BuildPrecompLargeRoot,
    ComputeCosts,
    ComputeXNorm2,
    Context,
    DynamicIcmWithIlsAbsNoNormal,
    DynamicIcmWithIlsNoAbsNoNormal,
    EncodeBase,
    EncodeBaseStreaming,
    EncodeBaseStreamingF32,
    EncodeConfig,
    SolveLeastSquaresAll,
)
