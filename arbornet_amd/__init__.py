"""arbornet_amd -- MI355X-native token sampling for ArborNet.

The product is ``libarbor_hip.so`` (HIP kernels for gfx950 behind the C ABI in
include/arbor_sampling.h); ``arbornet_amd.sampling`` binds it and exposes the
``Sampling.sample`` op, ``arbornet_amd.synthetic`` generates the benchmark workloads.
"""
from .sampling import (  # noqa: F401
    ARBOR_ID_BAD_HISTORY,
    ARBOR_ID_EMPTY,
    ARBOR_ID_INVALID,
    ArborSamplingError,
    Sampling,
    SamplingParams,
)
