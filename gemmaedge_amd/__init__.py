"""gemmaedge_amd — MI355X (gfx950) token-sampling path for GemmaEdge.

The product is the HIP library lib/libgemmaedge_sampler.so with the C ABI in
include/gemmaedge_sampler.h and the C++ drop-in in include/gemmaedge/sampling.h.
This package is its Python binding (``sampler``) and the synthetic workloads of
the benchmark configurations (``workloads``).
"""
from .sampler import (  # noqa: F401
    GE_DTYPE_BF16,
    GE_DTYPE_F32,
    GE_FLAG_NEAR_BOUNDARY,
    GE_FLAG_UNSUPPORTED,
    LIB_PATH,
    SampleArgs,
    SampleParams,
    Sampler,
    SamplerError,
    SamplingConfig,
    available,
    last_error,
    load_library,
    max_top_k,
)
