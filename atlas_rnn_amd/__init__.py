"""atlas_rnn_amd: MI355X-native memory-layer recurrence of atlas-rnn's Titans/OmegaNet RNN cells.

The hot path (delta, window aggregation, scalar-gated momentum/state scan, retrieval, and their
backward) runs as hand-written gfx950 HIP kernels in libatlas_mem.so behind the C ABI of
include/atlas_mem.h. Module classes mirror atlas_pytorch.rnn_memory / omega / affine_scan.
"""

from .functional import (  # noqa: F401
    memory_recurrence,
    memory_step_factored,
    buffer_factors,
    expand_buffer_factors,
    AtlasOmegaFunction,
    atlas_omega_forward,
    check_cuda_availability,
    get_cuda_status,
    assoc_scan,
    AssocScan,
    window_sum,
    affine_associative_scan,
)
from .rnn_memory import (  # noqa: F401
    RNNMemState,
    state_detach,
    PolynomialFeatureMap,
    MultiheadRMSNorm,
    RNNMemoryCell,
    OmegaRNNMemoryCell,
    RNNMemory,
    OmegaRNNMemory,
)

__all__ = [
    "memory_recurrence",
    "memory_step_factored",
    "buffer_factors",
    "expand_buffer_factors",
    "AtlasOmegaFunction",
    "atlas_omega_forward",
    "check_cuda_availability",
    "get_cuda_status",
    "assoc_scan",
    "AssocScan",
    "window_sum",
    "affine_associative_scan",
    "RNNMemState",
    "state_detach",
    "PolynomialFeatureMap",
    "MultiheadRMSNorm",
    "RNNMemoryCell",
    "OmegaRNNMemoryCell",
    "RNNMemory",
    "OmegaRNNMemory",
]
