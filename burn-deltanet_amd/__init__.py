"""burn-deltanet's delta-rule core, MI355X-native.

The product is libdeltanet_core.so (HIP kernels for gfx950 behind the C ABI
in include/deltanet_core.h). This package is its Python host side: `abi`
binds the C ABI, `delta` mirrors the reference's interface (DeltaInput,
DeltaPath, delta_step, DeltaChunkBackendExt::delta_chunk_recalculated,
combined_backward, unit_lower_inverse), `frontend` its projection front-end
(QkvProjection), output norm (OutNorm) and the fused decode step of a block
(block_step).
"""

from . import abi
from .abi import DeltaError
from .delta import (DeltaChunkFunction, DeltaChunkGrads, DeltaInput, DeltaPath, TriSolve,
                    beta_gates, combined_backward, delta_chunk_recalculated, delta_step,
                    unit_lower_inverse)
from .frontend import (ConvActivation, OutNorm, QkActivation, QkNorm, Qkv, QkvProjection,
                       QkvStep, ShortConv, WriteGate, block_step)

__all__ = [
    "abi", "DeltaError", "DeltaChunkFunction", "DeltaChunkGrads", "DeltaInput", "DeltaPath",
    "TriSolve", "beta_gates", "combined_backward", "delta_chunk_recalculated", "delta_step",
    "unit_lower_inverse",
    "ConvActivation", "OutNorm", "QkActivation", "QkNorm", "Qkv", "QkvProjection", "QkvStep",
    "ShortConv", "WriteGate", "block_step",
]
