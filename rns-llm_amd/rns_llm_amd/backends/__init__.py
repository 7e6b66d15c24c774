from .hip_backend import (
    AdaptiveMetadata,
    HipRNSBackend,
    PreparedAdaptiveRNSWeight,
    PreparedRNSWeight,
    RNSRequestBatchWorkspace,
    RNSWorkspace,
    hip_extension_available,
)

__all__ = [
    "AdaptiveMetadata",
    "HipRNSBackend",
    "PreparedAdaptiveRNSWeight",
    "PreparedRNSWeight",
    "RNSRequestBatchWorkspace",
    "RNSWorkspace",
    "hip_extension_available",
]
