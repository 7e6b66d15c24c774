"""rns_llm_amd: MI355X-native backend for the RNS linear / fused-QKV path of
Nek1tt/rns-llm.  Public names mirror ``rns_llm`` (``src/rns_llm/__init__.py``,
``backends/__init__.py``, ``layers/__init__.py``)."""
from .backends import (
    AdaptiveMetadata,
    HipRNSBackend,
    PreparedAdaptiveRNSWeight,
    PreparedRNSWeight,
    RNSRequestBatchWorkspace,
    RNSWorkspace,
    hip_extension_available,
)
from .layers import (
    CachedRNSQKV,
    InstalledQKVFusion,
    RNSLinear,
    RNSQKVProjection,
    install_opt_qkv_fusion,
    replace_opt_attention_blocks,
)
from .moduli import (
    DENSE_COPRIME_MODULI,
    LARGE_PRIME_MODULI,
    SMALL_PRIME_MODULI,
    choose_moduli_for_dot,
    minimal_prefix_channels,
    safe_l1_dot_bound,
    signed_capacity,
    validate_moduli,
)

__all__ = [
    "AdaptiveMetadata", "HipRNSBackend", "PreparedAdaptiveRNSWeight", "PreparedRNSWeight",
    "RNSRequestBatchWorkspace", "RNSWorkspace", "hip_extension_available", "CachedRNSQKV",
    "InstalledQKVFusion", "RNSLinear", "RNSQKVProjection", "install_opt_qkv_fusion",
    "replace_opt_attention_blocks",
    "DENSE_COPRIME_MODULI", "LARGE_PRIME_MODULI", "SMALL_PRIME_MODULI", "choose_moduli_for_dot",
    "minimal_prefix_channels", "safe_l1_dot_bound", "signed_capacity", "validate_moduli",
]
