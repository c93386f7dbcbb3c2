"""MI355X-native ETHOS expert-layer forward: product-key routing, hypernetwork expert
generation over the unique experts, reordered execution and weighted scatter-back,
as gfx950 HIP kernels behind a C-ABI (include/ethos_hip.h).

The layer classes are drop-ins for the reference's (wrmedford/ETHOS model.py and
kernels.py); see ethos_amd.layer.
"""
from .layer import (  # noqa: F401
    EthosExpertLayer,
    ExpertGenerationNetwork,
    FusedLowRankMoE_Reordered,
    ProductKeyRouter,
    SimplifiedHypernetMoE,
)

__all__ = [
    "EthosExpertLayer",
    "ExpertGenerationNetwork",
    "FusedLowRankMoE_Reordered",
    "ProductKeyRouter",
    "SimplifiedHypernetMoE",
]
