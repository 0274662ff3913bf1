from .implicit_hashfly_gemm import ConvHashOnTheFlyImplicitGEMM, InputGradLookup
from .implicit_precomputed_gemm import ConvPrecomputedNeighborGEMM

__all__ = ["ConvHashOnTheFlyImplicitGEMM", "ConvPrecomputedNeighborGEMM", "InputGradLookup"]
