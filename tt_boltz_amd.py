"""Import name for the ``tt-boltz_amd/`` package directory.

The directory name contains a hyphen, which Python cannot import directly; this
module turns itself into that package by pointing ``__path__`` at it, so
``import tt_boltz_amd`` and ``from tt_boltz_amd.pairformer import ...`` work from
the repository root.
"""
import os as _os

__path__ = [_os.path.join(_os.path.dirname(_os.path.abspath(__file__)), "tt-boltz_amd")]

from tt_boltz_amd.pairformer import (  # noqa: E402,F401
    AttentionPairBias, Module, Options, Pairformer, PairformerLayer, PairformerModule, Transition,
    TriangleAttention, TriangleMultiplication, TrunkRecycler, WeightScope, get_device, set_fast_mode,
)
from tt_boltz_amd.msa import MSA, MSALayer, MSAModule, OuterProductMean, PairWeightedAveraging  # noqa: E402,F401
from tt_boltz_amd.diffusion import (  # noqa: E402,F401
    DiffusionPairConditioning, PairwiseConditioning, TokenTransformerPairBias,
)
from tt_boltz_amd import ops  # noqa: E402,F401
