"""fp32 CPU restatement of the pair side of the reference diffusion conditioning (test oracle).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

Same conventions as ``pairformer_ref``: plain tensors, flat weight mappings keyed by the
reference state-dict names relative to the module, torch fp32 on the CPU.  Citations are
``path:line`` inside the tt-bio (moritztng/tt-boltz) source tree.
"""
from __future__ import annotations

from typing import Mapping

import torch

from .pairformer_ref import layer_norm, linear, sub, transition

Tensor = torch.Tensor
Weights = Mapping[str, Tensor]


def pairwise_conditioning(z_trunk: Tensor, rel_pos: Tensor, w: Weights, n_transitions: int = 2) -> Tensor:
    """``PairwiseConditioning.forward`` (``tt_bio/boltz2.py:1344-1355``): z = Linear(LN(cat(z_trunk,
    rel_pos))) (``dim_pairwise_init_proj``, 1330-1333), then z = transition(z) + z per transition."""
    z = torch.cat((z_trunk, rel_pos), dim=-1)
    z = linear(layer_norm(z, w["dim_pairwise_init_proj.0.weight"], w["dim_pairwise_init_proj.0.bias"]),
               w["dim_pairwise_init_proj.1.weight"])
    for i in range(n_transitions):
        z = transition(z, sub(w, f"transitions.{i}")) + z
    return z


def token_trans_bias(z: Tensor, w: Weights, depth: int) -> Tensor:
    """``token_trans_bias`` of ``DiffusionConditioning.forward`` (``tt_bio/boltz2.py:2472-2475``):
    cat over the ``depth`` layers of ``token_trans_proj_z.{l}`` = Sequential(LayerNorm(c_z),
    Linear(c_z, heads, bias=False)) (2434-2441) applied to z, along the last axis."""
    return torch.cat([linear(layer_norm(z, w[f"token_trans_proj_z.{l}.0.weight"], w[f"token_trans_proj_z.{l}.0.bias"]),
                             w[f"token_trans_proj_z.{l}.1.weight"]) for l in range(depth)], dim=-1)
