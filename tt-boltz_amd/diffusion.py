"""Pair side of the diffusion conditioning on the MI355X kernels.

``DiffusionConditioning.forward`` (``tt_bio/boltz2.py:2373-2476``) turns the trunk's pair
representation into (i) the conditioned pair tensor of ``PairwiseConditioning``
(``boltz2.py:1318-1355``) and (ii) ``token_trans_bias``, the per-layer, per-head attention
bias of the diffusion token transformer: LN_l(z)·W_lᵀ for each of its layers, concatenated
(``boltz2.py:2434-2441, 2472-2475``; the ttnn ``compute_bias`` that replays it across
sampling steps, ``tt_bio/tenstorrent.py:714-728``).  Both are N²-sized and fixed for every
sampling step, so they run once per trunk output.  The atom-side outputs (atom encoder,
atom biases) are not part of this path.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import nn

from . import ops
from .pairformer import Module, Options, Transition, WeightScope, get_device

C_Z = 128


class PairwiseConditioning(Module):
    """``boltz2.py:1318-1355``: z = Linear(LN(cat(z_trunk, rel_pos))); z = transition_i(z) + z."""

    def __init__(self, state_dict, options: Optional[Options] = None, n_transitions: int = 2):
        super().__init__(state_dict, options)
        if self.weights["dim_pairwise_init_proj.1.weight"].shape != (C_Z, 2 * C_Z):
            raise NotImplementedError(f"only c_z = {C_Z} with a {C_Z}-channel relative position feature is supported")
        self.ln_w = self.vec("dim_pairwise_init_proj.0.weight")
        self.ln_b = self.vec("dim_pairwise_init_proj.0.bias")
        self.w = self.mat("dim_pairwise_init_proj.1.weight")
        self.transitions = [Transition(self.scope(f"transitions.{i}"), self.options, allow_fast=False)
                            for i in range(n_transitions)]

    def __call__(self, z_trunk: torch.Tensor, rel_pos: torch.Tensor,
                 out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Device fp32 [B, N, N, 128] inputs; returns the conditioned pair tensor."""
        if out is None:
            out = torch.empty_like(z_trunk)
        ops.launch_pair_cond_proj(z_trunk, rel_pos, self.ln_w, self.ln_b, self.w, out, self.options.eps, self.variant)
        for t in self.transitions:
            nb = t.workspace_bytes(out.numel() // C_Z)   # 0: the fused pair transition needs none
            t(out, out=out, accumulate=True, ws=ops.workspace(nb, out.device) if nb else None)
        return out


class TokenTransformerPairBias(Module):
    """``token_trans_proj_z`` (``boltz2.py:2434-2441``) applied to z and concatenated
    (``boltz2.py:2472-2475``): out[..., l*H + h] = LN_l(z)·W_l[h]."""

    def __init__(self, depth: int, state_dict, options: Optional[Options] = None):
        super().__init__(state_dict, options)
        self.depth = depth
        w = self.weights
        self.heads = w["token_trans_proj_z.0.1.weight"].shape[0]
        self.ln_w = ops.f32(torch.stack([w[f"token_trans_proj_z.{l}.0.weight"] for l in range(depth)]), self.device)
        self.ln_b = ops.f32(torch.stack([w[f"token_trans_proj_z.{l}.0.bias"] for l in range(depth)]), self.device)
        self.w = ops.opw(torch.cat([w[f"token_trans_proj_z.{l}.1.weight"] for l in range(depth)]), self.device,
                         self.variant)

    def __call__(self, z: torch.Tensor, layout: int = 0, scale: float = 1.0,
                 out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """layout 0: [B, N, N, L*H] (the reference layout); layout 1: [L*H, B, N, N]."""
        M = self.depth * self.heads
        if out is None:
            shape = (*z.shape[:-1], M) if layout == 0 else (M, *z.shape[:-1])
            out = torch.empty(shape, dtype=torch.float32, device=z.device)
        ops.launch_token_pair_bias(z, self.ln_w, self.ln_b, self.w, out, self.depth, self.heads, layout, scale,
                                   self.options.eps, self.variant)
        return out


class DiffusionPairConditioning(nn.Module):
    """The pair outputs of ``DiffusionConditioning`` (``boltz2.py:2443-2476``):
    ``forward(z_trunk, relative_position_encoding) -> (z, token_trans_bias)``, with the weights
    of ``diffusion_conditioning.{pairwise_conditioner, token_trans_proj_z}``.  CPU tensors in,
    CPU fp32 out; device tensors stay on the device."""

    def __init__(self, token_transformer_depth: int = 24, n_transitions: int = 2,
                 options: Optional[Options] = None):
        super().__init__()
        self.depth, self.n_transitions = token_transformer_depth, n_transitions
        self.options = options or Options()
        self.conditioner: Optional[PairwiseConditioning] = None
        self.bias: Optional[TokenTransformerPairBias] = None

    def _load_from_state_dict(self, state_dict, prefix, _local_metadata, _strict, _missing_keys,
                              _unexpected_keys, _error_msgs):
        scope = WeightScope.wrap(state_dict).child(prefix[:-1]) if prefix else WeightScope.wrap(state_dict)
        self.conditioner = PairwiseConditioning(scope.child("pairwise_conditioner"), self.options, self.n_transitions)
        self.bias = TokenTransformerPairBias(self.depth, scope, self.options)

    def forward(self, z_trunk: torch.Tensor, relative_position_encoding: torch.Tensor):
        if self.conditioner is None:
            raise RuntimeError("DiffusionPairConditioning has no weights: call load_state_dict() first")
        dev = get_device()
        zt = z_trunk.to(dev, torch.float32).contiguous()
        rp = relative_position_encoding.to(dev, torch.float32).contiguous()
        z = self.conditioner(zt, rp)
        bias = self.bias(z)
        return z.to(z_trunk.device), bias.to(z_trunk.device)
