"""MSA module on the MI355X kernels (widening beyond the Pairformer).

Mirrors the ttnn ``MSA`` / ``MSALayer`` / ``OuterProductMean`` /
``PairWeightedAveraging`` stack (``tt_bio/tenstorrent.py:1632-1855``) and its
drop-in wrapper ``MSAModule`` (``tenstorrent.py:2524-2621``) at the ``Boltz2``
call site (``tt_bio/boltz2.py:4993-5009, 5230``), with the CPU reference's
semantics (``tt_bio/reference.py:1150-1398``): per-pair mask counts in the outer
product mean, the token and MSA masks from ``feats``.  Device tensors are fp32,
matrices in the MFMA operand type; every op is a HIP kernel behind the C ABI.
"""
from __future__ import annotations

from typing import Mapping, Optional

import torch
from torch import nn

from . import ops
from .pairformer import Module, Options, PairformerLayer, Transition, WeightScope, get_device

#: token vocabulary of the one-hot MSA feature (``tt_bio/data/const.py:100-157``)
NUM_TOKENS = 33


class OuterProductMean(Module):
    """``tenstorrent.py:1632-1720`` / ``reference.py:571-664``: z += OPM(m)."""

    def __init__(self, state_dict, options: Optional[Options] = None):
        super().__init__(state_dict, options)
        self.w = {k: self.vec(k) for k in ("norm.weight", "norm.bias", "proj_o.bias")}
        self.w.update({k: self.mat(k) for k in ("proj_a.weight", "proj_b.weight", "proj_o.weight")})

    def workspace_bytes(self, B: int, S: int, N: int) -> int:
        return ops.opm_workspace_bytes(B, S, N, self.variant)

    def __call__(self, m: torch.Tensor, msa_mask: Optional[torch.Tensor], z: torch.Tensor,
                 ws: Optional[torch.Tensor] = None) -> torch.Tensor:
        B, S, N, _ = m.shape
        if ws is None:
            ws = ops.workspace(self.workspace_bytes(B, S, N), m.device)
        ops.launch_opm(m, msa_mask, z, self.w, ws, True, self.options.eps, self.variant)
        return z


class PairWeightedAveraging(Module):
    """``reference.py:672-790`` (the ttnn version is called from ``tenstorrent.py:1757-1796``):
    m += PWA(m, z, pair_mask)."""

    def __init__(self, head_dim: int, n_heads: int, state_dict, options: Optional[Options] = None):
        super().__init__(state_dict, options)
        self.head_dim, self.n_heads = head_dim, n_heads
        self.w = {k: self.vec(k) for k in ("norm_m.weight", "norm_m.bias", "norm_z.weight", "norm_z.bias")}
        self.w.update({k: self.mat(k) for k in ("proj_m.weight", "proj_g.weight", "proj_z.weight", "proj_o.weight")})

    def workspace_bytes(self, B: int, S: int, N: int) -> int:
        return ops.pwa_workspace_bytes(B, S, N, self.variant)

    def __call__(self, m: torch.Tensor, z: torch.Tensor, pair_mask: Optional[torch.Tensor],
                 ws: Optional[torch.Tensor] = None) -> torch.Tensor:
        B, S, N, _ = m.shape
        if ws is None:
            ws = ops.workspace(self.workspace_bytes(B, S, N), m.device)
        ops.launch_pwa(m, z, pair_mask, m, self.w, ws, True, self.options.eps, self.variant)
        return m


class MSALayer(Module):
    """``tenstorrent.py:1723-1795`` / ``reference.py:1311-1398``:
    m += PWA(m, z); m += Tr(m); z += OPM(m); z = PairformerNoSeqLayer(z)."""

    def __init__(self, avg_head_dim: int, avg_n_heads: int, tri_att_head_dim: int, tri_att_n_heads: int,
                 state_dict, options: Optional[Options] = None):
        super().__init__(state_dict, options)
        self.msa_transition = Transition(self.scope("msa_transition"), self.options)
        self.pair_weighted_averaging = PairWeightedAveraging(avg_head_dim, avg_n_heads,
                                                             self.scope("pair_weighted_averaging"), self.options)
        self.outer_product_mean = OuterProductMean(self.scope("outer_product_mean"), self.options)
        self.pairformer_layer = PairformerLayer(tri_att_head_dim, tri_att_n_heads, None, None, False,
                                                self.scope("pairformer_layer"), self.options)

    def workspace_bytes(self, B: int, S: int, N: int) -> int:
        return max(self.pair_weighted_averaging.workspace_bytes(B, S, N),
                   self.msa_transition.workspace_bytes(B * S * N),
                   self.outer_product_mean.workspace_bytes(B, S, N),
                   self.pairformer_layer.workspace_bytes(B, N))

    def __call__(self, z: torch.Tensor, m: torch.Tensor, pair_mask: Optional[torch.Tensor],
                 msa_mask: Optional[torch.Tensor], ws: torch.Tensor, n_valid: int = 0):
        self.pair_weighted_averaging(m, z, pair_mask, ws)
        self.msa_transition(m, out=m, accumulate=True, ws=ws)
        self.outer_product_mean(m, msa_mask, z, ws)
        self.pairformer_layer(None, z, pair_mask, None, ws, n_valid)
        return z, m


class MSA(Module):
    """``tenstorrent.py:1798-1852``: input embedding and the block stack on padded device tensors."""

    def __init__(self, n_blocks: int, avg_head_dim: int, avg_n_heads: int, tri_att_head_dim: int,
                 tri_att_n_heads: int, state_dict, options: Optional[Options] = None):
        super().__init__(state_dict, options)
        self.s_proj = self.mat("s_proj.weight")
        # msa_proj stays fp32 and transposed: the one-hot product is a column gather
        self.msa_proj_t = ops.f32(self.weights["msa_proj.weight"], self.device).t().contiguous()
        self.blocks = [MSALayer(avg_head_dim, avg_n_heads, tri_att_head_dim, tri_att_n_heads,
                                self.scope(f"layers.{i}"), self.options) for i in range(n_blocks)]

    def workspace_bytes(self, B: int, S: int, N: int) -> int:
        return max((b.workspace_bytes(B, S, N) for b in self.blocks), default=16)

    def __call__(self, z: torch.Tensor, emb: torch.Tensor, msa: torch.Tensor, has_deletion: torch.Tensor,
                 deletion_value: torch.Tensor, msa_paired: torch.Tensor, pair_mask: Optional[torch.Tensor],
                 msa_mask: Optional[torch.Tensor], n_valid: int = 0) -> torch.Tensor:
        """Padded device tensors (N % 64 == 0): updates and returns z.  With padding
        (``n_valid`` < N) and no ``pair_mask`` the padding is masked out."""
        B, S, N = msa.shape
        if pair_mask is None and 0 < n_valid < N:
            pair_mask = ops.valid_pair_mask(B, N, n_valid, z.device)
        c_m = self.s_proj.shape[0]
        s_emb = torch.empty((B, N, c_m), dtype=torch.float32, device=z.device)
        ops.launch_linear(emb, self.s_proj, None, None, s_emb, self.variant)
        m = torch.empty((B, S, N, c_m), dtype=torch.float32, device=z.device)
        ops.launch_msa_embed(msa, has_deletion, deletion_value, msa_paired, s_emb, self.msa_proj_t, m, self.variant)
        ws = ops.workspace(self.workspace_bytes(B, S, N), z.device)
        for block in self.blocks:
            z, m = block(z, m, pair_mask, msa_mask, ws, n_valid)
        return z


def device_inputs(emb: torch.Tensor, feats: Mapping[str, torch.Tensor], n_pad: int,
                  device: torch.device) -> dict:
    """The MSA features of ``feats`` and ``emb`` (``s_inputs``) zero-padded to ``n_pad`` tokens
    on ``device``: the keyword arguments of ``MSA.__call__`` other than z, the pair mask and
    ``n_valid``."""
    B, S, N = feats["msa"].shape

    def per_row(key, dtype):
        t = torch.zeros((B, S, n_pad), dtype=dtype, device=device)
        t[:, :, :N] = feats[key].to(device, dtype)
        return t

    emb_dev = torch.zeros((B, n_pad, emb.shape[-1]), dtype=torch.float32, device=device)
    emb_dev[:, :N] = emb.to(device, torch.float32)
    return {"emb": emb_dev, "msa": per_row("msa", torch.int32), "has_deletion": per_row("has_deletion", torch.float32),
            "deletion_value": per_row("deletion_value", torch.float32),
            "msa_paired": per_row("msa_paired", torch.float32), "msa_mask": per_row("msa_mask", torch.float32)}


class MSAModule(nn.Module):
    """Drop-in for ``tenstorrent.MSAModule`` (``tenstorrent.py:2524-2621``) at
    ``boltz2.py:4993-5009``: ``forward(z, emb, feats) -> z_out`` (the caller adds it to z,
    ``boltz2.py:5230``).  CPU tensors in, CPU fp32 out; device tensors stay on device."""

    def __init__(self, n_blocks: int, avg_head_dim: int, avg_n_heads: int, tri_att_head_dim: int,
                 tri_att_n_heads: int, options: Optional[Options] = None):
        super().__init__()
        self.n_blocks = n_blocks
        self.avg_head_dim, self.avg_n_heads = avg_head_dim, avg_n_heads
        self.tri_att_head_dim, self.tri_att_n_heads = tri_att_head_dim, tri_att_n_heads
        self.options = options or Options()
        self.module: Optional[MSA] = None

    def _load_from_state_dict(self, state_dict, prefix, _local_metadata, _strict, _missing_keys,
                              _unexpected_keys, _error_msgs):
        self.module = MSA(self.n_blocks, self.avg_head_dim, self.avg_n_heads, self.tri_att_head_dim,
                          self.tri_att_n_heads, WeightScope.wrap(state_dict).child(prefix[:-1]), self.options)

    def reset_static_cache(self):
        """Nothing is cached across calls (kept for call-site compatibility)."""

    def forward(self, z: torch.Tensor, emb: torch.Tensor, feats: Mapping[str, torch.Tensor],
                use_kernels: bool = False) -> torch.Tensor:
        if self.module is None:
            raise RuntimeError("MSAModule has no weights: call load_state_dict() first")
        dev = get_device()
        B, N = z.shape[0], z.shape[1]
        n_pad = ops.padded_len(N)
        z_dev = ops.to_device_padded(z, n_pad, dev, pair=True)
        inputs = device_inputs(emb, feats, n_pad, dev)
        tok = torch.zeros((B, n_pad), dtype=torch.float32, device=dev)
        tok[:, :N] = feats["token_pad_mask"].to(dev, torch.float32)
        pair_mask = (tok[:, :, None] * tok[:, None, :]).contiguous()
        z_dev = self.module(z_dev, pair_mask=pair_mask, n_valid=N, **inputs)
        if z.device.type == "cpu":
            return ops.to_host(z_dev[:, :N, :N])
        return z_dev[:, :N, :N].to(z.device)
