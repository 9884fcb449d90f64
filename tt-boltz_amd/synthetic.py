"""Seeded synthetic weights and inputs for the benchmark/parity configurations.

The reference constructors zero every output projection and gate
(``tt_bio/boltz2.py:107-115``, ``tt_bio/reference.py:409-420``), so a freshly
constructed reference module produces identically-zero updates.  Checkpoints are
not available offline.  Weights are therefore drawn with an explicit,
non-degenerate init, in sorted state-dict-key order from one
``torch.Generator`` seeded with the configuration seed:

* every Linear weight (2-D): Xavier-uniform, gain 1;
* LayerNorm weights (1-D ``*.weight``): ``1 + 0.1 * U(-1, 1)``;
* LayerNorm biases and ``proj_q.bias`` (1-D ``*.bias``): ``0.1 * U(-1, 1)``.

Inputs are drawn in fp32 on the CPU from a separate ``torch.Generator`` with the
same seed, so the oracle and the GPU see identical bits.
"""
from __future__ import annotations

import hashlib
from typing import Dict

import torch


def layer_shapes(c_z: int = 128, c_s: int = 384, tri_heads: int = 4, tri_dim: int = 32, att_heads: int = 16,
                 transform_s: bool = True) -> Dict[str, tuple]:
    """State-dict keys and shapes of one PairformerLayer (reference.py:822-863, boltz2.py:307-341, 1188-1225)."""
    hd = tri_heads * tri_dim
    sh = {}
    for d in ("tri_mul_out", "tri_mul_in"):
        sh.update({f"{d}.norm_in.weight": (c_z,), f"{d}.norm_in.bias": (c_z,),
                   f"{d}.p_in.weight": (2 * c_z, c_z), f"{d}.g_in.weight": (2 * c_z, c_z),
                   f"{d}.norm_out.weight": (c_z,), f"{d}.norm_out.bias": (c_z,),
                   f"{d}.p_out.weight": (c_z, c_z), f"{d}.g_out.weight": (c_z, c_z)})
    for d in ("tri_att_start", "tri_att_end"):
        sh.update({f"{d}.layer_norm.weight": (c_z,), f"{d}.layer_norm.bias": (c_z,),
                   f"{d}.linear.weight": (tri_heads, c_z),
                   f"{d}.mha.linear_q.weight": (hd, c_z), f"{d}.mha.linear_k.weight": (hd, c_z),
                   f"{d}.mha.linear_v.weight": (hd, c_z), f"{d}.mha.linear_g.weight": (hd, c_z),
                   f"{d}.mha.linear_o.weight": (c_z, hd)})
    sh.update({"transition_z.norm.weight": (c_z,), "transition_z.norm.bias": (c_z,),
               "transition_z.fc1.weight": (4 * c_z, c_z), "transition_z.fc2.weight": (4 * c_z, c_z),
               "transition_z.fc3.weight": (c_z, 4 * c_z)})
    if transform_s:
        sh.update({"pre_norm_s.weight": (c_s,), "pre_norm_s.bias": (c_s,),
                   "attention.proj_q.weight": (c_s, c_s), "attention.proj_q.bias": (c_s,),
                   "attention.proj_k.weight": (c_s, c_s), "attention.proj_v.weight": (c_s, c_s),
                   "attention.proj_g.weight": (c_s, c_s), "attention.proj_o.weight": (c_s, c_s),
                   "attention.proj_z.0.weight": (c_z,), "attention.proj_z.0.bias": (c_z,),
                   "attention.proj_z.1.weight": (att_heads, c_z),
                   "transition_s.norm.weight": (c_s,), "transition_s.norm.bias": (c_s,),
                   "transition_s.fc1.weight": (4 * c_s, c_s), "transition_s.fc2.weight": (4 * c_s, c_s),
                   "transition_s.fc3.weight": (c_s, 4 * c_s)})
    return sh


def msa_layer_shapes(c_m: int = 64, c_z: int = 128, avg_heads: int = 8, avg_dim: int = 32, opm_hidden: int = 32,
                     tri_heads: int = 4, tri_dim: int = 32) -> Dict[str, tuple]:
    """State-dict keys and shapes of one MSALayer (reference.py:1311-1351): pair weighted
    averaging, msa transition, outer product mean and a no-seq PairformerLayer."""
    hd = avg_heads * avg_dim
    sh = {"pair_weighted_averaging.norm_m.weight": (c_m,), "pair_weighted_averaging.norm_m.bias": (c_m,),
          "pair_weighted_averaging.norm_z.weight": (c_z,), "pair_weighted_averaging.norm_z.bias": (c_z,),
          "pair_weighted_averaging.proj_m.weight": (hd, c_m), "pair_weighted_averaging.proj_g.weight": (hd, c_m),
          "pair_weighted_averaging.proj_z.weight": (avg_heads, c_z),
          "pair_weighted_averaging.proj_o.weight": (c_m, hd),
          "msa_transition.norm.weight": (c_m,), "msa_transition.norm.bias": (c_m,),
          "msa_transition.fc1.weight": (4 * c_m, c_m), "msa_transition.fc2.weight": (4 * c_m, c_m),
          "msa_transition.fc3.weight": (c_m, 4 * c_m),
          "outer_product_mean.norm.weight": (c_m,), "outer_product_mean.norm.bias": (c_m,),
          "outer_product_mean.proj_a.weight": (opm_hidden, c_m), "outer_product_mean.proj_b.weight": (opm_hidden, c_m),
          "outer_product_mean.proj_o.weight": (c_z, opm_hidden * opm_hidden),
          "outer_product_mean.proj_o.bias": (c_z,)}
    sh.update({f"pairformer_layer.{k}": v for k, v in layer_shapes(c_z, tri_heads=tri_heads, tri_dim=tri_dim,
                                                                    transform_s=False).items()})
    return sh


def msa_module_shapes(n_blocks: int, c_m: int = 64, c_z: int = 128, c_s: int = 384, n_feat: int = 36) -> Dict[str, tuple]:
    """MSAModule (reference.py:1150-1203): s_proj, msa_proj and ``layers.{i}.*``."""
    sh = {"s_proj.weight": (c_m, c_s), "msa_proj.weight": (c_m, n_feat)}
    one = msa_layer_shapes(c_m, c_z)
    for i in range(n_blocks):
        sh.update({f"layers.{i}.{k}": v for k, v in one.items()})
    return sh


def diffusion_pair_shapes(c_z: int = 128, depth: int = 24, heads: int = 16, n_transitions: int = 2,
                          prefix: str = "") -> Dict[str, tuple]:
    """Pair side of DiffusionConditioning (boltz2.py:2396-2441): ``pairwise_conditioner.*``
    (LN + projection of cat(z, rel_pos), transitions with hidden 2 c_z) and
    ``token_trans_proj_z.{l}.*`` (LN + Linear(c_z, heads) per token-transformer layer)."""
    sh = {"pairwise_conditioner.dim_pairwise_init_proj.0.weight": (2 * c_z,),
          "pairwise_conditioner.dim_pairwise_init_proj.0.bias": (2 * c_z,),
          "pairwise_conditioner.dim_pairwise_init_proj.1.weight": (c_z, 2 * c_z)}
    for i in range(n_transitions):
        p = f"pairwise_conditioner.transitions.{i}."
        sh.update({p + "norm.weight": (c_z,), p + "norm.bias": (c_z,), p + "fc1.weight": (2 * c_z, c_z),
                   p + "fc2.weight": (2 * c_z, c_z), p + "fc3.weight": (c_z, 2 * c_z)})
    for l in range(depth):
        sh.update({f"token_trans_proj_z.{l}.0.weight": (c_z,), f"token_trans_proj_z.{l}.0.bias": (c_z,),
                   f"token_trans_proj_z.{l}.1.weight": (heads, c_z)})
    return {prefix + k: v for k, v in sh.items()}


def recycle_shapes(c_z: int = 128, c_s: int = 384) -> Dict[str, tuple]:
    """Boltz2 recycling parameters (boltz2.py:4961-4968)."""
    return {"s_norm.weight": (c_s,), "s_norm.bias": (c_s,), "z_norm.weight": (c_z,), "z_norm.bias": (c_z,),
            "s_recycle.weight": (c_s, c_s), "z_recycle.weight": (c_z, c_z)}


def draw(shapes: Dict[str, tuple], seed: int) -> Dict[str, torch.Tensor]:
    """Explicit non-degenerate init in sorted key order from one seeded generator."""
    g = torch.Generator().manual_seed(seed)
    out = {}
    for key in sorted(shapes):
        shape = shapes[key]
        if len(shape) == 2:
            fan_out, fan_in = shape
            bound = (6.0 / (fan_in + fan_out)) ** 0.5
            out[key] = (torch.rand(shape, generator=g) * 2 - 1) * bound
        elif key.endswith(".weight"):
            out[key] = 1.0 + 0.1 * (torch.rand(shape, generator=g) * 2 - 1)
        else:
            out[key] = 0.1 * (torch.rand(shape, generator=g) * 2 - 1)
    return out


def stack_weights(n_blocks: int, seed: int, **kw) -> Dict[str, torch.Tensor]:
    """Weights of a ``n_blocks`` stack with keys ``layers.{i}.*``."""
    shapes = {}
    one = layer_shapes(**kw)
    for i in range(n_blocks):
        shapes.update({f"layers.{i}.{k}": v for k, v in one.items()})
    return draw(shapes, seed)


def fingerprint(w: Dict[str, torch.Tensor]) -> str:
    """SHA-256 over the fp32 bytes of the weights in sorted key order."""
    h = hashlib.sha256()
    for k in sorted(w):
        h.update(k.encode())
        h.update(w[k].detach().to(torch.float32).contiguous().numpy().tobytes())
    return h.hexdigest()


def pair_inputs(N: int, seed: int, c_z: int = 128, c_s: int = 384, z_scale: float = 1.0, pad_tail: int = 0,
                with_s: bool = True):
    """z [1,N,N,c_z] ~ z_scale*N(0,1), s [1,N,c_s] ~ N(0,1); token mask zero on the last ``pad_tail``."""
    g = torch.Generator().manual_seed(seed)
    z = torch.randn((1, N, N, c_z), generator=g) * z_scale
    s = torch.randn((1, N, c_s), generator=g) if with_s else None
    mask = torch.ones((1, N))
    if pad_tail:
        mask[:, N - pad_tail:] = 0.0
    pair_mask = mask[:, :, None] * mask[:, None, :]
    return s, z, mask, pair_mask


#: The five BASELINE.json configurations (shape parameters only).
CONFIGS = {
    0: dict(N=128, seed=0, z_scale=1.0, pad_tail=0, what="one PairformerLayer, fp32 oracle"),
    1: dict(N=512, seed=1, z_scale=1.0, pad_tail=51, what="triangle multiplication out/in"),
    2: dict(N=512, seed=2, z_scale=1.0, pad_tail=51, what="triangle attention start/end"),
    3: dict(N=768, seed=3, z_scale=0.5, pad_tail=0, what="64-layer stack, 4 recycling passes"),
    4: dict(N=1024, seed=4, z_scale=1.0, pad_tail=0, what="--fast block-fp8 trunk"),
}
