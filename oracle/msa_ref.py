"""fp32 CPU restatement of the reference Boltz-2 MSA module (test oracle).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

Same conventions as ``pairformer_ref``: plain tensors, a flat weight mapping keyed by
the reference state-dict names relative to the module, torch fp32 on the CPU in the
order the reference writes it, dropout the identity (inference).

Reference citations are ``path:line`` inside the tt-bio (moritztng/tt-boltz) source
tree.  The eval-mode chunked branches the reference takes for N > 384
(``tt_bio/reference.py:1233-1247``: head-by-head pair averaging, channel-chunked outer
product) compute the same sums in a different order; this restatement follows the
unchunked branches.
"""
from __future__ import annotations

from typing import Mapping

import torch
import torch.nn.functional as F

from .pairformer_ref import layer_norm, linear, pairformer_layer, sub, transition, chunk_size_for

Tensor = torch.Tensor
Weights = Mapping[str, Tensor]

#: ``tt_bio/data/const.py:100-157``: 2 + 20 + 11 residue / nucleotide tokens.
NUM_TOKENS = 33


def outer_product_mean(m: Tensor, msa_mask: Tensor, w: Weights) -> Tensor:
    """``OuterProductMean.forward`` (``reference.py:596-664``, unchunked branch 653-664).

    m [B,S,N,c_m], msa_mask [B,S,N].  a = proj_a(LN(m))*mask, b = proj_b(LN(m))*mask;
    z[i,j] = proj_o(vec_{c,d}(sum_s a[s,i,c] b[s,j,d]) / max(1, sum_s mask[s,i] mask[s,j])).
    """
    mask = msa_mask.unsqueeze(-1).to(m)
    mn = layer_norm(m, w["norm.weight"], w["norm.bias"])
    a = linear(mn, w["proj_a.weight"]) * mask
    b = linear(mn, w["proj_b.weight"]) * mask
    pm = mask[:, :, None, :] * mask[:, :, :, None]
    num_mask = pm.sum(1).clamp(min=1)
    z = torch.einsum("bsic,bsjd->bijcd", a.float(), b.float())
    z = z.reshape(*z.shape[:3], -1)
    z = z / num_mask
    return linear(z.to(m), w["proj_o.weight"], w["proj_o.bias"])


def pair_weighted_averaging(m: Tensor, z: Tensor, pair_mask: Tensor, w: Weights, num_heads: int = 8,
                            c_h: int = 32, inf: float = 1e6) -> Tensor:
    """``PairWeightedAveraging.forward`` (``reference.py:715-790``, unchunked branch 779-790).

    v = proj_m(LN_m(m)) per head, weights = softmax_j(proj_z(LN_z(z)) - inf*(1 - mask)),
    o[s,i] = sum_j w[h,i,j] v[s,j,h]; proj_o(sigmoid(proj_g(LN_m(m))) * o).
    """
    m = layer_norm(m, w["norm_m.weight"], w["norm_m.bias"])
    z = layer_norm(z, w["norm_z.weight"], w["norm_z.bias"])
    v = linear(m, w["proj_m.weight"])
    v = v.reshape(*v.shape[:3], num_heads, c_h).permute(0, 3, 1, 2, 4)     # b h s j d
    b = linear(z, w["proj_z.weight"]).permute(0, 3, 1, 2)                  # b h i j
    b = b + (1 - pair_mask[:, None]) * -inf
    wts = torch.softmax(b, dim=-1)
    g = torch.sigmoid(linear(m, w["proj_g.weight"]))
    o = torch.einsum("bhij,bhsjd->bhsid", wts, v)
    o = o.permute(0, 2, 3, 1, 4)
    o = o.reshape(*o.shape[:3], num_heads * c_h)
    return linear(g * o, w["proj_o.weight"])


def msa_layer(z: Tensor, m: Tensor, pair_mask: Tensor, msa_mask: Tensor, w: Weights, chunk_size=None,
              avg_heads: int = 8, avg_head_dim: int = 32, tri_att_heads: int = 4, tri_att_head_dim: int = 32):
    """``MSALayer.forward`` (``reference.py:1353-1398``): m += PWA(m, z); m += Tr(m);
    z += OPM(m); z = PairformerNoSeqLayer(z)."""
    m = m + pair_weighted_averaging(m, z, pair_mask, sub(w, "pair_weighted_averaging"), avg_heads, avg_head_dim)
    m = m + transition(m, sub(w, "msa_transition"))
    z = z + outer_product_mean(m, msa_mask, sub(w, "outer_product_mean"))
    _, z = pairformer_layer(None, z, None, pair_mask, sub(w, "pairformer_layer"), chunk_size,
                            tri_att_heads, tri_att_head_dim)
    return z, m


def msa_input(msa: Tensor, has_deletion: Tensor, deletion_value: Tensor, msa_paired: Tensor, emb: Tensor,
              w: Weights) -> Tensor:
    """``MSAModule.forward`` input embedding (``reference.py:1253-1276``, use_paired_feature):
    m = msa_proj([one_hot(msa), has_deletion, deletion_value, is_paired]) + s_proj(emb)."""
    m = torch.cat([F.one_hot(msa, num_classes=NUM_TOKENS).float(), has_deletion.unsqueeze(-1).float(),
                   deletion_value.unsqueeze(-1).float(), msa_paired.unsqueeze(-1).float()], dim=-1)
    return linear(m, w["msa_proj.weight"]) + linear(emb, w["s_proj.weight"]).unsqueeze(1)


def msa_module(z: Tensor, emb: Tensor, feats: Mapping[str, Tensor], w: Weights, n_blocks: int, **kw) -> Tensor:
    """``MSAModule.forward`` in eval mode without subsampling (``reference.py:1205-1307``);
    returns the updated z (the caller adds it to z, ``boltz2.py:5230``)."""
    m = msa_input(feats["msa"], feats["has_deletion"], feats["deletion_value"], feats["msa_paired"], emb, w)
    tm = feats["token_pad_mask"].float()
    pair_mask = tm[:, :, None] * tm[:, None, :]
    chunk = chunk_size_for(z.shape[1])
    for i in range(n_blocks):
        z, m = msa_layer(z, m, pair_mask, feats["msa_mask"].float(), sub(w, f"layers.{i}"), chunk, **kw)
    return z
