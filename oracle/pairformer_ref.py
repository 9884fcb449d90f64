"""fp32 CPU restatement of the reference Boltz-2 Pairformer (test oracle).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

Every function takes plain tensors plus a flat weight mapping whose keys are the
reference state-dict names relative to the module (e.g. ``"norm_in.weight"`` for
a triangle multiplication, ``"tri_mul_out.norm_in.weight"`` for a layer), so a
checkpoint slice loads unchanged.  All arithmetic is torch fp32 on the CPU, in
the order the reference writes it.  Dropout is the identity (inference,
``tt_bio/boltz2.py:293-304`` with ``training=False``) and ``use_kernels=False``
(the cuequivariance branch is never taken).

Reference citations are ``path:line`` inside the tt-bio (moritztng/tt-boltz)
source tree.
"""
from __future__ import annotations

from contextlib import contextmanager
from math import ceil, log2, sqrt
from typing import Mapping, Optional

import torch
import torch.nn.functional as F

Tensor = torch.Tensor
Weights = Mapping[str, Tensor]

#: ``tt_bio/data/const.py:775`` -- above this N the reference chunks triangle
#: attention rows by 128, otherwise by 512 (``tt_bio/reference.py:982-988``).
CHUNK_SIZE_THRESHOLD = 384


#: Rounding of product operands: None (exact fp32, the reference semantics) or a 16-bit torch
#: dtype.  ``operand_rounding(torch.float16)`` turns the oracle into a precision model of a
#: 16-bit-operand implementation (operands of every matmul / einsum rounded once, products
#: accumulated and everything else computed in fp32); tests use it to bound the drift that the
#: operand format alone causes.  It is not the reference and is off by default.
_OPERAND: Optional[torch.dtype] = None

#: Operand families of the precision model.  Every rounding site carries one name
#: ``"<family>.<x|w>"`` (activation or weight side); a selector rounds the sites it matches.
FAMILIES = (
    "tm_in",    # trimul: LN_in(z) . p_in
    "tm_gin",   # trimul: LN_in(z) . g_in
    "tm_ab",    # trimul: the gated planes a, b of the contraction
    "tm_x",     # trimul: the stored contraction output X
    "tm_out",   # trimul: LN_out(X) . p_out
    "tm_gate",  # trimul: LN_in(z) . g_out
    "ta_in",    # triangle attention: LN(z) . W_q / W_k / W_v
    "ta_g",     # triangle attention: LN(z) . W_g
    "ta_bias",  # triangle attention: LN(z) . W_bias (the per-head triangle bias)
    "ta_qk",    # triangle attention: q, k of the logits
    "ta_p",     # triangle attention: the probabilities P of P.v
    "ta_v",     # triangle attention: v of P.v
    "ta_o",     # triangle attention: the stored attention output o
    "ta_out",   # triangle attention: o . sigmoid(g) . W_o
    "tr_in",    # pair transition: LN(z) . fc1 / fc2
    "tr_hid",   # pair transition: silu(fc1) * fc2 . fc3
    "s_apb",    # single track: attention with pair bias (projections, logits, P.v, z bias)
    "s_tr",     # single track: transition
    "rec",      # pair recycling projection z_recycle(z_norm(z))
    "s_rec",    # single recycling projection s_recycle(s_norm(s))
    "misc",     # every other linear (MSA module, diffusion conditioning)
)
_SELECT: Optional[frozenset] = None

#: The precision model of this build's 16-bit kernels (``operand_rounding(dtype, **BUILD_MODEL)``):
#: every product operand rounded to the operand type, except where the kernels carry a weight as
#: a 16-bit hi + lo pair -- the trimul output projection p_out, the triangle attention's gate and
#: output projections, the pair recycling projection (its activation too) -- and with the mean
#: correction at the trimul's LN_in-side weights (p_in, g_in, g_out), the triangle attention's
#: q / k / v and bias projections and the pair transition's fc3 (the kernels take those means
#: over sampled positions; the model over all of them).
BUILD_MODEL = {"families": ("!tm_out.w", "!ta_out.w", "!ta_g.w", "!rec"),
               "mean_fix": ("tm_in", "tm_gin", "tm_gate", "ta_in", "ta_bias", "tr_hid")}
_MEAN_FIX = None          # None, or the selector of weight sites whose error gets the mean correction
_MEAN_SAMPLE = 1          # the correction's mean is taken over every k-th position


def _parse_selector(families):
    if families is None:
        return None
    families = frozenset(families)
    unknown = {f for f in families
               if f.lstrip("!") not in ("x", "w") and f.lstrip("!").split(".")[0] not in FAMILIES}
    if unknown:
        raise ValueError(f"unknown operand families {sorted(unknown)}")
    return families


def _matches(select, site: str) -> bool:
    if select is None:
        return True
    fam, side = site.split(".")
    names = (fam, site, side)
    if any("!" + n in select for n in names):
        return False
    if all(f.startswith("!") for f in select):
        return True
    return any(n in select for n in names)


@contextmanager
def operand_rounding(dtype: Optional[torch.dtype], families=None, mean_fix=False, mean_sample: int = 1):
    """Round the operands of the sites selected by ``families`` to ``dtype`` (all sites when
    None).  A selector item is a family name from ``FAMILIES`` (both sides), a site name
    ``"<family>.x"`` / ``"<family>.w"``, or ``"x"`` / ``"w"`` (that side of every family); an
    item starting with ``"!"`` excludes what it names (with exclusions only, every other site
    is selected).  ``mean_fix`` (True, or a selector of weight sites): at those rounded weights
    the rounding error only meets the activation's deviation from its mean over positions (the
    model of an implementation that adds (W - round(W)) . mean(x) in fp32), the mean taken over
    every ``mean_sample``-th position."""
    global _OPERAND, _SELECT, _MEAN_FIX, _MEAN_SAMPLE
    families = _parse_selector(families)
    fix = None if mean_fix is False or mean_fix is None else (
        frozenset() if mean_fix is True else _parse_selector(mean_fix))
    prev = _OPERAND, _SELECT, _MEAN_FIX, _MEAN_SAMPLE
    _OPERAND, _SELECT, _MEAN_FIX, _MEAN_SAMPLE = dtype, families, fix, int(mean_sample)
    try:
        yield
    finally:
        _OPERAND, _SELECT, _MEAN_FIX, _MEAN_SAMPLE = prev


def _selected(site: str) -> bool:
    return _OPERAND is not None and _matches(_SELECT, site)


def _mean_fixed(site: str) -> bool:
    return _MEAN_FIX is not None and _selected(site) and (not _MEAN_FIX or _matches(_MEAN_FIX, site))


def _op(t: Tensor, site: str) -> Tensor:
    """A product operand at rounding site ``site``, rounded to the operand type when the
    precision model selects that site."""
    return t.to(_OPERAND).to(t.dtype) if _selected(site) else t


def _op_scaled(t: Tensor, site: str) -> Tensor:
    """A stored intermediate (the trimul contraction output) rounded to the operand type under
    a power-of-two scale that keeps its largest value in the type's normal range."""
    if not _selected(site):
        return t
    amax = float(t.abs().max())
    if amax == 0.0:
        return t
    scale = 2.0 ** (15 - ceil(log2(amax)))
    return (t * scale).to(_OPERAND).to(t.dtype) / scale


def sub(w: Weights, prefix: str) -> dict:
    """Slice ``w`` to the keys under ``prefix.`` with the prefix removed."""
    p = prefix + "."
    return {k[len(p):]: v for k, v in w.items() if k.startswith(p)}


def layer_norm(x: Tensor, weight: Tensor, bias: Tensor, eps: float = 1e-5) -> Tensor:
    """``nn.LayerNorm`` / ``tt_bio/boltz2.py:738-768`` (fp32 branch)."""
    return F.layer_norm(x, (x.shape[-1],), weight, bias, eps)


def linear(x: Tensor, weight: Tensor, bias: Optional[Tensor] = None, fam: str = "misc") -> Tensor:
    """``nn.Linear`` / ``tt_bio/boltz2.py:720-731`` (fp32 branch); ``fam`` names the
    operand family of the precision model."""
    y = F.linear(_op(x, fam + ".x"), _op(weight, fam + ".w"), bias)
    if _mean_fixed(fam + ".w") and x.dim() > 2:
        flat = x.reshape(x.shape[0], -1, x.shape[-1])[:, ::_MEAN_SAMPLE]
        mu = flat.mean(dim=1).view((x.shape[0],) + (1,) * (x.dim() - 2) + (x.shape[-1],))
        y = y + F.linear(mu, weight - _op(weight, fam + ".w"))
    return y


# --------------------------------------------------------------------------------------
# Triangle multiplication  (tt_bio/reference.py:387-472 outgoing, 476-561 incoming)
# --------------------------------------------------------------------------------------
def triangle_multiplication(z: Tensor, pair_mask: Tensor, w: Weights, direction: str) -> Tensor:
    """Return the update of ``TriangleMultiplication{Outgoing,Incoming}.forward``.

    ``reference.py:455-472`` (outgoing) / ``544-561`` (incoming):
    LN_in -> p_in * sigmoid(g_in) -> * pair_mask -> split a|b (fp32) ->
    einsum ``bikd,bjkd->bijd`` (outgoing) or ``bkid,bkjd->bijd`` (incoming) ->
    p_out(LN_out(x)) * sigmoid(g_out(LN_in(z))).
    """
    if direction not in ("outgoing", "incoming"):
        raise ValueError(f"direction must be 'outgoing' or 'incoming', got {direction!r}")
    x = layer_norm(z, w["norm_in.weight"], w["norm_in.bias"])              # reference.py:456
    x_in = x                                                                # :457
    x = linear(x, w["p_in.weight"], fam="tm_in") * torch.sigmoid(linear(x, w["g_in.weight"], fam="tm_gin"))  # :458
    x = x * pair_mask.unsqueeze(-1)                                         # :461
    a, b = torch.chunk(x.float(), 2, dim=-1)                                # :464
    a, b = _op(a, "tm_ab.x"), _op(b, "tm_ab.x")
    if direction == "outgoing":
        x = torch.einsum("bikd,bjkd->bijd", a, b)                           # :467
    else:
        x = torch.einsum("bkid,bkjd->bijd", a, b)                           # :556
    x = _op_scaled(x, "tm_x.x")
    x = linear(layer_norm(x, w["norm_out.weight"], w["norm_out.bias"]), w["p_out.weight"], fam="tm_out")
    return x * torch.sigmoid(linear(x_in, w["g_out.weight"], fam="tm_gate"))  # :470


def triangle_multiplication_mx8(z: Tensor, pair_mask: Tensor, w: Weights, direction: str) -> Tensor:
    """Fast-mode (``--fast``, ``tt_bio/tenstorrent.py:60-61, 389-407, 431-503``) restatement
    of :func:`triangle_multiplication` with this build's MXFP8 format (``fp8_emu``) at
    the points the GPU quantizes: LN_in(z) and p_in/g_in along channels; the gated a, b
    along the contraction index k; LN_out(x) and p_out, LN_in(z) and g_out along
    channels.  Everything else is fp32, as in the fp32 oracle."""
    from .fp8_emu import fake_quant_mx8 as fq, linear_mx8
    if direction not in ("outgoing", "incoming"):
        raise ValueError(f"direction must be 'outgoing' or 'incoming', got {direction!r}")
    x = layer_norm(z, w["norm_in.weight"], w["norm_in.bias"])
    x_in = x
    x = linear_mx8(x, w["p_in.weight"]) * torch.sigmoid(linear_mx8(x, w["g_in.weight"]))
    x = x * pair_mask.unsqueeze(-1)
    a, b = torch.chunk(x.float(), 2, dim=-1)
    if direction == "outgoing":
        # x_ij = sum_k a_ik b_jk: blocks along k = dim 2 of [b, i, k, d]
        a = fq(a.transpose(2, 3)).transpose(2, 3)
        b = fq(b.transpose(2, 3)).transpose(2, 3)
        x = torch.einsum("bikd,bjkd->bijd", a, b)
    else:
        # x_ij = sum_k a_ki b_kj: blocks along k = dim 1 of [b, k, i, d]
        a = fq(a.permute(0, 2, 3, 1)).permute(0, 3, 1, 2)
        b = fq(b.permute(0, 2, 3, 1)).permute(0, 3, 1, 2)
        x = torch.einsum("bkid,bkjd->bijd", a, b)
    x = linear_mx8(layer_norm(x, w["norm_out.weight"], w["norm_out.bias"]), w["p_out.weight"])
    return x * torch.sigmoid(linear_mx8(x_in, w["g_out.weight"]))


# --------------------------------------------------------------------------------------
# Triangle attention  (tt_bio/reference.py:219-376 + Attention 33-194 + boltz2.py:790-810)
# --------------------------------------------------------------------------------------
def _mha_rows(x: Tensor, tri_bias: Tensor, mask_bias: Tensor, w: Weights,
              n_heads: int, head_dim: int, fq=None) -> Tensor:
    """``Attention.forward`` with ``use_kernels=False`` on a block of rows.

    x [B,I,J,C]; tri_bias [B,1,H,J,K]; mask_bias [B,I,1,1,K].
    ``reference.py:96-121`` (_prep_qkv: q scaled by 1/sqrt(d) before QK^T),
    ``boltz2.py:790-810`` (_attention: a = qk; a += mask_bias; a += tri_bias;
    softmax; a @ v), ``reference.py:123-136`` (_wrap_up: sigmoid gate, flatten,
    linear_o).  ``fq`` (fast mode): the quantizer applied, along channels, to the q, k,
    v and g projections and to linear_o's output (``tenstorrent.py:580-590, 603-614``).
    """
    fq = fq or (lambda t: t)
    shp = x.shape[:-1]
    q = fq(linear(x, w["linear_q.weight"], fam="ta_in")).view(shp + (n_heads, head_dim)).transpose(-2, -3)
    k = fq(linear(x, w["linear_k.weight"], fam="ta_in")).view(shp + (n_heads, head_dim)).transpose(-2, -3)
    v = fq(linear(x, w["linear_v.weight"], fam="ta_in")).view(shp + (n_heads, head_dim)).transpose(-2, -3)
    q = q / sqrt(head_dim)
    a = torch.matmul(_op(q, "ta_qk.x"), _op(k, "ta_qk.x").transpose(-1, -2))      # [B,I,H,J,K]
    a = a + mask_bias
    a = a + tri_bias
    a = torch.softmax(a, dim=-1)
    o = torch.matmul(_op(a, "ta_p.x"), _op(v, "ta_v.x")).transpose(-2, -3)      # [B,I,J,H,d]
    g = torch.sigmoid(fq(linear(x, w["linear_g.weight"], fam="ta_g"))).view(shp + (n_heads, head_dim))
    o = (_op(o, "ta_o.x") * g).reshape(shp + (n_heads * head_dim,))
    return fq(linear(o, w["linear_o.weight"], fam="ta_out"))


def triangle_attention(z: Tensor, pair_mask: Optional[Tensor], w: Weights, starting: bool = True,
                       chunk_size: Optional[int] = None, n_heads: int = 4, head_dim: int = 32,
                       inf: float = 1e9, fast: bool = False) -> Tensor:
    """Return the update of ``TriangleAttention{Starting,Ending}Node.forward``.

    ``reference.py:294-365``: transpose for the ending node; LN; additive
    ``inf*(mask-1)`` per (row, key); per-head bias ``linear(x)`` shared across
    rows; row-chunked ``mha`` (``chunk_layer``, ``boltz2.py:542-628``, which is
    an exact partition of the row batch); transpose back.

    Weight keys are those of the reference module: ``layer_norm.*``,
    ``linear.weight`` and ``mha.linear_{q,k,v,g,o}.weight``.

    ``fast``: the fast-mode (``--fast``) restatement in this build's MXFP8 format
    (``fp8_emu``) at the reference's block-fp8 points (``tenstorrent.py:526-539, 580-590,
    603-614, 628-639``): linear_{q,k,v,g}.weight along their input channels, the q, k, v, g
    projections along channels (one block per head) and linear_o's output along channels.
    The LayerNorm output, the triangle bias and linear_o.weight stay exact.
    """
    if pair_mask is None:
        pair_mask = z.new_ones(z.shape[:-1])
    if not starting:
        z = z.transpose(-2, -3)
        pair_mask = pair_mask.transpose(-1, -2)
    x = layer_norm(z, w["layer_norm.weight"], w["layer_norm.bias"])      # :331
    mask = pair_mask[..., :, None, None, :]                              # :334
    mask_bias = inf * (mask - 1)                                         # :335
    tri_bias = linear(x, w["linear.weight"], fam="ta_bias").permute(0, 3, 1, 2).unsqueeze(-4)  # :338-341
    mw = sub(w, "mha")
    fq = None
    if fast:
        from .fp8_emu import fake_quant_mx8 as fq
        mw = {k: (fq(t) if k in ("linear_q.weight", "linear_k.weight", "linear_v.weight", "linear_g.weight")
                  else t) for k, t in mw.items()}
    n_rows = x.shape[1]
    step = n_rows if chunk_size is None else chunk_size
    outs = []
    for r0 in range(0, n_rows, step):
        r1 = min(r0 + step, n_rows)
        outs.append(_mha_rows(x[:, r0:r1], tri_bias, mask_bias[:, r0:r1], mw, n_heads, head_dim, fq))
    out = torch.cat(outs, dim=1)
    if not starting:
        out = out.transpose(-2, -3)
    return out


def triangle_attention_core(q: Tensor, k: Tensor, v: Tensor, tri_bias: Tensor,
                            mask: Tensor, scale: float) -> Tensor:
    """Masked biased attention with the signature of the fused-op contract
    ``kernel_triangular_attn(q, k, v, tri_bias, mask, scale)`` (``boltz2.py:815-817``).

    q, k, v [B,I,H,J,d]; tri_bias [B,1,H,J,K]; mask [B,I,1,1,K] (bool or 0/1).
    Semantics are those of the ``use_kernels=False`` path it replaces
    (``reference.py:176-190`` + ``boltz2.py:790-810``): logits =
    (scale*q) k^T + 1e9*(mask-1) + tri_bias, fp32 softmax over keys.
    """
    mask_bias = 1e9 * (mask.to(torch.float32) - 1.0)
    a = torch.matmul(q * scale, k.transpose(-1, -2))
    a = a + mask_bias
    a = a + tri_bias
    return torch.matmul(torch.softmax(a, dim=-1), v)


# --------------------------------------------------------------------------------------
# Transition  (tt_bio/boltz2.py:1188-1258)
# --------------------------------------------------------------------------------------
def transition(x: Tensor, w: Weights, fam: str = "tr") -> Tensor:
    """``Transition.forward`` with ``chunk_size=None`` (``boltz2.py:1240-1245``):
    LN -> silu(fc1) * fc2 -> fc3 (no biases).  ``fam``: the precision model's family prefix
    (``<fam>_in`` for fc1 / fc2, ``<fam>_hid`` for fc3; "s_tr" / "misc" as one family)."""
    f_in, f_hid = (fam + "_in", fam + "_hid") if fam == "tr" else (fam, fam)
    x = layer_norm(x, w["norm.weight"], w["norm.bias"])
    x = F.silu(linear(x, w["fc1.weight"], fam=f_in)) * linear(x, w["fc2.weight"], fam=f_in)
    return linear(x, w["fc3.weight"], fam=f_hid)


def transition_mx8(x: Tensor, w: Weights) -> Tensor:
    """Fast-mode transition (``tt_bio/tenstorrent.py:879-906``) in this build's MXFP8
    format: LN(x) and fc1/fc2 along channels, silu(fc1)*fc2 and fc3 along the hidden axis."""
    from .fp8_emu import linear_mx8
    x = layer_norm(x, w["norm.weight"], w["norm.bias"])
    x = F.silu(linear_mx8(x, w["fc1.weight"])) * linear_mx8(x, w["fc2.weight"])
    return linear_mx8(x, w["fc3.weight"])


# --------------------------------------------------------------------------------------
# Single attention with pair bias  (tt_bio/boltz2.py:307-367)
# --------------------------------------------------------------------------------------
def attention_pair_bias(s: Tensor, z: Tensor, mask: Tensor, k_in: Tensor, w: Weights,
                        num_heads: int = 16, inf: float = 1e6, fast: bool = False) -> Tensor:
    """``AttentionPairBias.forward`` (``boltz2.py:343-367``), multiplicity 1.

    q = proj_q(s) (+bias), k/v from ``k_in``; bias = proj_z(z) =
    Linear(LN(z)) -> [B,H,N,N]; logits = qk^T/sqrt(d) + bias - inf*(1-mask_key);
    softmax; o = P v; proj_o(sigmoid(proj_g(s)) * o).  ``fast``: sigmoid(g) * o in this
    build's MXFP8 format along channels before proj_o (``tenstorrent.py:846``).
    """
    B, N, c_s = s.shape
    d = c_s // num_heads
    q = linear(s, w["proj_q.weight"], w["proj_q.bias"], fam="s_apb").view(B, -1, num_heads, d)
    k = linear(k_in, w["proj_k.weight"], fam="s_apb").view(B, -1, num_heads, d)
    v = linear(k_in, w["proj_v.weight"], fam="s_apb").view(B, -1, num_heads, d)
    bias = linear(layer_norm(z, w["proj_z.0.weight"], w["proj_z.0.bias"]), w["proj_z.1.weight"], fam="s_apb")
    bias = bias.permute(0, 3, 1, 2)                                       # "b ... h -> b h ..."
    g = torch.sigmoid(linear(s, w["proj_g.weight"], fam="s_apb"))
    attn = torch.einsum("bihd,bjhd->bhij", _op(q.float(), "s_apb.x"), _op(k.float(), "s_apb.x"))
    attn = attn / (d ** 0.5) + bias.float()
    attn = attn + (1 - mask[:, None, None].float()) * -inf
    attn = attn.softmax(dim=-1)
    o = torch.einsum("bhij,bjhd->bihd", _op(attn, "s_apb.x"), _op(v.float(), "s_apb.x")).to(v.dtype)
    o = o.reshape(B, -1, c_s)
    go = g * o
    if fast:
        from .fp8_emu import fake_quant_mx8
        go = fake_quant_mx8(go)
    return linear(go, w["proj_o.weight"], fam="s_apb")


# --------------------------------------------------------------------------------------
# Layer / stack  (tt_bio/reference.py:822-1003, no-seq 1007-1139)
# --------------------------------------------------------------------------------------
def chunk_size_for(n: int) -> int:
    """``reference.py:982-988``: eval-mode triangle-attention row chunk."""
    return 128 if n > CHUNK_SIZE_THRESHOLD else 512


def pairformer_layer(s: Optional[Tensor], z: Tensor, mask: Optional[Tensor], pair_mask: Tensor,
                     w: Weights, chunk_size: Optional[int] = None,
                     tri_att_heads: int = 4, tri_att_head_dim: int = 32, att_heads: int = 16,
                     fast: bool = False):
    """``PairformerLayer.forward`` (``reference.py:865-914``); ``s=None`` gives
    ``PairformerNoSeqLayer.forward`` (``reference.py:1035-1072``).

    z += TMo; z += TMi; z += TAs; z += TAe; z += Tr_z;
    s_n = LN(s); s += APB(s_n, z, mask, k_in=s_n); s += Tr_s(s).
    ``fast``: the reference's fast mode in MXFP8: the triangle multiplications, the triangle
    attentions' block-fp8 points, the pair transition and the single track's gated
    attention output.
    """
    tm = triangle_multiplication_mx8 if fast else triangle_multiplication
    z = z + tm(z, pair_mask, sub(w, "tri_mul_out"), "outgoing")
    z = z + tm(z, pair_mask, sub(w, "tri_mul_in"), "incoming")
    z = z + triangle_attention(z, pair_mask, sub(w, "tri_att_start"), True, chunk_size,
                               tri_att_heads, tri_att_head_dim, fast=fast)
    z = z + triangle_attention(z, pair_mask, sub(w, "tri_att_end"), False, chunk_size,
                               tri_att_heads, tri_att_head_dim, fast=fast)
    z = z + (transition_mx8 if fast else transition)(z, sub(w, "transition_z"))
    if s is None:
        return None, z
    s_normed = layer_norm(s.float(), w["pre_norm_s.weight"], w["pre_norm_s.bias"])
    s = s.float() + attention_pair_bias(s_normed, z.float(), mask.float(), s_normed,
                                        sub(w, "attention"), att_heads, fast=fast)
    s = s + transition(s, sub(w, "transition_s"), fam="s_tr")
    return s, z


def pairformer_stack(s: Optional[Tensor], z: Tensor, mask: Optional[Tensor], pair_mask: Tensor,
                     w: Weights, n_blocks: int, **kw):
    """``PairformerModule.forward`` / ``PairformerNoSeqModule.forward`` in eval
    mode (``reference.py:958-1003``, ``1106-1139``)."""
    chunk = chunk_size_for(z.shape[1])
    for i in range(n_blocks):
        s, z = pairformer_layer(s, z, mask, pair_mask, sub(w, f"layers.{i}"), chunk, **kw)
    return s, z


def recycle(s_init: Tensor, z_init: Tensor, mask: Tensor, w_stack: Weights, w_rec: Weights,
            n_blocks: int, recycling_steps: int, msa=None, pass_hook=None, **kw):
    """Trunk recycling loop of ``Boltz2.forward`` (``boltz2.py:5189-5248``) without the
    template module: s, z start at zero; each of the ``recycling_steps + 1`` passes does
    s = s_init + s_recycle(s_norm(s)), z = z_init + z_recycle(z_norm(z)) (5213-5214), with
    ``msa = (w_msa, emb, feats, msa_blocks)`` z = z + msa_module(z, emb, feats) (5230), then
    the Pairformer stack (5239-5245).

    ``w_rec`` keys: ``s_norm.*``, ``z_norm.*``, ``s_recycle.weight``, ``z_recycle.weight``.
    ``pass_hook(i, s, z)`` (optional) sees the state after each pass.
    """
    pair_mask = mask[:, :, None] * mask[:, None, :]
    s = torch.zeros_like(s_init)
    z = torch.zeros_like(z_init)
    for i in range(recycling_steps + 1):
        s = s_init + linear(layer_norm(s, w_rec["s_norm.weight"], w_rec["s_norm.bias"]),
                            w_rec["s_recycle.weight"], fam="s_rec")
        z = z_init + linear(layer_norm(z, w_rec["z_norm.weight"], w_rec["z_norm.bias"]),
                            w_rec["z_recycle.weight"], fam="rec")
        if msa is not None:
            from .msa_ref import msa_module
            w_msa, emb, feats, msa_blocks = msa
            z = z + msa_module(z, emb, feats, w_msa, msa_blocks)
        s, z = pairformer_stack(s, z, mask, pair_mask, w_stack, n_blocks, **kw)
        if pass_hook is not None:
            pass_hook(i, s, z)
    return s, z
