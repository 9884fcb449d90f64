"""Emulator of this build's ``--fast`` block-fp8 format (test oracle).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

The reference's fast mode uses Tenstorrent ``bfloat8_b`` (``tt_bio/tenstorrent.py:60-61``)
and has no CPU emulation (``--fast`` is ignored off-Tenstorrent,
``tt_bio/main.py:1648-1649``).  This build's fast mode maps to CDNA4's scaled
fp8 MFMA, i.e. the OCP Microscaling (MX) MXFP8-E4M3 format:

* blocks of 32 contiguous elements along the contraction (K) axis;
* one shared power-of-two scale per block: the smallest ``X = 2**e`` with
  ``amax / X <= 448`` (448 = 1.75 * 2**8, the largest e4m3 value), i.e.
  ``e = floor(log2(amax)) - 8``, plus one when amax's significand exceeds 1.75.
  The OCP MX rule ``floor(log2(amax)) - 8`` alone would clamp a block maximum in
  (448, 512) * X to 448 (up to 12.5 % off); this rule never saturates a block's
  elements.  Stored as an E8M0 byte (biased exponent, bias 127);
* elements ``v / X`` rounded to OCP e4m3 (FN variant: no infinities, max 448,
  subnormals down to 2**-9) with round-to-nearest-even and saturation to +-448.

A block of all zeros gets scale 2**-127 (E8M0 byte 0) and zero elements.
"""
from __future__ import annotations

import torch

E4M3_MAX = 448.0
E4M3_EMAX = 8          # floor(log2(448))
E4M3_MIN_NORMAL_EXP = -6
E4M3_MANT_BITS = 3
BLOCK = 32


def round_e4m3(y: torch.Tensor) -> torch.Tensor:
    """Round fp32 values to the nearest e4m3 (FN) value, ties to even, saturating at +-448."""
    y = y.to(torch.float32)
    a = y.abs()
    # exponent of each value; subnormal range shares the minimum normal exponent
    e = torch.floor(torch.log2(torch.where(a > 0, a, torch.ones_like(a))))
    e = torch.clamp(e, min=E4M3_MIN_NORMAL_EXP)
    ulp = torch.exp2(e - E4M3_MANT_BITS)
    q = torch.round(a / ulp) * ulp            # torch.round: half to even
    q = torch.clamp(q, max=E4M3_MAX)
    return torch.copysign(q, y)


def block_scale_exp(x: torch.Tensor) -> torch.Tensor:
    """Shared exponent per 32-block along the last axis (int32, unbiased): the smallest e
    with amax <= 448 * 2**e."""
    if x.shape[-1] % BLOCK:
        raise ValueError(f"last dim {x.shape[-1]} is not a multiple of {BLOCK}")
    xb = x.reshape(x.shape[:-1] + (x.shape[-1] // BLOCK, BLOCK)).to(torch.float32)
    amax = xb.abs().amax(dim=-1)
    # amax = f * 2**ex with 0.5 <= f < 1: floor(log2(amax)) = ex - 1, significand 2f
    f, ex = torch.frexp(torch.where(amax > 0, amax, torch.ones_like(amax)))
    e = (ex - 1 - E4M3_EMAX).to(torch.float32) + (f > 0.875).to(torch.float32)
    e = torch.where(amax > 0, e, torch.full_like(e, -127.0))
    return torch.clamp(e, -127, 127).to(torch.int32)


def quantize_mx8(x: torch.Tensor):
    """Return (elements as fp32 e4m3 values, unbiased scale exponents) for blocks along the last axis."""
    e = block_scale_exp(x)
    xb = x.reshape(x.shape[:-1] + (x.shape[-1] // BLOCK, BLOCK)).to(torch.float32)
    q = round_e4m3(xb / torch.exp2(e.to(torch.float32)).unsqueeze(-1))
    return q.reshape(x.shape), e


def fake_quant_mx8(x: torch.Tensor) -> torch.Tensor:
    """Quantize-dequantize along the last axis (what a scaled fp8 MFMA sees).

    A last axis that is not a multiple of 32 ends in a partial block; it is quantized
    as if zero-padded to 32 (zeros change neither the block maximum nor the other
    elements), which is what the GPU does on a zero-padded token grid."""
    K = x.shape[-1]
    if K % BLOCK:
        pad = BLOCK - K % BLOCK
        xp = torch.cat([x, torch.zeros(x.shape[:-1] + (pad,), dtype=x.dtype, device=x.device)], dim=-1)
        return fake_quant_mx8(xp)[..., :K]
    q, e = quantize_mx8(x)
    qb = q.reshape(x.shape[:-1] + (x.shape[-1] // BLOCK, BLOCK))
    return (qb * torch.exp2(e.to(torch.float32)).unsqueeze(-1)).reshape(x.shape)


def linear_mx8(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """fp32-accumulated ``x @ weight.T`` with both operands MXFP8-quantized along K."""
    return torch.nn.functional.linear(fake_quant_mx8(x), fake_quant_mx8(weight))
