"""Pin the CPU oracle (oracle/pairformer_ref.py) independently of its own formulas.

Each oracle function is checked against at least one of: the scalar-loop
restatement in oracle/brute.py (float64, explicit (i, j, k) indexing), a library
routine (torch.nn.functional.scaled_dot_product_attention / layer_norm /
float8_e4m3fn casts), or an invariant that a plausible mistake breaks
(transposition identities, mask invariance, chunking invariance, closed-form
special cases).  The reference ships no golden vectors for this path.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import brute, fp8_emu
from oracle import pairformer_ref as ref
from tt_boltz_amd import synthetic


def _w(shapes, seed):
    return synthetic.draw(shapes, seed)


def _trimul_w(c, seed=0):
    return _w({"norm_in.weight": (c,), "norm_in.bias": (c,), "p_in.weight": (2 * c, c), "g_in.weight": (2 * c, c),
               "norm_out.weight": (c,), "norm_out.bias": (c,), "p_out.weight": (c, c), "g_out.weight": (c, c)}, seed)


def _triatt_w(c, H, D, seed=0):
    return _w({"layer_norm.weight": (c,), "layer_norm.bias": (c,), "linear.weight": (H, c),
               "mha.linear_q.weight": (H * D, c), "mha.linear_k.weight": (H * D, c),
               "mha.linear_v.weight": (H * D, c), "mha.linear_g.weight": (H * D, c),
               "mha.linear_o.weight": (c, H * D)}, seed)


def _rand_mask(N, seed, p=0.3):
    g = torch.Generator().manual_seed(seed)
    return (torch.rand((1, N, N), generator=g) > p).float()


def _close(a, b, tol=2e-5):
    a = torch.as_tensor(np.asarray(a), dtype=torch.float64)
    b = torch.as_tensor(np.asarray(b), dtype=torch.float64)
    scale = b.abs().max().clamp_min(1e-6)
    assert ((a - b).abs().max() / scale).item() < tol, ((a - b).abs().max().item(), scale.item())


# ----------------------------------------------------------------------------- trimul
@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_trimul_matches_brute(direction):
    N, c = 5, 8
    z = torch.randn((1, N, N, c), generator=torch.Generator().manual_seed(1))
    m = _rand_mask(N, 2)
    w = _trimul_w(c, 3)
    _close(ref.triangle_multiplication(z, m, w, direction), brute.triangle_multiplication(z, m, w, direction))


def test_trimul_transpose_identity():
    """incoming(z^T) == outgoing(z) when the output gate is constant (g_out = 0):
    x_ij = sum_k a_ik b_jk is the same sum in both einsum strings after transposing z."""
    N, c = 7, 16
    z = torch.randn((1, N, N, c), generator=torch.Generator().manual_seed(4))
    w = _trimul_w(c, 5)
    w["g_out.weight"] = torch.zeros_like(w["g_out.weight"])
    ones = torch.ones((1, N, N))
    out = ref.triangle_multiplication(z, ones, w, "outgoing")
    inc = ref.triangle_multiplication(z.transpose(1, 2), ones, w, "incoming")
    _close(inc, out, 1e-5)
    # and the two directions differ for a non-symmetric z (catches a swapped einsum)
    assert (ref.triangle_multiplication(z, ones, w, "incoming") - out).abs().max() > 1e-3


def test_trimul_symmetric_input():
    N, c = 6, 8
    z = torch.randn((1, N, N, c), generator=torch.Generator().manual_seed(6))
    z = 0.5 * (z + z.transpose(1, 2))
    w = _trimul_w(c, 7)
    ones = torch.ones((1, N, N))
    _close(ref.triangle_multiplication(z, ones, w, "incoming"), ref.triangle_multiplication(z, ones, w, "outgoing"), 1e-5)


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_trimul_masked_token_invariance(direction):
    """With pair_mask = m m^T and m_r = 0, z at pairs touching token r cannot change
    the update at pairs (i, j) with i, j != r (both a and b are masked)."""
    N, c, r = 6, 8, 2
    g = torch.Generator().manual_seed(8)
    z = torch.randn((1, N, N, c), generator=g)
    m = torch.ones((1, N)); m[0, r] = 0
    pm = m[:, :, None] * m[:, None, :]
    w = _trimul_w(c, 9)
    z2 = z.clone()
    z2[0, r, :] += torch.randn((N, c), generator=g)
    z2[0, :, r] += torch.randn((N, c), generator=g)
    keep = torch.ones(N, dtype=torch.bool); keep[r] = False
    o1 = ref.triangle_multiplication(z, pm, w, direction)[0][keep][:, keep]
    o2 = ref.triangle_multiplication(z2, pm, w, direction)[0][keep][:, keep]
    _close(o2, o1, 1e-6)


# ----------------------------------------------------------------------------- triatt
@pytest.mark.parametrize("starting", [True, False])
def test_triatt_matches_brute(starting):
    N, c, H, D = 4, 8, 2, 4
    z = torch.randn((1, N, N, c), generator=torch.Generator().manual_seed(10))
    m = _rand_mask(N, 11, 0.25)
    w = _triatt_w(c, H, D, 12)
    _close(ref.triangle_attention(z, m, w, starting, None, H, D),
           brute.triangle_attention(z, m, w, starting, H, D))


def test_triatt_chunking_invariance():
    N, c, H, D = 9, 16, 2, 8
    z = torch.randn((1, N, N, c), generator=torch.Generator().manual_seed(13))
    m = _rand_mask(N, 14)
    w = _triatt_w(c, H, D, 15)
    full = ref.triangle_attention(z, m, w, True, None, H, D)
    for ch in (1, 2, 4, N):
        _close(ref.triangle_attention(z, m, w, True, ch, H, D), full, 1e-6)


def test_triatt_ending_is_transposed_starting():
    N, c, H, D = 6, 16, 2, 8
    z = torch.randn((1, N, N, c), generator=torch.Generator().manual_seed(16))
    m = _rand_mask(N, 17)
    w = _triatt_w(c, H, D, 18)
    end = ref.triangle_attention(z, m, w, False, None, H, D)
    start_t = ref.triangle_attention(z.transpose(1, 2), m.transpose(1, 2), w, True, None, H, D).transpose(1, 2)
    _close(end, start_t, 1e-6)


def test_triatt_core_matches_sdpa():
    """Masked biased attention vs torch's scaled_dot_product_attention (library routine)."""
    g = torch.Generator().manual_seed(19)
    B, I, H, J, D = 1, 5, 3, 7, 8
    q, k, v = (torch.randn((B, I, H, J, D), generator=g) for _ in range(3))
    bias = torch.randn((B, 1, H, J, J), generator=g)
    mask = (torch.rand((B, I, 1, 1, J), generator=g) > 0.3).float()
    mask[..., 0] = 1.0
    scale = 0.3
    o = ref.triangle_attention_core(q, k, v, bias, mask, scale)
    o_lib = F.scaled_dot_product_attention(q, k, v, attn_mask=bias + 1e9 * (mask - 1), scale=scale)
    _close(o, o_lib, 1e-5)


def test_triatt_core_all_masked_row_is_uniform():
    """A fully masked row softmaxes to the uniform average of v (fp32 -1e9 saturation,
    tt_bio/reference.py:334-335)."""
    g = torch.Generator().manual_seed(20)
    B, I, H, J, D = 1, 3, 2, 6, 4
    q, k, v = (torch.randn((B, I, H, J, D), generator=g) for _ in range(3))
    bias = torch.randn((B, 1, H, J, J), generator=g)
    mask = torch.ones((B, I, 1, 1, J)); mask[:, 1] = 0.0
    o = ref.triangle_attention_core(q, k, v, bias, mask, D ** -0.5)
    expect = v[:, 1].mean(dim=-2, keepdim=True).expand(B, H, J, D)
    _close(o[:, 1], expect, 1e-6)


def test_triatt_core_scalar_softmax():
    """H = 1, D = 1: o_j = sum_k softmax_k(scale*q_j*k_k + b_jk) v_k, by explicit loops."""
    J = 5
    g = torch.Generator().manual_seed(21)
    q, k, v = (torch.randn((1, 1, 1, J, 1), generator=g) for _ in range(3))
    bias = torch.randn((1, 1, 1, J, J), generator=g)
    o = ref.triangle_attention_core(q, k, v, bias, torch.ones((1, 1, 1, 1, J)), 0.7)
    for j in range(J):
        lg = [0.7 * q[0, 0, 0, j, 0].item() * k[0, 0, 0, kk, 0].item() + bias[0, 0, 0, j, kk].item() for kk in range(J)]
        mx = max(lg)
        e = [math.exp(x - mx) for x in lg]
        want = sum(ei * v[0, 0, 0, kk, 0].item() for kk, ei in enumerate(e)) / sum(e)
        assert abs(o[0, 0, 0, j, 0].item() - want) < 1e-5


# ----------------------------------------------------------------------------- transition / APB / LN
def test_transition_matches_brute():
    c, hdn = 8, 16
    x = torch.randn((1, 3, 4, c), generator=torch.Generator().manual_seed(22))
    w = _w({"norm.weight": (c,), "norm.bias": (c,), "fc1.weight": (hdn, c), "fc2.weight": (hdn, c),
            "fc3.weight": (c, hdn)}, 23)
    _close(ref.transition(x, w), brute.transition(x, w))


def test_layer_norm_matches_brute():
    x = torch.randn((3, 5, 16), generator=torch.Generator().manual_seed(24)) * 3 + 1
    w, b = torch.rand(16) + 0.5, torch.randn(16)
    _close(ref.layer_norm(x, w, b), brute.layer_norm(x, w, b))


def _apb_w(c_s, c_z, H, seed):
    return _w({"proj_q.weight": (c_s, c_s), "proj_q.bias": (c_s,), "proj_k.weight": (c_s, c_s),
               "proj_v.weight": (c_s, c_s), "proj_g.weight": (c_s, c_s), "proj_o.weight": (c_s, c_s),
               "proj_z.0.weight": (c_z,), "proj_z.0.bias": (c_z,), "proj_z.1.weight": (H, c_z)}, seed)


def test_apb_matches_brute():
    N, c_s, c_z, H = 5, 8, 8, 2
    g = torch.Generator().manual_seed(25)
    s = torch.randn((1, N, c_s), generator=g)
    z = torch.randn((1, N, N, c_z), generator=g)
    mask = torch.ones((1, N)); mask[0, 3] = 0
    w = _apb_w(c_s, c_z, H, 26)
    _close(ref.attention_pair_bias(s, z, mask, s, w, H), brute.attention_pair_bias(s, z, mask, s, w, H))


# ----------------------------------------------------------------------------- layer / stack
def _small_layer_weights(seed):
    return synthetic.draw(synthetic.layer_shapes(c_z=8, c_s=8, tri_heads=2, tri_dim=4, att_heads=2), seed)


def test_layer_matches_brute_composition():
    """The oracle layer equals the layer composed from independently written scalar ops
    in reference.py:877-912 order (catches a wrong order, a missing residual or a
    sub-block wired to the wrong weights)."""
    N = 4
    g = torch.Generator().manual_seed(27)
    s = torch.randn((1, N, 8), generator=g)
    z = torch.randn((1, N, N, 8), generator=g)
    mask = torch.ones((1, N)); mask[0, 3] = 0
    pm = mask[:, :, None] * mask[:, None, :]
    w = _small_layer_weights(28)
    so, zo = ref.pairformer_layer(s, z, mask, pm, w, None, 2, 4, 2)
    sb, zb = brute.pairformer_layer(s, z, mask, pm, w, 2, 4, 2)
    _close(zo, zb)
    _close(so, sb)


def test_stack_chunk_size_rule():
    assert ref.chunk_size_for(384) == 512 and ref.chunk_size_for(385) == 128


def test_noseq_layer_is_seq_layer_z():
    N = 5
    g = torch.Generator().manual_seed(29)
    s = torch.randn((1, N, 8), generator=g)
    z = torch.randn((1, N, N, 8), generator=g)
    mask = torch.ones((1, N))
    pm = mask[:, :, None] * mask[:, None, :]
    w = _small_layer_weights(30)
    _, z1 = ref.pairformer_layer(s, z, mask, pm, w, None, 2, 4, 2)
    s2, z2 = ref.pairformer_layer(None, z, None, pm, w, None, 2, 4, 2)
    assert s2 is None
    _close(z2, z1, 1e-7)


def test_recycle_zero_passes_is_one_stack_call():
    """recycling_steps = 0: s = s_init + W LN(0) = s_init + W b_norm (LN of zeros is its bias)."""
    N = 4
    g = torch.Generator().manual_seed(31)
    s_init = torch.randn((1, N, 8), generator=g)
    z_init = torch.randn((1, N, N, 8), generator=g)
    mask = torch.ones((1, N))
    w_stack = synthetic.draw({f"layers.0.{k}": v for k, v in synthetic.layer_shapes(
        c_z=8, c_s=8, tri_heads=2, tri_dim=4, att_heads=2).items()}, 32)
    w_rec = synthetic.draw(synthetic.recycle_shapes(c_z=8, c_s=8), 33)
    s_r, z_r = ref.recycle(s_init, z_init, mask, w_stack, w_rec, 1, 0, tri_att_heads=2, tri_att_head_dim=4,
                           att_heads=2)
    s0 = s_init + w_rec["s_norm.bias"] @ w_rec["s_recycle.weight"].T
    z0 = z_init + w_rec["z_norm.bias"] @ w_rec["z_recycle.weight"].T
    pm = mask[:, :, None] * mask[:, None, :]
    s_e, z_e = ref.pairformer_layer(s0, z0, mask, pm, ref.sub(w_stack, "layers.0"), 512, 2, 4, 2)
    _close(z_r, z_e, 1e-6)
    _close(s_r, s_e, 1e-6)


def test_recycle_msa_handoff_adds_the_returned_pair():
    """The MSA hand-off is z = z + msa_module(z) and the module returns the full updated z
    (boltz2.py:5230): with zero MSA blocks the module returns z itself, so one pass equals
    the stack on 2 (z_init + W b_norm)."""
    N, S = 4, 3
    g = torch.Generator().manual_seed(35)
    s_init = torch.randn((1, N, 8), generator=g)
    z_init = torch.randn((1, N, N, 8), generator=g)
    mask = torch.ones((1, N))
    w_stack = synthetic.draw({f"layers.0.{k}": v for k, v in synthetic.layer_shapes(
        c_z=8, c_s=8, tri_heads=2, tri_dim=4, att_heads=2).items()}, 36)
    w_rec = synthetic.draw(synthetic.recycle_shapes(c_z=8, c_s=8), 37)
    w_msa = synthetic.draw(synthetic.msa_module_shapes(0, c_m=8, c_z=8, c_s=8), 38)
    feats = {"msa": torch.randint(0, msa_ref.NUM_TOKENS, (1, S, N), generator=g),
             "has_deletion": torch.zeros((1, S, N)), "deletion_value": torch.zeros((1, S, N)),
             "msa_paired": torch.zeros((1, S, N)), "msa_mask": torch.ones((1, S, N)), "token_pad_mask": mask}
    emb = torch.randn((1, N, 8), generator=g)
    kw = dict(tri_att_heads=2, tri_att_head_dim=4, att_heads=2)
    s_r, z_r = ref.recycle(s_init, z_init, mask, w_stack, w_rec, 1, 0, msa=(w_msa, emb, feats, 0), **kw)
    s0 = s_init + w_rec["s_norm.bias"] @ w_rec["s_recycle.weight"].T
    z0 = z_init + w_rec["z_norm.bias"] @ w_rec["z_recycle.weight"].T
    pm = mask[:, :, None] * mask[:, None, :]
    s_e, z_e = ref.pairformer_layer(s0, 2 * z0, mask, pm, ref.sub(w_stack, "layers.0"), 512, 2, 4, 2)
    _close(z_r, z_e, 1e-6)
    _close(s_r, s_e, 1e-6)


# ----------------------------------------------------------------------------- fp8 emulator
def test_e4m3_rounding_matches_torch_cast():
    g = torch.Generator().manual_seed(34)
    x = torch.randn(20000, generator=g) * torch.exp2(torch.randint(-12, 9, (20000,), generator=g).float())
    x = x.clamp(-448, 448)
    ours = fp8_emu.round_e4m3(x)
    lib = x.to(torch.float8_e4m3fn).to(torch.float32)
    assert torch.equal(ours, lib)


def test_e4m3_representable_roundtrip_and_saturation():
    vals = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).to(torch.float32)
    vals = vals[torch.isfinite(vals)]
    assert torch.equal(fp8_emu.round_e4m3(vals), vals)
    assert fp8_emu.round_e4m3(torch.tensor([1e6, -500.0, 449.0])).tolist() == [448.0, -448.0, 448.0]


def test_mx8_scale_rule_and_block_independence():
    g = torch.Generator().manual_seed(35)
    x = torch.randn((4, 64), generator=g)
    x[1, :32] *= 1000.0
    # block maxima with significands on both sides of 1.75 (448 = 1.75 * 2^8)
    x[3] *= 2.0 ** -6                # |x| < 0.07: the planted values below are the block maxima
    x[3, 0], x[3, 32] = 1.9 * 2.0 ** 3, 1.74 * 2.0 ** -2
    x[0, 5] = 1.75 * 2.0 ** 4        # exactly 448 * 2^-4: stays at the floor exponent
    q, e = fp8_emu.quantize_mx8(x)
    amax = x.reshape(4, 2, 32).abs().amax(-1)
    # the smallest power of two X with amax / X <= 448, by search over exponents
    want = torch.empty_like(e)
    for idx in range(amax.numel()):
        a = float(amax.view(-1)[idx])
        k = -140
        while a / 2.0 ** k > 448.0:
            k += 1
        want.view(-1)[idx] = k
    assert torch.equal(e, want)
    assert e[3, 0].item() == 3 - 7 and e[3, 1].item() == -2 - 8 and e[0, 0].item() == 4 - 8
    # blocks are quantized independently: scaling one block does not change another
    x2 = x.clone(); x2[2, 32:] *= 64.0
    q2, _ = fp8_emu.quantize_mx8(x2)
    assert torch.equal(q2[2, :32], q[2, :32]) and torch.equal(q2[:2], q[:2])
    fq = fp8_emu.fake_quant_mx8(x)
    # no element saturates; RNE with 3 mantissa bits: half an ulp is <= |x| * 2^-4 in the
    # normal range and 2^-10 * scale (half the subnormal spacing 2^-9) below it
    scale = torch.exp2(e.float()).repeat_interleave(32, dim=-1)
    assert (q.abs() <= 448.0).all()
    bound = torch.maximum(x.abs() * 2 ** -4, scale * 2 ** -10)
    assert ((fq - x).abs() <= bound).all()
    assert torch.equal(fp8_emu.fake_quant_mx8(torch.zeros(32)), torch.zeros(32))


# ----------------------------------------------------------------------------- fast mode (MXFP8)
def test_brute_e4m3_table_matches_torch_cast():
    """The scalar table search of brute.py agrees with torch's float8_e4m3fn cast."""
    g = torch.Generator().manual_seed(41)
    v = torch.cat([torch.randn(4000, generator=g) * s for s in (0.01, 1.0, 40.0, 300.0)])
    want = v.clamp(-448, 448).to(torch.float8_e4m3fn).to(torch.float32)
    got = torch.tensor([brute._e4m3_nearest(float(x)) for x in v])
    assert torch.equal(got, want)


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_trimul_mx8_matches_brute(direction):
    """Emulated-fp8 triangle multiplication vs the scalar-loop version (independent
    quantizer), N = 32 (one MX block along k), c = 32, random mask."""
    N, c = 32, 32
    w = _trimul_w(c, seed=51)
    z = torch.randn((1, N, N, c), generator=torch.Generator().manual_seed(52))
    pm = _rand_mask(N, 53)
    got = ref.triangle_multiplication_mx8(z, pm, w, direction)
    want = brute.triangle_multiplication_mx8(z, pm, w, direction)
    _close(got, want, 1e-4)
    # and it is a genuine perturbation of the fp32 op (quantization error well above fp32 noise)
    exact = ref.triangle_multiplication(z, pm, w, direction)
    rel = ((got - exact).abs().mean() / exact.abs().mean()).item()
    assert 1e-3 < rel < 0.15, rel


@pytest.mark.parametrize("starting", [True, False])
def test_triatt_mx8_matches_brute(starting):
    """Emulated-fp8 triangle attention vs the scalar-loop version (independent quantizer):
    weights, q/k/v/g and the output quantized along channels (c = 32: one MX block)."""
    N, c, H, D = 4, 32, 2, 16
    z = torch.randn((1, N, N, c), generator=torch.Generator().manual_seed(60))
    m = _rand_mask(N, 61, 0.25)
    w = _triatt_w(c, H, D, 62)
    got = ref.triangle_attention(z, m, w, starting, None, H, D, fast=True)
    _close(got, brute.triangle_attention(z, m, w, starting, H, D, fast=True), 1e-4)
    exact = ref.triangle_attention(z, m, w, starting, None, H, D)
    rel = ((got - exact).abs().mean() / exact.abs().mean()).item()
    assert 1e-3 < rel < 0.15, rel


def test_triatt_mx8_quantization_points():
    """With the quantizer replaced by the identity the fast triangle attention is the fp32
    one, and it quantizes exactly: the four projection weights, then per row chunk q, k, v,
    g and the output (a dropped or extra point changes the count or the shapes)."""
    N, c, H, D = 6, 32, 2, 16
    z = torch.randn((1, N, N, c), generator=torch.Generator().manual_seed(63))
    m = _rand_mask(N, 64)
    w = _triatt_w(c, H, D, 65)
    seen = []

    def ident(t):
        seen.append(tuple(t.shape))
        return t

    real = fp8_emu.fake_quant_mx8
    fp8_emu.fake_quant_mx8 = ident
    try:
        got = ref.triangle_attention(z, m, w, True, 3, H, D, fast=True)
    finally:
        fp8_emu.fake_quant_mx8 = real
    assert torch.equal(got, ref.triangle_attention(z, m, w, True, 3, H, D))
    assert seen == [(H * D, c)] * 4 + ([(1, 3, N, H * D)] * 4 + [(1, 3, N, c)]) * 2, seen


def test_apb_mx8_matches_brute():
    N, c_s, c_z, H = 5, 32, 8, 2
    g = torch.Generator().manual_seed(66)
    s = torch.randn((1, N, c_s), generator=g)
    z = torch.randn((1, N, N, c_z), generator=g)
    mask = torch.ones((1, N)); mask[0, 2] = 0
    w = _apb_w(c_s, c_z, H, 67)
    got = ref.attention_pair_bias(s, z, mask, s, w, H, fast=True)
    _close(got, brute.attention_pair_bias(s, z, mask, s, w, H, fast=True), 1e-4)
    exact = ref.attention_pair_bias(s, z, mask, s, w, H)
    rel = ((got - exact).abs().mean() / exact.abs().mean()).item()
    assert 1e-3 < rel < 0.15, rel


def test_transition_mx8_matches_brute():
    c = 32
    w = _w({"norm.weight": (c,), "norm.bias": (c,), "fc1.weight": (4 * c, c), "fc2.weight": (4 * c, c),
            "fc3.weight": (c, 4 * c)}, 54)
    x = torch.randn((1, 3, 5, c), generator=torch.Generator().manual_seed(55))
    got = ref.transition_mx8(x, w)
    _close(got, brute.transition_mx8(x, w), 1e-4)
    exact = ref.transition(x, w)
    rel = ((got - exact).abs().mean() / exact.abs().mean()).item()
    assert 1e-3 < rel < 0.15, rel


def test_mx8_quantization_axis_of_trimul():
    """The a/b quantization runs along the contraction index: scaling one k-slice of a
    block changes only that block's scale, so outputs for (i, j) pairs whose blocks
    are untouched stay identical (outgoing: blocks along k = z column)."""
    N, c = 64, 32
    w = _trimul_w(c, seed=56)
    z = torch.randn((1, N, N, c), generator=torch.Generator().manual_seed(57))
    pm = torch.ones((1, N, N))
    base = ref.triangle_multiplication_mx8(z, pm, w, "outgoing")
    # masking one column block of k for row i=3 only changes x[3, :] (a rows) and x[:, 3] (b rows)
    pm2 = pm.clone(); pm2[0, 3, 32:] = 0.0
    moved = ref.triangle_multiplication_mx8(z, pm2, w, "outgoing")
    keep = torch.ones((N, N), dtype=torch.bool); keep[3, :] = False; keep[:, 3] = False
    assert torch.equal(moved[0][keep], base[0][keep])


def test_mx8_partial_block_equals_zero_padding():
    """A partial last block quantizes like the zero-padded block (the GPU's padded grid)."""
    g = torch.Generator().manual_seed(58)
    x = torch.randn((5, 70), generator=g) * 3
    padded = torch.cat([x, torch.zeros((5, 26))], dim=1)
    assert torch.equal(fp8_emu.fake_quant_mx8(x), fp8_emu.fake_quant_mx8(padded)[:, :70])
    assert torch.equal(fp8_emu.fake_quant_mx8(x)[:, :64], fp8_emu.fake_quant_mx8(x[:, :64]))
    # and the scalar quantizer of brute.py agrees on the partial block
    want = torch.tensor([brute.mx8_vec([float(v) for v in row]) for row in x], dtype=torch.float64)
    assert torch.allclose(fp8_emu.fake_quant_mx8(x).double(), want, rtol=0, atol=0)


# ----------------------------------------------------------------------------- MSA module
from oracle import msa_ref  # noqa: E402


def _opm_w(c_m, hh, c_z, seed):
    return _w({"norm.weight": (c_m,), "norm.bias": (c_m,), "proj_a.weight": (hh, c_m),
               "proj_b.weight": (hh, c_m), "proj_o.weight": (c_z, hh * hh), "proj_o.bias": (c_z,)}, seed)


def _pwa_w(c_m, c_z, H, ch, seed):
    return _w({"norm_m.weight": (c_m,), "norm_m.bias": (c_m,), "norm_z.weight": (c_z,), "norm_z.bias": (c_z,),
               "proj_m.weight": (H * ch, c_m), "proj_g.weight": (H * ch, c_m), "proj_z.weight": (H, c_z),
               "proj_o.weight": (c_m, H * ch)}, seed)


def test_opm_matches_brute():
    """Outer product mean: pairwise mask counts (with a fully masked sequence and a token
    masked in some sequences), channel order c*H + d, bias."""
    B, S, N, c_m, hh, c_z = 1, 4, 5, 8, 3, 6
    g = torch.Generator().manual_seed(61)
    m = torch.randn((B, S, N, c_m), generator=g)
    mask = (torch.rand((B, S, N), generator=g) > 0.3).float()
    mask[:, 1] = 0.0
    w = _opm_w(c_m, hh, c_z, 62)
    _close(msa_ref.outer_product_mean(m, mask, w), brute.outer_product_mean(m, mask, w))


def test_opm_single_sequence_closed_form():
    """S = 1, all ones: z[i,j] = Wo vec(a_i outer b_j) + bo (mean over one sequence)."""
    c_m, hh, c_z, N = 8, 4, 5, 3
    g = torch.Generator().manual_seed(63)
    m = torch.randn((1, 1, N, c_m), generator=g)
    w = _opm_w(c_m, hh, c_z, 64)
    mn = F.layer_norm(m, (c_m,), w["norm.weight"], w["norm.bias"])
    a, b = mn @ w["proj_a.weight"].T, mn @ w["proj_b.weight"].T
    want = torch.einsum("ic,jd->ijcd", a[0, 0], b[0, 0]).reshape(N, N, -1) @ w["proj_o.weight"].T + w["proj_o.bias"]
    _close(msa_ref.outer_product_mean(m, torch.ones((1, 1, N)), w)[0], want)


def test_pwa_matches_brute():
    """Pair weighted averaging: softmax over j (not s), per-head slices, masked pairs."""
    B, S, N, c_m, c_z, H, ch = 1, 3, 5, 8, 6, 2, 3
    g = torch.Generator().manual_seed(65)
    m = torch.randn((B, S, N, c_m), generator=g)
    z = torch.randn((B, N, N, c_z), generator=g)
    tok = torch.ones((B, N)); tok[:, -1] = 0
    pm = tok[:, :, None] * tok[:, None, :]
    w = _pwa_w(c_m, c_z, H, ch, 66)
    got = msa_ref.pair_weighted_averaging(m, z, pm, w, H, ch)
    want = brute.pair_weighted_averaging(m, z, pm, w, H, ch)
    # the fully masked row (i = N-1) is fp32 rounding of logit - 1e6 in the reference
    # (ulp 0.0625), which the float64 loops do not reproduce: compared separately, loosely
    _close(got[:, :, :-1], want[:, :, :-1])
    _close(got[:, :, -1:], want[:, :, -1:], tol=5e-2)


def test_pwa_uniform_bias_is_mean():
    """proj_z = 0 and no mask: every weight is 1/N, so o = sigmoid(g) * mean_j v."""
    B, S, N, c_m, c_z, H, ch = 1, 2, 4, 8, 6, 2, 3
    g = torch.Generator().manual_seed(67)
    m = torch.randn((B, S, N, c_m), generator=g)
    z = torch.randn((B, N, N, c_z), generator=g)
    w = _pwa_w(c_m, c_z, H, ch, 68)
    w["proj_z.weight"] = torch.zeros_like(w["proj_z.weight"])
    mn = F.layer_norm(m, (c_m,), w["norm_m.weight"], w["norm_m.bias"])
    v, gg = mn @ w["proj_m.weight"].T, torch.sigmoid(mn @ w["proj_g.weight"].T)
    want = (gg * v.mean(dim=2, keepdim=True)) @ w["proj_o.weight"].T
    _close(msa_ref.pair_weighted_averaging(m, z, torch.ones((B, N, N)), w, H, ch), want)


def test_msa_input_is_column_gather():
    """One-hot projection = the weight column of the token, plus the three feature columns
    and the s projection broadcast over sequences."""
    S, N, c_m, c_s = 3, 4, 6, 5
    g = torch.Generator().manual_seed(69)
    msa = torch.randint(0, msa_ref.NUM_TOKENS, (1, S, N), generator=g)
    hd, dv, pr = (torch.rand((1, S, N), generator=g) for _ in range(3))
    emb = torch.randn((1, N, c_s), generator=g)
    w = _w({"msa_proj.weight": (c_m, msa_ref.NUM_TOKENS + 3), "s_proj.weight": (c_m, c_s)}, 70)
    W = w["msa_proj.weight"]
    want = (W[:, msa[0]].permute(1, 2, 0) + hd[0, ..., None] * W[:, 33] + dv[0, ..., None] * W[:, 34]
            + pr[0, ..., None] * W[:, 35] + (emb[0] @ w["s_proj.weight"].T)[None])
    _close(msa_ref.msa_input(msa, hd, dv, pr, emb, w)[0], want)


# ----------------------------------------------------------------------------- diffusion conditioning (pair side)
from oracle import diffusion_ref  # noqa: E402


def test_pairwise_conditioning_matches_brute():
    g = torch.Generator().manual_seed(90)
    w = synthetic.draw(synthetic.diffusion_pair_shapes(c_z=8, depth=1, heads=2), 91)
    w = ref.sub(w, "pairwise_conditioner")
    zt = torch.randn((1, 3, 3, 8), generator=g)
    rp = torch.randn((1, 3, 3, 8), generator=g)
    got = diffusion_ref.pairwise_conditioning(zt, rp, w)
    _close(got, torch.from_numpy(brute.pairwise_conditioning(zt, rp, w)), 1e-5)


def test_token_trans_bias_matches_brute():
    """Output l*H + h is layer l's own LayerNorm and head-h row (a swapped layer/head order or
    a shared LayerNorm fails this)."""
    g = torch.Generator().manual_seed(92)
    w = synthetic.draw(synthetic.diffusion_pair_shapes(c_z=8, depth=3, heads=2, n_transitions=0), 93)
    z = torch.randn((1, 3, 4, 8), generator=g)
    got = diffusion_ref.token_trans_bias(z, w, 3)
    assert got.shape == (1, 3, 4, 6)
    _close(got, torch.from_numpy(brute.token_trans_bias(z, w, 3)), 1e-5)


def test_token_trans_bias_constant_rows_closed_form():
    """A constant pair row normalises to zero, so layer l's bias is W_l . beta_l."""
    w = synthetic.draw(synthetic.diffusion_pair_shapes(c_z=8, depth=2, heads=3, n_transitions=0), 94)
    z = torch.full((1, 2, 2, 8), 0.7)
    got = diffusion_ref.token_trans_bias(z, w, 2)
    want = torch.cat([w[f"token_trans_proj_z.{l}.1.weight"] @ w[f"token_trans_proj_z.{l}.0.bias"] for l in range(2)])
    _close(got, want.expand(1, 2, 2, 6), 1e-6)


# ----------------------------------------------------------------------------- operand-precision model
def test_operand_rounding_is_off_by_default_and_restored():
    g = torch.Generator().manual_seed(120)
    x, w = torch.randn(5, 16, generator=g), torch.randn(8, 16, generator=g)
    exact = F.linear(x, w)
    assert torch.equal(ref.linear(x, w), exact)
    with ref.operand_rounding(torch.float16):
        assert torch.equal(ref.linear(x, w), F.linear(x.half().float(), w.half().float()))
        with ref.operand_rounding(None):
            assert torch.equal(ref.linear(x, w), exact)
    assert ref._OPERAND is None and torch.equal(ref.linear(x, w), exact)


def test_operand_rounding_layer_drift_scales_with_operand_precision():
    """One layer under the 16-bit-operand precision model drifts from fp32 by about the
    operand type's relative precision: fp16 (2^-11) well below bf16 (2^-8), both far above
    fp32 noise -- a rounding site dropped from the model or applied twice breaks the ratio."""
    N = 24
    w = ref.sub(synthetic.stack_weights(1, 121), "layers.0")
    s, z, mask, pm = synthetic.pair_inputs(N, 122)
    s0, z0 = ref.pairformer_layer(s, z, mask, pm, w)
    err = {}
    for dt in (torch.float16, torch.bfloat16):
        with ref.operand_rounding(dt):
            s1, z1 = ref.pairformer_layer(s, z, mask, pm, w)
        upd = z0 - z
        err[dt] = ((z1 - z0).abs().mean() / upd.pow(2).mean().sqrt()).item()
    assert 1e-5 < err[torch.float16] < 3e-3, err
    assert 4 < err[torch.bfloat16] / err[torch.float16] < 16, err
