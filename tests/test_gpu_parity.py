"""GPU parity: every HIP path against the fp32 CPU oracle on identical seeded inputs.

Tolerance (bf16 compute vs fp32 reference), with
errors normalised by the RMS of the reference output:
    max |gpu - ref| <= 2e-2 * rms(ref)   and   mean |gpu - ref| <= 2e-3 * rms(ref).
Masked configurations report the valid region and the full tensor separately;
both must meet the bar.
"""
import math

import pytest
import torch

from oracle import pairformer_ref as ref
from tt_boltz_amd import ops, pairformer, synthetic

pytestmark = pytest.mark.gpu

MAX_TOL, MEAN_TOL = 2e-2, 2e-3


def stats(gpu_t, ref_t):
    g = gpu_t.detach().double().cpu()
    r = ref_t.detach().double().cpu()
    rms = r.pow(2).mean().sqrt().clamp_min(1e-12)
    d = (g - r).abs()
    return (d.max() / rms).item(), (d.mean() / rms).item()


def check(name, gpu_t, ref_t, max_tol=MAX_TOL, mean_tol=MEAN_TOL):
    mx, mn = stats(gpu_t, ref_t)
    print(f"[parity] {name}: max/rms={mx:.3e} mean/rms={mn:.3e}", flush=True)
    assert torch.isfinite(gpu_t).all(), f"{name}: non-finite output"
    assert mx <= max_tol and mn <= mean_tol, f"{name}: max/rms={mx:.3e} mean/rms={mn:.3e}"


def _sub_w(seed, prefix):
    return ref.sub(synthetic.draw({k: v for k, v in synthetic.layer_shapes().items()
                                   if k.startswith(prefix + ".")}, seed), prefix)


def _dev_w(w, dev, strip="", variant=ops.DEFAULT_VARIANT):
    return ops.convert_weights(w, dev, variant, strip)


def _inputs(N, seed, pad_tail=0, rand_mask=False):
    s, z, mask, pm = synthetic.pair_inputs(N, seed, pad_tail=pad_tail)
    if rand_mask:
        g = torch.Generator().manual_seed(seed + 100)
        pm = pm * (torch.rand(pm.shape, generator=g) > 0.15).float()
    return s, z, mask, pm


# ------------------------------------------------------------------------------ contraction
@pytest.mark.parametrize("variant", ["fp16", "bf16"])
@pytest.mark.parametrize("N", [64, 192, 256, 384, 448, 512, 640])
def test_contract_matches_fp32_matmul(gpu, N, variant):
    """The MFMA contraction on operand-type planes equals an fp32 matmul of the same
    (already rounded) values up to summation order; the scaled operand-type output is
    that result rounded once.  N < 448 runs the 128x128-tile kernel, N >= 448 the
    256x256-tile LDS-DMA kernel (448 and 640 end in partial edge tiles)."""
    g = torch.Generator().manual_seed(N)
    dt = ops.TORCH_DTYPE[variant]
    A = torch.randn((3, N, N), generator=g).to(dt)
    Bm = torch.randn((3, N, N), generator=g).to(dt)
    want = torch.bmm(A.float(), Bm.float().transpose(1, 2))
    X = torch.empty((3, N, N), dtype=torch.float32, device=gpu)
    ops.launch_trimul_contract(A.to(gpu), Bm.to(gpu), X, variant)
    mx, _ = stats(X, want)
    print(f"[parity] contract {variant} N={N}: max/rms={mx:.3e}", flush=True)
    assert mx < 1e-5
    Xh = torch.empty((3, N, N), dtype=dt, device=gpu)
    ops.launch_trimul_contract(A.to(gpu), Bm.to(gpu), Xh, variant)
    # one rounding of each element: |err| <= 2^-11 (fp16) / 2^-9 (bf16) of |x| (round to
    # nearest), checked elementwise with a 2x margin plus the fp32 summation-order slack
    got = Xh.float().cpu() * 256.0
    rel = 2 ** -10 if variant == "fp16" else 2 ** -8
    slack = 1e-5 * want.pow(2).mean().sqrt()
    assert bool(((got - want).abs() <= rel * want.abs() + slack).all())


def test_contract_768_full_chip(gpu):
    """128 planes at N = 768 (the north-star stack's contraction, edge-free 256x256 tiles
    over 4.5 rounds of the chip) against an fp32 matmul of the same operand-type values on
    the device (one rounding of the fp16 output)."""
    N = 768
    g = torch.Generator().manual_seed(768)
    A = torch.randn((128, N, N), generator=g).half().to(gpu)
    Bm = torch.randn((128, N, N), generator=g).half().to(gpu)
    want = torch.bmm(A.float(), Bm.float().transpose(1, 2).contiguous())
    X = torch.empty((128, N, N), dtype=torch.float16, device=gpu)
    ops.launch_trimul_contract(A, Bm, X, "fp16")
    got = X.float() * 256.0
    slack = 1e-5 * want.pow(2).mean().sqrt()
    bad = ((got - want).abs() > 2 ** -10 * want.abs() + slack).sum().item()
    print(f"[parity] contract N=768 x128: elements outside one rounding: {bad}", flush=True)
    assert bad == 0


# ------------------------------------------------------------------------------ triangle multiplication
@pytest.mark.parametrize("N,direction,rand_mask", [(64, "outgoing", False), (64, "incoming", True),
                                                   (192, "outgoing", True), (192, "incoming", False)])
def test_trimul_small(gpu, N, direction, rand_mask):
    prefix = "tri_mul_out" if direction == "outgoing" else "tri_mul_in"
    w = _sub_w(7, prefix)
    _, z, _, pm = _inputs(N, 11, pad_tail=N // 8, rand_mask=rand_mask)
    want = ref.triangle_multiplication(z, pm, w, direction)
    got = ops.triangle_multiplicative_update(z.to(gpu), direction, pm.to(gpu), **{
        "norm_in_weight": w["norm_in.weight"], "norm_in_bias": w["norm_in.bias"], "p_in_weight": w["p_in.weight"],
        "g_in_weight": w["g_in.weight"], "norm_out_weight": w["norm_out.weight"], "norm_out_bias": w["norm_out.bias"],
        "p_out_weight": w["p_out.weight"], "g_out_weight": w["g_out.weight"]})
    check(f"trimul {direction} N={N} rand_mask={rand_mask}", got, want)


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_trimul_config1(gpu, direction):
    """N=512, last 51 tokens padded, seed 1."""
    cfg = synthetic.CONFIGS[1]
    prefix = "tri_mul_out" if direction == "outgoing" else "tri_mul_in"
    w = _sub_w(cfg["seed"], prefix)
    _, z, _, pm = _inputs(cfg["N"], cfg["seed"], pad_tail=cfg["pad_tail"])
    want = ref.triangle_multiplication(z, pm, w, direction)
    zd = z.to(gpu)
    out = torch.empty_like(zd)
    ws = ops.workspace(ops.trimul_workspace_bytes(1, cfg["N"]), gpu)
    ops.launch_trimul(zd, out, pm.to(gpu).contiguous(), _dev_w(w, gpu), 0 if direction == "outgoing" else 1, ws,
                      accumulate=False)
    nv = cfg["N"] - cfg["pad_tail"]
    check(f"config1 trimul {direction} valid", out[:, :nv, :nv], want[:, :nv, :nv])
    check(f"config1 trimul {direction} full", out, want)


def test_trimul_inplace_accumulate(gpu):
    """In place (out aliases z_in) and into a separate buffer, accumulate=True equals the
    plain update added to z: up to the single rounding of a fused multiply-add (the kernel
    may form z + p*sigmoid(g) with one rounding), i.e. within a few ulps of |z| + |update|."""
    N = 128
    w = _dev_w(_sub_w(5, "tri_mul_out"), gpu)
    _, z, _, _ = _inputs(N, 12)
    zd = z.to(gpu)
    ws = ops.workspace(ops.trimul_workspace_bytes(1, N), gpu)
    upd = torch.empty_like(zd)
    ops.launch_trimul(zd, upd, None, w, 0, ws, accumulate=False)
    want = zd + upd
    ulp = 2.0 ** -23 * (zd.abs() + upd.abs())
    zi = zd.clone()
    ops.launch_trimul(zi, zi, None, w, 0, ws, accumulate=True)            # in place
    assert bool(((zi - want).abs() <= 4 * ulp).all())
    zo = zd.clone()
    zsrc = zd.clone()
    ops.launch_trimul(zsrc, zo, None, w, 0, ws, accumulate=True)          # out != z_in: out += update
    assert bool(((zo - want).abs() <= 4 * ulp).all())


# ------------------------------------------------------------------------------ triangle attention
@pytest.mark.parametrize("N,ending,rand_mask", [(64, False, False), (64, True, True), (192, False, True),
                                                (192, True, False)])
def test_triatt_small(gpu, N, ending, rand_mask):
    prefix = "tri_att_end" if ending else "tri_att_start"
    w = _sub_w(9, prefix)
    _, z, _, pm = _inputs(N, 13, pad_tail=N // 8, rand_mask=rand_mask)
    want = ref.triangle_attention(z, pm, w, not ending, None)
    zd = z.to(gpu)
    out = torch.empty_like(zd)
    ws = ops.workspace(ops.triatt_workspace_bytes(1, N), gpu)
    ops.launch_triatt(zd, out, pm.to(gpu).contiguous(), _dev_w(w, gpu, "mha."), ending, ws, accumulate=False)
    check(f"triatt ending={ending} N={N} rand_mask={rand_mask}", out, want)


@pytest.mark.parametrize("ending", [False, True])
def test_triatt_config2(gpu, ending):
    """N=512, last 51 tokens padded, seed 2; oracle unchunked fp32 (all 512
    rows in one attention call, evaluated on the device: [1, 512, 4, 512, 512] fp32 logits)."""
    cfg = synthetic.CONFIGS[2]
    prefix = "tri_att_end" if ending else "tri_att_start"
    w = _sub_w(cfg["seed"], prefix)
    _, z, _, pm = _inputs(cfg["N"], cfg["seed"], pad_tail=cfg["pad_tail"])
    with torch.no_grad():
        want = ref.triangle_attention(z.to(gpu), pm.to(gpu), {k: v.to(gpu) for k, v in w.items()}, not ending,
                                      None).cpu()
    zd = z.to(gpu)
    out = torch.empty_like(zd)
    ws = ops.workspace(ops.triatt_workspace_bytes(1, cfg["N"]), gpu)
    ops.launch_triatt(zd, out, pm.to(gpu).contiguous(), _dev_w(w, gpu, "mha."), ending, ws, accumulate=False)
    nv = cfg["N"] - cfg["pad_tail"]
    check(f"config2 triatt ending={ending} valid", out[:, :nv, :nv], want[:, :nv, :nv])
    check(f"config2 triatt ending={ending} full", out, want)


@pytest.mark.parametrize("N", [64, 96, 100, 128, 192, 256])
def test_tri_attention_core(gpu, N):
    """N = 100 runs padded to 128 with n_valid = 100: the fully masked row's mean of v then
    leaves out the padded keys, and the padded rows take the same path.  N = 128 needs no
    padding, so the caller's bias and mask go to the kernel as they are.  These launches fill
    less than half of the chip, so their blocks run split over workgroups of 2 heads (N = 64:
    one 64-key step per head, 192, 256) or of 1 head (96, 100, 128)."""
    g = torch.Generator().manual_seed(3)
    B, H, D = 1, 4, 32
    q, k, v = (torch.randn((B, N, H, N, D), generator=g) for _ in range(3))
    bias = torch.randn((B, 1, H, N, N), generator=g)
    mask = (torch.rand((B, N, 1, 1, N), generator=g) > 0.2).float()
    mask[:, 5] = 0.0   # a fully masked row: uniform average of v
    want = ref.triangle_attention_core(q, k, v, bias, mask, D ** -0.5)
    got = ops.triangle_attention(q.to(gpu), k.to(gpu), v.to(gpu), bias.to(gpu), mask.to(gpu))
    check("tri_attention core", got, want)
    check("tri_attention core masked row", got[:, 5], v[:, 5].mean(dim=-2, keepdim=True).expand(B, H, N, D))


# ------------------------------------------------------------------------------ transition / APB
def test_transition_pair(gpu):
    w = _sub_w(4, "transition_z")
    _, z, _, _ = _inputs(64, 14)
    want = ref.transition(z, w)
    got = ops.transition(z.to(gpu), w["norm.weight"], w["norm.bias"], w["fc1.weight"], w["fc2.weight"],
                         w["fc3.weight"])
    check("transition z", got, want)


def test_transition_single(gpu):
    w = _sub_w(4, "transition_s")
    s, _, _, _ = _inputs(100, 15)
    want = ref.transition(s, w)
    got = ops.transition(s.to(gpu), w["norm.weight"], w["norm.bias"], w["fc1.weight"], w["fc2.weight"],
                         w["fc3.weight"])
    check("transition s", got, want)


@pytest.mark.parametrize("N", [100, 128])
def test_attention_pair_bias(gpu, N):
    """N = 100 is padded to 128 inside the wrapper; N = 128 goes to the kernels as given."""
    w = _sub_w(6, "attention")
    s, z, mask, _ = _inputs(N, 16, pad_tail=7)
    want = ref.attention_pair_bias(s, z, mask, s, w, 16)
    got = ops.attention_pair_bias(s.to(gpu), z.to(gpu), mask.to(gpu), s.to(gpu), w, 16)
    check(f"attention_pair_bias N={N}", got[:, :N - 7], want[:, :N - 7])


# ------------------------------------------------------------------------------ layer / module
def test_layer_config0(gpu):
    """one full PairformerLayer, N=128, seed 0, masks all ones."""
    cfg = synthetic.CONFIGS[0]
    w = synthetic.stack_weights(1, cfg["seed"])
    s, z, mask, pm = _inputs(cfg["N"], cfg["seed"])
    s_ref, z_ref = ref.pairformer_stack(s, z, mask, pm, w, 1)
    mod = pairformer.PairformerModule(1, 32, 4, 24, 16, True)
    mod.load_state_dict(w)
    s_got, z_got = mod(s.to(gpu), z.to(gpu), mask.to(gpu), pm.to(gpu))
    check("config0 layer z", z_got, z_ref)
    check("config0 layer s", s_got, s_ref)


def test_layer_config0_bf16_operands(gpu):
    """Same layer with the bf16-operand library.  bf16 keeps 8 significant bits, so each
    MFMA operand rounding costs ~2^-9 relative; its bar is the looser
    max 5e-2 / mean 6e-3 of the rms (measured ~2.2e-2 / 3.0e-3)."""
    cfg = synthetic.CONFIGS[0]
    w = synthetic.stack_weights(1, cfg["seed"])
    s, z, mask, pm = _inputs(cfg["N"], cfg["seed"])
    s_ref, z_ref = ref.pairformer_stack(s, z, mask, pm, w, 1)
    mod = pairformer.PairformerModule(1, 32, 4, 24, 16, True, options=pairformer.Options(operand="bf16"))
    mod.load_state_dict(w)
    s_got, z_got = mod(s.to(gpu), z.to(gpu), mask.to(gpu), pm.to(gpu))
    check("config0 layer z (bf16 operands)", z_got, z_ref, 5e-2, 6e-3)
    check("config0 layer s (bf16 operands)", s_got, s_ref, 5e-2, 6e-3)


def test_module_dropin_padding(gpu):
    """Drop-in on CPU tensors (like the reference's tests/test_tenstorrent.py:31-43):
    2 blocks, N=100 (padded to 128 inside), outputs returned on the CPU."""
    w = synthetic.stack_weights(2, 21)
    s, z, mask, pm = _inputs(100, 22)
    s_ref, z_ref = ref.pairformer_stack(s, z, mask, pm, w, 2)
    mod = pairformer.PairformerModule(2, 32, 4, 24, 16, True)
    mod.load_state_dict(w)
    s_got, z_got = mod(s, z)
    assert s_got.device.type == "cpu" and z_got.shape == z.shape and s_got.shape == s.shape
    check("module N=100 z", z_got, z_ref)
    check("module N=100 s", s_got, s_ref)


def test_module_noseq_affinity_masks(gpu):
    """No-seq stack with a permuted half-masked token set (cf. tests/test_tenstorrent.py:55-66)."""
    N = 96
    w = synthetic.stack_weights(2, 23, transform_s=False)
    _, z, _, _ = _inputs(N, 24)
    g = torch.Generator().manual_seed(25)
    m = torch.ones((1, N)); m[0, : N // 2] = 0
    m = m[:, torch.randperm(N, generator=g)]
    pm = m[:, :, None] * m[:, None, :]
    _, z_ref = ref.pairformer_stack(None, z, None, pm, w, 2)
    mod = pairformer.PairformerModule(2, 32, 4, None, None, False, affinity=True)
    mod.load_state_dict(w)
    _, z_got = mod(None, z.to(gpu), pair_mask=pm.to(gpu))
    check("module no-seq affinity z", z_got, z_ref)


def test_module_out_of_memory_raises(gpu):
    """A request beyond the device's memory surfaces as a RuntimeError containing "out of
    memory", the text boltz2.py:5584-5591 catches to skip a batch.  z is a stride-0 view of a
    512 GiB pair tensor (512 real bytes), so the module's padded device copy cannot be
    allocated and nothing runs; the module works normally afterwards."""
    w = synthetic.stack_weights(1, 26, transform_s=False)
    mod = pairformer.PairformerModule(1, 32, 4, None, None, False)
    mod.load_state_dict(w)
    N = 32768
    huge = torch.zeros((1, 1, 1, 128), device=gpu).expand(1, N, N, 128)
    with pytest.raises(RuntimeError, match="out of memory"):
        mod(None, huge)
    del huge
    torch.cuda.empty_cache()
    _, z, _, pm = _inputs(64, 27)
    _, z_ref = ref.pairformer_stack(None, z, None, pm, w, 1)
    mod.reset_static_cache()
    _, z_got = mod(None, z.to(gpu))
    check("module after an out-of-memory error z", z_got, z_ref)


def test_recycler(gpu):
    N = 64
    w = synthetic.stack_weights(1, 26)
    w_rec = synthetic.draw(synthetic.recycle_shapes(), 27)
    s_init, z_init, mask, _ = _inputs(N, 28)
    s_ref, z_ref = ref.recycle(s_init, z_init, mask, w, w_rec, 1, 1)
    pf = pairformer.Pairformer(1, 32, 4, 24, 16, True, w)
    rec = pairformer.TrunkRecycler(pf, w_rec)
    s_got, z_got = rec(s_init.to(gpu), z_init.to(gpu), mask.to(gpu), 1)
    check("recycler z", z_got, z_ref)
    check("recycler s", s_got, s_ref)


def test_recycler_msa(gpu):
    """Recycling loop with the MSA hand-off on the device (z = z + MSA(z) before the stack,
    boltz2.py:5203-5245): 2 passes, 1 MSA block, 1 Pairformer block, N = 64, 24 MSA rows."""
    from tt_boltz_amd import msa as msa_mod
    N, S = 64, 24
    w = synthetic.stack_weights(1, 29)
    w_rec = synthetic.draw(synthetic.recycle_shapes(), 30)
    w_msa = synthetic.draw(synthetic.msa_module_shapes(1), 31)
    s_init, z_init, mask, _ = _inputs(N, 32)
    emb = torch.randn((1, N, 384), generator=torch.Generator().manual_seed(33))
    feats = _msa_feats(S, N, 34)
    feats["token_pad_mask"] = mask
    feats["msa_mask"] = feats["msa_mask"] * mask[:, None, :]
    s_ref, z_ref = ref.recycle(s_init, z_init, mask, w, w_rec, 1, 1, msa=(w_msa, emb, feats, 1))
    pf = pairformer.Pairformer(1, 32, 4, 24, 16, True, w)
    msa_dev = msa_mod.MSA(1, 32, 8, 32, 4, w_msa)
    rec = pairformer.TrunkRecycler(pf, w_rec, msa=msa_dev)
    inputs = msa_mod.device_inputs(emb, feats, N, gpu)
    s_got, z_got = rec(s_init.to(gpu), z_init.to(gpu), mask.to(gpu), 1, msa_inputs=inputs)
    check("recycler+MSA z", z_got, z_ref)
    check("recycler+MSA s", s_got, s_ref)


def test_single_track_overlap_identical(gpu):
    """The single track on a second stream (overlapped with the next layer's pair
    operations, started after 0, 1, 2 or 4 of them) gives bit-identical s and z to the same
    stack run in reference order on one stream: same kernels, same inputs, only the schedule
    differs."""
    N, n_blocks = 128, 3
    w = synthetic.stack_weights(n_blocks, 31)
    s, z, mask, pm = _inputs(N, 32)
    out = {}
    for key, opts in (("serial", pairformer.Options(overlap_single=False)),
                      *((d, pairformer.Options(single_delay=d)) for d in (0, 1, 2, 4))):
        pf = pairformer.Pairformer(n_blocks, 32, 4, 24, 16, True, w, options=opts)
        s_d, z_d = s.to(gpu).contiguous(), z.to(gpu).contiguous()
        out[key] = pf(s_d, z_d, pm.to(gpu), mask.to(gpu))
        torch.cuda.synchronize()
    for d in (0, 1, 2, 4):
        assert torch.equal(out[d][0], out["serial"][0]) and torch.equal(out[d][1], out["serial"][1]), d
    s_ref, z_ref = ref.pairformer_stack(s, z, mask, pm, w, n_blocks)
    check("overlapped 3-layer stack z", out[1][1], z_ref)
    check("overlapped 3-layer stack s", out[1][0], s_ref)


def test_transition_fused_pair_bias(gpu):
    """pf_transition_pair_bias_fwd: z is bit-identical to pf_transition_fwd, and the pair
    bias it writes matches pf_apb_pair_bias on that z (same formula, different summation
    order and LayerNorm lane layout) and the fp32 oracle's proj_z."""
    N, c_s, H = 96, 384, 16
    w_tr = _sub_w(41, "transition_z")
    w_apb = _sub_w(42, "attention")
    s, z, mask, _ = _inputs(N, 43)
    tr = pairformer.Transition(w_tr)
    apb = pairformer.AttentionPairBias(24, H, w_apb)
    z1, z2 = z.to(gpu).contiguous(), z.to(gpu).contiguous()
    s_d = s.to(gpu).contiguous()
    nb = apb.workspace_bytes(1, N)
    ws1, ws2 = ops.workspace(nb, gpu), ops.workspace(nb, gpu)
    tr(z1, out=z1, accumulate=True)
    apb(s_d, z1, None, out=s_d.clone(), ws=ws1, part="bias")
    tr(z2, out=z2, accumulate=True, pair_bias=(apb, s_d, ws2))
    torch.cuda.synchronize()
    assert torch.equal(z1, z2)
    off = 5 * N * c_s * 4
    b1 = ws1[off: off + H * N * N * 4].view(torch.float32).view(H, N, N)
    b2 = ws2[off: off + H * N * N * 4].view(torch.float32).view(H, N, N)
    check("fused pair bias vs pf_apb_pair_bias", b2, b1, 1e-2, 1e-3)
    zn = torch.nn.functional.layer_norm(z2.cpu().double()[0], (128,), w_apb["proj_z.0.weight"].double(),
                                        w_apb["proj_z.0.bias"].double(), 1e-5)
    want = torch.einsum("ijc,hc->hij", zn, w_apb["proj_z.1.weight"].double()) * math.log2(math.e)
    check("fused pair bias vs fp64 proj_z", b2, want)


def test_layer_batch2_matches_single(gpu):
    """B = 2 through the whole layer (every kernel's batch indexing: trimul planes,
    attention rows/bias, transitions, the single track) equals the two proteins run one at
    a time, bit for bit, and the fp32 oracle on the batch.  The mean correction of the
    16-bit input-side weights is a single-protein (B = 1) feature, so the bit-for-bit part
    runs without it; with the default options a batch (exact beta offsets, no correction) is
    checked against the oracle as well."""
    N = 64
    w = synthetic.stack_weights(1, 51)
    s0, z0, m0, pm0 = _inputs(N, 52)
    s1, z1, m1, pm1 = _inputs(N, 53, pad_tail=9)
    S, Z, M, PM = (torch.cat(t, 0) for t in ((s0, s1), (z0, z1), (m0, m1), (pm0, pm1)))
    pf = pairformer.Pairformer(1, 32, 4, 24, 16, True, w, pairformer.Options(mean_correction=False))
    s_b, z_b = pf(S.to(gpu).contiguous(), Z.to(gpu).contiguous(), PM.to(gpu).contiguous(), M.to(gpu).contiguous())
    pf_default = pairformer.Pairformer(1, 32, 4, 24, 16, True, w)
    s_d, z_d = pf_default(S.to(gpu).contiguous(), Z.to(gpu).contiguous(), PM.to(gpu).contiguous(),
                          M.to(gpu).contiguous())
    check("batch-2 layer z, default options", z_d, ref.pairformer_stack(S, Z, M, PM, w, 1)[1])
    for i, (s, z, m, pm) in enumerate(((s0, z0, m0, pm0), (s1, z1, m1, pm1))):
        s_1, z_1 = pf(s.to(gpu).contiguous(), z.to(gpu).contiguous(), pm.to(gpu).contiguous(),
                      m.to(gpu).contiguous())
        assert torch.equal(s_b[i:i + 1], s_1) and torch.equal(z_b[i:i + 1], z_1), f"batch element {i} differs"
    s_ref, z_ref = ref.pairformer_stack(S, Z, M, PM, w, 1)
    check("batch-2 layer z", z_b, z_ref)
    check("batch-2 layer s", s_b, s_ref)


@pytest.mark.parametrize("P,M,Nc,K", [(3, 96, 320, 192), (2, 512, 256, 1024), (1, 288, 800, 64),
                                     (70, 320, 512, 128)])
def test_batched_nt_gemm(gpu, P, M, Nc, K):
    """Rectangular form of the contraction kernel (partial 256-tiles in both dimensions):
    fp32 output equals an fp32 product of the same rounded operands up to summation order;
    the operand-type output is that result (times scale) rounded once.  70 x 320 x 512 has
    280 tiles: on 256 CUs the last 24 run as 128-row halves, one of each pair partly and one
    wholly past M."""
    g = torch.Generator().manual_seed(M + Nc + K)
    A = torch.randn((P, M, K), generator=g).half()
    Bm = torch.randn((P, Nc, K), generator=g).half()
    want = torch.bmm(A.float(), Bm.float().transpose(1, 2).contiguous())
    X = torch.empty((P, M, Nc), dtype=torch.float32, device=gpu)
    ops.launch_batched_nt_gemm(A.to(gpu), Bm.to(gpu), X)
    mx, _ = stats(X, want)
    assert mx < 1e-5, mx
    Xh = torch.empty((P, M, Nc), dtype=torch.float16, device=gpu)
    ops.launch_batched_nt_gemm(A.to(gpu), Bm.to(gpu), Xh, 0.25)
    err = (Xh.float().cpu() - 0.25 * want).abs()
    assert (err <= 2 ** -10 * (0.25 * want).abs() + 1e-3).all()


# ------------------------------------------------------------------------------ MSA module
from oracle import msa_ref  # noqa: E402


def _msa_sub(seed, prefix, c_m=64, c_z=128):
    shapes = synthetic.msa_layer_shapes(c_m, c_z)
    return ref.sub(synthetic.draw({k: v for k, v in shapes.items() if k.startswith(prefix + ".")}, seed), prefix)


def test_transition_msa(gpu):
    """C = 64 / hidden = 256 (the MSA transition's persistent fused kernel): a row count that
    is not a multiple of the 32-row tile, then in place with accumulate (m += Tr(m))."""
    w = _msa_sub(72, "msa_transition")
    g = torch.Generator().manual_seed(72)
    m = torch.randn((3, 37, 41, 64), generator=g)
    want = ref.transition(m, w)
    got = ops.transition(m.to(gpu), w["norm.weight"], w["norm.bias"], w["fc1.weight"], w["fc2.weight"],
                         w["fc3.weight"])
    check("transition msa", got, want)
    wd = ops.convert_weights(w, gpu)
    x = m.to(gpu).contiguous()
    assert ops.transition_workspace_bytes(x.numel() // 64, 64, 256) == 0
    ops.launch_transition(x, x, wd, None, accumulate=True)
    check("transition msa in place", x, m + want)


@pytest.mark.parametrize("S,N", [(40, 64), (130, 96)])
def test_outer_product_mean(gpu, S, N):
    """pf_opm_fwd vs the fp32 oracle: S padded to 64 inside, random sequence mask (with a
    fully masked sequence and tokens missing from some sequences), z += update."""
    w = _msa_sub(71, "outer_product_mean")
    g = torch.Generator().manual_seed(S + N)
    m = torch.randn((1, S, N, 64), generator=g)
    mask = (torch.rand((1, S, N), generator=g) > 0.2).float()
    mask[:, 3] = 0.0
    z = torch.randn((1, N, N, 128), generator=g)
    want = z + msa_ref.outer_product_mean(m, mask, w)
    zd = z.to(gpu).contiguous()
    wd = _dev_w(w, gpu)
    ws = ops.workspace(ops.opm_workspace_bytes(1, S, N), gpu)
    ops.launch_opm(m.to(gpu).contiguous(), mask.to(gpu).contiguous(), zd, wd, ws)
    check(f"outer product mean S={S} N={N}", zd, want)


@pytest.mark.parametrize("S,N", [(40, 64), (33, 128)])
def test_pair_weighted_averaging(gpu, S, N):
    """pf_pwa_fwd vs the fp32 oracle, m += update in place, a padded token tail (its row of
    weights is fully masked: compared on the valid tokens, where the reference's fp32
    rounding of logit - 1e6 does not enter)."""
    w = _msa_sub(72, "pair_weighted_averaging")
    g = torch.Generator().manual_seed(S * N)
    m = torch.randn((1, S, N, 64), generator=g)
    z = torch.randn((1, N, N, 128), generator=g)
    tok = torch.ones((1, N)); tok[:, N - 7:] = 0
    pm = tok[:, :, None] * tok[:, None, :]
    want = m + msa_ref.pair_weighted_averaging(m, z, pm, w)
    md = m.to(gpu).contiguous()
    wd = _dev_w(w, gpu)
    ws = ops.workspace(ops.pwa_workspace_bytes(1, S, N), gpu)
    ops.launch_pwa(md, z.to(gpu).contiguous(), pm.to(gpu).contiguous(), md, wd, ws)
    check(f"pair weighted averaging S={S} N={N} (valid tokens)", md[:, :, : N - 7], want[:, :, : N - 7])


def _msa_feats(S, N, seed, pad_tail=0):
    g = torch.Generator().manual_seed(seed)
    tok = torch.ones((1, N))
    if pad_tail:
        tok[:, N - pad_tail:] = 0
    return {"msa": torch.randint(0, msa_ref.NUM_TOKENS, (1, S, N), generator=g),
            "has_deletion": (torch.rand((1, S, N), generator=g) > 0.8).float(),
            "deletion_value": torch.rand((1, S, N), generator=g),
            "msa_paired": (torch.rand((1, S, N), generator=g) > 0.5).float(),
            "msa_mask": (torch.rand((1, S, N), generator=g) > 0.1).float() * tok[:, None, :],
            "token_pad_mask": tok}


def test_msa_module_dropin(gpu):
    """MSAModule drop-in (2 blocks) on CPU tensors: N = 50 padded to 64 inside, 20 MSA rows,
    a masked token tail and random sequence masks, vs the fp32 oracle (valid tokens)."""
    from tt_boltz_amd import msa as msa_mod
    N, S, nb = 50, 20, 2
    w = synthetic.draw(synthetic.msa_module_shapes(nb), 81)
    g = torch.Generator().manual_seed(82)
    z = torch.randn((1, N, N, 128), generator=g)
    emb = torch.randn((1, N, 384), generator=g)
    feats = _msa_feats(S, N, 83, pad_tail=6)
    want = msa_ref.msa_module(z, emb, feats, w, nb)
    mod = msa_mod.MSAModule(nb, 32, 8, 32, 4)
    mod.load_state_dict(w)
    got = mod(z, emb, feats)
    assert got.device.type == "cpu" and got.shape == z.shape
    v = N - 6
    check("MSA module 2 blocks (valid tokens)", got[:, :v, :v], want[:, :v, :v])


# ------------------------------------------------------------------------------ diffusion conditioning (pair side)
from oracle import diffusion_ref  # noqa: E402


@pytest.mark.parametrize("shape,depth,heads", [((1, 64, 64), 24, 16), ((1, 37, 41), 2, 16), ((2, 32, 32), 4, 8)])
def test_token_pair_bias(gpu, shape, depth, heads):
    """pf_token_pair_bias_fwd (LN statistics once, each layer's affine folded into its
    weights) vs the oracle's per-layer LayerNorm + Linear, both layouts; a row count that is
    not a multiple of the 32-pair tile; the attention's log2(e) scale."""
    from tt_boltz_amd import diffusion
    w = synthetic.draw(synthetic.diffusion_pair_shapes(depth=depth, heads=heads, n_transitions=0), 95)
    g = torch.Generator().manual_seed(96)
    z = torch.randn((*shape, 128), generator=g) * 2 + 0.5
    want = diffusion_ref.token_trans_bias(z, w, depth)
    mod = diffusion.TokenTransformerPairBias(depth, w)
    zd = z.to(gpu).contiguous()
    check(f"token pair bias {shape} L={depth} H={heads} layout 0", mod(zd), want)
    got1 = mod(zd, layout=1, scale=math.log2(math.e))
    check(f"token pair bias {shape} layout 1", got1, want.permute(3, 0, 1, 2) * math.log2(math.e))


def test_pairwise_conditioning(gpu):
    from tt_boltz_amd import diffusion
    w = ref.sub(synthetic.draw(synthetic.diffusion_pair_shapes(depth=1), 97), "pairwise_conditioner")
    g = torch.Generator().manual_seed(98)
    zt = torch.randn((1, 64, 64, 128), generator=g)
    rp = torch.randn((1, 64, 64, 128), generator=g) * 0.5
    want = diffusion_ref.pairwise_conditioning(zt, rp, w)
    got = diffusion.PairwiseConditioning(w)(zt.to(gpu).contiguous(), rp.to(gpu).contiguous())
    check("pairwise conditioning", got, want)


def test_diffusion_pair_conditioning_dropin(gpu):
    """The drop-in module on CPU tensors (N = 50, no padding needed): (z, token_trans_bias)."""
    from tt_boltz_amd import diffusion
    w = synthetic.draw(synthetic.diffusion_pair_shapes(depth=24, heads=16), 99)
    g = torch.Generator().manual_seed(100)
    zt = torch.randn((1, 50, 50, 128), generator=g)
    rp = torch.randn((1, 50, 50, 128), generator=g)
    z_want = diffusion_ref.pairwise_conditioning(zt, rp, ref.sub(w, "pairwise_conditioner"))
    b_want = diffusion_ref.token_trans_bias(z_want, w, 24)
    mod = diffusion.DiffusionPairConditioning(24)
    mod.load_state_dict(w)
    z_got, b_got = mod(zt, rp)
    assert z_got.device.type == "cpu" and b_got.shape == (1, 50, 50, 384)
    check("diffusion conditioning z", z_got, z_want)
    check("diffusion conditioning token bias", b_got, b_want)


# ------------------------------------------------------------------------------ template stack (c_z = 64)
def _sub_w64(seed, prefix):
    return ref.sub(synthetic.draw({k: v for k, v in synthetic.layer_shapes(c_z=64, transform_s=False).items()
                                   if k.startswith(prefix + ".")}, seed), prefix)


@pytest.mark.parametrize("N,direction", [(64, "outgoing"), (128, "incoming"), (448, "outgoing")])
def test_trimul_c64(gpu, N, direction):
    """c_z = 64 (the template stack's pair width): the same kernels built for 64 channels;
    random pair mask with a padded tail; N = 448 takes the 256x256-tile contraction."""
    prefix = "tri_mul_out" if direction == "outgoing" else "tri_mul_in"
    w = _sub_w64(40 + N, prefix)
    _, z, _, pm = synthetic.pair_inputs(N, 41 + N, c_z=64, pad_tail=N // 8, with_s=False)
    pm = pm * (torch.rand(pm.shape, generator=torch.Generator().manual_seed(N)) > 0.15).float()
    want = ref.triangle_multiplication(z, pm, w, direction)
    mod = pairformer.TriangleMultiplication(direction == "incoming", w)
    got = mod(z.to(gpu).contiguous(), pm.to(gpu).contiguous())
    check(f"trimul c_z=64 {direction} N={N}", got, want)


@pytest.mark.parametrize("N,ending", [(64, False), (128, True)])
def test_triatt_c64(gpu, N, ending):
    prefix = "tri_att_end" if ending else "tri_att_start"
    w = _sub_w64(42 + N, prefix)
    _, z, _, pm = synthetic.pair_inputs(N, 43 + N, c_z=64, pad_tail=N // 8, with_s=False)
    want = ref.triangle_attention(z, pm, w, not ending, None)
    mod = pairformer.TriangleAttention(32, 4, ending, {k[4:] if k.startswith("mha.") else k: v for k, v in w.items()})
    got = mod(z.to(gpu).contiguous(), pm.to(gpu).contiguous())
    check(f"triatt c_z=64 ending={ending} N={N}", got, want)


def test_template_pairformer_module(gpu):
    """The template stack's Pairformer (tenstorrent.PairformerModule(2, 32, 4, None, None, False)
    on c_z = 64 weights, boltz2.py:3748-3761): N = 50 padded to 64 inside, masked tail."""
    N = 50
    w = synthetic.stack_weights(2, 44, c_z=64, transform_s=False)
    _, z, _, _ = synthetic.pair_inputs(N, 45, c_z=64, with_s=False)
    m = torch.ones((1, N)); m[0, 44:] = 0
    pm = m[:, :, None] * m[:, None, :]
    _, z_ref = ref.pairformer_stack(None, z, None, pm, w, 2)
    mod = pairformer.PairformerModule(2, 32, 4, None, None, False)
    mod.load_state_dict(w)
    _, z_got = mod(None, z, pair_mask=pm)
    check("template pairformer (c_z=64) valid", z_got[:, :44, :44], z_ref[:, :44, :44])
    check("template pairformer (c_z=64) full", z_got, z_ref)


def test_confidence_config_stack(gpu):
    """The confidence module's stack (tenstorrent.PairformerModule(8, 32, 4, 24, 16, True),
    boltz2.py:4502-4510): 8 layers with the single track, N = 64, masked tail."""
    N = 64
    w = synthetic.stack_weights(8, 46)
    s, z, mask, pm = _inputs(N, 47, pad_tail=7)
    s_ref, z_ref = ref.pairformer_stack(s, z, mask, pm, w, 8)
    pf = pairformer.Pairformer(8, 32, 4, 24, 16, True, w)
    s_got, z_got = pf(s.to(gpu).contiguous(), z.to(gpu).contiguous(), pm.to(gpu).contiguous(), mask.to(gpu),
                      n_valid=N - 7)
    nv = N - 7
    check("confidence 8-layer stack z (valid)", z_got[:, :nv, :nv], z_ref[:, :nv, :nv])
    check("confidence 8-layer stack s (valid)", s_got[:, :nv], s_ref[:, :nv])


def test_msa_module_batch2(gpu):
    """Two structures in one batch (B = 2, different masks and MSA depths' padding) through
    the device MSA stack, each compared with the oracle run on its own."""
    from tt_boltz_amd import msa as msa_mod
    N, S = 64, 24
    w = synthetic.draw(synthetic.msa_module_shapes(1), 84)
    g = torch.Generator().manual_seed(85)
    z = torch.randn((2, N, N, 128), generator=g)
    emb = torch.randn((2, N, 384), generator=g)
    f0, f1 = _msa_feats(S, N, 86, pad_tail=5), _msa_feats(S, N, 87)
    f1["msa_mask"][:, S - 6:] = 0.0   # the second structure has fewer sequences
    feats = {k: torch.cat([f0[k], f1[k]]) for k in f0}
    want = torch.cat([msa_ref.msa_module(z[i:i + 1], emb[i:i + 1], f, w, 1) for i, f in enumerate((f0, f1))])
    mod = msa_mod.MSAModule(1, 32, 8, 32, 4)
    mod.load_state_dict(w)
    got = mod(z, emb, feats)
    check("MSA module B=2 (structure 0, valid)", got[0, :N - 5, :N - 5], want[0, :N - 5, :N - 5])
    check("MSA module B=2 (structure 1)", got[1], want[1])


def test_template_stack_batch(gpu):
    """c_z = 64 stack on a batch of 3 templates (the template module's batch axis), each
    against the oracle on its own."""
    N = 64
    w = synthetic.stack_weights(1, 48, c_z=64, transform_s=False)
    z = torch.randn((3, N, N, 64), generator=torch.Generator().manual_seed(49))
    pm = torch.ones((1, N, N))
    want = torch.cat([ref.pairformer_stack(None, z[i:i + 1], None, pm, w, 1)[1] for i in range(3)])
    pf = pairformer.Pairformer(1, 32, 4, None, None, False, w)
    _, got = pf(None, z.to(gpu).contiguous(), None, None)
    check("template stack batch of 3", got, want)


def test_msa_ops_deep_msa(gpu):
    """A deep MSA (S = 4096 sequences, N = 256): the outer product mean (K = 4096 in its
    contraction, mask counts up to 4096) and the pair weighted averaging against the fp32
    oracle evaluated on the GPU (the same torch code, fp32 on the device for speed)."""
    S, N = 4096, 256
    g = torch.Generator().manual_seed(88)
    m = torch.randn((1, S, N, 64), generator=g).to(gpu)
    mask = (torch.rand((1, S, N), generator=g) > 0.3).float().to(gpu)
    z = torch.randn((1, N, N, 128), generator=g).to(gpu)
    w_o = {k: v.to(gpu) for k, v in _msa_sub(73, "outer_product_mean").items()}
    want = z + msa_ref.outer_product_mean(m, mask, w_o)
    zd = z.clone()
    ws = ops.workspace(ops.opm_workspace_bytes(1, S, N), gpu)
    ops.launch_opm(m.contiguous(), mask.contiguous(), zd, _dev_w(w_o, gpu), ws)
    check(f"outer product mean S={S} N={N}", zd, want)
    del ws, want, zd
    w_p = {k: v.to(gpu) for k, v in _msa_sub(74, "pair_weighted_averaging").items()}
    pm = torch.ones((1, N, N), device=gpu)
    want = m + msa_ref.pair_weighted_averaging(m, z, pm, w_p)
    md = m.clone()
    ws = ops.workspace(ops.pwa_workspace_bytes(1, S, N), gpu)
    ops.launch_pwa(md, z, pm, md, _dev_w(w_p, gpu), ws)
    check(f"pair weighted averaging S={S} N={N}", md, want)


@pytest.mark.parametrize("ending", [False, True])
def test_triatt_n1024(gpu, ending):
    """N = 1024 (the flash kernel never materialises the N^3 logits), padded tail of 100
    tokens, against the fp32 oracle evaluated on the device in row chunks of 64."""
    N, pad = 1024, 100
    prefix = "tri_att_end" if ending else "tri_att_start"
    w = _sub_w(60, prefix)
    _, z, _, pm = _inputs(N, 61, pad_tail=pad)
    zd, pmd = z.to(gpu).contiguous(), pm.to(gpu).contiguous()
    want = ref.triangle_attention(zd, pmd, {k: v.to(gpu) for k, v in w.items()}, not ending, 64)
    out = torch.empty_like(zd)
    ws = ops.workspace(ops.triatt_workspace_bytes(1, N), gpu)
    ops.launch_triatt(zd, out, pmd, _dev_w(w, gpu, "mha."), ending, ws, accumulate=False)
    nv = N - pad
    check(f"triatt N=1024 ending={ending} valid", out[:, :nv, :nv], want[:, :nv, :nv])
    check(f"triatt N=1024 ending={ending} full", out, want)


@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_trimul_n1024(gpu, direction):
    """16-bit triangle multiplication at N = 1024 (contraction past the ridge point), random
    pair mask with a padded tail, against the fp32 oracle evaluated on the device."""
    N = 1024
    prefix = "tri_mul_out" if direction == "outgoing" else "tri_mul_in"
    w = _sub_w(62, prefix)
    _, z, _, pm = _inputs(N, 63, pad_tail=80, rand_mask=True)
    zd, pmd = z.to(gpu).contiguous(), pm.to(gpu).contiguous()
    want = ref.triangle_multiplication(zd, pmd, {k: v.to(gpu) for k, v in w.items()}, direction)
    out = torch.empty_like(zd)
    ws = ops.workspace(ops.trimul_workspace_bytes(1, N), gpu)
    ops.launch_trimul(zd, out, pmd, _dev_w(w, gpu), 0 if direction == "outgoing" else 1, ws, accumulate=False)
    check(f"trimul N=1024 {direction}", out, want)


def test_layer_n768(gpu):
    """One full PairformerLayer (pair and single tracks) at the north-star size N = 768
    against the fp32 oracle evaluated on the device (z ~ 0.5 N(0,1) as in the stack config)."""
    N = 768
    w = synthetic.stack_weights(1, 64)
    s, z, mask, pm = synthetic.pair_inputs(N, 65, z_scale=0.5)
    wd = {k: v.to(gpu) for k, v in ref.sub(w, "layers.0").items()}
    s_ref, z_ref = ref.pairformer_layer(s.to(gpu), z.to(gpu), mask.to(gpu), pm.to(gpu), wd, ref.chunk_size_for(N))
    pf = pairformer.Pairformer(1, 32, 4, 24, 16, True, w)
    s_got, z_got = pf(s.to(gpu).contiguous(), z.to(gpu).contiguous(), pm.to(gpu).contiguous(), mask.to(gpu))
    check("layer N=768 z", z_got, z_ref)
    check("layer N=768 s", s_got, s_ref)


def test_layer_n2048_padded(gpu):
    """The largest size tested: one full PairformerLayer at N = 2048 (z 2 GB fp32, the
    triangle attention's q/k/v/o 4 GB), the last 37 tokens masked, against the fp32 oracle
    evaluated on the device (attention in row chunks): byte offsets past 2^31 in the
    attention's workspace, and the fully masked rows' path at this size."""
    N, pad = 2048, 37
    w = synthetic.stack_weights(1, 66)
    s, z, mask, pm = synthetic.pair_inputs(N, 67, z_scale=0.5, pad_tail=pad)
    wd = {k: v.to(gpu) for k, v in ref.sub(w, "layers.0").items()}
    with torch.no_grad():
        s_ref, z_ref = ref.pairformer_layer(s.to(gpu), z.to(gpu), mask.to(gpu), pm.to(gpu), wd, 64)
    torch.cuda.empty_cache()
    pf = pairformer.Pairformer(1, 32, 4, 24, 16, True, w)
    s_got, z_got = pf(s.to(gpu).contiguous(), z.to(gpu).contiguous(), pm.to(gpu).contiguous(), mask.to(gpu))
    nv = N - pad
    check("layer N=2048 z (valid)", z_got[:, :nv, :nv], z_ref[:, :nv, :nv])
    check("layer N=2048 z", z_got, z_ref)
    check("layer N=2048 s", s_got, s_ref)


def test_layer_config1_bf16_operands(gpu):
    """The bf16-operand library (the metric's dtype) on one full PairformerLayer at the
    config 1/2 shape: N = 512 with the last 51 tokens masked, against the fp32 oracle evaluated
    on the device.  Bar as for config 0 with bf16 operands: max 5e-2 / mean 6e-3 of the rms."""
    cfg = synthetic.CONFIGS[1]
    N = cfg["N"]
    w = synthetic.stack_weights(1, cfg["seed"])
    s, z, mask, pm = synthetic.pair_inputs(N, cfg["seed"], pad_tail=cfg["pad_tail"])
    wd = {k: v.to(gpu) for k, v in ref.sub(w, "layers.0").items()}
    s_ref, z_ref = ref.pairformer_layer(s.to(gpu), z.to(gpu), mask.to(gpu), pm.to(gpu), wd, ref.chunk_size_for(N))
    mod = pairformer.PairformerModule(1, 32, 4, 24, 16, True, options=pairformer.Options(operand="bf16"))
    mod.load_state_dict(w)
    s_got, z_got = mod(s.to(gpu), z.to(gpu), mask.to(gpu), pm.to(gpu))
    check("config1 layer z (bf16 operands, 51 masked tokens)", z_got, z_ref, 5e-2, 6e-3)
    check("config1 layer s (bf16 operands, 51 masked tokens)", s_got, s_ref, 5e-2, 6e-3)


# ------------------------------------------------------------------------------ boundary regressions
def test_module_mask_cache_tracks_n(gpu):
    """N = 100 and then N = 120 without reset_static_cache(): both pad to 128, so the cached
    masks must be keyed on N as well (the second call needs 120 valid tokens, not 100)."""
    w = synthetic.stack_weights(1, 110)
    mod = pairformer.PairformerModule(1, 32, 4, 24, 16, True)
    mod.load_state_dict(w)
    for N, seed in ((100, 111), (120, 112)):
        s, z, mask, pm = _inputs(N, seed)
        s_ref, z_ref = ref.pairformer_stack(s, z, mask, pm, w, 1)
        s_got, z_got = mod(s, z)
        check(f"module N={N} after N=100 (no reset) z", z_got, z_ref)
        check(f"module N={N} after N=100 (no reset) s", s_got, s_ref)


def test_padded_stack_without_mask(gpu):
    """A padded stack (n_valid < N) called without any mask must still exclude the padding
    from the contractions: Pairformer and TrunkRecycler build the valid-token pair mask."""
    N, nv = 128, 100
    w = synthetic.stack_weights(1, 113)
    w_rec = synthetic.draw(synthetic.recycle_shapes(), 114)
    s, z, mask, pm = _inputs(nv, 115)
    s_ref, z_ref = ref.pairformer_stack(s, z, mask, pm, w, 1)
    s_pad = torch.zeros((1, N, 384)); s_pad[:, :nv] = s
    z_pad = torch.zeros((1, N, N, 128)); z_pad[:, :nv, :nv] = z
    pf = pairformer.Pairformer(1, 32, 4, 24, 16, True, w)
    s_got, z_got = pf(s_pad.to(gpu), z_pad.to(gpu), None, None, n_valid=nv)
    check("stack n_valid=100 of 128, no mask: z", z_got[:, :nv, :nv], z_ref)
    check("stack n_valid=100 of 128, no mask: s", s_got[:, :nv], s_ref)
    s_ref, z_ref = ref.recycle(s, z, mask, w, w_rec, 1, 1)
    rec = pairformer.TrunkRecycler(pf, w_rec)
    s_got, z_got = rec(s_pad.to(gpu), z_pad.to(gpu), None, 1, n_valid=nv)
    check("recycler n_valid=100 of 128, no mask: z", z_got[:, :nv, :nv], z_ref)
    check("recycler n_valid=100 of 128, no mask: s", s_got[:, :nv], s_ref)


@pytest.mark.parametrize("scale", [1 / 64, 16.0])
@pytest.mark.parametrize("direction", ["outgoing", "incoming"])
def test_trimul_weight_scale_headroom(gpu, direction, scale):
    """The contraction planes X are 16-bit with a per-call power-of-two scale: p_in / g_in
    scaled by 1/64 (|X| ~ 1e-4, deep in fp16's subnormal range for a fixed 2^-8 scale) or
    by 16 (|X| ~ 1e3) must meet the same bar as the unit-scale weights."""
    N = 256
    prefix = "tri_mul_out" if direction == "outgoing" else "tri_mul_in"
    w = _sub_w(116, prefix)
    for k in ("p_in.weight", "g_in.weight"):
        w[k] = w[k] * scale
    _, z, _, pm = _inputs(N, 117, pad_tail=20)
    want = ref.triangle_multiplication(z, pm, w, direction)
    out = torch.empty((1, N, N, 128), device=gpu)
    ws = ops.workspace(ops.trimul_workspace_bytes(1, N), gpu)
    ops.launch_trimul(z.to(gpu), out, pm.to(gpu), _dev_w(w, gpu), 0 if direction == "outgoing" else 1, ws,
                      accumulate=False)
    check(f"trimul {direction} weights x{scale}", out, want)
