"""GPU checks of the kernels' weight-precision paths.

* hi + lo weights (``ta_out`` gate / output projection, ``tm_out`` output projection, the pair
  recycling projection): wiring is checked by feeding the residual equal to the 16-bit weight
  itself, which must give the result of the plain kernel on the doubled weight (an exact
  doubling in the operand type) up to fp32 summation order; accuracy by the recycling
  projection's agreement with fp32 to ~1e-6 (both sides split).
* the mean correction of the trimul's LN_in-side weights: on a pair tensor whose rows share a
  strong channel pattern, the per-channel mean over positions of the GPU's update error (the
  coherent part that a deep stack accumulates) must fall well below the uncorrected kernel's.
"""
import pytest
import torch

from oracle import pairformer_ref as ref
from tt_boltz_amd import ops, synthetic

from test_gpu_parity import _dev_w, _inputs, _sub_w, check, stats

pytestmark = pytest.mark.gpu


def _same(a, b, name, mean_tol=2e-6):
    """Equal up to fp32 summation order: hi.x + lo.x and (2 hi).x differ in the last bits of an
    fp32 sum, which now and then moves a later 16-bit rounding by one step (max ~1e-4 of the
    rms); a wiring mistake (wrong row, pitch or operand) moves every element by O(1)."""
    mx, mn = stats(a, b)
    print(f"[precision] {name}: max/rms={mx:.3e} mean/rms={mn:.3e}", flush=True)
    assert torch.isfinite(a).all() and mx <= 2e-3 and mn <= mean_tol, f"{name}: max/rms={mx:.3e} mean/rms={mn:.3e}"


@pytest.mark.parametrize("ending", [False, True])
def test_triatt_residual_weights_wiring(gpu, ending):
    """ta_out with (hi, lo) = (W16, W16) equals the plain kernel on 2 W16 (gate and output)."""
    N = 192
    prefix = "tri_att_end" if ending else "tri_att_start"
    w = _dev_w(_sub_w(21, prefix), gpu, "mha.")
    _, z, _, pm = _inputs(N, 22, pad_tail=13)
    zd, pmd = z.to(gpu), pm.to(gpu).contiguous()
    ws = ops.workspace(ops.triatt_workspace_bytes(1, N), gpu)
    hilo = dict(w)
    hilo["linear_g.weight.lo"] = w["linear_g.weight"]
    hilo["linear_o.weight.lo"] = w["linear_o.weight"]
    doubled = dict(w)
    doubled["linear_g.weight"] = (2 * w["linear_g.weight"].float()).to(w["linear_g.weight"].dtype)
    doubled["linear_o.weight"] = (2 * w["linear_o.weight"].float()).to(w["linear_o.weight"].dtype)
    a, b = torch.empty_like(zd), torch.empty_like(zd)
    ops.launch_triatt(zd, a, pmd, hilo, ending, ws, accumulate=False)
    ops.launch_triatt(zd, b, pmd, doubled, ending, ws, accumulate=False)
    _same(a, b, f"triatt hi+lo(=hi) vs doubled weights ending={ending}")
    # and the true residual brings the update to the fp32 oracle at least as close as before
    true_lo = dict(w)
    raw = _sub_w(21, prefix)
    for k in ("linear_g.weight", "linear_o.weight"):
        true_lo[k + ".lo"] = ops.opw_lo(raw["mha." + k], gpu)
    c = torch.empty_like(zd)
    ops.launch_triatt(zd, c, pmd, true_lo, ending, ws, accumulate=False)
    want = ref.triangle_attention(z, pm, raw, not ending, None)
    check(f"triatt with weight residuals ending={ending}", c, want)


@pytest.mark.parametrize("direction", [0, 1])
def test_trimul_residual_weight_wiring(gpu, direction):
    """tm_out with p_out given as (W16, W16) equals the plain kernel on 2 W16; the two-fill X
    stage of that path is covered by the same comparison."""
    N = 256
    prefix = "tri_mul_out" if direction == 0 else "tri_mul_in"
    w = _dev_w(_sub_w(23, prefix), gpu)
    _, z, _, pm = _inputs(N, 24, pad_tail=17, rand_mask=True)
    zd, pmd = z.to(gpu), pm.to(gpu).contiguous()
    ws = ops.workspace(ops.trimul_workspace_bytes(1, N), gpu)
    hilo = dict(w)
    hilo["p_out.weight.lo"] = w["p_out.weight"]
    doubled = dict(w)
    doubled["p_out.weight"] = (2 * w["p_out.weight"].float()).to(w["p_out.weight"].dtype)
    a, b = torch.empty_like(zd), torch.empty_like(zd)
    ops.launch_trimul(zd, a, pmd, hilo, direction, ws, accumulate=False)
    ops.launch_trimul(zd, b, pmd, doubled, direction, ws, accumulate=False)
    _same(a, b, f"trimul p_out hi+lo(=hi) vs doubled direction={direction}")


def test_pair_recycling_projection_is_fp32_accurate(gpu):
    """base + W . LN(x) with both W and LN(x) split hi + lo agrees with fp64 to ~2e-7 of the
    update's rms in the mean (measured 2.2e-7; the plain 16-bit path: 2.4e-4), including the
    pass-start case x = 0 where LN(x) is the same beta at every pair."""
    g = torch.Generator().manual_seed(31)
    rows = 64 * 64
    w = synthetic.draw(synthetic.recycle_shapes(), 32)
    W, lnw, lnb = w["z_recycle.weight"], w["z_norm.weight"], w["z_norm.bias"]
    for name, x in (("random z", torch.randn((rows, 128), generator=g)), ("z = 0", torch.zeros((rows, 128)))):
        base = torch.randn((rows, 128), generator=g)
        want = ref.layer_norm(x.double(), lnw.double(), lnb.double()) @ W.double().t()
        xd, bd = x.to(gpu), base.to(gpu)
        out = torch.empty_like(bd)
        ops.launch_pair_ln_linear(xd, bd, lnw.to(gpu), lnb.to(gpu), ops.opw(W, gpu), out, 1e-5, "fp16",
                                  ops.opw_lo(W, gpu))
        upd = out.double().cpu() - base.double()
        mx, mn = stats(upd, want)
        plain = torch.empty_like(bd)
        ops.launch_pair_ln_linear(xd, bd, lnw.to(gpu), lnb.to(gpu), ops.opw(W, gpu), plain, 1e-5, "fp16")
        pmx, pmn = stats(plain.double().cpu() - base.double(), want)
        print(f"[precision] recycling projection, {name}: hi+lo max/rms={mx:.2e} mean/rms={mn:.2e}; "
              f"plain max/rms={pmx:.2e} mean/rms={pmn:.2e}", flush=True)
        assert mx < 1e-5 and mn < 1e-6, (name, mx, mn)
        assert pmn > 100 * mn


@pytest.mark.parametrize("direction", [0, 1])
def test_trimul_mean_correction_removes_coherent_error(gpu, direction):
    """z rows share a strong channel pattern (so the normalized rows have a large mean over
    positions).  The error of the 16-bit weights then has a large coherent part: the same
    offset at every position.  With the exact beta offsets and the mean correction, the
    per-channel mean over positions of the update's error must drop well below the plain
    kernel's, and the update must stay within the parity bar.  (The corrected run also carries
    p_out as hi + lo, as the module does: the contraction output's LayerNorm has a mean over
    positions too.)"""
    N = 256
    prefix = "tri_mul_out" if direction == 0 else "tri_mul_in"
    raw = _sub_w(25, prefix)
    g = torch.Generator().manual_seed(26)
    pattern = 3.0 * torch.randn(128, generator=g)
    z = pattern + torch.randn((1, N, N, 128), generator=g)
    pm = torch.ones((1, N, N))
    want = ref.triangle_multiplication(z.to(gpu), pm.to(gpu), {k: v.to(gpu) for k, v in raw.items()},
                                       "outgoing" if direction == 0 else "incoming").cpu()
    w = _dev_w(raw, gpu)
    beta = raw["norm_in.bias"].double()
    fixed = dict(w)
    fixed["in_offsets"] = torch.cat([raw[k].double() @ beta for k in ("p_in.weight", "g_in.weight",
                                                                      "g_out.weight")]).float().to(gpu)
    for k in ("p_in.weight", "g_in.weight", "g_out.weight", "p_out.weight"):
        fixed[k + ".lo"] = ops.opw_lo(raw[k], gpu)
    zd = z.to(gpu).contiguous()
    ws = ops.workspace(ops.trimul_workspace_bytes(1, N), gpu)
    a, b = torch.empty_like(zd), torch.empty_like(zd)
    ops.launch_trimul(zd, a, None, w, direction, ws, accumulate=False)
    ops.launch_trimul(zd, b, None, fixed, direction, ws, accumulate=False)
    rms = want.pow(2).mean().sqrt()
    coh_plain = ((a.cpu() - want).mean(dim=(0, 1, 2)).abs().mean() / rms).item()
    coh_fixed = ((b.cpu() - want).mean(dim=(0, 1, 2)).abs().mean() / rms).item()
    print(f"[precision] trimul direction={direction}: coherent error plain {coh_plain:.3e}, "
          f"mean-corrected {coh_fixed:.3e}", flush=True)
    check(f"trimul mean-corrected direction={direction}", b, want)
    assert coh_fixed < 0.35 * coh_plain


@pytest.mark.parametrize("N", [64, 128, 192, 256])
def test_pair_stats_sample_mean(gpu, N):
    """The statistics the mean correction starts from: after a mean-corrected trimul call the
    workspace holds 64 partial sums (after the three operand planes and the 1024 amax partials)
    that add up to the mean over the sampled positions of the rows normalized without their
    affine part.  The sample is every tile of 32 consecutive positions when there are at most
    1024 tiles (N = 64, 128: a whole-grid mean) and otherwise the 1024 tiles
    k * 2654435761 mod n_tiles (N = 192: 1152 tiles, some drawn twice; N = 256: half of the
    2048 tiles, each once)."""
    raw = _sub_w(27, "tri_mul_out")
    g = torch.Generator().manual_seed(28)
    z = 2.0 * torch.randn(128, generator=g) + torch.randn((1, N, N, 128), generator=g)
    w = dict(_dev_w(raw, gpu))
    w["in_offsets"] = torch.zeros(3 * 128, device=gpu)
    for k in ("p_in.weight", "g_in.weight", "g_out.weight"):
        w[k + ".lo"] = ops.opw_lo(raw[k], gpu)
    zd = z.to(gpu).contiguous()
    ws = ops.workspace(ops.trimul_workspace_bytes(1, N), gpu)
    ops.launch_trimul(zd, torch.empty_like(zd), None, w, 0, ws, accumulate=False)
    torch.cuda.synchronize()
    start = 3 * 128 * N * N * 2 + 1024 * 4
    mu = ws[start:start + 64 * 128 * 4].cpu().view(torch.float32).view(64, 128).double().sum(0)
    ntiles = N * N // 32
    tiles = range(ntiles) if ntiles <= 1024 else [k * 2654435761 % ntiles for k in range(1024)]
    rows = z.double().reshape(-1, 32, 128)[list(tiles)].reshape(-1, 128)
    xhat = (rows - rows.mean(1, keepdim=True)) / (rows.var(1, unbiased=False, keepdim=True) + 1e-5).sqrt()
    want = xhat.mean(0)
    err = (mu - want).abs().max().item()
    print(f"[precision] pair stats N={N}: |mu| max {want.abs().max().item():.3f}, max error {err:.2e}", flush=True)
    assert err < 1e-5


@pytest.mark.parametrize("with_bias", [False, True])
def test_transition_residual_weight_wiring(gpu, with_bias):
    """tr_pair with fc3 given as (W16, W16) equals the plain kernel on 2 W16 (the four-block
    ring of that path, with and without the fused single-track pair bias)."""
    N = 128
    w = _dev_w(_sub_w(27, "transition_z"), gpu)
    _, z, _, _ = _inputs(N, 28)
    s = torch.randn((1, N, 384), generator=torch.Generator().manual_seed(29)).to(gpu)
    zd = z.to(gpu).contiguous()
    hilo = dict(w)
    hilo["fc3.weight.lo"] = w["fc3.weight"]
    doubled = dict(w)
    doubled["fc3.weight"] = (2 * w["fc3.weight"].float()).to(w["fc3.weight"].dtype)
    outs, biases = [], []
    for ww in (hilo, doubled):
        out = zd.clone()   # out += update, as in the layer
        pb = None
        if with_bias:
            apb = _dev_w(_sub_w(30, "attention"), gpu)
            apb_ws = ops.workspace(ops.apb_workspace_bytes(1, N, 384, 16), gpu)
            pb = (s, apb, 16, apb_ws, 1e-5)
        ops.launch_transition(zd, out, ww, None, accumulate=True, pair_bias=pb)
        outs.append(out)
        if with_bias:
            off = 5 * N * 384 * 4   # q, k, v, g, o.g [N][384] fp32, then the bias [16][N][N]
            biases.append(apb_ws[off: off + 16 * N * N * 4].view(torch.float32).clone())
    _same(outs[0], outs[1], f"transition fc3 hi+lo(=hi) vs doubled (pair bias {with_bias})")
    if with_bias:
        # the bias is a 16-bit product of LN(z): each flipped z rounding moves it again (measured 2.7e-6)
        _same(biases[0], biases[1], "transition fused pair bias with fc3 hi+lo(=hi) vs doubled", 1e-5)


def _tr_sample_tiles(rows):
    """The tiles of 32 rows the pair transition's sampling pass takes (at most 256, by
    k * 2654435761 mod n_tiles when there are more)."""
    ntiles = rows // 32
    return list(range(ntiles)) if ntiles <= 256 else [k * 2654435761 % ntiles for k in range(256)]


@pytest.mark.parametrize("N,with_bias", [(64, False), (192, False), (256, True)])
def test_transition_mean_correction(gpu, N, with_bias):
    """fc3_mean_fix: fc3_16 plus corr = (fc3 - fc3_16) . mean(h) over the sampled tiles.
    corr (kept in the workspace after the 512 x 128 partial sums) must match fp64 on the same
    tiles to 1% of its size (the kernel's h comes from 16-bit operands).  On z rows that share a
    strong channel pattern (so h has a large mean), the fc3 rounding error alone is the plain
    kernel's difference to the hi + lo one; its per-channel mean over positions (what a deep
    stack accumulates) must mostly vanish from the mean-corrected kernel's difference to hi + lo
    (all 128 tiles sampled at N = 64; 256 of 1152 / 2048 at N = 192 / 256).  The update must meet
    the parity bar, and with the fused single-track pair bias it must be the same bits."""
    raw = _sub_w(33, "transition_z")
    g = torch.Generator().manual_seed(34)
    z = 2.0 * torch.randn(128, generator=g) + torch.randn((1, N, N, 128), generator=g)
    zd = z.to(gpu).contiguous()
    want = ref.transition(zd, {k: v.to(gpu) for k, v in raw.items()}).cpu()
    w = _dev_w(raw, gpu)
    fixed = dict(w)
    fixed["fc3.weight.lo"] = ops.opw_lo(raw["fc3.weight"], gpu)
    rows = N * N
    ws = ops.workspace(ops.transition_workspace_bytes(rows, 128, 512), gpu)
    a, b, hl = torch.empty_like(zd), torch.empty_like(zd), torch.empty_like(zd)
    ops.launch_transition(zd, a, w, None, accumulate=False)
    ops.launch_transition(zd, hl, fixed, None, accumulate=False)
    ops.launch_transition(zd, b, fixed, ws, accumulate=False, fc3_mean_fix=True)
    torch.cuda.synchronize()
    corr = ws[512 * 128 * 4: 513 * 128 * 4].cpu().view(torch.float32).double()
    x = z.double().reshape(-1, 32, 128)[_tr_sample_tiles(rows)].reshape(-1, 128)
    xn = ref.layer_norm(x, raw["norm.weight"].double(), raw["norm.bias"].double())
    hmean = (torch.nn.functional.silu(xn @ raw["fc1.weight"].double().t()) * (xn @ raw["fc2.weight"].double().t())).mean(0)
    corr_want = fixed["fc3.weight.lo"].double().cpu() @ hmean
    cerr = (corr - corr_want).abs().max().item() / corr_want.abs().max().item()
    rms = want.pow(2).mean().sqrt()
    coh_plain = ((a - hl).mean(dim=(0, 1, 2)).abs().mean().cpu() / rms).item()
    coh_fixed = ((b - hl).mean(dim=(0, 1, 2)).abs().mean().cpu() / rms).item()
    print(f"[precision] transition mean fix N={N}: corr max {corr_want.abs().max().item():.2e}, rel error "
          f"{cerr:.2e}; coherent fc3 error plain {coh_plain:.3e}, mean-corrected {coh_fixed:.3e}", flush=True)
    assert cerr < 1e-2
    check(f"transition mean-corrected N={N}", b, want)
    assert coh_fixed < 0.2 * coh_plain
    if with_bias:
        s = torch.randn((1, N, 384), generator=torch.Generator().manual_seed(35)).to(gpu)
        apb = _dev_w(_sub_w(36, "attention"), gpu)
        apb_ws = ops.workspace(ops.apb_workspace_bytes(1, N, 384, 16), gpu)
        c = torch.empty_like(zd)
        ops.launch_transition(zd, c, fixed, ws, accumulate=False, pair_bias=(s, apb, 16, apb_ws, 1e-5),
                              fc3_mean_fix=True)
        assert torch.equal(b, c)
