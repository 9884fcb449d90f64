"""GPU checks of the benchmark's measurement aids: in-layer launch timing (one event pair per
launch of the chosen kernel, and only while switched on) and the MFMA rate probes (finite
results, positive rates)."""
import pytest
import torch

from tt_boltz_amd import ops

pytestmark = pytest.mark.gpu


def test_contract8_timing_counts_each_launch(gpu):
    N = 128
    g = torch.Generator(device=gpu).manual_seed(41)
    qa, sa = ops.quantize_mx8(torch.randn((128 * N, N), device=gpu, generator=g))
    qb, sb = ops.quantize_mx8(torch.randn((128 * N, N), device=gpu, generator=g))
    X = torch.empty((128, N, N), dtype=torch.float32, device=gpu)
    run = lambda: ops.launch_trimul_mx8_contract(qa.view(128, N, N), qb.view(128, N, N), sa.view(128, N, N // 32),
                                                 sb.view(128, N, N // 32), X)
    run()   # not recorded
    ops.kernel_timing(ops.TIMED_CONTRACT8, True)
    for _ in range(3):
        run()
    ms, n = ops.kernel_timing_read(ops.TIMED_CONTRACT8)
    ops.kernel_timing(ops.TIMED_CONTRACT8, False)
    run()   # not recorded either
    ms2, n2 = ops.kernel_timing_read(ops.TIMED_CONTRACT8)
    print(f"[measure] contract8 timing: {n} launches, {ms:.3f} ms", flush=True)
    assert n == 3 and ms > 0 and (n2, ms2) == (n, ms)
    # the attention kind saw none of them
    ops.kernel_timing(ops.TIMED_ATTEND, True)
    run()
    assert ops.kernel_timing_read(ops.TIMED_ATTEND) == (0.0, 0)
    ops.kernel_timing(ops.TIMED_ATTEND, False)


def test_contract_timing_inside_trimul(gpu):
    """PF_TIMED_CONTRACT brackets the 16-bit contraction of each pf_trimul_fwd call (and only
    that: the standalone pf_trimul_contract is not recorded)."""
    from tt_boltz_amd import pairformer, synthetic
    N = 128
    pf = pairformer.Pairformer(1, 32, 4, 24, 16, True, synthetic.stack_weights(1, 0))
    tm = pf.blocks[0].triangle_multiplication_start
    _, z_cpu, _, _ = synthetic.pair_inputs(N, 0, with_s=False)
    z = z_cpu.to(gpu).contiguous()
    out = torch.empty_like(z)
    ws = ops.workspace(tm.workspace_bytes(1, N), gpu)
    A = torch.randn((128, N, N), device=gpu).half()
    X = torch.empty_like(A)
    ops.kernel_timing(ops.TIMED_CONTRACT, True)
    for _ in range(2):
        tm(z, None, out=out, ws=ws)
    ops.launch_trimul_contract(A, A, X)
    ms, n = ops.kernel_timing_read(ops.TIMED_CONTRACT)
    ops.kernel_timing(ops.TIMED_CONTRACT, False)
    print(f"[measure] contract timing inside trimul: {n} launches, {ms:.3f} ms", flush=True)
    assert n == 2 and ms > 0


@pytest.mark.parametrize("fp8", [False, True])
def test_mfma_rate_probe(gpu, fp8):
    r = ops.mfma_rate_probe(gpu, iters=256, per_cu=1, reps=1, fp8=fp8)
    print(f"[measure] mfma rate probe fp8={fp8}: {r}", flush=True)
    assert r["finite"] and r["tflops"] > 0
