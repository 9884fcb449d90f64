"""The layer under HIP graph capture: the library allocates nothing and records no memset, so
one PairformerLayer step captured with torch.cuda.graph replays like the eager call.  Each
replay is checked against an eager step from the same state, with eager work on other tensors
between the replays."""
import pytest
import torch

from tt_boltz_amd import ops, pairformer, synthetic

pytestmark = pytest.mark.gpu


def test_layer_graph_replays_match_eager(gpu):
    N = 128
    w = synthetic.stack_weights(1, 0)
    s_cpu, z_cpu, mask_cpu, pm_cpu = synthetic.pair_inputs(N, 0, pad_tail=9)
    pf = pairformer.Pairformer(1, 32, 4, 24, 16, True, w)
    layer = pf.blocks[0]
    ws = ops.workspace(pf.workspace_bytes(1, N), gpu)
    mask, pm = mask_cpu.to(gpu).contiguous(), pm_cpu.to(gpu).contiguous()
    z, s = z_cpu.to(gpu).contiguous(), s_cpu.to(gpu).contiguous()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        layer(s, z, pm, mask, ws)   # first call on the capture stream outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side), torch.cuda.graph(g, stream=side):
        layer(s, z, pm, mask, ws)
    torch.cuda.synchronize()
    # an eager copy of the layer's state, stepped alongside the graph
    ze, se = z.clone(), s.clone()
    ws_e = ops.workspace(pf.workspace_bytes(1, N), gpu)
    for rep in range(3):
        layer(se, ze, pm, mask, ws_e)          # eager step
        g.replay()                              # the captured step on z, s
        torch.cuda.synchronize()
        print(f"[graph] replay {rep}: z equal {torch.equal(z, ze)}, s equal {torch.equal(s, se)}", flush=True)
        assert torch.equal(z, ze) and torch.equal(s, se), f"replay {rep} differs from the eager step"
        junk = torch.randn((1 << 20,), device=gpu).sum()   # unrelated eager work between replays
        assert torch.isfinite(junk)
