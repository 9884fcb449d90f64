"""pf_apb_fwd_noalloc (the allocation-free variant of pf_apb_fwd, scratch in a static device
array) against pf_apb_fwd with a caller workspace, through the C-ABI: two calls in a row on
one GPU, the second smaller (and masked) so it runs over the first call's leftover scratch.
Both entry points run the same kernels on the same inputs, so the outputs must be identical.
A shape whose scratch exceeds the static size is refused with a message, before any launch."""
import ctypes

import pytest
import torch

from tt_boltz_amd import _lib, ops, synthetic

pytestmark = pytest.mark.gpu


def _inputs(dev, B, N, c_s, seed, n_valid):
    g = torch.Generator().manual_seed(seed)
    s = torch.randn((B, N, c_s), generator=g).to(dev)
    z = torch.randn((B, N, N, 128), generator=g).to(dev)
    mask = torch.zeros((B, N))
    mask[:, :n_valid] = 1.0
    return s, z, mask.to(dev)


def _weights(dev, seed):
    shapes = {k: v for k, v in synthetic.layer_shapes().items() if k.startswith("attention.")}
    w = {k[len("attention."):]: v for k, v in synthetic.draw(shapes, seed).items()}
    return ops.convert_weights(w, dev)


def _run(lib, fn, s, z, mask, w, H, ws, n_valid):
    out = torch.full_like(s, float("nan"))
    a = ops._apb_args(s, s, z, mask, out, w, H, ws if ws is not None else s, False, 1e-5, n_valid)
    if ws is None:   # the no-alloc entry point takes no workspace
        a.workspace, a.workspace_bytes = None, 0
    rc = getattr(lib, fn)(ctypes.byref(a))
    _lib.check(rc, fn)
    torch.cuda.synchronize()
    return out


def test_noalloc_matches_workspace_entry_point(gpu):
    lib = _lib.load()
    H, c_s = 16, 384
    cases = [(1, 512, 512, 11), (1, 256, 200, 12)]   # (B, N, n_valid, seed): the second is smaller
    for B, N, n_valid, seed in cases:
        print(f"[no_alloc] B={B} N={N} n_valid={n_valid} seed={seed}", flush=True)
        s, z, mask = _inputs(gpu, B, N, c_s, seed, n_valid)
        w = _weights(gpu, seed)
        ws = ops.workspace(ops.apb_workspace_bytes(B, N, c_s, H), gpu)
        want = _run(lib, "pf_apb_fwd", s, z, mask, w, H, ws, n_valid)
        got = _run(lib, "pf_apb_fwd_noalloc", s, z, mask, w, H, None, n_valid)
        assert torch.isfinite(want).all()
        assert torch.equal(got, want), (N, (got - want).abs().max().item())


def test_noalloc_refuses_oversize(gpu):
    lib = _lib.load()
    B, N, c_s, H = 1, 1024, 384, 16
    need = lib.pf_apb_workspace_size(B, N, c_s, H)
    assert need > (24 << 20)
    # dummy non-null pointers: the shape and pointers pass, the scratch size is refused before any
    # launch (nothing is dereferenced)
    ptrs = {f: 16 for f, ty in _lib.ApbArgs._fields_ if ty is ctypes.c_void_p and f not in ("stream", "workspace")}
    a = _lib.ApbArgs(B=B, N=N, c_s=c_s, C=128, H=H, **ptrs)
    assert lib.pf_apb_fwd_noalloc(ctypes.byref(a)) == -1
    assert "above the static" in lib.pf_last_error().decode()
