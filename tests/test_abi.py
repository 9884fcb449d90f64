"""C-ABI boundary checks that need no GPU: the library loads, exports every symbol
include/pairformer_hip.h declares, reports its ABI version, and rejects bad
arguments with a status code and a message before launching anything."""
import ctypes
import os
import re

import pytest

from tt_boltz_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "pairformer_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pf_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    names = _declared()
    for must in ("pf_trimul_fwd", "pf_triatt_fwd", "pf_tri_attention", "pf_transition_fwd", "pf_apb_fwd",
                 "pf_layernorm_fwd", "pf_linear_fwd", "pf_last_error", "pf_abi_version", "pf_quantize_mx8",
                 "pf_trimul_mx8_fwd", "pf_transition_mx8_fwd"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), name
    assert set(_declared()) == set(_lib.SIGNATURES), "ctypes signature table out of sync with the header"


def test_abi_version():
    assert _lib.load().pf_abi_version() == _lib.ABI_VERSION == 3


def test_struct_layouts_match_header_order():
    # the ctypes structs mirror the C structs field by field; spot-check sizes/offsets
    assert _lib.TrimulArgs.z_in.offset == 32 and ctypes.sizeof(_lib.TrimulArgs) == 32 + 19 * 8
    assert _lib.TransitionArgs.x_in.offset == 24 and ctypes.sizeof(_lib.TransitionArgs) == 24 + 12 * 8   # 11 pointers, fc3_mean_fix (padded)
    assert _lib.TriattArgs.z_in.offset == 40
    assert _lib.TrimulMx8Args.z_in.offset == 32 and ctypes.sizeof(_lib.TrimulMx8Args) == 32 + 18 * 8
    assert _lib.TransitionMx8Args.x_in.offset == 24 and ctypes.sizeof(_lib.TransitionMx8Args) == 24 + 11 * 8


def _err():
    return _lib.load().pf_last_error().decode()


def test_rejects_null_and_bad_shapes_without_launching():
    lib = _lib.load()
    assert lib.pf_trimul_fwd(None) == -1 and "null args" in _err()
    a = _lib.TrimulArgs(B=1, N=100, C=128, hidden=128, direction=0)
    assert lib.pf_trimul_fwd(ctypes.byref(a)) == -1 and "multiple of 64" in _err()
    a = _lib.TrimulArgs(B=1, N=128, C=96, hidden=96, direction=0)
    assert lib.pf_trimul_fwd(ctypes.byref(a)) == -1 and "128 or 64" in _err()
    a = _lib.TrimulArgs(B=1, N=128, C=64, hidden=128, direction=0)
    assert lib.pf_trimul_fwd(ctypes.byref(a)) == -1 and "hidden must equal c_z" in _err()
    t = _lib.TriattArgs(B=1, N=128, C=128, H=8, D=16)
    assert lib.pf_triatt_fwd(ctypes.byref(t)) == -1 and "H=4" in _err()
    assert lib.pf_layernorm_fwd(None, None, None, None, 4, 8, 1e-5, None) == -1
    assert lib.pf_linear_fwd(1, 1, None, None, 1, 4, 15, 32, None) == -1 and "K % 16" in _err()
    m = _lib.TrimulMx8Args(B=1, N=192, C=128, hidden=128, direction=0)
    assert lib.pf_trimul_mx8_fwd(ctypes.byref(m)) == -1 and "multiple of 128" in _err()
    assert lib.pf_quantize_mx8(1, 4, 48, 0, 1, 1, None) == -1 and "multiple of 32" in _err()
    assert lib.pf_quantize_mx8(1, 4, 64, 2, 1, 1, None) == -1 and "perm" in _err()
    tr = _lib.TransitionMx8Args(rows=16, C=384, hidden=1536)
    assert lib.pf_transition_mx8_fwd(ctypes.byref(tr)) == -1 and "C = 128" in _err()
    # the fc3 mean correction needs the residual and its workspace (dummy pointers: no launch)
    d = 4096
    t = _lib.TransitionArgs(rows=4096, C=128, hidden=512, x_in=d, out=d, norm_w=d, norm_b=d, fc1_w=d, fc2_w=d,
                            fc3_w=d, fc3_mean_fix=1)
    assert lib.pf_transition_fwd(ctypes.byref(t)) == -1 and "needs the fc3 residual" in _err()
    t.fc3_lo = d
    t.workspace, t.workspace_bytes = d, lib.pf_transition_workspace_size(4096, 128, 512) - 1
    assert lib.pf_transition_fwd(ctypes.byref(t)) == -1 and "needs a workspace" in _err()
    t.hidden, t.workspace_bytes = 480, lib.pf_transition_workspace_size(4096, 128, 480)
    assert lib.pf_transition_fwd(ctypes.byref(t)) == -1 and "multiple of 64" in _err()
    t.C, t.hidden, t.fc3_mean_fix = 384, 1536, 0
    assert lib.pf_transition_fwd(ctypes.byref(t)) == -1 and "C = 128 only" in _err()
    # with the fused pair bias, the transition's sums may not share the attention's workspace
    apb_bytes = lib.pf_apb_workspace_size(1, 64, 384, 16)
    apb = _lib.ApbArgs(B=1, N=64, c_s=384, C=128, H=16, zln_w=d, zln_b=d, w_z=d, workspace=1 << 20,
                       workspace_bytes=apb_bytes)
    t = _lib.TransitionArgs(rows=64 * 64, C=128, hidden=512, x_in=d, out=d, norm_w=d, norm_b=d, fc1_w=d, fc2_w=d,
                            fc3_w=d, fc3_lo=d, fc3_mean_fix=1, workspace=(1 << 20) + apb_bytes - 256,
                            workspace_bytes=lib.pf_transition_workspace_size(64 * 64, 128, 512))
    assert lib.pf_transition_pair_bias_fwd(ctypes.byref(t), ctypes.byref(apb)) == -1 and "overlaps" in _err()


def test_fast_mode_entry_points_reject_bad_arguments_without_launching():
    """pf_triatt_mx8_fwd, pf_apb_fwd_mx8 / pf_apb_attend_mx8, pf_transition_mx8_pair_bias_fwd
    and pf_trimul_mx8_contract check shapes, pointers, workspace and n_valid before any HIP
    call (dummy non-null pointers are never dereferenced on these paths)."""
    lib = _lib.load()
    assert lib.pf_triatt_mx8_fwd(None) == -1 and "null args" in _err()
    t = _lib.TriattMx8Args(B=1, N=128, C=64, H=4, D=32)
    assert lib.pf_triatt_mx8_fwd(ctypes.byref(t)) == -1 and "only C = 128" in _err()
    t = _lib.TriattMx8Args(B=1, N=96, C=128, H=4, D=32)
    assert lib.pf_triatt_mx8_fwd(ctypes.byref(t)) == -1 and "multiple of 64" in _err()
    t = _lib.TriattMx8Args(B=1, N=128, C=128, H=4, D=32)
    assert lib.pf_triatt_mx8_fwd(ctypes.byref(t)) == -1 and "null pointer" in _err()
    dummy = {f: 16 for f, ty in _lib.TriattMx8Args._fields_ if ty is ctypes.c_void_p and f not in ("pair_mask", "stream")}
    t = _lib.TriattMx8Args(B=1, N=128, C=128, H=4, D=32, workspace_bytes=16, **dummy)
    assert lib.pf_triatt_mx8_fwd(ctypes.byref(t)) == -1 and "workspace too small" in _err()
    need = lib.pf_triatt_mx8_workspace_size(1, 128, 128, 4, 32)
    assert need > 0
    t = _lib.TriattMx8Args(B=1, N=128, C=128, H=4, D=32, workspace_bytes=need, n_valid=129, **dummy)
    assert lib.pf_triatt_mx8_fwd(ctypes.byref(t)) == -1 and "n_valid 129 outside" in _err()

    assert lib.pf_apb_fwd_mx8(None) == -1 and "null args" in _err()
    # the allocation-free entry point names an unsupported shape as such (not as a scratch size)
    a = _lib.ApbArgs(B=1, N=100, c_s=384, C=128, H=16)
    assert lib.pf_apb_fwd_noalloc(ctypes.byref(a)) == -1 and "unsupported shape" in _err()
    a = _lib.ApbArgs(B=1, N=4096, c_s=384, C=128, H=16, **{f: 16 for f, ty in _lib.ApbArgs._fields_
                                                         if ty is ctypes.c_void_p and f not in ("stream", "workspace")})
    assert lib.pf_apb_fwd_noalloc(ctypes.byref(a)) == -1 and "bytes of scratch" in _err()
    a = _lib.ApbArgs(B=1, N=100, c_s=384, C=128, H=16)
    assert lib.pf_apb_attend_mx8(ctypes.byref(a)) == -1 and "unsupported shape" in _err()

    tr_ptrs = {f: 16 for f, ty in _lib.TransitionMx8Args._fields_ if ty is ctypes.c_void_p and f != "stream"}
    tr = _lib.TransitionMx8Args(rows=128 * 128 - 128, C=128, hidden=512, **tr_ptrs)
    apb = _lib.ApbArgs(B=1, N=128, c_s=384, C=128, H=16, zln_w=16, zln_b=16, w_z=16, workspace=16,
                       workspace_bytes=lib.pf_apb_workspace_size(1, 128, 384, 16))
    assert lib.pf_transition_mx8_pair_bias_fwd(ctypes.byref(tr), ctypes.byref(apb)) == -1
    assert "must equal B*N*N" in _err()
    tr = _lib.TransitionMx8Args(rows=128 * 128, C=128, hidden=500, **tr_ptrs)
    assert lib.pf_transition_mx8_pair_bias_fwd(ctypes.byref(tr), ctypes.byref(apb)) == -1
    assert "hidden a multiple of 128" in _err()

    assert lib.pf_trimul_mx8_contract(16, 16, 16, 16, 16, 2, 100, None) == -1 and "multiple of 128" in _err()
    assert lib.pf_trimul_mx8_contract(16, 16, 16, 16, 16, 1 << 20, 4096, None) == -1 and "2^31" in _err()


def test_both_operand_variants_load():
    for variant, code in _lib.OPERAND_CODE.items():
        lib = _lib.load(variant)
        assert lib.pf_operand_dtype() == code and lib.pf_abi_version() == 3
        for name in _declared():
            assert hasattr(lib, name), (variant, name)


def test_workspace_sizes():
    lib = _lib.load()
    # a, b and X planes (16-bit) + 1024 per-workgroup operand maxima (fp32) for X's scale + the
    # 64 x 128 partial sums of the mean correction (fp32)
    assert lib.pf_trimul_workspace_size(1, 512, 128) == 128 * 512 * 512 * (2 + 2 + 2) + 1024 * 4 + 64 * 128 * 4
    assert lib.pf_triatt_workspace_size(1, 64, 128, 4, 32) > 0
    assert lib.pf_triatt_workspace_size(1, 64, 128, 8, 16) == 0
    assert lib.pf_transition_workspace_size(4096, 128, 512) == 513 * 128 * 4   # fused: the fc3 mean-fix sums
    assert lib.pf_transition_workspace_size(100, 384, 1536) == 100 * (384 + 1536) * 4
    # e4m3 a/b planes + their E8M0 scales + the fp16 contraction output
    planes = 128 * 512 * 512
    assert lib.pf_trimul_mx8_workspace_size(1, 512, 128) == 2 * planes + 2 * planes // 32 + 2 * planes


def test_measurement_aids_reject_bad_arguments_without_launching():
    lib = _lib.load()
    assert lib.pf_kernel_timing(3, 1) == -1 and "unknown kind 3" in _err()
    assert lib.pf_kernel_timing(-1, 0) == -1 and "unknown kind" in _err()
    ms, n = ctypes.c_double(0.0), ctypes.c_int(0)
    assert lib.pf_kernel_timing_read(7, ctypes.byref(ms), ctypes.byref(n)) == -1 and "unknown kind 7" in _err()
    assert lib.pf_kernel_timing_read(0, None, None) == -1 and "null output pointer" in _err()
    assert lib.pf_mfma8_rate_probe(4, 6, 16, None) == -1 and "multiple of 4" in _err()
    assert lib.pf_mfma_rate_probe(0, 8, 16, None) == -1 and "workgroups > 0" in _err()
    # timing switched on and off without any launch records nothing
    assert lib.pf_kernel_timing(1, 1) == 0 and lib.pf_kernel_timing(1, 0) == 0
    assert lib.pf_kernel_timing_read(1, ctypes.byref(ms), ctypes.byref(n)) == 0 and n.value == 0 and ms.value == 0.0


def test_python_check_raises_with_message():
    lib = _lib.load()
    lib.pf_trimul_fwd(None)
    with pytest.raises(RuntimeError, match="null args"):
        _lib.check(-1, "pf_trimul_fwd")


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus 2 prints why and runs nothing (no GPU needed)."""
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120, cwd=root)
    assert "exactly one GPU" in r.stdout + r.stderr
    assert '"metric"' not in r.stdout


def test_options_validate_schedule_and_operand():
    """Host-side option checks: the single-track delay is 0-4 and the operand type is known."""
    from tt_boltz_amd import pairformer
    assert pairformer.Options().single_delay == 1 and pairformer.Options().overlap_single
    for bad in (-1, 5):
        with pytest.raises(ValueError, match="single_delay"):
            pairformer.Options(single_delay=bad)
    with pytest.raises(ValueError, match="operand"):
        pairformer.Options(operand="fp8")


def test_failed_block_drops_deferred_single_track():
    """A block that raises leaves no deferred single-track closure behind on the cached
    second stream (the next call would otherwise run it on the failed call's tensors), and a
    stale closure found at the start of a call is dropped, not run."""
    import types

    import torch
    from tt_boltz_amd import pairformer

    class FakeSingle:
        def __init__(self):
            self.pending, self.joined = None, False

        def discard(self):
            self.pending = None

        def join(self):
            self.joined = True

    single, ran = FakeSingle(), []
    single.pending = lambda: ran.append("stale from an earlier call")

    def good(s, z, *rest):
        single.pending = lambda: ran.append("deferred of this call")
        return s, z

    def bad(*rest):
        raise RuntimeError("launch failed")

    fake = types.SimpleNamespace(blocks=[good, bad], single_track=lambda *a: single, workspace_bytes=lambda B, N: 16)
    s, z = torch.zeros(1, 4, 8), torch.zeros(1, 4, 4, 8)
    with pytest.raises(RuntimeError, match="launch failed"):
        pairformer.Pairformer.__call__(fake, s, z, ws=torch.zeros(1))
    assert single.pending is None and not single.joined and ran == []
    fake.blocks = [good]
    pairformer.Pairformer.__call__(fake, s, z, ws=torch.zeros(1))
    assert single.joined and single.pending is not None and ran == []   # join() of the fake issues nothing


def test_weight_conversion_cache_follows_the_source_tensor():
    """The fused-op wrappers convert a weight once per tensor: the copy is reused while the
    source lives unmodified, redone after an in-place change, and dropped with the source."""
    import gc
    import torch
    from tt_boltz_amd import ops
    cpu = torch.device("cpu")
    w = torch.randn(64, 32)
    a = ops.opw(w, cpu, "fp16")
    assert a.dtype == torch.float16 and torch.equal(a.float(), w.half().float())
    assert ops.opw(w, cpu, "fp16") is a                      # reused
    assert ops.opw(w, cpu, "bf16") is not a                  # another operand type: its own copy
    w.mul_(2.0)                                              # in place: the version counter moves
    b = ops.opw(w, cpu, "fp16")
    assert b is not a and torch.equal(b.float(), w.half().float())
    n = len(ops._CONVERTED)
    del w, a, b
    gc.collect()
    assert len(ops._CONVERTED) < n                           # entries die with their source
    h = torch.randn(8, 8).half()
    assert ops.opw(h, cpu, "fp16").data_ptr() == h.data_ptr()   # nothing to convert, nothing kept
    assert all(e[0]() is not h for e in ops._CONVERTED.values())
    v = torch.randn(16)
    assert ops.f32(v, cpu).data_ptr() == v.data_ptr()
    with torch.inference_mode():
        t = torch.randn(4, 4)
    assert torch.equal(ops.opw(t, cpu, "fp16").float(), t.half().float())   # no version counter: converted each time
