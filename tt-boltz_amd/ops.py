"""Operator-level API: the Pairformer hot-path ops on PyTorch-ROCm device tensors.

Each public function mirrors a reference operator (same argument names and
meaning) and runs the HIP kernels of ``libpairformer_hip`` through the C ABI.
Tensors must live on a ROCm GPU; there is no CPU path.  Token counts that are not
a multiple of 64 are zero-padded internally (padding excluded from every softmax
and masked out of every contraction) and sliced back, like the reference's
Tenstorrent boundary pads (``tt_bio/tenstorrent.py:2235-2246``).

``variant`` selects the MFMA operand type: ``"fp16"`` (default, IEEE binary16)
or ``"bf16"``.  Accumulation and every statistic are fp32 in both.

The ``launch_*`` functions are the thin layer the modules use: they take
already-padded contiguous device tensors and pre-converted weights (operand-type
matrices, fp32 LayerNorm parameters and biases) and enqueue work on the current
stream.
"""
from __future__ import annotations

import ctypes
import weakref
from typing import Mapping, Optional

import torch

from . import _lib

PAD = 64
C_Z = 128
DEFAULT_VARIANT = _lib.DEFAULT_VARIANT
TORCH_DTYPE = {"fp16": torch.float16, "bf16": torch.bfloat16}


# --------------------------------------------------------------------------------------
# plumbing
# --------------------------------------------------------------------------------------
def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _require_gpu(*ts: Optional[torch.Tensor]) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(f"tensor on {t.device}: the HIP kernels need ROCm device tensors")
        dev = t.device
    if dev is None:
        raise RuntimeError("no device tensor given")
    return dev


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=device)


#: converted copies of weight tensors: id(source) -> (weakref to the source, its version counter
#: at conversion, device, dtype, the copy).  An entry lives as long as its source tensor and is
#: used only while the source is unmodified (same version), so the per-call fused-op wrappers
#: convert (or upload) a given weight once.
_CONVERTED: dict = {}


def _converted(w: torch.Tensor, device: torch.device, dtype: torch.dtype) -> torch.Tensor:
    try:
        version = w._version
    except RuntimeError:   # inference tensors keep no version counter: convert every time
        version = None
    key = id(w)
    e = _CONVERTED.get(key) if version is not None else None
    if e is not None and e[0]() is w and e[1] == version and e[2] == torch.device(device) and e[3] == dtype:
        return e[4]
    out = w.detach().to(device=device, dtype=dtype).contiguous()
    if version is None or out.data_ptr() == w.data_ptr():
        return out   # already in place: nothing to keep (and no reference that keeps w alive)
    try:
        ref = weakref.ref(w, lambda _r, k=key: _CONVERTED.pop(k, None))
    except TypeError:
        return out
    _CONVERTED[key] = (ref, version, torch.device(device), dtype, out)
    return out


def opw(w: torch.Tensor, device: torch.device, variant: str = DEFAULT_VARIANT) -> torch.Tensor:
    """A weight matrix in the MFMA operand type of ``variant`` (converted once per tensor)."""
    return _converted(w, device, TORCH_DTYPE[variant])


def opw_lo(w: torch.Tensor, device: torch.device, variant: str = DEFAULT_VARIANT) -> torch.Tensor:
    """The residual of ``opw``: w - float(opw(w)), itself in the operand type, so that hi + lo
    carries w to ~2^-22 of its size (for kernels that take a weight as two MFMA operands)."""
    w32 = w.detach().to(device=device, dtype=torch.float32)
    dt = TORCH_DTYPE[variant]
    return (w32 - w32.to(dt).to(torch.float32)).to(dt).contiguous()


def f32(t: Optional[torch.Tensor], device: torch.device) -> Optional[torch.Tensor]:
    return None if t is None else _converted(t, device, torch.float32)


def convert_weights(w: Mapping[str, torch.Tensor], device: torch.device, variant: str = DEFAULT_VARIANT,
                    strip: str = "") -> dict:
    """1-D tensors (LayerNorm params, biases) -> fp32; matrices -> operand type."""
    out = {}
    for k, v in w.items():
        kk = k[len(strip):] if strip and k.startswith(strip) else k
        out[kk] = f32(v, device) if v.dim() == 1 else opw(v, device, variant)
    return out


def padded_len(n: int, pad: int = PAD) -> int:
    return -(-n // pad) * pad


def pad_pair(z: torch.Tensor, n_pad: int) -> torch.Tensor:
    """Zero-pad [B,N,N,C] to [B,n_pad,n_pad,C] (always returns a new contiguous fp32 tensor)."""
    B, N, _, C = z.shape
    out = torch.zeros((B, n_pad, n_pad, C), dtype=torch.float32, device=z.device)
    out[:, :N, :N] = z
    return out


#: row chunks of a host -> device pair copy: the host copy of one chunk into pinned memory
#: overlaps the DMA of the previous chunk
_H2D_CHUNKS = 4


def to_device_padded(x: torch.Tensor, n_pad: int, device: torch.device, pair: bool) -> torch.Tensor:
    """Zero-padded fp32 device copy of ``x``: [B,N,N,C] -> [B,n_pad,n_pad,C] (``pair``) or
    [B,N,C] -> [B,n_pad,C].  A CPU tensor moves through pinned staging buffers (torch's
    caching host allocator) in row chunks with asynchronous DMA, so the host copy of a
    chunk overlaps the transfer of the previous one; a device tensor is padded in place."""
    B, N = x.shape[0], x.shape[1]
    shape = (B, n_pad, n_pad, x.shape[-1]) if pair else (B, n_pad, x.shape[-1])
    out = torch.zeros(shape, dtype=torch.float32, device=device)
    dst = out[:, :N, :N] if pair else out[:, :N]
    if x.device.type != "cpu":
        dst.copy_(x)
        return out
    xf = x if x.dtype == torch.float32 else x.float()
    if xf.is_pinned():
        dst.copy_(xf, non_blocking=True)
        return out
    step = max(1, -(-N // _H2D_CHUNKS))
    for r0 in range(0, N, step):
        r1 = min(N, r0 + step)
        stage = torch.empty(xf[:, r0:r1].shape, dtype=torch.float32, pin_memory=True)
        stage.copy_(xf[:, r0:r1])
        dst[:, r0:r1].copy_(stage, non_blocking=True)
    return out


def to_host(x: torch.Tensor) -> torch.Tensor:
    """A CPU copy of device tensor ``x`` in pinned memory (one DMA, then a stream sync)."""
    out = torch.empty(x.shape, dtype=x.dtype, pin_memory=True)
    out.copy_(x, non_blocking=True)
    torch.cuda.current_stream(x.device).synchronize()
    return out


def valid_pair_mask(B: int, N: int, n_valid: int, device: torch.device) -> torch.Tensor:
    """[B,N,N] fp32 pair mask that is 1 on the first ``n_valid`` tokens' pairs and 0 on the
    boundary padding: what a padded stack uses when the caller gives no mask."""
    out = torch.zeros((B, N, N), dtype=torch.float32, device=device)
    out[:, :n_valid, :n_valid] = 1.0
    return out


def pad_pair_mask(pair_mask: Optional[torch.Tensor], B: int, N: int, n_pad: int,
                  device: torch.device) -> Optional[torch.Tensor]:
    """[B,N,N] 0/1 mask padded with zeros; None when no masking is needed."""
    if pair_mask is None and n_pad == N:
        return None
    out = torch.zeros((B, n_pad, n_pad), dtype=torch.float32, device=device)
    out[:, :N, :N] = 1.0 if pair_mask is None else pair_mask.to(device=device, dtype=torch.float32)
    return out


# --------------------------------------------------------------------------------------
# launchers (padded, contiguous, device-resident inputs; weights pre-converted)
# --------------------------------------------------------------------------------------
def trimul_workspace_bytes(B: int, N: int, variant: str = DEFAULT_VARIANT, C: int = C_Z) -> int:
    return _lib.load(variant).pf_trimul_workspace_size(B, N, C)


def launch_trimul(z_in: torch.Tensor, out: torch.Tensor, pair_mask: Optional[torch.Tensor],
                  w: Mapping[str, torch.Tensor], direction: int, ws: torch.Tensor,
                  accumulate: bool, eps: float = 1e-5, variant: str = DEFAULT_VARIANT) -> None:
    B, N, _, C = z_in.shape
    a = _lib.TrimulArgs(
        B=B, N=N, C=C, hidden=w["p_in.weight"].shape[0] // 2, direction=direction,
        accumulate=int(accumulate), eps=eps, z_in=_ptr(z_in), out=_ptr(out), pair_mask=_ptr(pair_mask),
        norm_in_w=_ptr(w["norm_in.weight"]), norm_in_b=_ptr(w["norm_in.bias"]),
        p_in_w=_ptr(w["p_in.weight"]), g_in_w=_ptr(w["g_in.weight"]),
        norm_out_w=_ptr(w["norm_out.weight"]), norm_out_b=_ptr(w["norm_out.bias"]),
        p_out_w=_ptr(w["p_out.weight"]), g_out_w=_ptr(w["g_out.weight"]),
        workspace=_ptr(ws), workspace_bytes=ws.numel(), stream=_stream(),
        p_out_lo=_ptr(w.get("p_out.weight.lo")), in_offsets=_ptr(w.get("in_offsets")),
        p_in_lo=_ptr(w.get("p_in.weight.lo")), g_in_lo=_ptr(w.get("g_in.weight.lo")),
        g_out_lo=_ptr(w.get("g_out.weight.lo")))
    _lib.check(_lib.load(variant).pf_trimul_fwd(ctypes.byref(a)), "pf_trimul_fwd", variant)


def triatt_workspace_bytes(B: int, N: int, H: int = 4, D: int = 32, variant: str = DEFAULT_VARIANT,
                           C: int = C_Z) -> int:
    return _lib.load(variant).pf_triatt_workspace_size(B, N, C, H, D)


def launch_triatt(z_in: torch.Tensor, out: torch.Tensor, pair_mask: Optional[torch.Tensor],
                  w: Mapping[str, torch.Tensor], ending: bool, ws: torch.Tensor, accumulate: bool,
                  n_heads: int = 4, head_dim: int = 32, eps: float = 1e-5, n_valid: int = 0,
                  variant: str = DEFAULT_VARIANT) -> None:
    B, N, _, C = z_in.shape
    a = _lib.TriattArgs(
        B=B, N=N, C=C, H=n_heads, D=head_dim, ending=int(ending), accumulate=int(accumulate), n_valid=n_valid,
        eps=eps, z_in=_ptr(z_in), out=_ptr(out), pair_mask=_ptr(pair_mask),
        ln_w=_ptr(w["layer_norm.weight"]), ln_b=_ptr(w["layer_norm.bias"]), w_bias=_ptr(w["linear.weight"]),
        w_q=_ptr(w["linear_q.weight"]), w_k=_ptr(w["linear_k.weight"]), w_v=_ptr(w["linear_v.weight"]),
        w_g=_ptr(w["linear_g.weight"]), w_o=_ptr(w["linear_o.weight"]),
        workspace=_ptr(ws), workspace_bytes=ws.numel(), stream=_stream(),
        w_g_lo=_ptr(w.get("linear_g.weight.lo")), w_o_lo=_ptr(w.get("linear_o.weight.lo")),
        in_offsets=_ptr(w.get("in_offsets")), w_q_lo=_ptr(w.get("linear_q.weight.lo")),
        w_k_lo=_ptr(w.get("linear_k.weight.lo")), w_v_lo=_ptr(w.get("linear_v.weight.lo")),
        w_bias_lo=_ptr(w.get("linear.weight.lo")))
    _lib.check(_lib.load(variant).pf_triatt_fwd(ctypes.byref(a)), "pf_triatt_fwd", variant)


def launch_triatt_attend(ws: torch.Tensor, B: int, N: int, n_valid: int = 0, variant: str = DEFAULT_VARIANT) -> None:
    """The flash-attention kernel alone on the operands the last ``launch_triatt`` call with
    the same (B, N) left in ``ws`` (measurement of the dominant kernel)."""
    _lib.check(_lib.load(variant).pf_triatt_attend_workspace(_ptr(ws), ws.numel(), B, N, n_valid, _stream()),
               "pf_triatt_attend_workspace", variant)


def attend_timing(enable: bool, variant: str = DEFAULT_VARIANT) -> None:
    """Start (clearing the record) or stop in-layer launch timing of the triangle-attention core
    on this host thread: every attention-core launch made meanwhile is bracketed by HIP events
    on its stream (a measurement aid; see ``attend_timing_read``)."""
    _lib.check(_lib.load(variant).pf_attend_timing(1 if enable else 0), "pf_attend_timing", variant)


def attend_timing_read(variant: str = DEFAULT_VARIANT):
    """(summed launch ms, launches) of the attention-core launches recorded since
    ``attend_timing(True)``; waits for the last one."""
    ms, n = ctypes.c_double(0.0), ctypes.c_int(0)
    _lib.check(_lib.load(variant).pf_attend_timing_read(ctypes.byref(ms), ctypes.byref(n)),
               "pf_attend_timing_read", variant)
    return ms.value, n.value


TIMED_ATTEND, TIMED_CONTRACT8, TIMED_CONTRACT = 0, 1, 2   # pf_kernel_timing kinds (PF_TIMED_*)


def kernel_timing(kind: int, enable: bool, variant: str = DEFAULT_VARIANT) -> None:
    """``attend_timing`` for a chosen kernel kind (TIMED_ATTEND, TIMED_CONTRACT8, TIMED_CONTRACT)."""
    _lib.check(_lib.load(variant).pf_kernel_timing(kind, 1 if enable else 0), "pf_kernel_timing", variant)


def kernel_timing_read(kind: int, variant: str = DEFAULT_VARIANT):
    """(summed launch ms, launches) of the kind's launches recorded since ``kernel_timing``."""
    ms, n = ctypes.c_double(0.0), ctypes.c_int(0)
    _lib.check(_lib.load(variant).pf_kernel_timing_read(kind, ctypes.byref(ms), ctypes.byref(n)),
               "pf_kernel_timing_read", variant)
    return ms.value, n.value


def mfma_rate_probe(device: torch.device, iters: int = 20000, per_cu: int = 2, reps: int = 3,
                    variant: str = DEFAULT_VARIANT, fp8: bool = False) -> dict:
    """Sustained MFMA rate of the chip under load (pseudo-random operands, every SIMD issuing
    back-to-back 32x32x16 16-bit MFMAs, or with ``fp8`` block-scaled 32x32x64 e4m3 MFMAs, from
    ``4 * per_cu`` waves), timed with HIP events: the best of ``reps`` launches after one
    warm-up."""
    lib = _lib.load(variant)
    probe, flop_per_mfma = (lib.pf_mfma8_rate_probe, 131072) if fp8 else (lib.pf_mfma_rate_probe, 32768)
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    wgs = cus * per_cu
    waves = lib.pf_mfma_rate_probe_waves(wgs)
    sink = torch.empty(waves, dtype=torch.float32, device=device)
    stream = _stream()
    best = None
    for r in range(reps + 1):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        _lib.check(probe(wgs, iters, _ptr(sink), stream), "pf_mfma_rate_probe", variant)
        b.record()
        torch.cuda.synchronize()
        ms = a.elapsed_time(b)
        if r and (best is None or ms < best):
            best = ms
    flop = waves * iters * 4 * flop_per_mfma
    return {"tflops": round(flop / (best * 1e-3) / 1e12, 1), "launch_ms": round(best, 3), "waves": waves,
            "mfma_per_wave": iters * 4, "finite": bool(torch.isfinite(sink).all())}


def transition_workspace_bytes(rows: int, C: int, hidden: int, variant: str = DEFAULT_VARIANT) -> int:
    return _lib.load(variant).pf_transition_workspace_size(rows, C, hidden)


def launch_transition(x_in: torch.Tensor, out: torch.Tensor, w: Mapping[str, torch.Tensor],
                      ws: Optional[torch.Tensor], accumulate: bool, eps: float = 1e-5,
                      variant: str = DEFAULT_VARIANT, pair_bias: Optional[tuple] = None,
                      fc3_mean_fix: bool = False) -> None:
    """``pair_bias = (s, w_apb, n_heads, apb_ws, eps_apb)``: also write the single-track pair
    bias of ``out`` into ``apb_ws`` in the same kernel (pf_transition_pair_bias_fwd; c_z = 128).
    ``fc3_mean_fix``: use ``w["fc3.weight.lo"]`` through the sampled mean correction instead of
    the hi + lo product (needs ``ws``)."""
    C = x_in.shape[-1]
    rows = x_in.numel() // C
    a = _lib.TransitionArgs(
        rows=rows, C=C, hidden=w["fc1.weight"].shape[0], accumulate=int(accumulate), eps=eps,
        x_in=_ptr(x_in), out=_ptr(out), norm_w=_ptr(w["norm.weight"]), norm_b=_ptr(w["norm.bias"]),
        fc1_w=_ptr(w["fc1.weight"]), fc2_w=_ptr(w["fc2.weight"]), fc3_w=_ptr(w["fc3.weight"]),
        workspace=_ptr(ws), workspace_bytes=0 if ws is None else ws.numel(), stream=_stream(),
        fc3_lo=_ptr(w.get("fc3.weight.lo")), fc3_mean_fix=int(fc3_mean_fix))
    if pair_bias is None:
        _lib.check(_lib.load(variant).pf_transition_fwd(ctypes.byref(a)), "pf_transition_fwd", variant)
        return
    s, w_apb, n_heads, apb_ws, eps_apb = pair_bias
    b = _apb_args(s, s, out, None, s, w_apb, n_heads, apb_ws, False, eps_apb, 0)
    _lib.check(_lib.load(variant).pf_transition_pair_bias_fwd(ctypes.byref(a), ctypes.byref(b)),
               "pf_transition_pair_bias_fwd", variant)


def apb_workspace_bytes(B: int, N: int, c_s: int, H: int, variant: str = DEFAULT_VARIANT) -> int:
    return _lib.load(variant).pf_apb_workspace_size(B, N, c_s, H)


def _apb_args(s: torch.Tensor, k_in: torch.Tensor, z: torch.Tensor, mask: Optional[torch.Tensor],
              out: torch.Tensor, w: Mapping[str, torch.Tensor], n_heads: int, ws: torch.Tensor,
              accumulate: bool, eps: float, n_valid: int):
    B, N, c_s = s.shape
    return _lib.ApbArgs(
        B=B, N=N, c_s=c_s, C=z.shape[-1], H=n_heads, accumulate=int(accumulate), n_valid=n_valid, eps=eps,
        s=_ptr(s), k_in=_ptr(k_in), z=_ptr(z), mask=_ptr(mask), out=_ptr(out),
        w_q=_ptr(w["proj_q.weight"]), b_q=_ptr(w["proj_q.bias"]), w_k=_ptr(w["proj_k.weight"]),
        w_v=_ptr(w["proj_v.weight"]), w_g=_ptr(w["proj_g.weight"]), w_o=_ptr(w["proj_o.weight"]),
        zln_w=_ptr(w["proj_z.0.weight"]), zln_b=_ptr(w["proj_z.0.bias"]), w_z=_ptr(w["proj_z.1.weight"]),
        workspace=_ptr(ws), workspace_bytes=ws.numel(), stream=_stream())


def launch_apb(s: torch.Tensor, k_in: torch.Tensor, z: torch.Tensor, mask: Optional[torch.Tensor],
               out: torch.Tensor, w: Mapping[str, torch.Tensor], n_heads: int, ws: torch.Tensor,
               accumulate: bool, eps: float = 1e-5, n_valid: int = 0, variant: str = DEFAULT_VARIANT,
               part: str = "all", fast: bool = False) -> None:
    """AttentionPairBias on the current stream.  ``part``: "all" (pf_apb_fwd), "bias" (only
    the z-dependent pair bias into ``ws``, pf_apb_pair_bias) or "attend" (the rest, reading
    the bias a previous "bias" call left in ``ws``, pf_apb_attend).  ``fast``: the fast-mode
    entry points (o * sigmoid(g) in MXFP8 before the output projection)."""
    a = _apb_args(s, k_in, z, mask, out, w, n_heads, ws, accumulate, eps, n_valid)
    if fast:
        fn = {"all": "pf_apb_fwd_mx8", "bias": "pf_apb_pair_bias", "attend": "pf_apb_attend_mx8"}[part]
    else:
        fn = {"all": "pf_apb_fwd", "bias": "pf_apb_pair_bias", "attend": "pf_apb_attend"}[part]
    _lib.check(getattr(_lib.load(variant), fn)(ctypes.byref(a)), fn, variant)


def launch_layernorm(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor, out: torch.Tensor,
                     eps: float = 1e-5, variant: str = DEFAULT_VARIANT) -> None:
    C = x.shape[-1]
    _lib.check(_lib.load(variant).pf_layernorm_fwd(_ptr(x), _ptr(w), _ptr(b), _ptr(out), x.numel() // C, C, eps,
                                                   _stream()), "pf_layernorm_fwd", variant)


def launch_linear(x: torch.Tensor, w: torch.Tensor, bias: Optional[torch.Tensor],
                  resid: Optional[torch.Tensor], out: torch.Tensor, variant: str = DEFAULT_VARIANT) -> None:
    K = x.shape[-1]
    _lib.check(_lib.load(variant).pf_linear_fwd(_ptr(x), _ptr(w), _ptr(bias), _ptr(resid), _ptr(out),
                                                x.numel() // K, K, w.shape[0], _stream()), "pf_linear_fwd", variant)


def launch_pair_ln_linear(x: torch.Tensor, base: torch.Tensor, ln_w: torch.Tensor, ln_b: torch.Tensor,
                          w: torch.Tensor, out: torch.Tensor, eps: float = 1e-5,
                          variant: str = DEFAULT_VARIANT, w_lo: Optional[torch.Tensor] = None) -> None:
    """out = base + W . LN(x) per pair; with ``w_lo`` (``opw_lo`` of the weight) to ~fp32 accuracy."""
    C = x.shape[-1]
    _lib.check(_lib.load(variant).pf_pair_ln_linear_fwd(_ptr(x), _ptr(base), _ptr(ln_w), _ptr(ln_b), _ptr(w),
                                                        _ptr(w_lo), _ptr(out), x.numel() // C, C, eps, _stream()),
               "pf_pair_ln_linear_fwd", variant)


def launch_add(a: torch.Tensor, b: torch.Tensor, out: torch.Tensor, variant: str = DEFAULT_VARIANT) -> None:
    """out = a + b (fp32, same element count): the ``z = z + module(z)`` hand-off of the trunk loop."""
    if not (a.numel() == b.numel() == out.numel()):
        raise ValueError(f"launch_add: element counts differ ({a.numel()}, {b.numel()}, {out.numel()})")
    _lib.check(_lib.load(variant).pf_add_fwd(_ptr(a), _ptr(b), _ptr(out), a.numel(), _stream()), "pf_add_fwd",
               variant)


def launch_pair_cond_proj(z: torch.Tensor, rel_pos: torch.Tensor, ln_w: torch.Tensor, ln_b: torch.Tensor,
                          w: torch.Tensor, out: torch.Tensor, eps: float = 1e-5,
                          variant: str = DEFAULT_VARIANT) -> None:
    """out = W . LN(cat(z, rel_pos)) (PairwiseConditioning's input projection)."""
    C = z.shape[-1]
    _lib.check(_lib.load(variant).pf_pair_cond_proj_fwd(_ptr(z), _ptr(rel_pos), _ptr(ln_w), _ptr(ln_b), _ptr(w),
                                                        _ptr(out), z.numel() // C, C, eps, _stream()),
               "pf_pair_cond_proj_fwd", variant)


def launch_token_pair_bias(z: torch.Tensor, ln_w: torch.Tensor, ln_b: torch.Tensor, w: torch.Tensor,
                           out: torch.Tensor, n_layers: int, n_heads: int, layout: int = 0, scale: float = 1.0,
                           eps: float = 1e-5, variant: str = DEFAULT_VARIANT) -> None:
    """Token-transformer pair bias: out = scale * cat_l(LN_l(z) W_l^T) (layout 0: [..., L*H];
    layout 1: [L*H][rows])."""
    C = z.shape[-1]
    _lib.check(_lib.load(variant).pf_token_pair_bias_fwd(_ptr(z), _ptr(ln_w), _ptr(ln_b), _ptr(w), _ptr(out),
                                                         z.numel() // C, C, n_layers, n_heads, layout, scale, eps,
                                                         _stream()), "pf_token_pair_bias_fwd", variant)


def launch_batched_nt_gemm(A: torch.Tensor, B: torch.Tensor, X: torch.Tensor, scale: float = 1.0,
                           variant: str = DEFAULT_VARIANT) -> None:
    """X[p] = scale * A[p] @ B[p]^T (pf_batched_nt_gemm): A [P,M,K], B [P,Nc,K] operand type,
    X [P,M,Nc] fp32 or operand type."""
    P, M, K = A.shape
    Nc = B.shape[1]
    _lib.check(_lib.load(variant).pf_batched_nt_gemm(_ptr(A), _ptr(B), _ptr(X), int(X.dtype == torch.float32), P, M,
                                                     Nc, K, float(scale), _stream()), "pf_batched_nt_gemm", variant)


def launch_trimul_contract(opA: torch.Tensor, opB: torch.Tensor, X: torch.Tensor,
                           variant: str = DEFAULT_VARIANT) -> None:
    """X fp32 -> unscaled fp32 output; X in the operand dtype -> 2^-8-scaled (pf_trimul_fwd's format)."""
    planes, N = opA.shape[0], opA.shape[1]
    _lib.check(_lib.load(variant).pf_trimul_contract(_ptr(opA), _ptr(opB), _ptr(X), int(X.dtype == torch.float32),
                                                     planes, N, _stream()), "pf_trimul_contract", variant)


# --------------------------------------------------------------------------------------
# fast mode (MXFP8: e4m3 elements, one E8M0 scale per 32 along the contraction axis)
# --------------------------------------------------------------------------------------
FAST_PAD = 128     # the fp8 triangle multiplication works on N % 128 == 0


def quantize_mx8(x: torch.Tensor, perm: int = 0, variant: str = DEFAULT_VARIANT):
    """fp32 [rows, K] device tensor -> (e4m3 bytes uint8 [rows, K], E8M0 scales uint8 [rows, K/32]).
    ``perm=1`` stores each 32-block in accumulator order (the fc3.weight layout)."""
    _require_gpu(x)
    xf = x.detach().to(torch.float32).contiguous()
    rows, K = xf.shape
    q = torch.empty((rows, K), dtype=torch.uint8, device=xf.device)
    s = torch.empty((rows, K // 32), dtype=torch.uint8, device=xf.device)
    _lib.check(_lib.load(variant).pf_quantize_mx8(_ptr(xf), rows, K, perm, _ptr(q), _ptr(s), _stream()),
               "pf_quantize_mx8", variant)
    return q, s


def mx8_weights(w: Mapping[str, torch.Tensor], device: torch.device, keys_perm: Mapping[str, int],
                variant: str = DEFAULT_VARIANT) -> dict:
    """Quantize the matrices named in ``keys_perm`` (key -> perm) once, on the device:
    returns {key + ".q": bytes, key + ".s": scales}."""
    out = {}
    for k, perm in keys_perm.items():
        q, s = quantize_mx8(w[k].to(device=device, dtype=torch.float32), perm, variant)
        out[k + ".q"], out[k + ".s"] = q, s
    return out


def trimul_mx8_workspace_bytes(B: int, N: int, variant: str = DEFAULT_VARIANT) -> int:
    return _lib.load(variant).pf_trimul_mx8_workspace_size(B, N, C_Z)


def launch_trimul_mx8(z_in: torch.Tensor, out: torch.Tensor, pair_mask: Optional[torch.Tensor],
                      w: Mapping[str, torch.Tensor], direction: int, ws: torch.Tensor, accumulate: bool,
                      eps: float = 1e-5, variant: str = DEFAULT_VARIANT) -> None:
    """``w``: fp32 LayerNorm params plus ``p_in.weight.q`` / ``.s`` ... from mx8_weights."""
    B, N, _, C = z_in.shape
    a = _lib.TrimulMx8Args(
        B=B, N=N, C=C, hidden=C, direction=direction, accumulate=int(accumulate), eps=eps,
        z_in=_ptr(z_in), out=_ptr(out), pair_mask=_ptr(pair_mask),
        norm_in_w=_ptr(w["norm_in.weight"]), norm_in_b=_ptr(w["norm_in.bias"]),
        p_in_q=_ptr(w["p_in.weight.q"]), p_in_s=_ptr(w["p_in.weight.s"]),
        g_in_q=_ptr(w["g_in.weight.q"]), g_in_s=_ptr(w["g_in.weight.s"]),
        norm_out_w=_ptr(w["norm_out.weight"]), norm_out_b=_ptr(w["norm_out.bias"]),
        p_out_q=_ptr(w["p_out.weight.q"]), p_out_s=_ptr(w["p_out.weight.s"]),
        g_out_q=_ptr(w["g_out.weight.q"]), g_out_s=_ptr(w["g_out.weight.s"]),
        workspace=_ptr(ws), workspace_bytes=ws.numel(), stream=_stream())
    _lib.check(_lib.load(variant).pf_trimul_mx8_fwd(ctypes.byref(a)), "pf_trimul_mx8_fwd", variant)


def triatt_mx8_workspace_bytes(B: int, N: int, n_heads: int = 4, head_dim: int = 32,
                               variant: str = DEFAULT_VARIANT) -> int:
    return _lib.load(variant).pf_triatt_mx8_workspace_size(B, N, C_Z, n_heads, head_dim)


def launch_triatt_mx8(z_in: torch.Tensor, out: torch.Tensor, pair_mask: Optional[torch.Tensor],
                      w: Mapping[str, torch.Tensor], ending: bool, ws: torch.Tensor, accumulate: bool,
                      n_heads: int = 4, head_dim: int = 32, eps: float = 1e-5, n_valid: int = 0,
                      variant: str = DEFAULT_VARIANT) -> None:
    """``w``: fp32 LayerNorm params, op-type ``linear.weight`` / ``linear_o.weight`` and
    ``linear_{q,k,v,g}.weight.q`` / ``.s`` from mx8_weights."""
    B, N, _, C = z_in.shape
    a = _lib.TriattMx8Args(
        B=B, N=N, C=C, H=n_heads, D=head_dim, ending=int(ending), accumulate=int(accumulate), n_valid=n_valid,
        eps=eps, z_in=_ptr(z_in), out=_ptr(out), pair_mask=_ptr(pair_mask),
        ln_w=_ptr(w["layer_norm.weight"]), ln_b=_ptr(w["layer_norm.bias"]), w_bias=_ptr(w["linear.weight"]),
        w_q_q=_ptr(w["linear_q.weight.q"]), w_q_s=_ptr(w["linear_q.weight.s"]),
        w_k_q=_ptr(w["linear_k.weight.q"]), w_k_s=_ptr(w["linear_k.weight.s"]),
        w_v_q=_ptr(w["linear_v.weight.q"]), w_v_s=_ptr(w["linear_v.weight.s"]),
        w_g_q=_ptr(w["linear_g.weight.q"]), w_g_s=_ptr(w["linear_g.weight.s"]), w_o=_ptr(w["linear_o.weight"]),
        workspace=_ptr(ws), workspace_bytes=ws.numel(), stream=_stream())
    _lib.check(_lib.load(variant).pf_triatt_mx8_fwd(ctypes.byref(a)), "pf_triatt_mx8_fwd", variant)


def launch_transition_mx8(x_in: torch.Tensor, out: torch.Tensor, w: Mapping[str, torch.Tensor],
                          accumulate: bool, eps: float = 1e-5, variant: str = DEFAULT_VARIANT,
                          pair_bias: Optional[tuple] = None) -> None:
    """``pair_bias`` as in :func:`launch_transition` (pf_transition_mx8_pair_bias_fwd)."""
    C = x_in.shape[-1]
    a = _lib.TransitionMx8Args(
        rows=x_in.numel() // C, C=C, hidden=w["fc1.weight.q"].shape[0], accumulate=int(accumulate), eps=eps,
        x_in=_ptr(x_in), out=_ptr(out), norm_w=_ptr(w["norm.weight"]), norm_b=_ptr(w["norm.bias"]),
        fc1_q=_ptr(w["fc1.weight.q"]), fc1_s=_ptr(w["fc1.weight.s"]),
        fc2_q=_ptr(w["fc2.weight.q"]), fc2_s=_ptr(w["fc2.weight.s"]),
        fc3_q=_ptr(w["fc3.weight.q"]), fc3_s=_ptr(w["fc3.weight.s"]), stream=_stream())
    if pair_bias is None:
        _lib.check(_lib.load(variant).pf_transition_mx8_fwd(ctypes.byref(a)), "pf_transition_mx8_fwd", variant)
        return
    s, w_apb, n_heads, apb_ws, eps_apb = pair_bias
    b = _apb_args(s, s, out, None, s, w_apb, n_heads, apb_ws, False, eps_apb, 0)
    _lib.check(_lib.load(variant).pf_transition_mx8_pair_bias_fwd(ctypes.byref(a), ctypes.byref(b)),
               "pf_transition_mx8_pair_bias_fwd", variant)


def launch_trimul_mx8_contract(A8: torch.Tensor, B8: torch.Tensor, SA: torch.Tensor, SB: torch.Tensor,
                               X: torch.Tensor, variant: str = DEFAULT_VARIANT) -> None:
    planes, N = A8.shape[0], A8.shape[1]
    _lib.check(_lib.load(variant).pf_trimul_mx8_contract(_ptr(A8), _ptr(B8), _ptr(SA), _ptr(SB), _ptr(X), planes,
                                                         N, _stream()), "pf_trimul_mx8_contract", variant)


TRIMUL_MX8_KEYS = {"p_in.weight": 0, "g_in.weight": 0, "p_out.weight": 0, "g_out.weight": 0}
#: fast-mode triangle attention: the q/k/v/g projections (the reference's bfloat8_b weights,
#: ``tenstorrent.py:526-539``); the triangle-bias and output weights stay 16-bit
TRIATT_MX8_KEYS = {"linear_q.weight": 0, "linear_k.weight": 0, "linear_v.weight": 0, "linear_g.weight": 0}
TRANSITION_MX8_KEYS = {"fc1.weight": 0, "fc2.weight": 0, "fc3.weight": 1}


# --------------------------------------------------------------------------------------
# public functional API (mirrors of the reference operators)
# --------------------------------------------------------------------------------------
def _as_b4(x: torch.Tensor):
    return (x.unsqueeze(0), True) if x.dim() == 3 else (x, False)


def triangle_multiplicative_update(x: torch.Tensor, direction: str = "outgoing",
                                   mask: Optional[torch.Tensor] = None,
                                   norm_in_weight=None, norm_in_bias=None, p_in_weight=None,
                                   g_in_weight=None, norm_out_weight=None, norm_out_bias=None,
                                   p_out_weight=None, g_out_weight=None, eps: float = 1e-5,
                                   variant: str = DEFAULT_VARIANT) -> torch.Tensor:
    """Fused triangle multiplicative update; the contract of
    ``kernel_triangular_mult`` (``tt_bio/boltz2.py:820-848``) with the semantics of
    ``TriangleMultiplication{Outgoing,Incoming}.forward(use_kernels=False)``
    (``tt_bio/reference.py:455-472, 544-561``).  Returns the update (fp32)."""
    if direction not in ("outgoing", "incoming"):
        raise ValueError(f"direction must be 'outgoing' or 'incoming', got {direction!r}")
    x, squeezed = _as_b4(x)
    dev = _require_gpu(x)
    B, N, _, C = x.shape
    n_pad = padded_len(N)
    zp = pad_pair(x.to(torch.float32), n_pad) if n_pad != N else x.to(torch.float32).contiguous()
    m3 = None if mask is None else (mask.unsqueeze(0) if mask.dim() == 2 else mask)
    if m3 is not None and n_pad == N and tuple(m3.shape) == (B, N, N):
        mp = m3.to(device=dev, dtype=torch.float32).contiguous()   # read-only: no padded copy needed
    else:
        mp = pad_pair_mask(m3, B, N, n_pad, dev)
    w = convert_weights({"norm_in.weight": norm_in_weight, "norm_in.bias": norm_in_bias,
                         "p_in.weight": p_in_weight, "g_in.weight": g_in_weight,
                         "norm_out.weight": norm_out_weight, "norm_out.bias": norm_out_bias,
                         "p_out.weight": p_out_weight, "g_out.weight": g_out_weight}, dev, variant)
    out = torch.empty_like(zp)
    ws = workspace(trimul_workspace_bytes(B, n_pad, variant), dev)
    launch_trimul(zp, out, mp, w, 0 if direction == "outgoing" else 1, ws, accumulate=False, eps=eps,
                  variant=variant)
    out = out[:, :N, :N] if n_pad != N else out
    return out[0] if squeezed else out


def triangle_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, bias: torch.Tensor,
                       mask: Optional[torch.Tensor] = None, scale: Optional[float] = None,
                       variant: str = DEFAULT_VARIANT) -> torch.Tensor:
    """Triangle attention core; the contract of ``kernel_triangular_attn(q, k, v,
    tri_bias, mask, scale)`` (``tt_bio/boltz2.py:815-817``) with the semantics of the
    ``use_kernels=False`` path (``tt_bio/reference.py:176-190``, ``boltz2.py:790-810``).

    q, k, v: [B, I, H, J, D]; bias: [B, 1, H, J, K]; mask: [B, I, 1, 1, K] (bool or
    0/1) or None; I = J = K.  Returns o [B, I, H, J, D] fp32."""
    dev = _require_gpu(q, k, v, bias)
    B, I, H, J, D = q.shape
    if not (I == J == k.shape[3] == v.shape[3]):
        raise ValueError("triangle_attention expects I == J == K (square pair grid)")
    if scale is None:
        scale = D ** -0.5
    N = J
    n_pad = padded_len(N)

    def padq(t):
        t = t.to(torch.float32)
        if n_pad == N:
            return t.contiguous()
        o = torch.zeros((B, n_pad, H, n_pad, D), dtype=torch.float32, device=dev)
        o[:, :N, :, :N] = t
        return o

    qp, kp, vp = padq(q), padq(k), padq(v)
    if n_pad == N:   # no padding: the caller's bias and mask as they are (fp32, contiguous)
        bp = bias.reshape(B, H, N, N).to(torch.float32).contiguous()
        mp = None if mask is None else mask.reshape(B, N, N).to(torch.float32).contiguous()
    else:
        bp = torch.zeros((B, H, n_pad, n_pad), dtype=torch.float32, device=dev)
        bp[:, :, :N, :N] = bias.reshape(B, H, N, N)
        mp = torch.zeros((B, n_pad, n_pad), dtype=torch.float32, device=dev)
        mp[:, :N, :N] = 1.0 if mask is None else mask.reshape(B, N, N).to(torch.float32)
    o = torch.empty((B, n_pad, H, n_pad, D), dtype=torch.float32, device=dev)
    lib = _lib.load(variant)
    ws = workspace(lib.pf_tri_attention_workspace_size(B, n_pad, H, D), dev)
    _lib.check(lib.pf_tri_attention(_ptr(qp), _ptr(kp), _ptr(vp), _ptr(bp), _ptr(mp), float(scale), _ptr(o),
                                    B, n_pad, H, D, N, _ptr(ws), ws.numel(), _stream()), "pf_tri_attention", variant)
    return o[:, :N, :, :N] if n_pad != N else o


def transition(x: torch.Tensor, norm_weight, norm_bias, fc1_weight, fc2_weight, fc3_weight,
               eps: float = 1e-5, variant: str = DEFAULT_VARIANT) -> torch.Tensor:
    """``Transition.forward`` (``tt_bio/boltz2.py:1227-1258``): returns fc3(silu(fc1 LN x) * fc2 LN x)."""
    dev = _require_gpu(x)
    xin = x.to(torch.float32).contiguous()
    w = convert_weights({"norm.weight": norm_weight, "norm.bias": norm_bias, "fc1.weight": fc1_weight,
                         "fc2.weight": fc2_weight, "fc3.weight": fc3_weight}, dev, variant)
    C = xin.shape[-1]
    out = torch.empty_like(xin)
    nb = transition_workspace_bytes(xin.numel() // C, C, fc1_weight.shape[0], variant)
    launch_transition(xin, out, w, workspace(nb, dev) if nb else None, accumulate=False, eps=eps, variant=variant)
    return out


def attention_pair_bias(s: torch.Tensor, z: torch.Tensor, mask: Optional[torch.Tensor], k_in: torch.Tensor,
                        weights: Mapping[str, torch.Tensor], num_heads: int = 16,
                        eps: float = 1e-5, variant: str = DEFAULT_VARIANT, fast: bool = False) -> torch.Tensor:
    """``AttentionPairBias.forward`` (``tt_bio/boltz2.py:343-367``, multiplicity 1).
    ``weights`` uses the module's state-dict keys (``proj_q.weight`` ...).  ``fast``: the
    fast-mode entry point (o * sigmoid(g) in MXFP8, ``tt_bio/tenstorrent.py:846``)."""
    dev = _require_gpu(s, z, k_in)
    B, N, c_s = s.shape
    n_pad = padded_len(N)

    def pad_tokens(t):   # [B, N, c] -> [B, n_pad, c] fp32; read-only, so no copy when N needs no padding
        if n_pad == N:
            return t.to(torch.float32).contiguous()
        o = torch.zeros((B, n_pad) + tuple(t.shape[2:]), dtype=torch.float32, device=dev)
        o[:, :N] = t
        return o
    sp, kp = pad_tokens(s), pad_tokens(k_in)
    zp = pad_pair(z.to(torch.float32), n_pad) if n_pad != N else z.to(torch.float32).contiguous()
    if mask is not None and n_pad == N:
        mp = mask.to(device=dev, dtype=torch.float32).contiguous()
    else:
        mp = torch.zeros((B, n_pad), dtype=torch.float32, device=dev)
        mp[:, :N] = 1.0 if mask is None else mask.to(torch.float32)
    w = convert_weights(weights, dev, variant)
    out = torch.empty_like(sp)
    ws = workspace(apb_workspace_bytes(B, n_pad, c_s, num_heads, variant), dev)
    launch_apb(sp, kp, zp, mp, out, w, num_heads, ws, accumulate=False, eps=eps, n_valid=N, variant=variant,
               fast=fast)
    return out[:, :N]


def layer_norm(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    dev = _require_gpu(x)
    xin = x.to(torch.float32).contiguous()
    out = torch.empty_like(xin)
    launch_layernorm(xin, f32(weight, dev), f32(bias, dev), out, eps)
    return out


def linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None,
           variant: str = DEFAULT_VARIANT) -> torch.Tensor:
    dev = _require_gpu(x)
    xin = x.to(torch.float32).contiguous()
    out = torch.empty(xin.shape[:-1] + (weight.shape[0],), dtype=torch.float32, device=dev)
    launch_linear(xin, opw(weight, dev, variant), f32(bias, dev), None, out, variant)
    return out


# --------------------------------------------------------------------------------------
# MSA module
# --------------------------------------------------------------------------------------
def opm_workspace_bytes(B: int, S: int, N: int, variant: str = DEFAULT_VARIANT) -> int:
    return _lib.load(variant).pf_opm_workspace_size(B, S, N)


def launch_opm(m: torch.Tensor, msa_mask: Optional[torch.Tensor], z: torch.Tensor, w: Mapping[str, torch.Tensor],
               ws: torch.Tensor, accumulate: bool = True, eps: float = 1e-5, variant: str = DEFAULT_VARIANT) -> None:
    """z (+)= OuterProductMean(m, msa_mask) (pf_opm_fwd); m [B,S,N,64], z [B,N,N,128]."""
    B, S, N, c_m = m.shape
    a = _lib.OpmArgs(
        B=B, S=S, N=N, c_m=c_m, c_hidden=w["proj_a.weight"].shape[0], C=z.shape[-1], accumulate=int(accumulate),
        eps=eps, m=_ptr(m), msa_mask=_ptr(msa_mask), z=_ptr(z), norm_w=_ptr(w["norm.weight"]),
        norm_b=_ptr(w["norm.bias"]), w_a=_ptr(w["proj_a.weight"]), w_b=_ptr(w["proj_b.weight"]),
        w_o=_ptr(w["proj_o.weight"]), b_o=_ptr(w["proj_o.bias"]),
        workspace=_ptr(ws), workspace_bytes=ws.numel(), stream=_stream())
    _lib.check(_lib.load(variant).pf_opm_fwd(ctypes.byref(a)), "pf_opm_fwd", variant)


def pwa_workspace_bytes(B: int, S: int, N: int, variant: str = DEFAULT_VARIANT) -> int:
    return _lib.load(variant).pf_pwa_workspace_size(B, S, N)


def launch_pwa(m: torch.Tensor, z: torch.Tensor, pair_mask: Optional[torch.Tensor], out: torch.Tensor,
               w: Mapping[str, torch.Tensor], ws: torch.Tensor, accumulate: bool = True, eps: float = 1e-5,
               variant: str = DEFAULT_VARIANT) -> None:
    """out = (m if accumulate) + PairWeightedAveraging(m, z, pair_mask) (pf_pwa_fwd)."""
    B, S, N, c_m = m.shape
    H = w["proj_z.weight"].shape[0]
    a = _lib.PwaArgs(
        B=B, S=S, N=N, c_m=c_m, C=z.shape[-1], H=H, c_h=w["proj_m.weight"].shape[0] // H,
        accumulate=int(accumulate), eps=eps, m=_ptr(m), out=_ptr(out), z=_ptr(z), pair_mask=_ptr(pair_mask),
        norm_m_w=_ptr(w["norm_m.weight"]), norm_m_b=_ptr(w["norm_m.bias"]), norm_z_w=_ptr(w["norm_z.weight"]),
        norm_z_b=_ptr(w["norm_z.bias"]), w_m=_ptr(w["proj_m.weight"]), w_g=_ptr(w["proj_g.weight"]),
        w_z=_ptr(w["proj_z.weight"]), w_o=_ptr(w["proj_o.weight"]),
        workspace=_ptr(ws), workspace_bytes=ws.numel(), stream=_stream())
    _lib.check(_lib.load(variant).pf_pwa_fwd(ctypes.byref(a)), "pf_pwa_fwd", variant)


def launch_msa_embed(msa: torch.Tensor, has_deletion: Optional[torch.Tensor], deletion_value: Optional[torch.Tensor],
                     msa_paired: Optional[torch.Tensor], s_emb: torch.Tensor, w_t: torch.Tensor, m: torch.Tensor,
                     variant: str = DEFAULT_VARIANT) -> None:
    """m = msa_proj(one_hot features) + s_emb (pf_msa_embed); msa int32 [B,S,N]."""
    B, S, N = msa.shape
    _lib.check(_lib.load(variant).pf_msa_embed(_ptr(msa), _ptr(has_deletion), _ptr(deletion_value), _ptr(msa_paired),
                                               _ptr(s_emb), _ptr(w_t), _ptr(m), B, S, N, m.shape[-1],
                                               w_t.shape[0] - 3, _stream()), "pf_msa_embed", variant)
