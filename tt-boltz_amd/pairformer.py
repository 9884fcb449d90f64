"""Drop-in Pairformer modules for MI355X (PyTorch-ROCm host, HIP kernels).

Mirrors the call surface of the Tenstorrent path in ``tt_bio/tenstorrent.py``:

* ``PairformerModule`` (``tenstorrent.py:2194-2284``, an ``nn.Module`` built by
  ``TorchWrapper``, ``2113-2191``): same constructor, ``load_state_dict`` (weights
  are taken from the state dict at load time, no parameters are registered),
  ``forward(s, z, mask=None, pair_mask=None, use_kernels=False) -> (s, z)`` and
  ``reset_static_cache()``; pads N to a multiple of 64 and slices back; masks are
  built on the first forward after a reset and reused.
* ``Pairformer`` / ``PairformerLayer`` / ``TriangleMultiplication`` /
  ``TriangleAttention`` / ``Transition`` / ``AttentionPairBias`` with the
  reference names and weight keys (``tenstorrent.py:351-1083``), operating on
  device-resident padded tensors.
* ``WeightScope``, ``get_device``, ``set_fast_mode``.

Numerics follow the reference CPU modules (``tt_bio/reference.py``), not the
Tenstorrent approximations: the pair mask multiplies both trimul operands
(``reference.py:461``), triangle attention masks per (row, key) with 1e9
(``reference.py:334-335``), single attention masks keys with 1e6
(``boltz2.py:362``), and the pair bias is added unscaled after q/sqrt(d)
(``reference.py:117-118``).  The residual stream z and s are fp32; MFMA operands
are fp16 by default (``Options(operand="bf16")`` selects bf16 operands).
"""
from __future__ import annotations

from types import MappingProxyType
from typing import Mapping, Optional

import torch
from torch import nn

from . import ops

_FAST_MODE = False
_device: Optional[torch.device] = None

C_Z = 128
#: pair widths the kernels are built for: the trunk (128) and the template stack (64)
C_Z_SUPPORTED = (128, 64)


def set_fast_mode(enabled: bool) -> None:
    """``tenstorrent.py:178-181``: process-global block-fp8 switch, read at module construction."""
    global _FAST_MODE
    _FAST_MODE = bool(enabled)


def get_device() -> torch.device:
    """The process's GPU (one device per process, like ``tenstorrent.py:213-243``)."""
    global _device
    if _device is None:
        if not torch.cuda.is_available():
            raise RuntimeError("no ROCm GPU visible: the Pairformer HIP kernels have no CPU path")
        _device = torch.device("cuda", torch.cuda.current_device())
    return _device


class WeightScope(Mapping):
    """Read-only state-dict view with the reference's scoping interface
    (``tenstorrent.py:261-293``: ``wrap``, ``data``, ``as_dict``, ``[key]``, ``child``).

    ``child("a.b", strip_prefix="mha.")`` re-roots the view at ``a.b.``: a key
    ``a.b.mha.linear_q.weight`` is seen as ``linear_q.weight``, ``a.b.layer_norm.weight`` as
    ``layer_norm.weight``; keys outside the scope are dropped."""

    __slots__ = ("_items",)

    def __init__(self, data: Mapping[str, torch.Tensor]):
        self._items = MappingProxyType(dict(data))

    @classmethod
    def wrap(cls, data) -> "WeightScope":
        if isinstance(data, WeightScope):
            return data
        return cls(data)

    @property
    def data(self) -> Mapping[str, torch.Tensor]:
        return self._items

    def as_dict(self) -> dict:
        return dict(self._items)

    def __getitem__(self, key: str) -> torch.Tensor:
        return self._items[key]

    def __iter__(self):
        return iter(self._items)

    def __len__(self) -> int:
        return len(self._items)

    @staticmethod
    def _relative(key: str, root: str, strip: str) -> Optional[str]:
        """``key`` seen from ``root`` (None if outside it), with a leading ``strip`` removed."""
        n = len(root)
        if key[n:n + 1] != "." or not key.startswith(root):
            return None
        rest = key[n + 1:]
        return rest[len(strip):] if strip and rest.startswith(strip) else rest

    def child(self, scope: str, strip_prefix: str = "") -> "WeightScope":
        if not scope:
            return self
        picked = {}
        for key, value in self._items.items():
            rel = self._relative(key, scope, strip_prefix)
            if rel:
                picked[rel] = value
        return WeightScope(picked)


class Options:
    """Replaces ttnn's ``compute_kernel_config``: numerics knobs shared by the kernels.

    ``operand``: MFMA operand type, ``"fp16"`` (default) or ``"bf16"``.
    ``overlap_single``: run each layer's single-track update on a second stream, overlapped
    with the next layer's pair operations (results are identical; default on).
    ``single_delay``: how many of the next layer's pair operations (0-4) go ahead of the
    overlapped single track (it then starts beside the following ones).  The default 1 keeps it
    off the outgoing triangle multiplication, whose contraction it slows the most (N = 512:
    1.254 vs 1.263 ms per layer with 0; 1.269 with 2, 1.308 with 4).
    ``weight_residuals``: the pair kernels whose weights fit twice in LDS (the triangle
    attention's gate and output projection, the triangle multiplication's output projection,
    the recycling projection; the pair transition's output projection when the mean correction
    is off or the batch is larger than one) take each 16-bit weight together with its rounding
    residual and multiply by both (default on).  A 16-bit weight's rounding error is the same at
    every position, so it adds up coherently through a deep stack; with the residual the
    weights are good to ~2^-22 of their size.
    ``mean_correction``: the weights after a LayerNorm whose LDS does not hold them twice (the
    triangle multiplication's p_in, g_in, g_out; the triangle attention's q, k, v and bias
    projections) get the exact W . beta offsets plus the mean correction
    (W - W16) . (gamma * mu), mu the mean over positions of the normalized input, estimated per
    call from sampled positions: the part of their rounding error that every position shares.
    The pair transition's fc3 then takes its residual the same way, (W - W16) . mean(h) over the
    hidden activations of sampled positions, instead of as the hi + lo product (default on;
    c_z = 128, batch 1)."""

    def __init__(self, eps: float = 1e-5, operand: str = ops.DEFAULT_VARIANT, overlap_single: bool = True,
                 single_delay: int = 1, weight_residuals: bool = True, mean_correction: bool = True):
        if operand not in ops.TORCH_DTYPE:
            raise ValueError(f"operand must be one of {sorted(ops.TORCH_DTYPE)}, got {operand!r}")
        if not 0 <= single_delay <= 4:
            raise ValueError(f"single_delay must be in 0..4, got {single_delay}")
        self.eps = eps
        self.operand = operand
        self.overlap_single = overlap_single
        self.single_delay = single_delay
        self.weight_residuals = weight_residuals
        self.mean_correction = mean_correction


class Module:
    """Base: holds a weight scope and converts weights to device tensors once.

    ``fast`` is the process-global fast mode at construction time (the reference reads
    it when it builds the modules, ``tenstorrent.py:537-539``): the triangle
    multiplications, the triangle attentions' q/k/v/g projections and the pair transition
    then keep MXFP8 weights and run the fast-mode kernels, and the single-track attention
    quantizes its gated output (``tenstorrent.py:846``)."""

    def __init__(self, state_dict, options: Optional[Options] = None):
        self.weights = WeightScope.wrap(state_dict)
        self.options = options or Options()
        self.device = get_device()
        self.fast = _FAST_MODE

    @property
    def variant(self) -> str:
        return self.options.operand

    def scope(self, scope: str, strip_prefix: str = "") -> WeightScope:
        return self.weights.child(scope, strip_prefix)

    def mat(self, key: str) -> torch.Tensor:
        return ops.opw(self.weights[key], self.device, self.variant)

    def mat_lo(self, key: str) -> torch.Tensor:
        """The rounding residual of ``mat(key)`` (``ops.opw_lo``)."""
        return ops.opw_lo(self.weights[key], self.device, self.variant)

    def vec(self, key: str) -> torch.Tensor:
        return ops.f32(self.weights[key], self.device)


class TriangleMultiplication(Module):
    """``tenstorrent.py:351-503``; ``ending=True`` is the incoming direction."""

    def __init__(self, ending: bool, state_dict, options: Optional[Options] = None):
        super().__init__(state_dict, options)
        self.ending = ending
        self.C = self.weights["p_in.weight"].shape[1]
        if self.C not in C_Z_SUPPORTED or self.weights["p_in.weight"].shape != (2 * self.C, self.C):
            raise NotImplementedError(f"only c_z in {C_Z_SUPPORTED} is supported "
                                      f"(p_in {tuple(self.weights['p_in.weight'].shape)})")
        # the fp8 kernels are built for c_z = 128; the template stack (c_z = 64) stays 16-bit
        self.fast = self.fast and self.C == C_Z
        self.w = {k: self.vec(k) for k in ("norm_in.weight", "norm_in.bias", "norm_out.weight", "norm_out.bias")}
        if self.fast:
            self.w.update(ops.mx8_weights(self.weights, self.device, ops.TRIMUL_MX8_KEYS, self.variant))
        else:
            self.w.update({k: self.mat(k) for k in ("p_in.weight", "g_in.weight", "p_out.weight", "g_out.weight")})
            if self.options.weight_residuals and self.C == C_Z:   # p_out to ~fp32 (hi + lo)
                self.w["p_out.weight.lo"] = self.mat_lo("p_out.weight")
            if self.options.mean_correction and self.C == C_Z:
                # the mean correction of the LN_in-side weights: exact W . beta offsets and the
                # residuals of p_in, g_in, g_out
                beta = self.weights["norm_in.bias"].detach().double().cpu()
                self.w["in_offsets"] = torch.cat([self.weights[k].detach().double().cpu() @ beta for k in
                                                  ("p_in.weight", "g_in.weight", "g_out.weight")]).to(
                    device=self.device, dtype=torch.float32)
                self.w.update({k + ".lo": self.mat_lo(k) for k in ("p_in.weight", "g_in.weight", "g_out.weight")})

    def workspace_bytes(self, B: int, N: int) -> int:
        if self.fast:
            return ops.trimul_mx8_workspace_bytes(B, N, self.variant)
        return ops.trimul_workspace_bytes(B, N, self.variant, self.C)

    def __call__(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
                 accumulate: bool = False, ws: Optional[torch.Tensor] = None) -> torch.Tensor:
        """x [B,N,N,c_z] fp32 device, N % 64 == 0 (N % 128 == 0 in fast mode).
        Returns the update (or ``out`` += update)."""
        B, N = x.shape[0], x.shape[1]
        if ws is None:
            ws = ops.workspace(self.workspace_bytes(B, N), x.device)
        if out is None:
            out = torch.empty_like(x)
        if self.fast:
            ops.launch_trimul_mx8(x, out, mask, self.w, int(self.ending), ws, accumulate, self.options.eps,
                                  self.variant)
        else:
            ops.launch_trimul(x, out, mask, self.w, int(self.ending), ws, accumulate, self.options.eps, self.variant)
        return out


class TriangleAttention(Module):
    """``tenstorrent.py:506-650``; weight scope with the ``mha.`` prefix stripped."""

    def __init__(self, head_dim: int, n_heads: int, ending: bool, state_dict, options: Optional[Options] = None,
                 affinity: bool = False):
        super().__init__(state_dict, options)
        if (head_dim, n_heads) != (32, 4):
            raise NotImplementedError(f"only 4 heads x 32 are supported (got {n_heads} x {head_dim})")
        self.head_dim, self.n_heads, self.ending, self.affinity = head_dim, n_heads, ending, affinity
        self.C = self.weights["layer_norm.weight"].shape[0]
        if self.C not in C_Z_SUPPORTED:
            raise NotImplementedError(f"only c_z in {C_Z_SUPPORTED} is supported (got {self.C})")
        # the fast-mode kernels are built for c_z = 128; the template stack (c_z = 64) stays 16-bit
        self.fast = self.fast and self.C == C_Z
        self.w = {k: self.vec(k) for k in ("layer_norm.weight", "layer_norm.bias")}
        self.w.update({k: self.mat(k) for k in ("linear.weight", "linear_o.weight")})
        if self.fast:
            self.w.update(ops.mx8_weights(self.weights, self.device, ops.TRIATT_MX8_KEYS, self.variant))
        else:
            self.w.update({k: self.mat(k) for k in ops.TRIATT_MX8_KEYS})
            if self.options.weight_residuals and self.C == C_Z:
                self.w.update({k + ".lo": self.mat_lo(k) for k in ("linear_g.weight", "linear_o.weight")})
            if self.options.mean_correction and self.C == C_Z:
                # the mean correction of the projection: exact W . beta offsets and the residuals of
                # the kernel's gamma-folded weights op(op(W) diag(gamma))
                keys = ("linear_q.weight", "linear_k.weight", "linear_v.weight", "linear.weight")
                beta = self.weights["layer_norm.bias"].detach().double().cpu()
                gamma = self.weights["layer_norm.weight"].detach().double().cpu()
                self.w["in_offsets"] = torch.cat([self.weights[k].detach().double().cpu() @ beta for k in keys]).to(
                    device=self.device, dtype=torch.float32)
                dt = ops.TORCH_DTYPE[self.variant]
                for k in keys:
                    w64 = self.weights[k].detach().double().cpu()
                    folded = (w64.to(dt).float() * gamma.float()).to(dt)   # as the kernel folds it
                    self.w[k + ".lo"] = (w64 * gamma - folded.double()).to(dt).to(self.device).contiguous()

    def workspace_bytes(self, B: int, N: int) -> int:
        if self.fast:
            return ops.triatt_mx8_workspace_bytes(B, N, self.n_heads, self.head_dim, self.variant)
        return ops.triatt_workspace_bytes(B, N, self.n_heads, self.head_dim, self.variant, self.C)

    def __call__(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
                 accumulate: bool = False, ws: Optional[torch.Tensor] = None, n_valid: int = 0) -> torch.Tensor:
        """``n_valid``: tokens at or beyond it are boundary padding (0 = none)."""
        B, N = x.shape[0], x.shape[1]
        if ws is None:
            ws = ops.workspace(self.workspace_bytes(B, N), x.device)
        if out is None:
            out = torch.empty_like(x)
        launch = ops.launch_triatt_mx8 if self.fast else ops.launch_triatt
        launch(x, out, mask, self.w, self.ending, ws, accumulate, self.n_heads, self.head_dim, self.options.eps,
               n_valid, self.variant)
        return out


class Transition(Module):
    """``tenstorrent.py:856-946`` / ``boltz2.py:1188-1258``."""

    def __init__(self, state_dict, options: Optional[Options] = None, allow_fast: bool = True):
        super().__init__(state_dict, options)
        self.w = {k: self.vec(k) for k in ("norm.weight", "norm.bias")}
        self.C = self.weights["fc1.weight"].shape[1]
        self.hidden = self.weights["fc1.weight"].shape[0]
        # fast mode covers the Pairformer's pair transition (c_z = 128); the single-track
        # one and those outside the Pairformer (allow_fast=False) stay 16-bit
        self.fast = self.fast and allow_fast and self.C == C_Z
        if self.fast:
            self.w.update(ops.mx8_weights(self.weights, self.device, ops.TRANSITION_MX8_KEYS, self.variant))
        else:
            self.w.update({k: self.mat(k) for k in ("fc1.weight", "fc2.weight", "fc3.weight")})
            if self.options.weight_residuals and allow_fast and self.C == C_Z:   # the pair transition
                self.w["fc3.weight.lo"] = self.mat_lo("fc3.weight")

    def workspace_bytes(self, rows: int) -> int:
        if self.fast:
            return 0
        return ops.transition_workspace_bytes(rows, self.C, self.hidden, self.variant)

    def fuses_pair_bias(self) -> bool:
        """Whether ``__call__`` can also produce the single-track pair bias of its output."""
        return self.C == C_Z

    def __call__(self, x: torch.Tensor, out: Optional[torch.Tensor] = None, accumulate: bool = False,
                 ws: Optional[torch.Tensor] = None, pair_bias: Optional[tuple] = None) -> torch.Tensor:
        """``pair_bias = (attention_pair_bias, s, apb_ws)`` (only if ``fuses_pair_bias()``): the
        same kernel also writes the attention's pair bias of the updated ``out`` into
        ``apb_ws``, as ``attention_pair_bias(s, out, ..., part="bias")`` would."""
        rows = x.numel() // self.C
        if out is None:
            out = torch.empty_like(x)
        pb = None
        if pair_bias is not None:
            apb, s, apb_ws = pair_bias
            pb = (s, apb.w, apb.n_heads, apb_ws, apb.options.eps)
        if self.fast:
            ops.launch_transition_mx8(x, out, self.w, accumulate, self.options.eps, self.variant, pb)
            return out
        if ws is None:
            nb = self.workspace_bytes(rows)
            ws = ops.workspace(nb, x.device) if nb else None
        # the sampled mean is one batch element's: batch 1 only (otherwise hi + lo)
        mean_fix = self.options.mean_correction and "fc3.weight.lo" in self.w and x.dim() == 4 and x.shape[0] == 1
        ops.launch_transition(x, out, self.w, ws, accumulate, self.options.eps, self.variant, pb, mean_fix)
        return out


class AttentionPairBias(Module):
    """``tenstorrent.py:653-853`` (non-atom branch, compute_pair_bias=True)."""

    def __init__(self, head_dim: int, n_heads: int, state_dict, options: Optional[Options] = None):
        super().__init__(state_dict, options)
        self.head_dim, self.n_heads = head_dim, n_heads
        self.w = {k: self.vec(k) for k in ("proj_q.bias", "proj_z.0.weight", "proj_z.0.bias")}
        self.w.update({k: self.mat(k) for k in ("proj_q.weight", "proj_k.weight", "proj_v.weight", "proj_g.weight",
                                                "proj_o.weight", "proj_z.1.weight")})
        self.c_s = self.weights["proj_q.weight"].shape[0]

    def workspace_bytes(self, B: int, N: int) -> int:
        return ops.apb_workspace_bytes(B, N, self.c_s, self.n_heads, self.variant)

    def __call__(self, s: torch.Tensor, z: torch.Tensor, mask: Optional[torch.Tensor] = None,
                 k_in: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None, accumulate: bool = False,
                 ws: Optional[torch.Tensor] = None, n_valid: int = 0, part: str = "all") -> torch.Tensor:
        """``part="bias"`` computes only the pair bias from z into ``ws``; ``part="attend"``
        runs the rest with the bias a previous "bias" call left in the same ``ws`` (the two
        halves may run on different streams, ordered by the caller)."""
        B, N, _ = s.shape
        if ws is None:
            if part != "all":
                raise ValueError("AttentionPairBias: part='bias'/'attend' need the caller's workspace")
            ws = ops.workspace(self.workspace_bytes(B, N), s.device)
        if out is None:
            out = torch.empty_like(s)
        ops.launch_apb(s, s if k_in is None else k_in, z, mask, out, self.w, self.n_heads, ws, accumulate,
                       self.options.eps, n_valid, self.variant, part, fast=self.fast)
        return out


class SingleTrackStream:
    """A second HIP stream (default priority) for the single-track half of each layer.

    The single track of layer L (pre_norm_s, attention with pair bias, transition_s) reads
    z only through the pair bias, which is computed on the caller's stream right after the
    layer's pair operations; the rest runs here, overlapped with layer L+1's pair
    operations, which never touch s.  ``ws`` is the single track's own workspace.  The
    next layer's pair bias (which overwrites the bias in ``ws``) and ``join()`` wait for
    the previous single track on the caller's stream.
    """

    def __init__(self, nbytes: int, device: torch.device, delay: int = 0):
        self.stream = torch.cuda.Stream(device=device)
        self.ws = ops.workspace(nbytes, device)
        self.done: Optional[torch.cuda.Event] = None
        self.delay = delay
        self.pending = None   # a single track waiting for `delay` pair operations to be queued

    def issue_pending(self) -> None:
        """Queue a deferred single track now (it starts after the caller's queued work)."""
        if self.pending is not None:
            fn, self.pending = self.pending, None
            fn()

    def wait_previous(self) -> None:
        self.issue_pending()
        if self.done is not None:
            torch.cuda.current_stream().wait_event(self.done)

    def join(self) -> None:
        """Make the caller's stream wait for every single-track update issued so far."""
        self.wait_previous()
        self.done = None

    def discard(self) -> None:
        """Drop a deferred single track that was never queued (its call raised)."""
        self.pending = None


class PairformerLayer(Module):
    """``tenstorrent.py:949-1046`` / ``reference.py:822-914`` (no-seq: ``1007-1072``).

    ``__call__(s, z, pair_mask, mask, ws, n_valid)`` updates the device tensors in
    place: z += TMo; z += TMi; z += TAs; z += TAe; z += Tr_z; then, with
    ``transform_s``, s += APB(LN(s), z, mask, k_in=LN(s)); s += Tr_s(s).
    """

    def __init__(self, tri_att_head_dim: int, tri_att_n_heads: int, att_head_dim: Optional[int],
                 att_n_heads: Optional[int], transform_s: bool, state_dict, options: Optional[Options] = None,
                 affinity: bool = False):
        super().__init__(state_dict, options)
        self.transform_s = transform_s
        self.triangle_multiplication_start = TriangleMultiplication(False, self.scope("tri_mul_out"), self.options)
        self.triangle_multiplication_end = TriangleMultiplication(True, self.scope("tri_mul_in"), self.options)
        self.triangle_attention_start = TriangleAttention(tri_att_head_dim, tri_att_n_heads, False,
                                                          self.scope("tri_att_start", "mha."), self.options, affinity)
        self.triangle_attention_end = TriangleAttention(tri_att_head_dim, tri_att_n_heads, True,
                                                        self.scope("tri_att_end", "mha."), self.options, affinity)
        self.transition_z = Transition(self.scope("transition_z"), self.options)
        if transform_s:
            self.pre_norm_s_weight = self.vec("pre_norm_s.weight")
            self.pre_norm_s_bias = self.vec("pre_norm_s.bias")
            self.attention_pair_bias = AttentionPairBias(att_head_dim, att_n_heads, self.scope("attention"),
                                                         self.options)
            self.transition_s = Transition(self.scope("transition_s"), self.options)

    def single_workspace_bytes(self, B: int, N: int) -> int:
        """Workspace of the single-track half (pre_norm_s output, then the attention's)."""
        if not self.transform_s:
            return 0
        c_s = self.attention_pair_bias.c_s
        return max(self.attention_pair_bias.workspace_bytes(B, N) + B * N * c_s * 4,
                   self.transition_s.workspace_bytes(B * N))

    def transition_workspace_bytes(self, B: int, N: int) -> int:
        """The pair transition's share at the start of the layer workspace (kept apart from
        the single track's, which its fused pair bias writes in the same launch)."""
        return (self.transition_z.workspace_bytes(B * N * N) + 255) // 256 * 256

    def workspace_bytes(self, B: int, N: int) -> int:
        n = max(self.triangle_multiplication_start.workspace_bytes(B, N),
                self.triangle_attention_start.workspace_bytes(B, N))
        return max(n, self.transition_workspace_bytes(B, N) + self.single_workspace_bytes(B, N))

    def __call__(self, s: Optional[torch.Tensor], z: torch.Tensor, pair_mask: Optional[torch.Tensor] = None,
                 mask: Optional[torch.Tensor] = None, ws: Optional[torch.Tensor] = None, n_valid: int = 0,
                 single: Optional[SingleTrackStream] = None):
        """With ``single``, the single-track update is left running on ``single.stream``
        (call ``single.join()`` before reading s); otherwise everything is on the current
        stream in reference order."""
        B, N = z.shape[0], z.shape[1]
        if ws is None:
            ws = ops.workspace(self.workspace_bytes(B, N), z.device)
        pair_ops = (
            lambda: self.triangle_multiplication_start(z, pair_mask, out=z, accumulate=True, ws=ws),
            lambda: self.triangle_multiplication_end(z, pair_mask, out=z, accumulate=True, ws=ws),
            lambda: self.triangle_attention_start(z, pair_mask, out=z, accumulate=True, ws=ws, n_valid=n_valid),
            lambda: self.triangle_attention_end(z, pair_mask, out=z, accumulate=True, ws=ws, n_valid=n_valid),
        )
        for i, op in enumerate(pair_ops):
            op()
            if single is not None and i + 1 == single.delay:
                single.issue_pending()   # the previous layer's single track starts beside the rest
        tr_nb = self.transition_workspace_bytes(B, N)
        tr_ws = ws[:tr_nb] if tr_nb else None
        if not (self.transform_s and s is not None):
            self.transition_z(z, out=z, accumulate=True, ws=tr_ws)
            return s, z
        c_s = s.shape[-1]
        sws = ws[tr_nb:] if single is None else single.ws
        s_norm = sws[: B * N * c_s * 4].view(torch.float32).view(B, N, c_s)
        apb_ws = sws[B * N * c_s * 4:]
        if single is not None:
            # the previous single track must be done with the workspace (and s) first
            single.wait_previous()
        # the single track reads z only through the pair bias of the final z: with the 16-bit
        # pair transition it comes out of the same kernel
        if self.transition_z.fuses_pair_bias():
            self.transition_z(z, out=z, accumulate=True, ws=tr_ws,
                              pair_bias=(self.attention_pair_bias, s, apb_ws))
        else:
            self.transition_z(z, out=z, accumulate=True, ws=tr_ws)
            self.attention_pair_bias(s, z, mask, out=s, ws=apb_ws, n_valid=n_valid, part="bias")
        if single is None:
            ops.launch_layernorm(s, self.pre_norm_s_weight, self.pre_norm_s_bias, s_norm, self.options.eps,
                                 self.variant)
            self.attention_pair_bias(s_norm, z, mask, k_in=s_norm, out=s, accumulate=True, ws=apb_ws,
                                     n_valid=n_valid, part="attend")
            self.transition_s(s, out=s, accumulate=True, ws=sws)
            return s, z
        def issue():
            ready = torch.cuda.Event()
            ready.record(torch.cuda.current_stream())
            with torch.cuda.stream(single.stream):
                single.stream.wait_event(ready)
                ops.launch_layernorm(s, self.pre_norm_s_weight, self.pre_norm_s_bias, s_norm, self.options.eps,
                                     self.variant)
                self.attention_pair_bias(s_norm, z, mask, k_in=s_norm, out=s, accumulate=True, ws=apb_ws,
                                         n_valid=n_valid, part="attend")
                self.transition_s(s, out=s, accumulate=True, ws=sws)
                done = torch.cuda.Event()
                done.record(single.stream)
            for t in (s, mask, sws):
                if t is not None:
                    t.record_stream(single.stream)
            single.done = done

        if single.delay == 0:
            issue()
        else:
            single.pending = issue
        return s, z


class Pairformer(Module):
    """``tenstorrent.py:1049-1083``: the block stack on device-resident padded tensors."""

    def __init__(self, n_blocks: int, tri_att_head_dim: int, tri_att_n_heads: int, att_head_dim: Optional[int],
                 att_n_heads: Optional[int], transform_s: bool, state_dict, options: Optional[Options] = None,
                 affinity: bool = False):
        super().__init__(state_dict, options)
        self.transform_s = transform_s
        self.blocks = [
            PairformerLayer(tri_att_head_dim, tri_att_n_heads, att_head_dim, att_n_heads, transform_s,
                            self.scope(f"layers.{i}"), self.options, affinity=affinity)
            for i in range(n_blocks)
        ]

    def workspace_bytes(self, B: int, N: int) -> int:
        return max((b.workspace_bytes(B, N) for b in self.blocks), default=16)

    def single_track(self, B: int, N: int, device: torch.device) -> Optional[SingleTrackStream]:
        """The (cached) second stream and workspace for overlapping the single track."""
        if not self.transform_s or not self.options.overlap_single:
            return None
        nb = max((b.single_workspace_bytes(B, N) for b in self.blocks), default=16)
        key = (B, N, str(device))
        if getattr(self, "_single_key", None) != key:
            self._single = SingleTrackStream(nb, device, self.options.single_delay)
            self._single_key = key
        return self._single

    def __call__(self, s: Optional[torch.Tensor], z: torch.Tensor, pair_mask: Optional[torch.Tensor] = None,
                 mask: Optional[torch.Tensor] = None, ws: Optional[torch.Tensor] = None, n_valid: int = 0):
        """Padded device tensors in; ``n_valid`` (0 = all) tokens are real.  With padding and
        no ``pair_mask`` the padding is masked out (the contractions have no ``n_valid``)."""
        B, N = z.shape[0], z.shape[1]
        if pair_mask is None and 0 < n_valid < N:
            pair_mask = ops.valid_pair_mask(B, N, n_valid, z.device)
        if ws is None:
            ws = ops.workspace(self.workspace_bytes(B, N), z.device)
        single = self.single_track(z.shape[0], z.shape[1], z.device) if s is not None else None
        if single is None:
            for block in self.blocks:
                s, z = block(s, z, pair_mask, mask, ws, n_valid, single)
            return s, z
        single.discard()   # a cached stream never carries a closure over another call's tensors
        try:
            for block in self.blocks:
                s, z = block(s, z, pair_mask, mask, ws, n_valid, single)
        except BaseException:
            single.discard()
            raise
        single.join()
        return s, z


class PairformerModule(nn.Module):
    """Drop-in for ``tenstorrent.PairformerModule`` (``tenstorrent.py:2194-2284``) and
    ``reference.PairformerModule`` / ``PairformerNoSeqModule`` at the
    ``Boltz2`` call sites (``boltz2.py:3750, 4502, 4688, 5015``)."""

    def __init__(self, n_blocks: int, tri_att_head_dim: int, tri_att_n_heads: int, att_head_dim: Optional[int],
                 att_n_heads: Optional[int], transform_s: bool, affinity: bool = False,
                 options: Optional[Options] = None):
        super().__init__()
        self.n_blocks = n_blocks
        self.tri_att_head_dim = tri_att_head_dim
        self.tri_att_n_heads = tri_att_n_heads
        self.att_head_dim = att_head_dim
        self.att_n_heads = att_n_heads
        self.transform_s = transform_s
        self.affinity = affinity
        self.module: Optional[Pairformer] = None
        self.options = options or Options()
        self._runtime_cache: dict = {}
        self._first_forward_pass = True

    def _load_from_state_dict(self, state_dict, prefix, _local_metadata, _strict, _missing_keys,
                              _unexpected_keys, _error_msgs):
        self.module = Pairformer(self.n_blocks, self.tri_att_head_dim, self.tri_att_n_heads, self.att_head_dim,
                                 self.att_n_heads, self.transform_s,
                                 WeightScope.wrap(state_dict).child(prefix[:-1]), self.options,
                                 affinity=self.affinity)

    def reset_static_cache(self):
        """Drop cached masks so they are rebuilt on the next forward (``tenstorrent.py:2182-2191``)."""
        self._runtime_cache.clear()
        self._first_forward_pass = True

    def _build_masks(self, B: int, N: int, n_pad: int, mask, pair_mask, dev) -> None:
        if pair_mask is None and mask is not None:
            m = mask.to(dev, torch.float32)
            pair_mask = m[:, :, None] * m[:, None, :]
        self._runtime_cache["pair_mask"] = ops.pad_pair_mask(pair_mask, B, N, n_pad, dev)
        if self.transform_s:
            tm = torch.zeros((B, n_pad), dtype=torch.float32, device=dev)
            tm[:, :N] = 1.0 if mask is None else mask.to(dev, torch.float32)
            self._runtime_cache["mask"] = tm
        # the masks depend on the unpadded length too: N = 100 and N = 120 share n_pad = 128
        self._runtime_cache["shape"] = (B, N, n_pad)

    def forward(self, s: Optional[torch.Tensor], z: torch.Tensor, mask: Optional[torch.Tensor] = None,
                pair_mask: Optional[torch.Tensor] = None, use_kernels: bool = False):
        """``(s [B,N,c_s] | None, z [B,N,N,c_z]) -> (s_out | None, z_out)``, fp32, on z's device.
        ``use_kernels`` is accepted for call-site compatibility and ignored.  CPU tensors
        move through pinned staging buffers; CPU results come back in pinned memory."""
        if self.module is None:
            raise RuntimeError("PairformerModule has no weights: call load_state_dict() first")
        dev = get_device()
        B, N = z.shape[0], z.shape[1]
        n_pad = ops.padded_len(N, ops.FAST_PAD if self.module.fast else ops.PAD)
        if self._first_forward_pass or self._runtime_cache.get("shape") != (B, N, n_pad):
            self._build_masks(B, N, n_pad, mask, pair_mask, dev)
            self._first_forward_pass = False
        z_dev = ops.to_device_padded(z, n_pad, dev, pair=True)
        s_dev = None
        if self.transform_s and s is not None:
            s_dev = ops.to_device_padded(s, n_pad, dev, pair=False)
        s_dev, z_dev = self.module(s_dev, z_dev, self._runtime_cache["pair_mask"], self._runtime_cache.get("mask"),
                                   n_valid=N)

        def back(t_dev, like):
            return ops.to_host(t_dev) if like.device.type == "cpu" else t_dev.to(like.device)

        z_out = back(z_dev[:, :N, :N], z)
        s_out = None if s_dev is None else back(s_dev[:, :N], s)
        if s is not None and not self.transform_s:
            s_out = s
        return s_out, z_out


class TrunkRecycler:
    """Device-resident trunk recycling loop of ``Boltz2.forward`` (``boltz2.py:5189-5248``)
    without the template module: s, z start at zero and each of the ``recycling_steps + 1``
    passes computes ``s = s_init + s_recycle(s_norm(s))``, ``z = z_init + z_recycle(z_norm(z))``
    (``boltz2.py:5213-5214``), with an MSA module ``z = z + msa(z, ...)`` (``boltz2.py:5230``),
    and runs the Pairformer stack, without leaving the GPU between passes.

    ``msa`` is a device ``MSA`` (``tt_boltz_amd.msa``); its padded inputs are passed to each
    call as ``msa_inputs`` (``tt_boltz_amd.msa.device_inputs``)."""

    def __init__(self, pairformer: Pairformer, state_dict, options: Optional[Options] = None, msa=None):
        w = WeightScope.wrap(state_dict)
        self.pairformer = pairformer
        self.msa = msa
        self.options = options or pairformer.options
        v = self.options.operand
        dev = get_device()
        self.s_norm_w, self.s_norm_b = ops.f32(w["s_norm.weight"], dev), ops.f32(w["s_norm.bias"], dev)
        self.z_norm_w, self.z_norm_b = ops.f32(w["z_norm.weight"], dev), ops.f32(w["z_norm.bias"], dev)
        self.s_rec = ops.opw(w["s_recycle.weight"], dev, v)
        self.z_rec = ops.opw(w["z_recycle.weight"], dev, v)
        # the pair recycling projection to ~fp32 (its input is the same beta at every pair at
        # a pass's start, so a 16-bit rounding would shift all of z alike)
        self.z_rec_lo = ops.opw_lo(w["z_recycle.weight"], dev, v) if self.options.weight_residuals else None

    def __call__(self, s_init: torch.Tensor, z_init: torch.Tensor, mask: Optional[torch.Tensor],
                 recycling_steps: int, pass_hook=None, n_valid: int = 0, msa_inputs: Optional[dict] = None):
        """Padded device tensors in (N % 64 == 0); returns device (s, z).  ``pass_hook(i, s, z)``
        (optional) is called after each pass with the device state (enqueued, not synchronized)."""
        if (self.msa is None) != (msa_inputs is None):
            raise ValueError("TrunkRecycler: msa_inputs must be given exactly when an MSA module is attached")
        B, N = z_init.shape[0], z_init.shape[1]
        v = self.options.operand
        dev = z_init.device
        if mask is not None:
            pair_mask = (mask[:, :, None] * mask[:, None, :]).contiguous()
        elif 0 < n_valid < N:
            pair_mask = ops.valid_pair_mask(B, N, n_valid, dev)
        else:
            pair_mask = None
        s = torch.zeros_like(s_init)
        z = torch.zeros_like(z_init)
        s_tmp = torch.empty_like(s_init)
        z_msa = None if self.msa is None else torch.empty_like(z_init)
        ws = ops.workspace(self.pairformer.workspace_bytes(B, N), dev)
        for i in range(recycling_steps + 1):
            ops.launch_layernorm(s, self.s_norm_w, self.s_norm_b, s_tmp, self.options.eps, v)
            ops.launch_linear(s_tmp, self.s_rec, None, s_init, s, v)
            ops.launch_pair_ln_linear(z, z_init, self.z_norm_w, self.z_norm_b, self.z_rec, z, self.options.eps, v,
                                      self.z_rec_lo)
            if self.msa is not None:
                z_msa.copy_(z)
                self.msa(z_msa, pair_mask=pair_mask, n_valid=n_valid, **msa_inputs)
                ops.launch_add(z, z_msa, z, v)
            s, z = self.pairformer(s, z, pair_mask, mask, ws, n_valid)
            if pass_hook is not None:
                pass_hook(i, s, z)
        return s, z
