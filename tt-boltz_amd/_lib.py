"""ctypes binding of libpairformer_hip (the C ABI in include/pairformer_hip.h).

Two builds of the same kernels live next to this file:
``libpairformer_hip.so`` (IEEE fp16 MFMA operands, the default) and
``libpairformer_hip_bf16.so`` (bf16 operands).  If the requested library is
missing, loading raises: there is no CPU or torch fallback for any operation of
this package.
"""
from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIBS = {"fp16": "libpairformer_hip.so", "bf16": "libpairformer_hip_bf16.so"}
OPERAND_CODE = {"fp16": 0, "bf16": 1}
DEFAULT_VARIANT = "fp16"
LIB_PATH = os.path.join(HERE, LIBS[DEFAULT_VARIANT])
ABI_VERSION = 3

c_int, c_float, c_long, c_size_t, c_void_p = ctypes.c_int, ctypes.c_float, ctypes.c_long, ctypes.c_size_t, ctypes.c_void_p


class TrimulArgs(ctypes.Structure):
    _fields_ = [
        ("B", c_int), ("N", c_int), ("C", c_int), ("hidden", c_int), ("direction", c_int),
        ("accumulate", c_int), ("eps", c_float),
        ("z_in", c_void_p), ("out", c_void_p), ("pair_mask", c_void_p),
        ("norm_in_w", c_void_p), ("norm_in_b", c_void_p), ("p_in_w", c_void_p), ("g_in_w", c_void_p),
        ("norm_out_w", c_void_p), ("norm_out_b", c_void_p), ("p_out_w", c_void_p), ("g_out_w", c_void_p),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t), ("stream", c_void_p),
        ("p_out_lo", c_void_p), ("in_offsets", c_void_p), ("p_in_lo", c_void_p), ("g_in_lo", c_void_p),
        ("g_out_lo", c_void_p),
    ]


class TriattArgs(ctypes.Structure):
    _fields_ = [
        ("B", c_int), ("N", c_int), ("C", c_int), ("H", c_int), ("D", c_int), ("ending", c_int),
        ("accumulate", c_int), ("n_valid", c_int), ("eps", c_float),
        ("z_in", c_void_p), ("out", c_void_p), ("pair_mask", c_void_p),
        ("ln_w", c_void_p), ("ln_b", c_void_p), ("w_bias", c_void_p),
        ("w_q", c_void_p), ("w_k", c_void_p), ("w_v", c_void_p), ("w_g", c_void_p), ("w_o", c_void_p),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t), ("stream", c_void_p),
        ("w_g_lo", c_void_p), ("w_o_lo", c_void_p), ("in_offsets", c_void_p), ("w_q_lo", c_void_p),
        ("w_k_lo", c_void_p), ("w_v_lo", c_void_p), ("w_bias_lo", c_void_p),
    ]


class TriattMx8Args(ctypes.Structure):
    _fields_ = [
        ("B", c_int), ("N", c_int), ("C", c_int), ("H", c_int), ("D", c_int), ("ending", c_int),
        ("accumulate", c_int), ("n_valid", c_int), ("eps", c_float),
        ("z_in", c_void_p), ("out", c_void_p), ("pair_mask", c_void_p),
        ("ln_w", c_void_p), ("ln_b", c_void_p), ("w_bias", c_void_p),
        ("w_q_q", c_void_p), ("w_q_s", c_void_p), ("w_k_q", c_void_p), ("w_k_s", c_void_p),
        ("w_v_q", c_void_p), ("w_v_s", c_void_p), ("w_g_q", c_void_p), ("w_g_s", c_void_p), ("w_o", c_void_p),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t), ("stream", c_void_p),
    ]


class TransitionArgs(ctypes.Structure):
    _fields_ = [
        ("rows", c_long), ("C", c_int), ("hidden", c_int), ("accumulate", c_int), ("eps", c_float),
        ("x_in", c_void_p), ("out", c_void_p), ("norm_w", c_void_p), ("norm_b", c_void_p),
        ("fc1_w", c_void_p), ("fc2_w", c_void_p), ("fc3_w", c_void_p),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t), ("stream", c_void_p),
        ("fc3_lo", c_void_p), ("fc3_mean_fix", c_int),
    ]


class ApbArgs(ctypes.Structure):
    _fields_ = [
        ("B", c_int), ("N", c_int), ("c_s", c_int), ("C", c_int), ("H", c_int),
        ("accumulate", c_int), ("n_valid", c_int), ("eps", c_float),
        ("s", c_void_p), ("k_in", c_void_p), ("z", c_void_p), ("mask", c_void_p), ("out", c_void_p),
        ("w_q", c_void_p), ("b_q", c_void_p), ("w_k", c_void_p), ("w_v", c_void_p), ("w_g", c_void_p),
        ("w_o", c_void_p), ("zln_w", c_void_p), ("zln_b", c_void_p), ("w_z", c_void_p),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t), ("stream", c_void_p),
    ]


class OpmArgs(ctypes.Structure):
    _fields_ = [
        ("B", c_int), ("S", c_int), ("N", c_int), ("c_m", c_int), ("c_hidden", c_int), ("C", c_int),
        ("accumulate", c_int), ("eps", c_float),
        ("m", c_void_p), ("msa_mask", c_void_p), ("z", c_void_p), ("norm_w", c_void_p), ("norm_b", c_void_p),
        ("w_a", c_void_p), ("w_b", c_void_p), ("w_o", c_void_p), ("b_o", c_void_p),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t), ("stream", c_void_p),
    ]


class PwaArgs(ctypes.Structure):
    _fields_ = [
        ("B", c_int), ("S", c_int), ("N", c_int), ("c_m", c_int), ("C", c_int), ("H", c_int), ("c_h", c_int),
        ("accumulate", c_int), ("eps", c_float),
        ("m", c_void_p), ("out", c_void_p), ("z", c_void_p), ("pair_mask", c_void_p),
        ("norm_m_w", c_void_p), ("norm_m_b", c_void_p), ("norm_z_w", c_void_p), ("norm_z_b", c_void_p),
        ("w_m", c_void_p), ("w_g", c_void_p), ("w_z", c_void_p), ("w_o", c_void_p),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t), ("stream", c_void_p),
    ]


class TrimulMx8Args(ctypes.Structure):
    _fields_ = [
        ("B", c_int), ("N", c_int), ("C", c_int), ("hidden", c_int), ("direction", c_int),
        ("accumulate", c_int), ("eps", c_float),
        ("z_in", c_void_p), ("out", c_void_p), ("pair_mask", c_void_p),
        ("norm_in_w", c_void_p), ("norm_in_b", c_void_p),
        ("p_in_q", c_void_p), ("p_in_s", c_void_p), ("g_in_q", c_void_p), ("g_in_s", c_void_p),
        ("norm_out_w", c_void_p), ("norm_out_b", c_void_p),
        ("p_out_q", c_void_p), ("p_out_s", c_void_p), ("g_out_q", c_void_p), ("g_out_s", c_void_p),
        ("workspace", c_void_p), ("workspace_bytes", c_size_t), ("stream", c_void_p),
    ]


class TransitionMx8Args(ctypes.Structure):
    _fields_ = [
        ("rows", c_long), ("C", c_int), ("hidden", c_int), ("accumulate", c_int), ("eps", c_float),
        ("x_in", c_void_p), ("out", c_void_p), ("norm_w", c_void_p), ("norm_b", c_void_p),
        ("fc1_q", c_void_p), ("fc1_s", c_void_p), ("fc2_q", c_void_p), ("fc2_s", c_void_p),
        ("fc3_q", c_void_p), ("fc3_s", c_void_p), ("stream", c_void_p),
    ]


#: name -> (restype, argtypes); every symbol include/pairformer_hip.h declares.
SIGNATURES = {
    "pf_abi_version": (c_int, []),
    "pf_last_error": (ctypes.c_char_p, []),
    "pf_operand_dtype": (c_int, []),
    "pf_trimul_workspace_size": (c_size_t, [c_int, c_int, c_int]),
    "pf_trimul_fwd": (c_int, [ctypes.POINTER(TrimulArgs)]),
    "pf_trimul_contract": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]),
    "pf_triatt_workspace_size": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "pf_triatt_fwd": (c_int, [ctypes.POINTER(TriattArgs)]),
    "pf_triatt_attend_workspace": (c_int, [c_void_p, c_size_t, c_int, c_int, c_int, c_void_p]),
    "pf_tri_attention_workspace_size": (c_size_t, [c_int, c_int, c_int, c_int]),
    "pf_tri_attention": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_float, c_void_p,
                                 c_int, c_int, c_int, c_int, c_int, c_void_p, c_size_t, c_void_p]),
    "pf_transition_workspace_size": (c_size_t, [c_long, c_int, c_int]),
    "pf_transition_fwd": (c_int, [ctypes.POINTER(TransitionArgs)]),
    "pf_apb_workspace_size": (c_size_t, [c_int, c_int, c_int, c_int]),
    "pf_apb_fwd": (c_int, [ctypes.POINTER(ApbArgs)]),
    "pf_apb_pair_bias": (c_int, [ctypes.POINTER(ApbArgs)]),
    "pf_apb_attend": (c_int, [ctypes.POINTER(ApbArgs)]),
    "pf_apb_fwd_noalloc": (c_int, [ctypes.POINTER(ApbArgs)]),
    "pf_apb_fwd_mx8": (c_int, [ctypes.POINTER(ApbArgs)]),
    "pf_apb_attend_mx8": (c_int, [ctypes.POINTER(ApbArgs)]),
    "pf_transition_pair_bias_fwd": (c_int, [ctypes.POINTER(TransitionArgs), ctypes.POINTER(ApbArgs)]),
    "pf_opm_workspace_size": (c_size_t, [c_int, c_int, c_int]),
    "pf_opm_fwd": (c_int, [ctypes.POINTER(OpmArgs)]),
    "pf_pwa_workspace_size": (c_size_t, [c_int, c_int, c_int]),
    "pf_pwa_fwd": (c_int, [ctypes.POINTER(PwaArgs)]),
    "pf_msa_embed": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                             c_int, c_int, c_int, c_void_p]),
    "pf_batched_nt_gemm": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_float,
                                   c_void_p]),
    "pf_layernorm_fwd": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_long, c_int, c_float, c_void_p]),
    "pf_linear_fwd": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_long, c_int, c_int, c_void_p]),
    "pf_pair_ln_linear_fwd": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                      c_long, c_int, c_float, c_void_p]),
    "pf_add_fwd": (c_int, [c_void_p, c_void_p, c_void_p, c_long, c_void_p]),
    "pf_pair_cond_proj_fwd": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_long, c_int,
                                      c_float, c_void_p]),
    "pf_token_pair_bias_fwd": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_long, c_int, c_int,
                                       c_int, c_int, c_float, c_float, c_void_p]),
    "pf_quantize_mx8": (c_int, [c_void_p, c_long, c_int, c_int, c_void_p, c_void_p, c_void_p]),
    "pf_trimul_mx8_workspace_size": (c_size_t, [c_int, c_int, c_int]),
    "pf_trimul_mx8_fwd": (c_int, [ctypes.POINTER(TrimulMx8Args)]),
    "pf_triatt_mx8_workspace_size": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "pf_triatt_mx8_fwd": (c_int, [ctypes.POINTER(TriattMx8Args)]),
    "pf_trimul_mx8_contract": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "pf_transition_mx8_fwd": (c_int, [ctypes.POINTER(TransitionMx8Args)]),
    "pf_transition_mx8_pair_bias_fwd": (c_int, [ctypes.POINTER(TransitionMx8Args), ctypes.POINTER(ApbArgs)]),
    "pf_attend_timing": (c_int, [c_int]),
    "pf_attend_timing_read": (c_int, [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(c_int)]),
    "pf_kernel_timing": (c_int, [c_int, c_int]),
    "pf_kernel_timing_read": (c_int, [c_int, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(c_int)]),
    "pf_mfma_rate_probe_waves": (c_long, [c_int]),
    "pf_mfma_rate_probe": (c_int, [c_int, c_int, c_void_p, c_void_p]),
    "pf_mfma8_rate_probe": (c_int, [c_int, c_int, c_void_p, c_void_p]),
}

_lock = threading.Lock()
_libs: dict = {}


def load(variant: str = DEFAULT_VARIANT) -> ctypes.CDLL:
    """Load (once) and return the library of ``variant`` ('fp16' or 'bf16')."""
    lib = _libs.get(variant)
    if lib is not None:
        return lib
    if variant not in LIBS:
        raise ValueError(f"unknown operand variant {variant!r}; expected one of {sorted(LIBS)}")
    with _lock:
        lib = _libs.get(variant)
        if lib is not None:
            return lib
        path = os.path.join(HERE, LIBS[variant])
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: build it with `python tt-boltz_amd/build.py` "
                               "(there is no fallback path)")
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        v = lib.pf_abi_version()
        if v != ABI_VERSION:
            raise RuntimeError(f"{path}: ABI {v} != expected {ABI_VERSION}; rebuild")
        if lib.pf_operand_dtype() != OPERAND_CODE[variant]:
            raise RuntimeError(f"{path}: operand dtype code {lib.pf_operand_dtype()} does not match {variant}")
        _libs[variant] = lib
    return lib


def check(rc: int, what: str, variant: str = DEFAULT_VARIANT) -> None:
    """Raise RuntimeError(pf_last_error()) for a non-zero status."""
    if rc != 0:
        msg = load(variant).pf_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")
