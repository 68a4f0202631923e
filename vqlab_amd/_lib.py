"""ctypes binding of libvqk.so (the C ABI declared in include/vqk.h).

The library is required: importing a kernel wrapper without it raises, there
is no CPU fallback. Status codes map onto the reference's exceptions
(NotImplementedError / ValueError / RuntimeError, see include/vqk.h).
"""
from __future__ import annotations

import ctypes
import os
import pathlib

# VQK_LIBRARY points at another build of the same ABI (A/B of kernel variants).
LIB_PATH = pathlib.Path(os.environ.get("VQK_LIBRARY") or
                        pathlib.Path(__file__).resolve().parent / "libvqk.so")

VQK_OK, VQK_ENOTIMPL, VQK_EINVAL, VQK_ESHARDED, VQK_EDEVICE, VQK_ENOSPACE = range(6)
VQK_F16, VQK_BF16, VQK_F32, VQK_U8, VQK_U16, VQK_U32, VQK_I32, VQK_I64 = range(8)
VQK_NOALLOC_SCRATCH_BYTES = 32 << 20     # include/vqk.h
VQK_MOE_HEADER_BYTES = 49152             # include/vqk.h: zero before a layer workspace's first call
VQK_VIA_F16 = 0x100                      # output type flag: round through fp16 first
VQK_X_KEEP = 0x200                       # x type flag (d=8 GEMV): x enters the products unrounded

c_i32, c_i64, c_p, c_sz = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p, ctypes.c_size_t


class VQKWeights(ctypes.Structure):
    _fields_ = [("codes", c_p), ("code_cols", c_i64), ("code_type", c_i32),
                ("pack_bits", c_i32), ("codebook", c_p), ("K", c_i64), ("D", c_i32),
                ("group", c_i32), ("scales", c_p), ("E", c_i64), ("OUT", c_i64),
                ("IN", c_i64), ("row_table", c_p), ("n_live", c_i64), ("k_expect", c_i64)]


class VQKMoeDesc(ctypes.Structure):
    _fields_ = [("gate", ctypes.POINTER(VQKWeights)), ("up", ctypes.POINTER(VQKWeights)),
                ("down", ctypes.POINTER(VQKWeights)), ("sh_gate", ctypes.POINTER(VQKWeights)),
                ("sh_up", ctypes.POINTER(VQKWeights)), ("sh_down", ctypes.POINTER(VQKWeights)),
                ("sh_gate_vec", c_p), ("sh_gate_vec_type", c_i32), ("top_k", c_i32),
                ("norm_topk", c_i32)]


class VQKOptions(ctypes.Structure):
    _fields_ = [("fused_max_n", c_i64), ("dense_fused_max_n", c_i64),
                ("decode_bf16io", c_i32), ("prefill_bf16io", c_i32),
                ("crowded_grouped", c_i32)]


# name -> (restype, argtypes), one entry per function of include/vqk.h
SIGNATURES = {
    "vqk_version": (ctypes.c_char_p, []),
    "vqk_last_error": (ctypes.c_char_p, []),
    "vqk_bits_for_k": (c_i32, [c_i64, ctypes.POINTER(c_i32)]),
    "vqk_words_per_row": (c_i64, [c_i64, c_i32]),
    "vqk_pack_bits_for": (c_i32, [c_i64, c_i64, c_i32, ctypes.POINTER(c_i32)]),
    "vqk_pack_host": (c_i32, [c_p, c_i64, c_i64, c_i32, c_p]),
    "vqk_unpack_host": (c_i32, [c_p, c_i64, c_i64, c_i32, c_p]),
    "vqk_pack": (c_i32, [c_p, c_i64, c_i64, c_i32, c_p, c_p]),
    "vqk_unpack": (c_i32, [c_p, c_i64, c_i64, c_i32, c_p, c_p]),
    "vqk_dequant": (c_i32, [ctypes.POINTER(VQKWeights), c_i64, c_i64, c_p, c_p]),
    "vqk_dequant_experts": (c_i32, [ctypes.POINTER(VQKWeights), c_p, c_i64, c_p, c_p]),
    "vqk_dense_gemv": (c_i32, [ctypes.POINTER(VQKWeights), c_p, c_i32, c_i64, c_p, c_i32, c_p]),
    "vqk_moe_expert_gemv": (c_i32, [ctypes.POINTER(VQKWeights), c_p, c_i32, c_i64, c_p, c_i64,
                                    c_i64, c_p, c_i32, c_p]),
    "vqk_grouped_gemm_workspace": (c_i32, [ctypes.POINTER(VQKWeights), c_i64,
                                           ctypes.POINTER(c_sz)]),
    "vqk_grouped_gemm": (c_i32, [ctypes.POINTER(VQKWeights), c_p, c_i32, c_i64, c_p, c_i64,
                                 c_i64, c_p, c_i32, c_p, c_sz, c_p]),
    "vqk_dense_gemm_workspace": (c_i32, [ctypes.POINTER(VQKWeights), c_i64,
                                         ctypes.POINTER(ctypes.c_size_t)]),
    "vqk_dense_gemm": (c_i32, [ctypes.POINTER(VQKWeights), c_p, c_i32, c_i64, c_p, c_i32, c_p,
                               ctypes.c_size_t, c_p]),
    "vqk_moe_decode_layer_workspace": (c_i32, [ctypes.POINTER(VQKMoeDesc), c_i64,
                                               ctypes.POINTER(c_sz)]),
    "vqk_moe_decode_layer": (c_i32, [ctypes.POINTER(VQKMoeDesc), c_p, c_i32, c_i64, c_p, c_p,
                                     c_i32, c_p, c_p, c_p, c_sz, c_p]),
    "vqk_moe_decode_layer_noalloc": (c_i32, [ctypes.POINTER(VQKMoeDesc), c_p, c_i32, c_i64, c_p,
                                             c_p, c_i32, c_p, c_p, c_p]),
    "vqk_moe_layer_status": (c_i32, [c_p, c_p]),
    "vqk_moe_layer_reset": (c_i32, [c_p, c_p]),
    "vqk_embed_gather": (c_i32, [ctypes.POINTER(VQKWeights), c_p, c_i32, c_i64, c_p, c_i32,
                                 c_p]),
    "vqk_dense_fits": (c_i32, [c_i64, c_i64, c_i32, c_i32]),
    "vqk_wdec_fits": (c_i32, [c_i32, c_i64, c_i32, c_i32]),
    "vqk_gemmseg_fits": (c_i32, [c_i32, c_i64, c_i32, c_i32, c_i64]),
    "vqk_skipzero_row_table_host": (c_i32, [c_p, c_i64, c_i64, c_p, ctypes.POINTER(c_i64)]),
    "vqk_options_default": (None, [ctypes.POINTER(VQKOptions)]),
    "vqk_options_from_env": (None, [ctypes.POINTER(VQKOptions)]),
    "vqk_switch_apply_workspace": (c_i32, [ctypes.POINTER(VQKWeights), c_i64,
                                           ctypes.POINTER(VQKOptions), ctypes.POINTER(c_sz)]),
    "vqk_switch_apply": (c_i32, [ctypes.POINTER(VQKWeights), c_p, c_i32, c_i64, c_p, c_i64,
                                 c_i64, c_p, c_i32, c_p, c_sz, ctypes.POINTER(VQKOptions), c_p]),
    "vqk_linear_apply_workspace": (c_i32, [ctypes.POINTER(VQKWeights), c_i64,
                                           ctypes.POINTER(VQKOptions), ctypes.POINTER(c_sz)]),
    "vqk_linear_apply": (c_i32, [ctypes.POINTER(VQKWeights), c_p, c_i32, c_i64, c_p, c_i32, c_p,
                                 c_sz, ctypes.POINTER(VQKOptions), c_p]),
}

_LIB = None


def lib():
    """The loaded library; raises ImportError when libvqk.so is not built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} is not built: run `python -m vqlab_amd.build` "
                              "(hipcc, gfx950). There is no CPU fallback.")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _LIB = L
    return _LIB


def options(from_env: bool = False, **fields) -> VQKOptions:
    """A vqk_options: the defaults, or (from_env) the defaults overridden by
    the reference's VQ_* variables where set; keyword fields override both."""
    o = VQKOptions()
    (lib().vqk_options_from_env if from_env else lib().vqk_options_default)(ctypes.byref(o))
    for k, v in fields.items():
        setattr(o, k, v)
    return o


def last_error() -> str:
    return lib().vqk_last_error().decode(errors="replace")


def check(rc: int, what: str = "") -> None:
    """Raise the reference's exception type for a non-OK status."""
    if rc == VQK_OK:
        return
    msg = f"{what}: {last_error()}" if what else last_error()
    if rc == VQK_ENOTIMPL:
        raise NotImplementedError(msg)
    if rc in (VQK_EINVAL, VQK_ENOSPACE):
        raise ValueError(msg)
    raise RuntimeError(msg)
