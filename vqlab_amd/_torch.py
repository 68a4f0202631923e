"""torch plumbing for the C ABI: tensors -> descriptor structs, dtype codes,
the current HIP stream. torch provides device memory and streams only; the
arithmetic runs in libvqk."""
from __future__ import annotations

import ctypes

import torch

from . import _lib as L

ACT_TYPES = {torch.float16: L.VQK_F16, torch.bfloat16: L.VQK_BF16, torch.float32: L.VQK_F32}


def act_type(t: torch.Tensor) -> int:
    try:
        return ACT_TYPES[t.dtype]
    except KeyError:
        raise ValueError(f"activations must be float16, bfloat16 or float32, got {t.dtype}")


def code_type(t: torch.Tensor) -> int:
    if t.dtype == torch.uint8:
        return L.VQK_U8
    if t.dtype in (torch.int16, torch.uint16):
        return L.VQK_U16
    if t.dtype in (torch.int32, torch.uint32):
        return L.VQK_U32
    raise ValueError(f"codes must be uint8, uint16 or uint32 words, got {t.dtype}")


def stream(device=None) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def require_cuda(*ts):
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("libvqk kernels take device (cuda) tensors")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")
    return dev


def as_fp16(t: torch.Tensor) -> torch.Tensor:
    return (t if t.dtype == torch.float16 else t.to(torch.float16)).contiguous()


def weights(codes, codebook, scales, group_size=64, pack_bits=0, in_features=None,
            row_table=None, k_expect=0, keep=None) -> L.VQKWeights:
    """Describe one VQ module. `keep` (a list) receives every tensor whose
    pointer the struct holds, so the caller can keep them alive."""
    codes = codes.contiguous()
    codebook = as_fp16(codebook)
    scales = as_fp16(scales)
    K, D = codebook.shape
    if row_table is not None:
        row_table = row_table.to(torch.int32).contiguous()
        E, OUT = row_table.shape
        n_live = codes.shape[0]
    elif codes.ndim == 3:
        E, OUT = codes.shape[0], codes.shape[1]
        n_live = 0
    elif codes.ndim == 2:
        E, OUT = 1, codes.shape[0]
        n_live = 0
    else:
        raise ValueError(f"codes must be [E, OUT, W] or [OUT, W], got {tuple(codes.shape)}")
    if pack_bits:
        if in_features is None:
            raise ValueError("packed codes need explicit in_features")
        IN = int(in_features)
    else:
        IN = codes.shape[-1] * D
    w = L.VQKWeights()
    w.codes = codes.data_ptr()
    w.code_cols = codes.shape[-1]
    w.code_type = code_type(codes)
    w.pack_bits = int(pack_bits)
    w.codebook = codebook.data_ptr()
    w.K = K
    w.D = D
    w.group = int(group_size)
    w.scales = scales.data_ptr()
    w.E, w.OUT, w.IN = E, OUT, IN
    w.row_table = 0 if row_table is None else row_table.data_ptr()
    w.n_live = n_live
    w.k_expect = int(k_expect)
    if keep is not None:
        keep.extend([codes, codebook, scales, row_table])
    return w
