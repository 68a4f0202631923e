"""Sub-byte packing of VQ codes -- the vq_pack interface (src/vqlab/runtime/vq_pack.py).

Same names, arguments and layout as the reference (vq_pack.py:11-27): codes
[E, OUT, NSUB] -> uint32 words [E, OUT, WPR], WPR = ceil(NSUB/32) * BITS,
32-code blocks of BITS words, code i of a block at bit i*BITS LSB first,
tail block zero-padded. numpy inputs are packed by libvqk's host routine,
torch device tensors by its HIP kernels. Precondition failures raise
AssertionError, as the reference's asserts do.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib as L

BLOCK = 32


def bits_for_k(k: int) -> int:
    """vq_pack.py:34-38: code width the codebook size K implies (K a power of two)."""
    b = ctypes.c_int32()
    rc = L.lib().vqk_bits_for_k(int(k), ctypes.byref(b))
    assert rc == L.VQK_OK, f"K={k} is not a power of two"
    return b.value


def words_per_row(nsub: int, bits: int) -> int:
    """vq_pack.py:41-45: ceil(NSUB/32) * BITS."""
    return int(L.lib().vqk_words_per_row(int(nsub), int(bits)))


def packed_bytes(e: int, out: int, nsub: int, bits: int) -> int:
    return e * out * words_per_row(nsub, bits) * 4


def _is_torch(a) -> bool:
    return type(a).__module__.startswith("torch")


def pack(codes, bits: int):
    """[E, OUT, NSUB] integer codes -> [E, OUT, WPR] uint32 (vq_pack.py:48-76)."""
    bits = int(bits)
    if _is_torch(codes):
        return _pack_device(codes, bits)
    codes = np.asarray(codes)
    assert codes.ndim == 3, codes.shape
    assert int(codes.max(initial=0)) < (1 << bits), "code exceeds bit width"
    e, out, nsub = codes.shape
    src = np.ascontiguousarray(codes, dtype=np.uint16)
    dst = np.zeros((e, out, words_per_row(nsub, bits)), np.uint32)
    L.check(L.lib().vqk_pack_host(src.ctypes.data, e * out, nsub, bits, dst.ctypes.data), "pack")
    return dst


def unpack(packed, nsub: int, bits: int):
    """Inverse of pack (vq_pack.py:79-97): uint8 for bits <= 8, else uint16."""
    bits, nsub = int(bits), int(nsub)
    if _is_torch(packed):
        return _unpack_device(packed, nsub, bits)
    packed = np.ascontiguousarray(packed, dtype=np.uint32)
    e, out, wpr = packed.shape
    assert wpr == words_per_row(nsub, bits), (wpr, nsub, bits)
    dst = np.zeros((e, out, nsub), np.uint8 if bits <= 8 else np.uint16)
    L.check(L.lib().vqk_unpack_host(packed.ctypes.data, e * out, nsub, bits, dst.ctypes.data),
            "unpack")
    return dst


def _pack_device(codes, bits):
    import torch
    from . import _torch as T
    assert codes.ndim == 3, tuple(codes.shape)
    T.require_cuda(codes)
    assert int(codes.max().item() if codes.numel() else 0) < (1 << bits), \
        "code exceeds bit width"
    e, out, nsub = codes.shape
    src = codes.to(torch.int32).to(torch.int16).contiguous()   # low 16 bits = the code
    dst = torch.empty((e, out, words_per_row(nsub, bits)), dtype=torch.int32, device=codes.device)
    L.check(L.lib().vqk_pack(T.ptr(src), e * out, nsub, bits, T.ptr(dst), T.stream(codes.device)),
            "pack")
    return dst


def _unpack_device(packed, nsub, bits):
    import torch
    from . import _torch as T
    T.require_cuda(packed)
    packed = packed.contiguous()
    e, out, wpr = packed.shape
    assert wpr == words_per_row(nsub, bits), (wpr, nsub, bits)
    dt = torch.uint8 if bits <= 8 else torch.int16
    dst = torch.empty((e, out, nsub), dtype=dt, device=packed.device)
    L.check(L.lib().vqk_unpack(T.ptr(packed), e * out, nsub, bits, T.ptr(dst),
                               T.stream(packed.device)), "unpack")
    return dst
