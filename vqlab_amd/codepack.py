"""The packing decision for MoE expert codes -- the codepack interface
(src/vqlab/core/artifacts/codepack.py), shared by re-packing and fixture
generation.

Rules (codepack.py:6-13, 22-30):
  * byte-aligned widths (K = 256, 65536) stay unpacked: packing saves no bytes;
  * NSUB % 32 != 0 stays unpacked unless `pack_unaligned`;
  * a packed tensor must round-trip through unpack before it is returned.

`pack_codes` takes numpy arrays (libvqk's host packer) or torch device
tensors (its HIP packer, round trip checked on the device).
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib as L
from . import vq_pack


def pack_bits_for(k: int, nsub: int, pack_unaligned: bool = False) -> int:
    """codepack.py:22-30: the width [.., NSUB] codes at codebook size K pack
    to, or 0 when they stay unpacked."""
    b = ctypes.c_int32()
    rc = L.lib().vqk_pack_bits_for(int(k), int(nsub), int(bool(pack_unaligned)), ctypes.byref(b))
    assert rc == L.VQK_OK, f"K={k} is not a power of two"
    return b.value


def pack_codes(mod: str, codes, k: int, pack_unaligned: bool = False):
    """codepack.py:33-52: (codes, pack_bits) for an [E, OUT, NSUB] integer
    array -- uint32 words and the width when it packs, else the input and 0.
    Raises SystemExit if the packed tensor does not round-trip (a packing
    error would decode to plausible garbage, not an error)."""
    nsub = int(codes.shape[2])
    bits = pack_bits_for(k, nsub, pack_unaligned)
    if not bits:
        return codes, 0
    if vq_pack._is_torch(codes):
        import torch
        c = codes.to(torch.int32)
        packed = vq_pack.pack(c, bits)
        back = vq_pack.unpack(packed, nsub, bits).to(torch.int32) & 0xFFFF
        ok = bool(torch.equal(back, c))
    else:
        c = np.asarray(codes).astype(np.uint16)
        packed = vq_pack.pack(c, bits)
        ok = np.array_equal(vq_pack.unpack(packed, nsub, bits).astype(np.uint16), c)
    if not ok:
        raise SystemExit(f"FATAL: {mod} did not round-trip through the packer")
    return packed, bits
