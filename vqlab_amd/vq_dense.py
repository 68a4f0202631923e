"""Dense VQ linears for PyTorch-ROCm -- the vq_dense interface
(src/vqlab/runtime/vq_dense.py) over libvqk's HIP kernels.

  VQLinear(codes, codebook, vq_scales, group_size, pack_bits, in_features)
                                                     vq_dense.py:315-441
  _fused_max_n(pack_bits, d)                         vq_dense.py:60-102
  _decode_matmul(xf, codes, codebook, scales, group_size, OUT, IN, pack_bits)
                                                     vq_dense.py:262-312
  VQEmbedding(codes, codebook, vq_scales, ...)       vq_dense.py:444-513

Small N runs the fused GEMV (vqk_dense_gemv). Large N runs the tiled
dequant-into-LDS matrix-core GEMM (vqk_dense_gemm), which never materialises
the fp16 weight.
"""
from __future__ import annotations

import ctypes
import os

import torch

from . import _lib as L
from . import _torch as T
from . import vq_switch as VS

# Rows up to which the fused GEMV beats the dequant + matrix-core GEMM on
# MI355X; keyed on pack state and d like the reference's cutoffs
# (vq_dense.py:55-102). VQ_DENSE_FUSED_MAX_N overrides for A/B.
_DENSE_FUSED_MAX_N_BY_D = {2: 32, 4: 32, 8: 32}


def _fused_max_n(pack_bits, d):
    if "VQ_DENSE_FUSED_MAX_N" in os.environ:
        return int(os.environ["VQ_DENSE_FUSED_MAX_N"])
    return _DENSE_FUSED_MAX_N_BY_D.get(int(d), 32)


def _decode_matmul(xf, codes_in, codebook, scales, group_size, OUT, IN, pack_bits):
    """xf @ decode(codes).T for large N: [N, OUT] in xf's dtype."""
    T.require_cuda(xf, codes_in, codebook, scales)
    keep = []
    w = T.weights(codes_in, codebook, scales, group_size, pack_bits, IN, keep=keep)
    xf = xf.contiguous()
    y = torch.empty((xf.shape[0], int(OUT)), dtype=xf.dtype, device=xf.device)
    ws = ctypes.c_size_t()
    L.check(L.lib().vqk_dense_gemm_workspace(ctypes.byref(w), xf.shape[0], ctypes.byref(ws)),
            "_decode_matmul")
    work = torch.empty(max(1, ws.value), dtype=torch.uint8, device=xf.device)
    L.check(L.lib().vqk_dense_gemm(ctypes.byref(w), T.ptr(xf), T.act_type(xf), xf.shape[0],
                                   T.ptr(y), T.act_type(y), T.ptr(work), ws.value,
                                   T.stream(xf.device)),
            "_decode_matmul")
    return y


class VQLinear(torch.nn.Module):
    """Drop-in for a bias-free nn.Linear whose weight is VQ-coded
    (vq_dense.py:315-441). codes [OUT, NSUB] (uint8/uint16) or [OUT, WPR]
    uint32 words of pack_bits-wide fields."""

    def __init__(self, codes, codebook, vq_scales, group_size=64, pack_bits=0,
                 in_features=None):
        super().__init__()
        if pack_bits and in_features is None:
            raise ValueError("packed codes need explicit in_features")
        self.codes = codes
        self.codebook = codebook
        self.vq_scales = vq_scales
        self.group_size = group_size
        self.pack_bits = pack_bits
        self._in_features = in_features
        self._k_expect = int(codebook.shape[0])

    @property
    def input_dims(self):
        if self.pack_bits:
            return int(self._in_features)
        return int(self.codes.shape[-1]) * int(self.codebook.shape[1])

    @property
    def output_dims(self):
        return int(self.codes.shape[0])

    def forward(self, x):
        if int(self.codebook.shape[0]) != self._k_expect:
            raise RuntimeError(
                f"VQ codebook was sharded: K={self.codebook.shape[0]}, expected "
                f"{self._k_expect}. The codebook is a SHARED lookup table and must be "
                f"REPLICATED across tensor-parallel ranks.")
        OUT, IN = self.output_dims, self.input_dims
        lead = x.shape[:-1]
        xf = x.reshape(-1, IN)
        N = xf.shape[0]
        K, d = int(self.codebook.shape[0]), int(self.codebook.shape[1])
        G = IN // int(self.vq_scales.shape[-1])
        if N <= _fused_max_n(self.pack_bits, d) and VS.dense_fits(K, IN, G, d):
            y = VS._dense_fused(xf, self.codes, self.codebook, self.vq_scales,
                                pack_bits=self.pack_bits, in_features=self._in_features)
        else:
            y = _decode_matmul(xf, self.codes, self.codebook, self.vq_scales, G, OUT, IN,
                               self.pack_bits)
        return y.reshape(*lead, OUT)


class VQEmbedding(torch.nn.Module):
    """Drop-in for nn.Embedding whose table is VQ-coded (vq_dense.py:444-513):
    decodes only the gathered rows, bit-exact, and returns out_dtype."""

    def __init__(self, codes, codebook, vq_scales, group_size=64, pack_bits=0,
                 in_features=None, out_dtype=torch.bfloat16):
        super().__init__()
        if pack_bits and in_features is None:
            raise ValueError("packed codes need explicit in_features")
        self.codes = codes
        self.codebook = codebook
        self.vq_scales = vq_scales
        self.group_size = group_size
        self.pack_bits = pack_bits
        self._in_features = in_features
        self.out_dtype = out_dtype
        self._k_expect = int(codebook.shape[0])

    @property
    def num_embeddings(self):
        return int(self.codes.shape[0])

    @property
    def dims(self):
        if self.pack_bits:
            return int(self._in_features)
        return int(self.codes.shape[1]) * int(self.codebook.shape[1])

    def forward(self, ids):
        if int(self.codebook.shape[0]) != self._k_expect:
            raise RuntimeError("VQ codebook was sharded; must be replicated.")
        flat = ids.reshape(-1)
        IN = self.dims
        # gather the touched rows on device, then decode just those rows
        rows = self.codes.index_select(0, flat)
        sc = self.vq_scales.index_select(0, flat)
        w = VS.wdec_decode(rows, self.codebook, sc, flat.numel(), IN, self.group_size,
                           self.pack_bits)
        return w.reshape(*ids.shape, IN).to(self.out_dtype)
