"""Dense VQ linears for PyTorch-ROCm -- the vq_dense interface
(src/vqlab/runtime/vq_dense.py) over libvqk's HIP kernels.

  VQLinear(codes, codebook, vq_scales, group_size, pack_bits, in_features)
                                                     vq_dense.py:315-441
  _fused_max_n(pack_bits, d)                         vq_dense.py:60-102
  _decode_matmul(xf, codes, codebook, scales, group_size, OUT, IN, pack_bits)
                                                     vq_dense.py:262-312
  VQEmbedding(codes, codebook, vq_scales, ...)       vq_dense.py:444-513

VQLinear dispatches through vqk_linear_apply: small N runs the fused GEMV
(vqk_dense_gemv), large N vqk_dense_gemm -- up to 64 rows W is decoded
straight into matrix-core operands; above, the weight is dequantised into a
workspace panel in x's arithmetic type and multiplied by libvqk's matrix-core
GEMM. VQEmbedding decodes only the gathered rows (vqk_embed_gather), in one
launch.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib as L
from . import _torch as T
from . import vq_switch as VS

def _fused_max_n(pack_bits, d):
    """Rows up to which VQLinear runs the fused GEMV (vq_dense.py:55-102): the
    options' dense_fused_max_n (VQ_DENSE_FUSED_MAX_N, default 32)."""
    return int(VS.options().dense_fused_max_n)


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
        T.require_cuda(xf, self.codes, self.codebook, self.vq_scales)
        N = xf.shape[0]
        G = IN // int(self.vq_scales.shape[-1])
        keep = []
        w = T.weights(self.codes, self.codebook, self.vq_scales, G, self.pack_bits, IN, keep=keep)
        xf = xf.contiguous()
        y = torch.empty((N, OUT), dtype=xf.dtype, device=xf.device)
        o = VS.options()
        ws = ctypes.c_size_t()
        L.check(L.lib().vqk_linear_apply_workspace(ctypes.byref(w), N, ctypes.byref(o),
                                                   ctypes.byref(ws)), "VQLinear")
        work = torch.empty(ws.value, dtype=torch.uint8, device=xf.device) if ws.value else None
        L.check(L.lib().vqk_linear_apply(ctypes.byref(w), T.ptr(xf), T.act_type(xf), N, T.ptr(y),
                                         T.act_type(y), T.ptr(work) if work is not None else None,
                                         ws.value, ctypes.byref(o), T.stream(xf.device)),
                "VQLinear")
        return y.reshape(*lead, OUT)


def embed_gather(w, keep, ids, out_dtype):
    """rows ids of the table `w` (a vqk_weights with E == 1), decoded and
    converted to out_dtype in one launch: [*ids.shape, IN]."""
    dev = T.require_cuda(ids, *[t for t in keep if t is not None])
    if out_dtype not in T.ACT_TYPES:
        raise ValueError(f"out_dtype must be float16, bfloat16 or float32, got {out_dtype}")
    flat = ids.reshape(-1)
    if flat.dtype not in (torch.int32, torch.int64):
        flat = flat.to(torch.int64)
    flat = flat.contiguous()
    out = torch.empty((flat.numel(), int(w.IN)), dtype=out_dtype, device=dev)
    L.check(L.lib().vqk_embed_gather(ctypes.byref(w), T.ptr(flat),
                                     L.VQK_I64 if flat.dtype == torch.int64 else L.VQK_I32,
                                     flat.numel(), T.ptr(out), T.ACT_TYPES[out_dtype],
                                     T.stream(dev)),
            "embedding gather")
    return out.reshape(*ids.shape, int(w.IN))


class VQEmbedding(torch.nn.Module):
    """Drop-in for nn.Embedding whose table is VQ-coded (vq_dense.py:444-513):
    decodes only the gathered rows, bit-exactly, and returns out_dtype.
    codes [rows, NSUB] uint8/uint16 or [rows, WPR] uint32 words of
    pack_bits-wide fields; vq_scales [rows, IN / group_size] fp16."""

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

    def _desc(self, keep):
        return T.weights(self.codes, self.codebook, self.vq_scales, self.group_size,
                         self.pack_bits, self._in_features, k_expect=self._k_expect,
                         keep=keep)

    def forward(self, ids):
        # a codebook whose K changed was sliced (vq_dense.py:491-494): the
        # library refuses it (VQK_ESHARDED -> RuntimeError) before any launch
        keep = []
        w = self._desc(keep)
        return embed_gather(w, keep, ids, self.out_dtype)

    def as_linear(self, x):
        """x @ W.T over the whole decoded table (vq_dense.py:508-513), for a
        tied output head: the dense large-N path of VQLinear."""
        OUT, IN = self.num_embeddings, self.dims
        lead = x.shape[:-1]
        xf = x.reshape(-1, IN)
        y = _decode_matmul(xf, self.codes, self.codebook, self.vq_scales, self.group_size,
                           OUT, IN, self.pack_bits)
        return y.reshape(*lead, OUT)
