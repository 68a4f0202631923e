"""VQ routed-expert runtime for PyTorch-ROCm -- the vq_switch interface
(src/vqlab/runtime/vq_switch.py) over libvqk's HIP kernels.

Module-level functions keep the reference's names and argument meaning:
  VQSwitchLinear(codes, codebook, vq_scales, group_size, pack_bits,
                 in_features, row_table)                vq_switch.py:5194-5423
  _fused(x, eidx, codes, codebook, scales, ...)         vq_switch.py:2919-3249
  _dense_fused(x, codes, codebook, scales, ...)         vq_switch.py:3339-3434
  wdec_decode(codes, codebook, scales, rows, IN, G, pack_bits, r0)
                                                        vq_switch.py:3517-3544
  _decode_chunk(codes, codebook, scales, eidx_chunk, pack_bits, in_features)
                                                        vq_switch.py:4725-4782
  dense_fits / wdec_fits / gemmseg_fits                 3290 / 3505 / 4469
  skipzero_row_table / skipzero_weights                 4958-5013
  VQPLEEmbedding(codes, codebook, vq_scales, group_size, packed_nsub)
                                                        vq_switch.py:5426-5495
Tensors are torch tensors on a ROCm device; every call launches on the
current stream and never synchronises with the host.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib as L
from . import _torch as T

# The reference's VQ_* dispatch flags -- VQ_FUSED_MAX_N (pairs at or below which
# decode runs the fused GEMV, vq_switch.py:43-45), VQ_DECODE_BF16IO and
# VQ_GEMMSEG_BF16IO (vq_switch.py:4372, 4421) -- read once at import as the
# reference does, and handed to libvqk as one explicit options struct.
OPTIONS = None


def options():
    global OPTIONS
    if OPTIONS is None:
        OPTIONS = L.options(from_env=True)
    return OPTIONS


# ------------------------------------------------------------ predicates
def dense_fits(K, IN, G, d=2) -> bool:
    return bool(L.lib().vqk_dense_fits(int(K), int(IN), int(G), int(d)))


def wdec_fits(D, NSUB, G, pack_bits) -> bool:
    return bool(L.lib().vqk_wdec_fits(int(D), int(NSUB), int(G), int(pack_bits)))


def gemmseg_fits(D, K, G, pack_bits, IN) -> bool:
    return bool(L.lib().vqk_gemmseg_fits(int(D), int(K), int(G), int(pack_bits), int(IN)))


def _group(IN, scales) -> int:
    ngrp = int(scales.shape[-1])
    if ngrp <= 0 or IN % ngrp:
        raise ValueError(f"scales have {ngrp} groups, which does not divide IN={IN}")
    return IN // ngrp


def _in_features(codes, codebook, pack_bits, in_features, scales):
    if pack_bits:
        if in_features is not None:
            return int(in_features)
        # the scales axis carries the true width for padded-tail packs
        return int(scales.shape[-1]) * 64
    return int(codes.shape[-1]) * int(codebook.shape[1])


# ---------------------------------------------------------------- kernels
def _fused(x, eidx, codes, codebook, scales, pack_bits=0, simd=None, d2_u32=None,
           xkrep=None, rowtbl=None, in_features=None, out_dtype=None):
    """[N, OUT] = fused VQ GEMV over (token, expert) pairs, in x's dtype
    (or out_dtype).

    x is [T, IN]; with xkrep, pair n reads token row n // xkrep, else x has
    one row per pair. eidx: [N] expert ids (device). simd / d2_u32 select
    Metal kernel twins in the reference and have no meaning here.
    """
    T.require_cuda(x, eidx, codes, codebook, scales, rowtbl)
    IN = int(x.shape[-1])
    if in_features is not None and int(in_features) != IN:
        raise ValueError(f"x is IN={IN} but the module says in_features={in_features}")
    G = _group(IN, scales)
    keep = []
    w = T.weights(codes, codebook, scales, G, pack_bits, IN, rowtbl, keep=keep)
    x = x.contiguous()
    e = eidx.reshape(-1).to(torch.int32).contiguous()
    N = e.numel()
    rep = int(xkrep) if xkrep is not None else 1
    Tt = x.shape[0]
    y = torch.empty((N, w.OUT), dtype=out_dtype or x.dtype, device=x.device)
    L.check(L.lib().vqk_moe_expert_gemv(ctypes.byref(w), T.ptr(x), T.act_type(x), Tt, T.ptr(e),
                                        N, rep, T.ptr(y), T.act_type(y), T.stream(x.device)),
            "_fused")
    return y


def _dense_fused(x, codes, codebook, scales, pack_bits=0, in_features=None):
    """Dense fused GEMV: y[N, OUT] = x[N, IN] @ decode(codes).T (vq_switch.py:3339)."""
    T.require_cuda(x, codes, codebook, scales)
    N, IN = x.shape
    if pack_bits and in_features is not None and int(in_features) != IN:
        raise ValueError(f"packed dense: x is IN={IN} but module says in_features={in_features}")
    G = _group(IN, scales)
    keep = []
    w = T.weights(codes, codebook, scales, G, pack_bits, IN, keep=keep)
    x = x.contiguous()
    y = torch.empty((N, w.OUT), dtype=x.dtype, device=x.device)
    L.check(L.lib().vqk_dense_gemv(ctypes.byref(w), T.ptr(x), T.act_type(x), N, T.ptr(y),
                                   T.act_type(y), T.stream(x.device)), "_dense_fused")
    return y


def wdec_decode(codes, codebook, scales, rows, IN, G, pack_bits, r0=0):
    """Rows [r0, r0+rows) of the (flattened) module -> [rows, IN] fp16, bit-exact."""
    T.require_cuda(codes, codebook, scales)
    keep = []
    w = T.weights(codes, codebook, scales, G, pack_bits, IN, keep=keep)
    out = torch.empty((int(rows), int(IN)), dtype=torch.float16, device=codes.device)
    L.check(L.lib().vqk_dequant(ctypes.byref(w), int(r0), int(rows), T.ptr(out),
                                T.stream(codes.device)), "wdec_decode")
    return out


def _decode_chunk(codes, codebook, scales, eidx_chunk, pack_bits=0, in_features=None,
                  rowtbl=None):
    """Experts eidx_chunk -> [NE, OUT, IN] fp16 weights, bit-exact."""
    T.require_cuda(codes, codebook, scales, eidx_chunk, rowtbl)
    IN = _in_features(codes, codebook, pack_bits, in_features, scales)
    G = _group(IN, scales)
    keep = []
    w = T.weights(codes, codebook, scales, G, pack_bits, IN, rowtbl, keep=keep)
    e = eidx_chunk.reshape(-1).to(torch.int32).contiguous()
    out = torch.empty((e.numel(), w.OUT, IN), dtype=torch.float16, device=codes.device)
    L.check(L.lib().vqk_dequant_experts(ctypes.byref(w), T.ptr(e), e.numel(), T.ptr(out),
                                        T.stream(codes.device)), "_decode_chunk")
    return out


def _gemmseg(x2, eidx, codes, codebook, scales, pack_bits, IN, xkrep, rowtbl=None,
             out_dtype=None):
    """Large-N routed path: device-sorted grouped GEMM on the matrix cores.
    Output rows are in the caller's pair order (the reference sorts on the
    host and un-permutes with y[inv], vq_switch.py:5383-5394)."""
    G = _group(IN, scales)
    keep = []
    w = T.weights(codes, codebook, scales, G, pack_bits, IN, rowtbl, keep=keep)
    x2 = x2.contiguous()
    e = eidx.reshape(-1).to(torch.int32).contiguous()
    N = e.numel()
    ws = ctypes.c_size_t()
    L.check(L.lib().vqk_grouped_gemm_workspace(ctypes.byref(w), N, ctypes.byref(ws)), "_gemmseg")
    work = torch.empty(max(1, ws.value), dtype=torch.uint8, device=x2.device)
    y = torch.empty((N, w.OUT), dtype=out_dtype or x2.dtype, device=x2.device)
    L.check(L.lib().vqk_grouped_gemm(ctypes.byref(w), T.ptr(x2), T.act_type(x2), x2.shape[0],
                                     T.ptr(e), N, int(xkrep), T.ptr(y), T.act_type(y),
                                     T.ptr(work), ws.value, T.stream(x2.device)), "_gemmseg")
    return y


def _float_staged(codebook, pack_bits) -> bool:
    """The reference's decode kernels that stage x as float and take bf16 x
    unrounded under VQ_DECODE_BF16IO: unpacked d4 with K <= 1024, d8 with
    K > 1024 (vq_switch.py:106-150, 2781, 3172-3185); libvqk's
    vqk_switch_apply applies the same rule."""
    K, D = int(codebook.shape[0]), int(codebook.shape[1])
    return (D == 8 and K > 1024) or (D == 4 and not pack_bits and K <= 1024)


def _switch_apply(x2, eidx, codes, codebook, scales, pack_bits, IN, xkrep, rowtbl=None,
                  out_dtype=None, opts=None):
    """VQSwitchLinear's dispatch through vqk_switch_apply with the module
    options (or `opts`); out_dtype (an extension) rounds once into it."""
    T.require_cuda(x2, eidx, codes, codebook, scales, rowtbl)
    G = _group(IN, scales)
    keep = []
    w = T.weights(codes, codebook, scales, G, pack_bits, IN, rowtbl, keep=keep)
    x2 = x2.contiguous()
    e = eidx.reshape(-1).to(torch.int32).contiguous()
    N = e.numel()
    o = opts or options()
    ws = ctypes.c_size_t()
    L.check(L.lib().vqk_switch_apply_workspace(ctypes.byref(w), N, ctypes.byref(o),
                                               ctypes.byref(ws)), "VQSwitchLinear")
    work = torch.empty(ws.value, dtype=torch.uint8, device=x2.device) if ws.value else None
    y = torch.empty((N, w.OUT), dtype=out_dtype or x2.dtype, device=x2.device)
    wk = T.ptr(work) if work is not None else None
    if out_dtype is not None:
        # the same dispatch (a workspace means the grouped GEMM), one rounding
        if ws.value:
            L.check(L.lib().vqk_grouped_gemm(ctypes.byref(w), T.ptr(x2), T.act_type(x2), x2.shape[0],
                                             T.ptr(e), N, int(xkrep), T.ptr(y), T.act_type(y), wk,
                                             ws.value, T.stream(x2.device)), "VQSwitchLinear")
        else:
            xt = T.act_type(x2)
            if o.decode_bf16io and x2.dtype == torch.bfloat16 and _float_staged(codebook, pack_bits):
                xt |= L.VQK_X_KEEP             # as vqk_switch_apply does
            L.check(L.lib().vqk_moe_expert_gemv(ctypes.byref(w), T.ptr(x2), xt,
                                                x2.shape[0], T.ptr(e), N, int(xkrep), T.ptr(y),
                                                T.act_type(y), T.stream(x2.device)), "VQSwitchLinear")
        return y
    L.check(L.lib().vqk_switch_apply(ctypes.byref(w), T.ptr(x2), T.act_type(x2), x2.shape[0],
                                     T.ptr(e), N, int(xkrep), T.ptr(y), T.act_type(y), wk,
                                     ws.value, ctypes.byref(o), T.stream(x2.device)), "VQSwitchLinear")
    return y


# ------------------------------------------------------------- skipzero
def skipzero_row_table(rowmask, E, OUT):
    """uint8 [E, ceil(OUT/8)] live-row mask (little bit order) -> int32 [E, OUT]
    compact row per (expert, row), -1 = dead (vq_switch.py:4958-4973). Built
    on the host like the reference's CPU-stream build; returned on rowmask's
    device."""
    dev = rowmask.device if isinstance(rowmask, torch.Tensor) else None
    rm = np.ascontiguousarray(
        rowmask.cpu().numpy() if isinstance(rowmask, torch.Tensor) else rowmask, np.uint8)
    table = np.empty((int(E), int(OUT)), np.int32)
    n = ctypes.c_int64()
    L.check(L.lib().vqk_skipzero_row_table_host(rm.ctypes.data, int(E), int(OUT),
                                                table.ctypes.data, ctypes.byref(n)),
            "skipzero_row_table")
    t = torch.from_numpy(table)
    return t.to(dev) if dev is not None else t


def skipzero_weights(weights, modules, shard=None):
    """On-disk skipzero tensors -> what VQSwitchLinear(row_table=...) loads
    (vq_switch.py:4988-5013); the conversion lives with the artifact loader
    (artifact.convert_skipzero), which applies the same per-module checks.
    `shard` = (rank, n) takes the rank's tensor-parallel slice first
    (artifact.skipzero_shard, vq_switch.py:5112-5147)."""
    from .artifact import convert_skipzero
    return convert_skipzero(weights, modules, shard)


def skipzero_shard(weights, modules, rank, n):
    """Rank `rank` of an n-way split of on-disk skipzero tensors
    (vq_switch.py:5112-5147); see artifact.skipzero_shard."""
    from .artifact import skipzero_shard as _shard
    return _shard(weights, modules, rank, n)


# ---------------------------------------------------------------- module
class VQSwitchLinear(torch.nn.Module):
    """Drop-in for mlx-lm's QuantizedSwitchLinear over VQ codes
    (vq_switch.py:5194-5423). No bias."""

    def __init__(self, codes, codebook, vq_scales, group_size: int = 64, pack_bits: int = 0,
                 in_features: int | None = None, row_table=None):
        super().__init__()
        if row_table is not None and (codes.ndim != 2 or vq_scales.ndim != 2):
            raise ValueError("skipzero codes/vq_scales must be compact 2-D")
        if pack_bits and in_features is None:
            raise ValueError("packed codes need explicit in_features: a packed row is WPR "
                             "words wide, so its shape no longer implies the input dimension")
        self.codes = codes
        self.codebook = codebook
        self.vq_scales = vq_scales
        self.row_table = row_table
        self.group_size = group_size
        self.pack_bits = pack_bits
        self._in_features = in_features
        self._k_expect = int(codebook.shape[0])

    @classmethod
    def from_weights(cls, codes, codebook, vq_scales):
        if codes.dtype in (torch.int32, torch.uint32):
            k = int(codebook.shape[0])
            bits = (k - 1).bit_length()
            return cls(codes, codebook, vq_scales, pack_bits=bits,
                       in_features=int(vq_scales.shape[-1]) * 64)
        return cls(codes, codebook, vq_scales)

    @property
    def skipzero(self):
        return self.row_table is not None

    @property
    def input_dims(self):
        if self.pack_bits:
            return int(self.vq_scales.shape[-1]) * self.group_size
        return int(self.codes.shape[-1]) * int(self.codebook.shape[1])

    @property
    def output_dims(self):
        return int(self.row_table.shape[1] if self.skipzero else self.codes.shape[1])

    @property
    def num_experts(self):
        return int(self.row_table.shape[0] if self.skipzero else self.codes.shape[0])

    def _check_codebook(self):
        k_now = int(self.codebook.shape[0])
        if k_now != self._k_expect:
            raise RuntimeError(
                f"VQ codebook was sharded: K={k_now}, expected {self._k_expect}. The codebook "
                f"is a SHARED lookup table and must be replicated across tensor-parallel "
                f"ranks, not sliced (codes and scales shard fine on the default axes).")

    def forward(self, x, indices, sorted_indices=False, out_dtype=None):
        """x [..., 1, 1, IN] (broadcast over indices [..., k]) -> [..., k, 1, OUT]
        in x's dtype, or out_dtype (an extension: callers that keep fp32
        intermediates skip one rounding)."""
        self._check_codebook()
        IN, OUT = self.input_dims, self.output_dims
        N = indices.numel()
        T_tok = x.numel() // IN
        if T_tok > 0 and N % T_tok == 0:
            x2, rep = x.reshape(T_tok, IN), N // T_tok
        else:
            lead = tuple(indices.shape)
            x2, rep = x.expand(*lead, 1, IN).reshape(N, IN), 1
        eidx = indices.reshape(-1)
        # libvqk's dispatch (vqk_switch_apply): the fused GEMV up to
        # VQ_FUSED_MAX_N pairs, else -- or, an extension beyond the
        # reference, when the pairs crowd onto few experts (N >= 4 and
        # N >= 2E) -- the grouped GEMM. By default the
        # outputs are rounded through fp16 like the reference's fp16 kernels
        # and cast; an explicit out_dtype keeps the single rounding.
        y = _switch_apply(x2, eidx, self.codes, self.codebook, self.vq_scales, self.pack_bits,
                          IN, rep, self.row_table, out_dtype=out_dtype)
        return y.reshape(*indices.shape, 1, OUT)


class VQPLEEmbedding(torch.nn.Module):
    """VQ-coded embedding / per-layer-embedding (PLE) table shard whose
    decode is a pure gather (vq_switch.py:5426-5495):
      codes      uint16 [rows, cols / dim] unpacked, or, with packed_nsub,
                 uint8 [rows, row_bytes]: packed_nsub codes of
                 BITS = max(1, bit_length(K - 1)) bits back to back, code j at
                 bits [j*BITS, (j+1)*BITS) of the row, LSB first
      codebook   fp16 [K, dim]
      vq_scales  fp16 [rows, cols / group_size]
    __call__(ids) -> [*ids.shape, cols] bfloat16: codebook[codes[ids]] times
    the row's group scales, rounded to fp16 and then to bf16, decoded in one
    launch of vqk_embed_gather. At BITS == 8 the byte stream is the codes
    themselves (vq_switch.py:5456-5467) and is read as plain uint8 codes."""

    def __init__(self, codes, codebook, vq_scales, group_size: int = 32,
                 packed_nsub: int = 0):
        super().__init__()
        self.codes = codes
        self.codebook = codebook
        self.vq_scales = vq_scales
        self.group_size = group_size
        self._pn = int(packed_nsub)
        self._bits = max(1, (int(codebook.shape[0]) - 1).bit_length())
        self._byte_codes = bool(packed_nsub) and self._bits == 8

    def _desc(self, keep):
        d = int(self.codebook.shape[1])
        if self._pn and not self._byte_codes:
            if self.codes.dtype != torch.uint8:
                raise ValueError(f"packed PLE rows must be uint8 bytes, got {self.codes.dtype}")
            w = T.weights(self.codes, self.codebook, self.vq_scales, self.group_size,
                          pack_bits=self._bits, in_features=self._pn * d, keep=keep)
            return w
        if self._pn and int(self.codes.shape[-1]) != self._pn:
            raise ValueError(f"byte-coded PLE rows are {self.codes.shape[-1]} bytes, "
                             f"expected {self._pn} codes")
        return T.weights(self.codes, self.codebook, self.vq_scales, self.group_size, keep=keep)

    def forward(self, ids):
        from .vq_dense import embed_gather
        keep = []
        w = self._desc(keep)
        return embed_gather(w, keep, ids, torch.bfloat16)
