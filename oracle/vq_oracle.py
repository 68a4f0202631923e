"""CPU oracle for the VQ weight-decode path -- TEST INFRASTRUCTURE ONLY.

This module restates, in numpy, what the reference computes on the fused VQ
decode path. It is the checker the HIP kernels are compared against. Only
`tests/`, `__graft_entry__.smoke()` and `bench.py`'s cpu_baseline leg may
import it; the product (`vqlab_amd`) never does, and has no CPU fallback.

Reference anchors (paths relative to the reference checkout):
  pack / unpack / bits_for_k / words_per_row   src/vqlab/runtime/vq_pack.py:34-97
  pack_bits_for (codepack rule)                src/vqlab/core/artifacts/codepack.py:22-30
  dequant  W = fp16(f32(cb[c]) * f32(s))       src/vqlab/runtime/vq_switch.py:3463-3493,
                                               vq_dense.py:132-137
  decode-then-matmul                           gate/kernel_reference.py:10-23,
                                               score/kernel_truth_moe.py:35-49
  expert GEMV semantics (x rows, xkrep, sz)    vq_switch.py:2919-2963, 4422-4451, 733-795
  router + SwitchGLU + combine                 bench/decode_ladder.py:107-119,
                                               tests/test_qwen3_5_parity.py:180-205
  skipzero compact form / row table            skipzero/skipzero_load.py:1-65,
                                               skipzero/sz_pack.py:77-113,
                                               vq_switch.py:4958-4973
  grouped-GEMM tile metadata                   vq_switch.py:4590-4610,
                                               tests/test_routing_memo.py:51-62
  embeddings (gather-only decode)              vq_dense.py:491-506 (VQEmbedding),
                                               vq_switch.py:5426-5495 (VQPLEEmbedding)

Pinning (what checks each function; see tests/test_oracle.py):
  pack/unpack      reference golden sha256 prefixes (bits 4) + bit-serial brute
                   force for every width 2..16 + byte-identity of widths 8/16
                   with little-endian u8/u16 arrays.
  dequant          numpy's own IEEE fp16 conversion is the single rounding;
                   cross-checked against the independent C restatement
                   (vq_oracle.c) including subnormal, inf and NaN inputs.
  decode_matmul    float64 brute-force loop on tiny shapes; closed forms
                   (one-hot codebook, constant scales).
  dequant_exact    equals dequant wherever s * cb is an fp16 value (scales
                   that are powers of two); per-group brute-force loop of the
                   reference's fused formula on tiny shapes.
  route            brute-force sort; weights sum to one; softmax invariance.
  moe_layer        identical-expert invariant (combine of equal experts ==
                   one expert), per-pair loop restatement; the shared-expert
                   term by closed forms (shared expert == the only routed
                   expert: a zero gate vector gives exactly 1.5x the routed
                   output, gate logits of +-1000 give 2x and 1x) in both
                   rounding modes.
  bf16_round,      torch's own float32 -> bfloat16 / float16 conversions
  fp16_round,      over 200k random bit patterns, bf16 ties and specials
  f32_to_bf16_bits (bit patterns, signed zeros included; NaN by its rule).
  skipzero         reference golden sha256 prefixes (sz_codes, sz_scales,
                   sz_rowmask, sz_shape) + cumsum brute force for the table.
  tile_meta        the reference test's double loop, restated.
  ple_unpack       bit-serial brute force over the byte stream (numpy
                   unpackbits) for widths 1..16 + the width-8 identity the
                   reference relies on (vq_switch.py:5456-5467).
  embed_rows       dequant of the gathered rows == the gathered rows of the
                   full-table dequant; f16_to_bf16 against torch's own
                   float -> bfloat16 conversion (round to nearest even) over
                   every fp16 bit pattern.
"""
from __future__ import annotations

import numpy as np

BLOCK = 32          # codes per packing block (vq_pack.py:31)
SZ_TINY = 6.2e-5    # dead-row threshold (skipzero_load.py:14, sz_pack.py:104)


# ----------------------------------------------------------------- a1: widths
def bits_for_k(k: int) -> int:
    """vq_pack.py:34-38: BITS = log2 K, K must be a power of two."""
    k = int(k)
    b = (k - 1).bit_length()
    if k < 1 or (1 << b) != k:
        raise ValueError(f"K={k} is not a power of two")
    return b


def words_per_row(nsub: int, bits: int) -> int:
    """vq_pack.py:41-45: ceil(NSUB/32) blocks of BITS words each."""
    return (int(nsub) + BLOCK - 1) // BLOCK * int(bits)


def pack_bits_for(k: int, nsub: int, pack_unaligned: bool = False) -> int:
    """codepack.py:22-30: byte-aligned widths and unaligned NSUB stay unpacked."""
    bits = bits_for_k(k)
    if nsub % BLOCK and not pack_unaligned:
        return 0
    if bits % 8 == 0:
        return 0
    return bits


# ----------------------------------------------------------- a2/a3: pack
def pack(codes: np.ndarray, bits: int) -> np.ndarray:
    """[..., NSUB] integer codes -> [..., WPR] uint32 (vq_pack.py:48-76).

    Code i of each 32-code block sits at bit i*BITS of the block, LSB first;
    a field may straddle two words but never leaves its block. The tail block
    of an unaligned row is zero-padded.
    """
    codes = np.asarray(codes)
    lead, nsub = codes.shape[:-1], codes.shape[-1]
    if codes.size and int(codes.max()) >= (1 << bits):
        raise ValueError("code exceeds bit width")
    nblk = (nsub + BLOCK - 1) // BLOCK
    padded = np.zeros(lead + (nblk * BLOCK,), np.uint64)
    padded[..., :nsub] = codes
    src = padded.reshape(lead + (nblk, BLOCK))
    out = np.zeros(lead + (nblk, bits), np.uint64)
    for i in range(BLOCK):
        w, sh = divmod(i * bits, 32)
        v = src[..., i] << np.uint64(sh)
        out[..., w] |= v & np.uint64(0xFFFFFFFF)
        if sh + bits > 32:
            out[..., w + 1] |= v >> np.uint64(32)
    return out.astype(np.uint32).reshape(lead + (nblk * bits,))


def unpack(packed: np.ndarray, nsub: int, bits: int) -> np.ndarray:
    """Inverse of pack (vq_pack.py:79-97): uint8 for bits <= 8, else uint16."""
    packed = np.asarray(packed, np.uint32)
    lead, wpr = packed.shape[:-1], packed.shape[-1]
    if wpr != words_per_row(nsub, bits):
        raise ValueError(f"WPR {wpr} != words_per_row({nsub}, {bits})")
    nblk = wpr // bits
    src = packed.reshape(lead + (nblk, bits)).astype(np.uint64)
    mask = np.uint64((1 << bits) - 1)
    out = np.zeros(lead + (nblk, BLOCK), np.uint64)
    for i in range(BLOCK):
        w, sh = divmod(i * bits, 32)
        v = src[..., w] >> np.uint64(sh)
        if sh + bits > 32:
            v = v | (src[..., w + 1] << np.uint64(32 - sh))
        out[..., i] = v & mask
    out = out.reshape(lead + (nblk * BLOCK,))[..., :nsub]
    return out.astype(np.uint16 if bits > 8 else np.uint8)


def unpack_bitserial(packed: np.ndarray, nsub: int, bits: int) -> np.ndarray:
    """The same layout read one bit at a time: bit k of code j lives at
    absolute bit (j//32)*32*BITS + (j%32)*BITS + k of the row. A second,
    structurally different reading of vq_pack.py:11-27 used to pin unpack."""
    packed = np.asarray(packed, np.uint32)
    lead = packed.shape[:-1]
    flat = packed.reshape(-1, packed.shape[-1])
    res = np.zeros((flat.shape[0], nsub), np.uint32)
    for j in range(nsub):
        base = (j // BLOCK) * BLOCK * bits + (j % BLOCK) * bits
        for k in range(bits):
            pos = base + k
            bit = (flat[:, pos // 32] >> np.uint32(pos % 32)) & np.uint32(1)
            res[:, j] |= bit << np.uint32(k)
    return res.reshape(lead + (nsub,))


# ------------------------------------------------------------- a4: dequant
def dequant(codes: np.ndarray, codebook: np.ndarray, scales: np.ndarray,
            group: int) -> np.ndarray:
    """W[r, j*d+u] = fp16_RNE(f32(cb[c_rj, u]) * f32(s[r, (j*d+u)//G])).

    vq_switch.py:3484-3492 (wdec) and vq_dense.py:132-137 (_decode): the
    fp16 x fp16 product is exact in fp32, so exactly one rounding happens.
    codes [..., NSUB] (unpacked), codebook [K, d] fp16, scales [..., IN/G]
    fp16 -> [..., IN] fp16.
    """
    codes = np.asarray(codes).astype(np.int64)
    cb = np.asarray(codebook, np.float16).astype(np.float32)
    s = np.asarray(scales, np.float16).astype(np.float32)
    d = cb.shape[1]
    lead, nsub = codes.shape[:-1], codes.shape[-1]
    w = cb[codes].reshape(lead + (nsub * d,))
    ngrp = s.shape[-1]
    with np.errstate(invalid="ignore", over="ignore"):
        if ngrp * group == nsub * d:
            # whole groups: broadcast each scale over its group (same products,
            # no repeated scale array)
            prod = w.reshape(lead + (ngrp, group)) * s[..., None]
            return prod.astype(np.float16).reshape(lead + (nsub * d,))
        sx = np.repeat(s, group, axis=-1)[..., : nsub * d]
        return (w * sx).astype(np.float16)


# ------------------------------------------------------ decode-then-matmul
def decode_matmul(x: np.ndarray, w16: np.ndarray, acc: str = "f64") -> np.ndarray:
    """y = x @ W.T with W the dequantized fp16 weight (vq_dense.py:267-294);
    accumulation in float64 ('f64', score/kernel_truth.py) or float32
    ('f32', gate/kernel_reference.py). x [N, IN] (any float dtype)."""
    dt = np.float64 if acc == "f64" else np.float32
    return np.asarray(x, np.float32).astype(dt) @ np.asarray(w16).astype(dt).T


def dequant_exact(codes: np.ndarray, codebook: np.ndarray, scales: np.ndarray,
                  group: int) -> np.ndarray:
    """W[r, j*d+u] = f64(cb[c_rj, u]) * f64(s[r, (j*d+u)//G]), unrounded.

    The fused decode kernels never form an fp16 weight: they sum the code
    dots <cb[c], x> of a scale group and scale that sum once
    (`acc = fma((float)srow[g], gacc, acc)`, vq_switch.py:1344-1350, 978-985),
    so in exact arithmetic their weight is this product (distributivity).
    """
    codes = np.asarray(codes).astype(np.int64)
    cb = np.asarray(codebook, np.float16).astype(np.float64)
    s = np.asarray(scales, np.float16).astype(np.float64)
    d = cb.shape[1]
    lead, nsub = codes.shape[:-1], codes.shape[-1]
    w = cb[codes].reshape(lead + (nsub * d,))
    sx = np.repeat(s, group, axis=-1)[..., : nsub * d]
    with np.errstate(invalid="ignore", over="ignore"):
        return w * sx


def expert_gemv(x, eidx, codes, codebook, scales, group, xkrep=1,
                row_table=None, acc="f64", weights="fp16"):
    """y[n, r] for pairs n: token row n // xkrep against expert eidx[n].

    Mirrors _fused's contract (vq_switch.py:2919-2963, XKREP 4422-4451):
    codes [E, OUT, NSUB] unpacked (or compact [NLIVE, NSUB] with a row
    table [E, OUT], -1 = dead row -> exact +0, vq_switch.py:760-771).
    weights "fp16": the dequantised fp16 weight (dequant); "exact": the
    fused kernels' per-group scaling unrounded (dequant_exact), for checks
    whose bar is tighter than one fp16 rounding of W. x is taken in
    float32 (bf16 values exactly); a path that stages it as fp16 gets it
    rounded by the caller.
    """
    x = np.asarray(x, np.float32)
    deq = dequant_exact if weights == "exact" else dequant
    eidx = np.asarray(eidx).astype(np.int64).reshape(-1)
    n_pairs = eidx.shape[0]
    if row_table is None:
        out = codes.shape[1]
    else:
        out = row_table.shape[1]
    dt = np.float64 if acc == "f64" else np.float32
    y = np.zeros((n_pairs, out), dt)
    cache = {}                      # expert -> its dequantized fp16 weight, widened once
    for n in range(n_pairs):
        e = int(eidx[n])
        if e not in cache:
            if row_table is None:
                w = deq(codes[e], codebook, scales[e], group)
            else:
                rt = np.asarray(row_table)[e]
                live = rt >= 0
                w = np.zeros((out, codes.shape[-1] * codebook.shape[1]),
                             np.float64 if weights == "exact" else np.float16)
                if live.any():
                    w[live] = deq(codes[rt[live]], codebook, scales[rt[live]], group)
            cache[e] = w.astype(dt)
        y[n] = x[n // xkrep].astype(dt) @ cache[e].T
    return y


# ------------------------------------------------------------ a15: MoE block
def route(logits: np.ndarray, top_k: int, norm: bool = True):
    """softmax (fp32) -> top-k -> renormalise (decode_ladder.py:107-113;
    test_qwen3_5_parity.py:187-191). Ties are broken towards the lower
    expert id (stable descending sort); on continuous logits they have
    probability zero. Returns (ids [T, k] int64 in descending-weight order,
    weights [T, k] float64).

    NaN logits (which make the reference's softmax NaN throughout) are this
    build's defined extension: they take no part in the softmax, rank below
    every other logit (-inf included) and are never selected; a row with
    fewer than top_k non-NaN logits fills its last selections with id -1 and
    weight 0. Every row needs a finite logit."""
    lg = np.asarray(logits, np.float64)
    nan = np.isnan(lg)
    lgm = np.where(nan, -np.inf, lg)
    pr = np.exp(lgm - lgm.max(-1, keepdims=True))
    pr = pr / pr.sum(-1, keepdims=True)
    pos = np.broadcast_to(np.arange(lg.shape[-1]), lg.shape)
    idx = np.stack([np.lexsort((pos[t], nan[t], -pr[t])) for t in range(lg.shape[0])])[:, :top_k]
    w = np.take_along_axis(pr, idx, -1)
    dead = np.take_along_axis(nan, idx, -1)
    idx = np.where(dead, -1, idx)
    w = np.where(dead, 0.0, w)
    if norm:
        w = w / w.sum(-1, keepdims=True)
    return idx, w


def silu(v):
    return v / (1.0 + np.exp(-v))


def sigmoid(v):
    return 1.0 / (1.0 + np.exp(-v))


def f32_to_bf16_bits(u) -> np.ndarray:
    """float32 bit patterns (uint32) -> bfloat16 bit patterns (uint16): round
    to nearest even on the bits; a NaN keeps its sign and top payload bits
    with the quiet bit set."""
    u = np.asarray(u, np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    return np.where(nan, (u >> 16) | 0x40, r).astype(np.uint16)


def bf16_round(v) -> np.ndarray:
    """Values -> the float64 values of their bfloat16 roundings: one RNE of
    the float32 value to 8 significand bits (what `.astype(bfloat16)` does to
    an fp32 array); NaN stays NaN."""
    u = np.asarray(v, np.float64).astype(np.float32).view(np.uint32)
    r = f32_to_bf16_bits(u)
    return (r.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def fp16_round(v) -> np.ndarray:
    """float64 -> float32 -> fp16 (RNE) -> float64: a kernel's fp32
    accumulator stored as an fp16 output."""
    with np.errstate(over="ignore"):
        return np.asarray(v, np.float64).astype(np.float32).astype(np.float16).astype(np.float64)


def moe_layer(x, logits, gate, up, down, top_k, norm=True, shared=None,
              shared_gate=None, h_round=None, rounding=None):
    """Qwen-style SparseMoeBlock over VQ experts.

    y[t] = sum_j w[t,j] * down_e(silu(gate_e(x_t)) * up_e(x_t))
           + sigmoid(shared_gate . x_t) * shared(x_t)
    (test_qwen3_5_parity.py:180-205; decode_ladder.py:107-119).

    gate/up/down are dicts {codes (unpacked [E,OUT,NSUB]), codebook, scales,
    group}; shared, if given, is a dict of three such (E=1) and shared_gate a
    float vector [H].

    Rounding of the intermediates (the dot products are float64 over the
    exact fp16 weights either way):
      rounding=None      float64 throughout; h_round, if given, is a numpy
                         float dtype the SwiGLU intermediate is rounded to
                         before down_proj (the fused kernels hand down_proj an
                         fp16 activation).
      rounding="reference"  the rounding points of the reference's bf16
                         decode path: each VQSwitchLinear's fp32 accumulator
                         leaves its kernel as fp16 and is cast back to x's
                         dtype, bf16 (vq_switch.py:5306-5308, 5423); SwiGLU
                         runs in bf16 (silu = g * sigmoid(g), each op rounded);
                         down_proj's bf16 input is cast to fp16 again; the
                         shared gate linear and its sigmoid give bf16
                         (decode_ladder.py:117-125); the weighted sum over
                         experts is float (scores are fp32 router outputs).
    Returns (y [T, H] float64, ids, weights).
    """
    x = np.asarray(x, np.float32).astype(np.float64)
    ids, w = route(logits, top_k, norm)
    T = x.shape[0]
    H = down["codes"].shape[1]
    y = np.zeros((T, H), np.float64)
    wcache = {}
    ref = rounding == "reference"
    if rounding not in (None, "reference"):
        raise ValueError(f"unknown rounding {rounding!r}")

    def W(p, e):
        key = (id(p), e)
        if key not in wcache:
            wcache[key] = dequant(p["codes"][e], p["codebook"], p["scales"][e],
                                  p["group"]).astype(np.float64)
        return wcache[key]

    def lin(p, e, v):
        out = W(p, e) @ v
        return bf16_round(fp16_round(out)) if ref else out

    def mlp(xt, g, u, dn, e):
        gv, uv = lin(g, e, xt), lin(u, e, xt)
        if ref:
            h = bf16_round(bf16_round(gv * bf16_round(sigmoid(gv))) * uv)
            h = fp16_round(h)
        else:
            h = silu(gv) * uv
            if h_round is not None:
                h = h.astype(h_round).astype(np.float64)
        return lin(dn, e, h)

    for t in range(T):
        for j in range(top_k):
            e = int(ids[t, j])
            if e >= 0:                     # -1: a selection left empty (NaN logits)
                y[t] += w[t, j] * mlp(x[t], gate, up, down, e)
        if shared is not None:
            z = float(np.asarray(shared_gate, np.float64) @ x[t])
            sg = float(bf16_round(sigmoid(bf16_round(z)))) if ref else sigmoid(z)
            y[t] += sg * mlp(x[t], shared["gate"], shared["up"], shared["down"], 0)
    return y, ids, w


# ------------------------------------------------------------ a14: skipzero
def skipzero_compact(codes: np.ndarray, scales: np.ndarray, tiny: float = SZ_TINY):
    """Expanded [E, OUT, W] codes / [E, OUT, NGRP] scales -> the on-disk
    skipzero tensors (sz_pack.py:77-113 dead-row rule; skipzero_load.py:8-16):
    a row is dead when every one of its scales is < tiny.
    Returns dict(sz_codes [NLIVE, W], sz_scales [NLIVE, NGRP],
    sz_rowmask uint8 [E, ceil(OUT/8)] little bit order, sz_shape int32[4])."""
    E, OUT = codes.shape[:2]
    live = ~(np.asarray(scales).astype(np.float32) < tiny).all(axis=-1)
    flat = live.reshape(-1)
    return {
        "sz_codes": np.ascontiguousarray(codes.reshape(E * OUT, -1)[flat]),
        "sz_scales": np.ascontiguousarray(scales.reshape(E * OUT, -1)[flat]),
        "sz_rowmask": np.packbits(live, axis=-1, bitorder="little"),
        "sz_shape": np.array([E, OUT, codes.shape[-1], scales.shape[-1]], np.int32),
    }


def skipzero_row_table(rowmask: np.ndarray, E: int, OUT: int) -> np.ndarray:
    """vq_switch.py:4958-4973: int32 [E, OUT], compact row of each live
    (expert, row) in expert-major order, -1 for a dead row."""
    bits = np.unpackbits(np.asarray(rowmask, np.uint8).reshape(E, -1), axis=-1,
                         bitorder="little")[:, :OUT]
    live = bits.reshape(-1).astype(np.int64)
    pos = np.cumsum(live) - 1
    return np.where(live > 0, pos, -1).astype(np.int32).reshape(E, OUT)


def skipzero_expand(shape, rowmask, compact):
    """skipzero_load.py:53-64: compact rows back to [E, OUT, W]; dead = 0."""
    E, OUT = int(shape[0]), int(shape[1])
    live = np.unpackbits(np.asarray(rowmask, np.uint8), axis=-1,
                         bitorder="little")[:, :OUT].astype(bool).reshape(-1)
    full = np.zeros((E * OUT,) + compact.shape[1:], compact.dtype)
    full[live] = compact
    return full.reshape((E, OUT) + compact.shape[1:])


# ---------------------------------------------- a12: grouped tile metadata
def sort_routing(idx: np.ndarray, k_rep: int):
    """vq_switch.py:5383-5388: stable argsort of the flat expert ids, its
    inverse, the source token row of each sorted pair and the sorted ids."""
    idx = np.asarray(idx).reshape(-1)
    order = np.argsort(idx, kind="stable")
    inv = np.argsort(order, kind="stable")
    src = (order // k_rep).astype(np.uint32)
    return order, inv, src, idx[order]


def tile_meta(idx_sorted: np.ndarray, E: int, rtile: int = 32) -> np.ndarray:
    """(expert, row_start, nrows) per tile of <= rtile sorted rows, experts
    ascending, tiles ascending within an expert (vq_switch.py:4590-4610;
    the reference loop in tests/test_routing_memo.py:51-62)."""
    idx_sorted = np.asarray(idx_sorted).astype(np.int64)
    counts = np.bincount(idx_sorted, minlength=E)
    metas = []
    start = 0
    for e in range(E):
        c = int(counts[e])
        for r0 in range(0, c, rtile):
            metas.append((e, start + r0, min(rtile, c - r0)))
        start += c
    return np.asarray(metas, np.int32).reshape(-1, 3)


# ------------------------------------------------------------- embeddings
def ple_unpack(rows_u8: np.ndarray, nsub: int, bits: int) -> np.ndarray:
    """PLE byte-stream rows [..., row_bytes] uint8 -> [..., nsub] codes:
    code j is the `bits`-wide field at bit j*bits of the row, LSB first, read
    through the 3-byte window at byte (j*bits)//8 with the row padded by two
    zero bytes (vq_switch.py:5449-5478)."""
    b = np.asarray(rows_u8, np.uint8).astype(np.uint32)
    pad = np.zeros(b.shape[:-1] + (2,), np.uint32)
    b = np.concatenate([b, pad], axis=-1)
    bit0 = np.arange(nsub, dtype=np.int64) * bits
    b0, sh = bit0 // 8, (bit0 % 8).astype(np.uint32)
    win = b[..., b0] | (b[..., b0 + 1] << np.uint32(8)) | (b[..., b0 + 2] << np.uint32(16))
    return (win >> sh) & np.uint32((1 << bits) - 1)


def f16_to_bf16(h: np.ndarray) -> np.ndarray:
    """fp16 values -> bfloat16 bit patterns (uint16), round to nearest even,
    NaN kept NaN: what .astype(bfloat16) does to an fp16 array
    (vq_dense.py:506, vq_switch.py:5495). fp16 -> fp32 is exact, so this is
    one rounding of the fp32 value to 8 significand bits."""
    u = np.asarray(h, np.float16).astype(np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


def bf16_values(h: np.ndarray) -> np.ndarray:
    """fp16 values -> the float32 values of their bfloat16 casts: the weight
    operand of the reference's GEMM when x is bf16 (`xf @ w.T.astype(xf.dtype)`,
    vq_dense.py:288, 294)."""
    return (f16_to_bf16(h).astype(np.uint32) << 16).view(np.float32)


def embed_rows(ids: np.ndarray, codes: np.ndarray, codebook: np.ndarray,
               scales: np.ndarray, group: int) -> np.ndarray:
    """Rows ids of a VQ table, decoded: fp16 [*ids.shape, IN]
    (vq_dense.py:491-506; vq_switch.py:5480-5495). codes are the unpacked
    [rows, NSUB] codes; ids must be valid rows."""
    ids = np.asarray(ids, np.int64)
    flat = ids.reshape(-1)
    w = dequant(np.asarray(codes)[flat], codebook, np.asarray(scales)[flat], group)
    return w.reshape(ids.shape + (w.shape[-1],))
