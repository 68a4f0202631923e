"""Regenerates the VQ tensors of the reference's writer-contract fixture.

The reference builds a tiny qwen3_5-shaped MoE artifact from numpy's seeded
PCG64 stream (tests/test_writer_contracts.py:160-176): E=2 experts, H=I=128,
group 64, L=3 layers x (gate_proj, up_proj, down_proj), codebook K (16 for
the "vq16" artifact the pack and sz-pack goldens are taken from), d=4.
Per (layer, projection), in this order, it draws
  scales   rr.random((E, out, in // 64)) + 0.5        -> fp16
  codes    rr.integers(0, K, (E, out, in // 4))       -> uint8 (K <= 256)
  codebook rr.standard_normal((K, 4)) * 0.05          -> fp16
with rr = np.random.default_rng(seed); layer 0 up_proj has sc[0, :5] = 0
(five dead rows for the skipzero writer). Each artifact's non-VQ skeleton
comes from a separate stream and does not perturb these draws.

The expected sha256[:16] of each tensor live in writer_hashes.json, copied
from the reference goldens by make_writer_hashes.py.
"""
from __future__ import annotations

import hashlib
import json
import pathlib

import numpy as np

E, H, I, G, L = 2, 128, 128, 64, 3
PROJS = ("gate_proj", "up_proj", "down_proj")
MOD = "model.language_model.layers.{li}.mlp.switch_mlp.{p}"
HASHES = pathlib.Path(__file__).resolve().parent / "writer_hashes.json"


def vq_tensors(K: int = 16, seed: int = 1):
    """{module: dict(codes, codebook, vq_scales)} in the fixture's draw order."""
    rr = np.random.default_rng(seed)
    out = {}
    for li in range(L):
        for p in PROJS:
            ins = I if p == "down_proj" else H
            outs = H if p == "down_proj" else I
            sc = (rr.random((E, outs, ins // G)) + .5).astype(np.float16)
            if li == 0 and p == "up_proj":
                sc[0, :5] = 0
            codes = rr.integers(0, K, (E, outs, ins // 4)).astype(
                np.uint8 if K <= 256 else np.uint16)
            cb = (rr.standard_normal((K, 4)) * .05).astype(np.float16)
            out[MOD.format(li=li, p=p)] = {"codes": codes, "codebook": cb,
                                           "vq_scales": sc}
    return out


def sha16(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()[:16]


def golden():
    return json.loads(HASHES.read_text())
