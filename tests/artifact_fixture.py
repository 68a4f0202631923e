"""Writes small VQLab-format artifacts for the loader tests.

The MoE part is the reference's writer-contract fixture (E=2, H=I=128, d4,
K16, three layers; tests/golden/writer_fixture.py regenerates its seeded
tensors) in the two on-disk forms the reference's goldens pin:
  form "pack"     packed uint32 codes, pack_bits 4 (writers/pack.json)
  form "sz_pack"  unpacked uint8 codes, layer 0 up_proj stored as skipzero
                  sz_codes / sz_scales / sz_rowmask / sz_shape
                  (writers/sz_pack.json)
Every VQ tensor written is checked against the golden sha256 prefix, so the
artifact is byte-for-byte what the reference's writers produce. On top come
a dense VQ linear, a VQ embedding and two PLE shards (config sections
vq_linear / vq_embed / vq_ple, add_model_file.py:130-150 and
dense_shim.py:53-83) with seeded tensors of this build's own, and one non-VQ
tensor. Tensors are spread over two shards with an index file."""
from __future__ import annotations

import json
import pathlib

import numpy as np

from golden import writer_fixture as wf
from oracle import vq_oracle as vo

PRE = "model.language_model."


def _extras(rng):
    """Dense linear, embedding and PLE tables: {prefix: tensors}, config."""
    t, cfg = {}, {"vq_linear": {}, "vq_embed": {}, "vq_ple": None}
    # dense linear, d8 K4096 packed 12-bit, 96 x 256
    codes = rng.integers(0, 4096, (96, 32)).astype(np.uint16)
    p = PRE + "layers.0.self_attn.o_proj"
    t[p] = {"codes": vo.pack(codes, 12), "codebook": (rng.standard_normal((4096, 8)) * .05)
            .astype(np.float16), "vq_scales": rng.uniform(.5, 1.5, (96, 4)).astype(np.float16),
            "_codes": codes}
    cfg["vq_linear"][p] = {"out": 96, "in": 256, "k": 4096, "dim": 8, "group": 64,
                           "pack_bits": 12}
    # embedding, d4 K256 uint8, 300 rows x 128
    codes = rng.integers(0, 256, (300, 32)).astype(np.uint8)
    p = PRE + "embed_tokens"
    t[p] = {"codes": codes, "codebook": (rng.standard_normal((256, 4)) * .05).astype(np.float16),
            "vq_scales": rng.uniform(.5, 1.5, (300, 2)).astype(np.float16), "_codes": codes}
    cfg["vq_embed"][p] = {"rows": 300, "in": 128, "k": 256, "dim": 4, "group": 64}
    # two PLE shards, K2048 d4, 40 codes of 11 bits = 55 bytes per row
    keys, shapes = [], {}
    for i in range(2):
        codes = rng.integers(0, 2048, (64, 40)).astype(np.uint32)
        bitmat = ((codes[..., None] >> np.arange(11, dtype=np.uint32)) & 1).astype(np.uint8)
        rows = np.packbits(bitmat.reshape(64, 440), axis=-1, bitorder="little")
        p = PRE + f"ngram_embedding.shard_{i}"
        t[p] = {"codes": rows, "codebook": (rng.standard_normal((2048, 4)) * .05)
                .astype(np.float16), "vq_scales": rng.uniform(.5, 1.5, (64, 5))
                .astype(np.float16), "_codes": codes}
        keys.append(p)
        shapes[p] = [64, 160]
    cfg["vq_ple"] = {"geometry": {"k": 2048, "dim": 4, "group": 32, "row_bytes": 55},
                     "keys": keys, "shapes": shapes}
    return t, cfg


def write(root, form="sz_pack"):
    """Writes the artifact under `root`; returns (config, {prefix: arrays})
    where arrays hold the unpacked codes ('_codes') and the stored tensors."""
    from safetensors.numpy import save_file
    root = pathlib.Path(root)
    root.mkdir(parents=True, exist_ok=True)
    gold = wf.golden()[form]
    mods = {}
    tensors = {}
    for m, t in wf.vq_tensors().items():
        mods[m] = dict(t, _codes=t["codes"])
        if form == "pack":
            tensors[m + ".codes"] = vo.pack(t["codes"], 4)
            tensors[m + ".codebook"] = t["codebook"]
            tensors[m + ".vq_scales"] = t["vq_scales"]
        elif m in (gold["vq_skipzero"] or {}):
            sz = vo.skipzero_compact(t["codes"], t["vq_scales"])
            for k, v in sz.items():
                tensors[m + "." + k] = v
            tensors[m + ".codebook"] = t["codebook"]
        else:
            tensors[m + ".codes"] = t["codes"]
            tensors[m + ".codebook"] = t["codebook"]
            tensors[m + ".vq_scales"] = t["vq_scales"]
    for k, v in tensors.items():
        g = gold["tensors"][k]
        assert list(v.shape) == g["shape"] and wf.sha16(v) == g["sha"], k
    rng = np.random.default_rng(2024)
    extra, ecfg = _extras(rng)
    for p, t in extra.items():
        mods[p] = t
        for k in ("codes", "codebook", "vq_scales"):
            tensors[p + "." + k] = t[k]
    tensors[PRE + "layers.0.input_layernorm.weight"] = np.ones(128, np.float16)
    cfg = {"model_type": "qwen3_5_moe", "dtype": "bfloat16",
           "vq_modules": {k: dict(v) for k, v in gold["vq_modules"].items()}, **ecfg}
    if gold["vq_skipzero"]:
        cfg["vq_skipzero"] = {"format": "vq-skipzero", "version": 1,
                              "modules": gold["vq_skipzero"]}
    keys = sorted(tensors)
    halves = (keys[: len(keys) // 2], keys[len(keys) // 2:])
    wm = {}
    for i, part in enumerate(halves):
        name = f"model-{i + 1:05d}-of-00002.safetensors"
        save_file({k: np.ascontiguousarray(tensors[k]) for k in part}, str(root / name))
        wm.update({k: name for k in part})
    (root / "model.safetensors.index.json").write_text(json.dumps({"weight_map": wm}))
    (root / "config.json").write_text(json.dumps(cfg, indent=1))
    return cfg, mods
