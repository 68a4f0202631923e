"""VQLab artifact loader: config.json + safetensors shards -> this package's
VQ modules on a ROCm device.

The reference attaches its VQ modules while the bundle's model.py builds the
model -- `vq_modules` (VQSwitchLinear, skipzero included) and `vq_ple`
(VQPLEEmbedding) in bundle/add_model_file.py:70-150, `vq_linear` (VQLinear)
and `vq_embed` (VQEmbedding) in runtime/dense_shim.py:53-83 -- with
zero-filled placeholders whose shapes a strict load then checks, and it
converts skipzero tensors on the way in (skipzero_weights,
vq_switch.py:4988-5013). Here the same config sections and tensor names
build the modules directly: each module's tensors are read from its shard,
checked against the shapes and dtypes the config implies (ValueError naming
the key otherwise, as a strict load would), moved to the device one module
at a time, and wrapped in VQSwitchLinear / VQLinear / VQEmbedding /
VQPLEEmbedding. Tensors that belong to no VQ module are listed, not loaded.

    art = load_artifact("/path/to/artifact", device="cuda")
    art.modules["model.language_model.layers.0.mlp.switch_mlp.gate_proj"]
    art.attach(model)          # install every module into a torch model tree
"""
from __future__ import annotations

import dataclasses
import json
import pathlib
import re

import numpy as np
import torch

from . import vq_pack
from .vq_dense import VQEmbedding, VQLinear
from .vq_switch import VQPLEEmbedding, VQSwitchLinear, skipzero_row_table

_DTYPES = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def read_config(path) -> dict:
    return json.loads((pathlib.Path(path) / "config.json").read_text())


def shard_map(path) -> dict:
    """tensor key -> shard file: model.safetensors.index.json's weight_map,
    else the keys of every *.safetensors file in the directory."""
    from safetensors import safe_open
    root = pathlib.Path(path)
    idx = root / "model.safetensors.index.json"
    if idx.exists():
        wm = json.loads(idx.read_text())["weight_map"]
        return {k: root / v for k, v in wm.items()}
    out = {}
    for f in sorted(root.glob("*.safetensors")):
        with safe_open(str(f), framework="pt") as sf:
            for k in sf.keys():
                out[k] = f
    return out


def _model_dtype(cfg) -> torch.dtype:
    """The artifact's activation dtype (dense_shim.py:40-44)."""
    name = (cfg.get("dtype") or cfg.get("torch_dtype")
            or cfg.get("text_config", {}).get("dtype") or "bfloat16")
    return _DTYPES[name]


def module_specs(cfg) -> list:
    """[(config path, kind, spec)] for every VQ module the config declares:
    kind 'switch' (vq_modules), 'linear' (vq_linear), 'embed' (vq_embed),
    'ple' (vq_ple keys, spec = geometry + that key's [rows, cols])."""
    out = [(p, "switch", m) for p, m in cfg.get("vq_modules", {}).items()]
    out += [(p, "linear", m) for p, m in cfg.get("vq_linear", {}).items()]
    out += [(p, "embed", m) for p, m in cfg.get("vq_embed", {}).items()]
    ple = cfg.get("vq_ple") or {}
    for key in ple.get("keys", []):
        rows, cols = ple["shapes"][key]
        out.append((key, "ple", dict(ple["geometry"], rows=int(rows), cols=int(cols))))
    return out


def _strip(p: str) -> str:
    """A module path without the layout prefixes the two module trees differ
    by (`language_model.`, a leading `model.`), so the mlx_lm and mlx_vlm
    spellings of one module compare equal (arch_resolve.py:186-240)."""
    p = re.sub(r"\.ngram_embedding\.shard_(\d+)$", r".ngram_embedding.shards.\1", p)
    p = p.replace("language_model.", "")
    while p.startswith("model."):
        p = p[len("model."):]
    return p


def _tensor_prefix(path: str, keys) -> str:
    """The weight-key prefix of the module at config path `path`: the path
    itself, else the unique module prefix that is the same module in the
    other layout's spelling."""
    if path + ".codebook" in keys:
        return path
    want = _strip(path)
    hits = sorted({k[: -len(".codebook")] for k in keys
                   if k.endswith(".codebook") and _strip(k[: -len(".codebook")]) == want})
    if len(hits) != 1:
        raise KeyError(f"no tensors for VQ module {path!r}" if not hits else
                       f"VQ module {path!r} matches several tensor prefixes: {hits}")
    return hits[0]


def _expect(key, t, shape, dtypes):
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{key}: expected shape {tuple(shape)}, the artifact holds "
                         f"{tuple(t.shape)}")
    if t.dtype not in dtypes:
        raise ValueError(f"{key}: expected dtype {dtypes[0]}, the artifact holds {t.dtype}")


def _code_layout(spec):
    """(columns, accepted dtypes, pack_bits) of a module's code rows."""
    nsub = int(spec["in"]) // int(spec["dim"])
    pb = int(spec.get("pack_bits", 0) or 0)
    if pb:
        return vq_pack.words_per_row(nsub, pb), (torch.uint32, torch.int32), pb
    if int(spec["k"]) <= 256:
        return nsub, (torch.uint8,), 0
    return nsub, (torch.uint16, torch.int16), 0


def _as_kernel_codes(t):
    # bit-identical signed views: the kernels read the words / halves as stored
    if t.dtype == torch.uint32:
        return t.view(torch.int32)
    if t.dtype == torch.uint16:
        return t.view(torch.int16)
    return t


class _Reader:
    """Reads single tensors from the shards, keeping each shard open."""

    def __init__(self, smap):
        self.smap = smap
        self._open = {}

    def __contains__(self, key):
        return key in self.smap

    def get(self, key):
        from safetensors import safe_open
        f = self.smap[key]
        if f not in self._open:
            self._open[f] = safe_open(str(f), framework="pt")
        return self._open[f].get_tensor(key)

    def close(self):
        self._open.clear()


# ------------------------------------------------------------- skipzero
# On-disk tensors of one skipzero module (docs/SKIPZERO.md in the reference):
# live rows of codes / scales, the [E, ceil(OUT/8)] live-row bit mask and the
# [E, OUT, W, NGRP] shape record.
SZ_SUFFIXES = (".sz_codes", ".sz_scales", ".sz_rowmask", ".sz_shape")


def skipzero_module(q, parts, E, OUT):
    """One module's skipzero tensors (`parts`: suffix -> tensor) -> (compact
    codes, compact scales, row table [E, OUT] int32) after checking the mask
    against (E, OUT), the shape record against the mask, and the compact
    row counts against the mask's live rows."""
    missing = [suf for suf in (".sz_codes", ".sz_scales", ".sz_rowmask") if suf not in parts]
    if missing:
        raise KeyError(f"{q}: skipzero tensors incomplete, missing {missing}")
    mask = parts[".sz_rowmask"]
    _expect(q + ".sz_rowmask", mask, (E, (OUT + 7) // 8), (torch.uint8,))
    if ".sz_shape" in parts:
        shp = [int(v) for v in torch.as_tensor(parts[".sz_shape"]).reshape(-1).tolist()]
        if shp[:2] != [E, OUT]:
            raise ValueError(f"{q}.sz_shape {shp} disagrees with (experts, out) = ({E}, {OUT})")
    table = skipzero_row_table(mask, E, OUT)
    n_live = int((table >= 0).sum())
    codes, sc = parts[".sz_codes"], parts[".sz_scales"]
    for suf, t in ((".sz_codes", codes), (".sz_scales", sc)):
        if t.ndim != 2 or t.shape[0] != n_live:
            raise ValueError(f"{q}{suf}: {tuple(t.shape)} rows, the mask has {n_live} live rows")
    return codes, sc, table


def _layout_match(modules, prefix):
    """The vq_skipzero entry of a tensor prefix: exact, else the one entry
    that names the same module in the other module-tree spelling."""
    if prefix in modules:
        return modules[prefix]
    want = _strip(prefix)
    hits = [v for k, v in modules.items() if _strip(k) == want]
    if len(hits) != 1:
        raise KeyError(f"skipzero tensors for {prefix!r} match {len(hits)} vq_skipzero entries")
    return hits[0]


# --------------------------------------------------- tensor-parallel split
# Leaves split on their output rows (each rank keeps its slice of every
# expert's rows) and on their input axis (rows stay whole), as the
# reference's skipzero_shard does (vq_switch.py:5025-5026).
SZ_ROW_SPLIT = ("gate_proj", "up_proj")
SZ_IN_SPLIT = ("down_proj",)


def skipzero_live(rowmask, E, OUT) -> np.ndarray:
    """Bit-packed uint8 [E, ceil(OUT/8)] live-row mask (little bit order) ->
    bool [E, OUT] (vq_switch.py:5029-5033); host side, the mask is small."""
    rm = rowmask.cpu().numpy() if isinstance(rowmask, torch.Tensor) else np.asarray(rowmask)
    rm = np.ascontiguousarray(rm, np.uint8).reshape(int(E), -1)
    return np.unpackbits(rm, axis=-1, bitorder="little")[:, : int(OUT)].astype(bool)


def _check_rank(rank, n):
    if not (isinstance(n, int) and n >= 1 and isinstance(rank, int) and 0 <= rank < n):
        raise ValueError(f"skipzero shard: bad rank/n {rank}/{n}")


def skipzero_shard_modules(modules, rank, n, rowmask):
    """Per-rank vq_skipzero entries for an n-way tensor split
    (vq_switch.py:5036-5075): gate_proj / up_proj get out = OUT / n and
    live_rows = the rank's live rows; down_proj entries come back unchanged
    once the input-axis cut is checked to fall on scale-group (and, packed,
    32-code block) boundaries, which needs the entry's vq_modules geometry
    (in, dim, group, pack_bits). `rowmask(key)` returns a module's
    sz_rowmask. ValueError for OUT % n != 0, an unaligned input cut or a
    leaf with no split rule; KeyError for a down_proj entry without its
    geometry."""
    _check_rank(rank, n)
    out = {}
    for key, m in modules.items():
        leaf = key.rsplit(".", 1)[-1]
        E, OUT = int(m["experts"]), int(m["out"])
        if leaf in SZ_ROW_SPLIT:
            if OUT % n:
                raise ValueError(f"skipzero shard: {key} OUT={OUT} does not divide into {n} ranks")
            lo, hi = rank * OUT // n, (rank + 1) * OUT // n
            live = skipzero_live(rowmask(key), E, OUT)[:, lo:hi]
            out[key] = dict(m, out=OUT // n, live_rows=int(live.sum()))
        elif leaf in SZ_IN_SPLIT:
            try:
                IN, D, G = int(m["in"]), int(m["dim"]), int(m.get("group", 64))
            except KeyError:
                raise KeyError(f"skipzero shard: {key} needs its vq_modules geometry "
                               f"(in, dim, group, pack_bits) to check the input-axis cut") from None
            pb = int(m.get("pack_bits") or 0)
            cut = IN // n
            ok = IN % n == 0 and cut % G == 0 and cut % D == 0 and (not pb or (cut // D) % 32 == 0)
            if not ok:
                raise ValueError(f"skipzero shard: {key} IN={IN} split {n} ways is not aligned to "
                                 f"group {G}" + (f" and 32-code blocks (d={D}, {pb}-bit words)"
                                                 if pb else ""))
            out[key] = dict(m)
        else:
            raise ValueError(f"skipzero shard: no tensor split rule for {key} (leaf {leaf!r})")
    return out


def _shard_rows(parts, E, OUT, rank, n):
    """One row-split module's on-disk skipzero tensors (suffix -> tensor) ->
    the rank's: compact rows of its output slice (taken through the mask, in
    the compact order), the sliced mask and the shape record."""
    lo, hi = rank * OUT // n, (rank + 1) * OUT // n
    live = skipzero_live(parts[".sz_rowmask"], E, OUT)
    pos = (np.cumsum(live.reshape(-1)) - 1).reshape(E, OUT)
    keep = torch.from_numpy(pos[:, lo:hi][live[:, lo:hi]].astype(np.int64))
    out = dict(parts)
    for suf in (".sz_codes", ".sz_scales"):
        t = parts[suf]
        out[suf] = t.index_select(0, keep.to(t.device))
    mask = parts[".sz_rowmask"]
    rm = torch.from_numpy(np.packbits(live[:, lo:hi], axis=-1, bitorder="little"))
    out[".sz_rowmask"] = rm.to(mask.device) if isinstance(mask, torch.Tensor) else rm
    if ".sz_shape" in parts:
        shp = torch.as_tensor(parts[".sz_shape"]).to(torch.int32).clone()
        shp.view(-1)[1] = hi - lo
        out[".sz_shape"] = shp
    return out


def skipzero_shard(weights, modules, rank, n):
    """Rank `rank` of an n-way tensor split of on-disk skipzero tensors,
    before convert_skipzero (the reference's skipzero_shard,
    vq_switch.py:5112-5147): gate_proj / up_proj keep the rank's output rows
    of every expert (sz_codes / sz_scales rows taken through the mask,
    sz_rowmask and sz_shape sliced); down_proj is left as it is (its input
    axis is cut like any expanded module's). Returns (weights of the same
    kind as given, per-rank modules as skipzero_shard_modules)."""
    _check_rank(rank, n)
    pairs = list(weights.items()) if isinstance(weights, dict) else list(weights)
    d = dict(pairs)
    pre = [k[: -len(".sz_rowmask")] for k in d if k.endswith(".sz_rowmask")]
    keyed = {}
    for q in pre:
        key = next((k for k in modules if k == q), None)
        if key is None:
            want = _strip(q)
            hits = [k for k in modules if _strip(k) == want]
            if len(hits) != 1:
                raise KeyError(f"skipzero tensors for {q!r} match {len(hits)} vq_skipzero entries")
            key = hits[0]
        keyed[q] = key
    by_key = {key: q for q, key in keyed.items()}
    smods = skipzero_shard_modules({key: modules[key] for key in by_key}, rank, n,
                                   lambda key: d[by_key[key] + ".sz_rowmask"])
    for q, key in keyed.items():
        if key.rsplit(".", 1)[-1] not in SZ_ROW_SPLIT:
            continue
        m = modules[key]
        parts = {suf: d[q + suf] for suf in SZ_SUFFIXES if q + suf in d}
        for suf, t in _shard_rows(parts, int(m["experts"]), int(m["out"]), rank, n).items():
            d[q + suf] = t
    mods = dict(modules)
    mods.update(smods)
    out = [(k, d[k]) for k, _ in pairs]
    return (dict(out) if isinstance(weights, dict) else out), mods


def convert_skipzero(weights, modules, shard=None):
    """On-disk skipzero tensors -> what VQSwitchLinear(row_table=...) loads
    (the reference's skipzero_weights, vq_switch.py:4988-5013): each module's
    {p}.sz_* tensors become {p}.codes / {p}.vq_scales (compact rows) and
    {p}.row_table; every other tensor passes through unchanged, and weights
    without skipzero tensors come back as given. `weights` is a dict or a
    list of (key, tensor) pairs (the same kind is returned); `modules` maps
    module prefixes to their vq_skipzero entries (experts, out). `shard` =
    (rank, n) applies skipzero_shard first, with the unsplit modules."""
    if shard is not None and any(k.endswith(".sz_rowmask") for k in
                                 (weights if isinstance(weights, dict) else dict(weights))):
        weights, modules = skipzero_shard(weights, modules, *shard)
    pairs = list(weights.items()) if isinstance(weights, dict) else list(weights)
    groups, kept = {}, []
    for key, val in pairs:
        suf = next((s for s in SZ_SUFFIXES if key.endswith(s)), None)
        if suf is None:
            kept.append((key, val))
        else:
            groups.setdefault(key[: -len(suf)], {})[suf] = val
    if not groups:
        return weights
    for prefix, parts in groups.items():
        entry = _layout_match(modules, prefix)
        codes, sc, table = skipzero_module(prefix, parts, int(entry["experts"]),
                                           int(entry["out"]))
        dev = codes.device if isinstance(codes, torch.Tensor) else None
        kept += [(prefix + ".codes", codes), (prefix + ".vq_scales", sc),
                 (prefix + ".row_table", table.to(dev) if dev is not None else table)]
    return dict(kept) if isinstance(weights, dict) else kept


def _build(path, kind, spec, rd, sz_mods, device, out_dtype, shard=None):
    q = _tensor_prefix(path, rd.smap)
    g = int(spec["group"])
    k, d = int(spec["k"]), int(spec["dim"])
    cb = rd.get(q + ".codebook")
    _expect(q + ".codebook", cb, (k, d), (torch.float16,))
    cb = cb.to(device)
    if kind == "ple":
        rows, cols = spec["rows"], spec["cols"]
        rb = spec.get("row_bytes")
        codes = rd.get(q + ".codes")
        if rb:
            _expect(q + ".codes", codes, (rows, int(rb)), (torch.uint8,))
        else:
            _expect(q + ".codes", codes, (rows, cols // d), (torch.uint16, torch.int16))
        sc = rd.get(q + ".vq_scales")
        _expect(q + ".vq_scales", sc, (rows, cols // g), (torch.float16,))
        return VQPLEEmbedding(_as_kernel_codes(codes).to(device), cb, sc.to(device),
                              group_size=g, packed_nsub=(cols // d) if rb else 0)

    IN = int(spec["in"])
    cols, cdt, pb = _code_layout(spec)
    infeat = IN if pb else None
    if kind == "switch" and q + ".sz_rowmask" in rd:
        # skipzero: compact live rows + [E, OUT] row table (vq_switch.py:4988-5013)
        szm = sz_mods.get(path, {})
        E = int(szm.get("experts", spec["experts"]))
        OUT = int(szm.get("out", spec["out"]))
        parts = {suf: rd.get(q + suf) for suf in SZ_SUFFIXES if q + suf in rd}
        if shard is not None:
            # the rank's output rows (gate / up); down_proj stays whole once
            # its input cut is checked (vq_switch.py:5112-5147)
            entry = dict(spec, experts=E, out=OUT)
            skipzero_shard_modules({path: entry}, *shard, lambda _: parts[".sz_rowmask"])
            if path.rsplit(".", 1)[-1] in SZ_ROW_SPLIT:
                parts = _shard_rows(parts, E, OUT, *shard)
                OUT //= shard[1]
        codes, sc, table = skipzero_module(q, parts, E, OUT)
        _expect(q + ".sz_codes", codes, (codes.shape[0], cols), cdt)
        _expect(q + ".sz_scales", sc, (codes.shape[0], IN // g), (torch.float16,))
        return VQSwitchLinear(_as_kernel_codes(codes).to(device), cb, sc.to(device),
                              group_size=g, pack_bits=pb, in_features=infeat,
                              row_table=table.to(device))
    codes, sc = rd.get(q + ".codes"), rd.get(q + ".vq_scales")
    if kind == "switch":
        E, OUT = int(spec["experts"]), int(spec["out"])
        _expect(q + ".codes", codes, (E, OUT, cols), cdt)
        _expect(q + ".vq_scales", sc, (E, OUT, IN // g), (torch.float16,))
        return VQSwitchLinear(_as_kernel_codes(codes).to(device), cb, sc.to(device),
                              group_size=g, pack_bits=pb, in_features=infeat)
    rows = int(spec["rows"] if kind == "embed" else spec["out"])
    _expect(q + ".codes", codes, (rows, cols), cdt)
    _expect(q + ".vq_scales", sc, (rows, IN // g), (torch.float16,))
    if kind == "linear":
        return VQLinear(_as_kernel_codes(codes).to(device), cb, sc.to(device), group_size=g,
                        pack_bits=pb, in_features=infeat)
    return VQEmbedding(_as_kernel_codes(codes).to(device), cb, sc.to(device), group_size=g,
                       pack_bits=pb, in_features=infeat, out_dtype=out_dtype)


def _candidates(path: str) -> list:
    """Spellings of a module path in the two module trees (arch_resolve.py:186-240):
    as written, with a leading `language_model.` added or removed, and -- for
    weight-key spellings such as `model.language_model.layers.N` -- with the
    inner `language_model.` level dropped."""
    c = [path]
    c.append(path[len("language_model."):] if path.startswith("language_model.")
             else "language_model." + path)
    flat = path.replace("language_model.", "")
    if flat not in c:
        c.append(flat)
    for p in list(c):
        m = re.search(r"\.ngram_embedding\.shard_(\d+)$", p)
        if m:
            c.append(p[: m.start()] + f".ngram_embedding.shards.{m.group(1)}")
    return c


def attach(root: torch.nn.Module, path: str, module: torch.nn.Module) -> None:
    """Install `module` at `path` of a torch module tree, trying the path as
    written, then with `language_model.` added or removed, then the PLE
    `shard_N` -> `shards.N` spelling; raises naming every candidate when none
    resolves (a module that silently fails to attach leaves a random dense
    layer in the model)."""
    cands = _candidates(path)
    for cand in cands:
        obj, parts, ok = root, cand.split("."), True
        for c in parts[:-1]:
            try:
                obj = obj[int(c)] if c.isdigit() else getattr(obj, c)
            except (AttributeError, IndexError, KeyError, TypeError):
                ok = False
                break
        leaf = parts[-1]
        if not ok:
            continue
        if leaf.isdigit() and isinstance(obj, (list, torch.nn.ModuleList)) and int(leaf) < len(obj):
            obj[int(leaf)] = module
            return
        if hasattr(obj, leaf):
            setattr(obj, leaf, module)
            return
    raise AttributeError(f"VQ module {path!r} does not resolve on {type(root).__name__}; "
                         f"tried {cands}")


@dataclasses.dataclass
class Artifact:
    path: pathlib.Path
    config: dict
    modules: dict            # config path -> VQ module (device tensors)
    other_keys: list         # tensors that belong to no VQ module (not loaded)

    def attach(self, model: torch.nn.Module) -> None:
        for p, m in self.modules.items():
            attach(model, p, m)


def load_artifact(path, device="cuda", only=None, shard=None) -> Artifact:
    """Builds every VQ module `path`'s config.json declares (or those whose
    config path is in `only`), reading each module's tensors from its shard
    and moving them to `device` one module at a time. `shard` = (rank, n)
    (default: the config's vq_skipzero.shard {"rank", "n"}, as the
    reference's loader reads it) builds rank `rank` of an n-way tensor split
    of the skipzero modules: gate_proj / up_proj with the rank's OUT / n
    output rows of every expert; down_proj whole, after checking that its
    input axis cuts on scale-group and code-block boundaries."""
    root = pathlib.Path(path)
    cfg = read_config(root)
    rd = _Reader(shard_map(root))
    szc = cfg.get("vq_skipzero") or {}
    sz_mods = szc.get("modules") or {}
    if shard is None and szc.get("shard"):
        shard = (int(szc["shard"]["rank"]), int(szc["shard"]["n"]))
    out_dtype = _model_dtype(cfg)
    mods, used = {}, set()
    try:
        for p, kind, spec in module_specs(cfg):
            if only is not None and p not in only:
                continue
            mods[p] = _build(p, kind, spec, rd, sz_mods, device, out_dtype, shard)
            q = _tensor_prefix(p, rd.smap)
            used.update(k for k in rd.smap if k.startswith(q + "."))
    finally:
        rd.close()
    other = sorted(k for k in rd.smap if k not in used)
    return Artifact(root, cfg, mods, other)
