"""The artifact loader (config.json + safetensors -> VQ modules) on the CPU:
module kinds, shapes, skipzero conversion, layout-tolerant lookups and the
strict-load refusals. The GPU test at the end runs every loaded module
against the oracle."""
import json

import numpy as np
import pytest

import artifact_fixture as af
from oracle import vq_oracle as vo

torch = pytest.importorskip("torch")


def _np(t):
    t = t.cpu().contiguous()
    if t.dtype in (torch.int32, torch.uint32):
        return t.view(torch.int32).numpy().view(np.uint32)
    if t.dtype in (torch.int16, torch.uint16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


@pytest.mark.parametrize("form", ["sz_pack", "pack"])
def test_load_builds_every_module(tmp_path, form):
    from vqlab_amd import artifact
    from vqlab_amd.vq_dense import VQEmbedding, VQLinear
    from vqlab_amd.vq_switch import VQPLEEmbedding, VQSwitchLinear
    cfg, mods = af.write(tmp_path, form)
    art = artifact.load_artifact(tmp_path, device="cpu")
    assert set(art.modules) == {p for p, _, _ in artifact.module_specs(cfg)}
    assert art.other_keys == [af.PRE + "layers.0.input_layernorm.weight"]
    sz = set((cfg.get("vq_skipzero") or {}).get("modules", {}))
    for p, m in art.modules.items():
        src = mods[p]
        if p in cfg["vq_modules"]:
            assert isinstance(m, VQSwitchLinear)
            assert m.num_experts == 2 and m.output_dims == 128 and m.input_dims == 128
            assert m.skipzero == (p in sz)
            stored = _np(m.codes)
            if p in sz:
                c = vo.skipzero_compact(src["codes"], src["vq_scales"])
                assert np.array_equal(stored, c["sz_codes"])
                assert np.array_equal(m.row_table.numpy(),
                                      vo.skipzero_row_table(c["sz_rowmask"], 2, 128))
                assert (m.row_table < 0).sum() == 5
            elif form == "pack":
                assert m.pack_bits == 4
                assert np.array_equal(vo.unpack(stored, 32, 4), src["codes"])
            else:
                assert np.array_equal(stored, src["codes"])
        elif p in cfg["vq_linear"]:
            assert isinstance(m, VQLinear) and m.input_dims == 256 and m.output_dims == 96
            assert np.array_equal(vo.unpack(_np(m.codes), 32, 12), src["_codes"])
        elif p in cfg["vq_embed"]:
            assert isinstance(m, VQEmbedding) and m.num_embeddings == 300 and m.dims == 128
            assert m.out_dtype == torch.bfloat16
        else:
            assert isinstance(m, VQPLEEmbedding) and m._pn == 40 and m._bits == 11
            assert np.array_equal(vo.ple_unpack(_np(m.codes), 40, 11), src["_codes"])


def test_shape_and_dtype_mismatch_refused(tmp_path):
    from safetensors.numpy import save_file
    from vqlab_amd import artifact
    af.write(tmp_path, "sz_pack")
    cfg = json.loads((tmp_path / "config.json").read_text())
    p = af.PRE + "layers.1.mlp.switch_mlp.gate_proj"
    cfg["vq_modules"][p]["out"] = 64
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    with pytest.raises(ValueError, match="gate_proj.codes: expected shape"):
        artifact.load_artifact(tmp_path, device="cpu", only={p})
    cfg["vq_modules"][p]["out"] = 128
    cfg["vq_modules"][p]["k"] = 4096          # uint16 codes expected for K > 256
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    with pytest.raises(ValueError, match="codebook: expected shape"):
        artifact.load_artifact(tmp_path, device="cpu", only={p})
    # a module the shards do not hold
    cfg["vq_modules"][p]["k"] = 16
    cfg["vq_modules"][af.PRE + "layers.7.mlp.switch_mlp.gate_proj"] = cfg["vq_modules"][p]
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    with pytest.raises(KeyError, match="no tensors"):
        artifact.load_artifact(tmp_path, device="cpu")
    assert save_file  # the loader reads what safetensors writes


def test_other_layout_spelling_resolves(tmp_path):
    from vqlab_amd import artifact
    af.write(tmp_path, "sz_pack")
    cfg = json.loads((tmp_path / "config.json").read_text())
    # config written against the mlx_lm tree (model.layers.N), tensors in the
    # mlx_vlm spelling (model.language_model.layers.N)
    cfg["vq_modules"] = {k.replace("language_model.", ""): v for k, v in cfg["vq_modules"].items()}
    cfg["vq_skipzero"]["modules"] = {k.replace("language_model.", ""): v
                                     for k, v in cfg["vq_skipzero"]["modules"].items()}
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    art = artifact.load_artifact(tmp_path, device="cpu")
    m = art.modules["model.layers.0.mlp.switch_mlp.up_proj"]
    assert m.skipzero and (m.row_table < 0).sum() == 5


def test_attach_into_module_tree(tmp_path):
    from vqlab_amd import artifact
    af.write(tmp_path, "sz_pack")
    art = artifact.load_artifact(tmp_path, device="cpu")
    nn = torch.nn

    class Mlp(nn.Module):
        def __init__(self):
            super().__init__()
            self.switch_mlp = nn.Module()
            for n in ("gate_proj", "up_proj", "down_proj"):
                setattr(self.switch_mlp, n, nn.Linear(1, 1))

    class Layer(nn.Module):
        def __init__(self):
            super().__init__()
            self.mlp = Mlp()
            self.self_attn = nn.Module()
            self.self_attn.o_proj = nn.Linear(1, 1)

    # the mlx_lm tree: model.layers.N (no language_model level), PLE shards
    # kept in a list (shards.N)
    root = nn.Module()
    root.model = nn.Module()
    root.model.layers = nn.ModuleList([Layer() for _ in range(3)])
    root.model.embed_tokens = nn.Embedding(2, 2)
    root.model.ngram_embedding = nn.Module()
    root.model.ngram_embedding.shards = nn.ModuleList([nn.Embedding(2, 2) for _ in range(2)])
    art.attach(root)
    assert root.model.layers[2].mlp.switch_mlp.down_proj is \
        art.modules[af.PRE + "layers.2.mlp.switch_mlp.down_proj"]
    assert root.model.ngram_embedding.shards[1] is art.modules[af.PRE + "ngram_embedding.shard_1"]
    assert root.model.embed_tokens is art.modules[af.PRE + "embed_tokens"]
    with pytest.raises(AttributeError, match="does not resolve"):
        artifact.attach(root, "model.layers.9.mlp.switch_mlp.gate_proj", nn.Linear(1, 1))


@pytest.mark.gpu
@pytest.mark.parametrize("form", ["sz_pack", "pack"])
def test_loaded_modules_match_oracle_on_gpu(tmp_path, form):
    from vq_cases import assert_close
    from vqlab_amd import artifact
    cfg, mods = af.write(tmp_path, form)
    art = artifact.load_artifact(tmp_path, device="cuda")
    rng = np.random.default_rng(11)
    for p, m in art.modules.items():
        print(f"artifact module {p}", flush=True)
        src = mods[p]
        if p in cfg["vq_modules"]:
            x = rng.standard_normal((3, 128)).astype(np.float32)
            idx = rng.integers(0, 2, (3, 2))
            y = m(torch.from_numpy(x).cuda()[:, None, None, :],
                  torch.from_numpy(idx).cuda(), out_dtype=torch.float32)
            w = vo.dequant(src["_codes"], src["codebook"], src["vq_scales"], 64)
            ref = np.einsum("ti,tkoi->tko", x.astype(np.float64), w[idx].astype(np.float64))
            assert_close(y.reshape(3, 2, 128).cpu().numpy(), ref, what=p)
        elif p in cfg["vq_linear"]:
            x = rng.standard_normal((2, 256)).astype(np.float32)
            y = m(torch.from_numpy(x).cuda())
            w = vo.dequant(src["_codes"], src["codebook"], src["vq_scales"], 64)
            assert_close(y.cpu().numpy(), vo.decode_matmul(x, w), what=p)
        else:
            G = 32 if "ngram" in p else 64
            ids = rng.integers(0, src["_codes"].shape[0], (4,))
            got = m(torch.from_numpy(ids).cuda())
            ref = vo.f16_to_bf16(vo.embed_rows(ids, src["_codes"], src["codebook"],
                                               src["vq_scales"], G))
            assert np.array_equal(got.cpu().view(torch.int16).numpy().view(np.uint16), ref), p


def test_skipzero_weights_converts_state_dicts(tmp_path):
    """vq_switch.skipzero_weights (vq_switch.py:4988-5013) over the reference
    golden's skipzero tensors: {p}.sz_* become compact codes / scales + the
    row table, other tensors pass through, a list stays a list, the module
    entry is found under the other module-tree spelling, weights without sz_
    tensors come back unchanged, and incomplete or inconsistent tensors are
    refused."""
    from safetensors.numpy import load_file
    from vqlab_amd.vq_switch import skipzero_weights
    cfg, mods = af.write(tmp_path, "sz_pack")
    flat = {}
    for f in sorted(tmp_path.glob("*.safetensors")):
        flat.update({k: torch.from_numpy(v) for k, v in load_file(str(f)).items()})
    szmods = cfg["vq_skipzero"]["modules"]
    out = skipzero_weights(flat, szmods)
    assert isinstance(out, dict) and not any(".sz_" in k for k in out)
    for p, spec in szmods.items():
        c = vo.skipzero_compact(mods[p]["codes"], mods[p]["vq_scales"])
        assert np.array_equal(_np(out[p + ".codes"]), c["sz_codes"])
        assert np.array_equal(_np(out[p + ".vq_scales"]), c["sz_scales"])
        assert np.array_equal(out[p + ".row_table"].numpy(),
                              vo.skipzero_row_table(c["sz_rowmask"], spec["experts"], spec["out"]))
    passthru = [k for k in flat if ".sz_" not in k]
    assert all(out[k] is flat[k] for k in passthru)
    # list in, list out; module entries spelled in the other layout
    other = {k.replace("model.language_model.", "language_model.model."): v
             for k, v in szmods.items()}
    lst = skipzero_weights(list(flat.items()), other)
    assert isinstance(lst, list) and dict(lst).keys() == out.keys()
    # nothing to convert: the same object back
    plain = {k: flat[k] for k in passthru}
    assert skipzero_weights(plain, szmods) is plain
    # a missing mask, and a compact row count the mask disagrees with
    p = next(iter(szmods))
    broken = {k: v for k, v in flat.items() if k != p + ".sz_rowmask"}
    with pytest.raises(KeyError, match="missing"):
        skipzero_weights(broken, szmods)
    bad = dict(flat)
    bad[p + ".sz_codes"] = flat[p + ".sz_codes"][1:]
    with pytest.raises(ValueError, match="live rows"):
        skipzero_weights(bad, szmods)


# ------------------------------------------------- tensor-parallel split
def _sz_ondisk(rng, E, OUT, W, NG, dead):
    """Expanded codes / scales with many dead rows (one expert all dead, one
    all live) and their on-disk skipzero tensors (torch, CPU)."""
    codes = rng.integers(0, 2**31, (E, OUT, W), dtype=np.int64).astype(np.uint32)
    sc = (rng.standard_normal((E, OUT, NG)) * 0.1 + 1).astype(np.float16)
    live = rng.random((E, OUT)) >= dead
    live[1, :] = False
    live[2, :] = True
    codes[~live] = 0
    sc[~live] = 0
    sz = vo.skipzero_compact(codes, sc)
    t = {".sz_codes": torch.from_numpy(sz["sz_codes"].view(np.int32)),
         ".sz_scales": torch.from_numpy(sz["sz_scales"]),
         ".sz_rowmask": torch.from_numpy(sz["sz_rowmask"]),
         ".sz_shape": torch.from_numpy(sz["sz_shape"])}
    return codes, sc, live, t


@pytest.mark.parametrize("OUT,n", [(96, 2), (96, 4), (102, 2), (64, 1), (128, 8)])
@pytest.mark.parametrize("leaf", ["gate_proj", "up_proj"])
def test_skipzero_shard_rows_concat_equal_unsplit(OUT, n, leaf):
    """skipzero_shard (vq_switch.py:5112-5147) on gate / up: each rank keeps
    its output slice of every expert's rows, taken through the mask; the
    ranks' converted modules, expanded and concatenated over OUT, are
    byte-equal to the unsplit module, and their live rows add up (the
    reference's test_sz_shard row-split check, on the tensors)."""
    from vqlab_amd.vq_switch import skipzero_shard, skipzero_weights
    rng = np.random.default_rng(OUT * 10 + n)
    E, W, NG = 8, 24, 8
    codes, sc, live, t = _sz_ondisk(rng, E, OUT, W, NG, 0.7)
    p = f"model.layers.3.mlp.switch_mlp.{leaf}"
    w = {p + k: v for k, v in t.items()}
    w["model.layers.3.mlp.other"] = torch.ones(3)
    mods = {p: {"experts": E, "out": OUT, "live_rows": int(live.sum())}}
    gc, gs, total = [], [], 0
    for rank in range(n):
        wr, mr = skipzero_shard(dict(w), mods, rank, n)
        assert mr[p]["out"] == OUT // n and mr[p]["experts"] == E
        assert wr[p + ".sz_codes"].shape[0] == mr[p]["live_rows"]
        assert wr[p + ".sz_shape"].tolist()[:2] == [E, OUT // n]
        assert wr["model.layers.3.mlp.other"] is w["model.layers.3.mlp.other"]
        total += mr[p]["live_rows"]
        out = skipzero_weights(wr, mr)
        rt = out[p + ".row_table"].numpy()
        assert rt.shape == (E, OUT // n)
        c = _np(out[p + ".codes"])
        gc.append(np.where(rt[..., None] >= 0, c[np.maximum(rt, 0)], 0))
        gs.append(np.where(rt[..., None] >= 0, _np(out[p + ".vq_scales"])[np.maximum(rt, 0)], 0))
    assert total == int(live.sum())
    assert np.array_equal(np.concatenate(gc, axis=1), codes)
    assert np.array_equal(np.concatenate(gs, axis=1).view(np.uint16), sc.view(np.uint16))
    # skipzero_weights(shard=) is skipzero_shard then the conversion
    one = skipzero_weights(list(w.items()), mods, shard=(n - 1, n))
    assert isinstance(one, list)
    two = skipzero_weights(*skipzero_shard(dict(w), mods, n - 1, n))
    assert all(torch.equal(v, two[k]) for k, v in one)


def test_skipzero_shard_down_untouched_and_refusals():
    """down_proj splits on its input axis: its skipzero tensors and entry
    come back as they were once the cut is checked against the scale groups
    and 32-code blocks; the refusals of skipzero_shard_modules
    (vq_switch.py:5036-5075): OUT % n, an unaligned input cut, a down entry
    without its geometry, a leaf with no split rule, a bad rank."""
    from vqlab_amd.vq_switch import skipzero_shard
    rng = np.random.default_rng(5)
    E, IN = 4, 512
    _, _, live, t = _sz_ondisk(rng, E, 96, 16, 8, 0.5)
    geo = {"experts": E, "out": 96, "live_rows": int(live.sum()), "in": IN, "dim": 4,
           "group": 64, "pack_bits": 12, "k": 4096}
    dp = "model.layers.0.mlp.switch_mlp.down_proj"
    wd = {dp + k: v for k, v in t.items()}
    wr, mr = skipzero_shard(dict(wd), {dp: geo}, 1, 4)    # 128 inputs = 32 codes per rank
    assert mr[dp] == geo and all(wr[k] is wd[k] for k in wd)
    with pytest.raises(ValueError, match="not aligned"):
        skipzero_shard(dict(wd), {dp: geo}, 0, 8)          # 16 codes per rank
    with pytest.raises(ValueError, match="not aligned"):
        skipzero_shard(dict(wd), {dp: geo}, 0, 3)
    skipzero_shard(dict(wd), {dp: dict(geo, pack_bits=0)}, 0, 8)   # unpacked: groups only
    with pytest.raises(KeyError, match="geometry"):
        skipzero_shard(dict(wd), {dp: {"experts": E, "out": 96}}, 0, 2)
    g = "model.layers.0.mlp.switch_mlp.gate_proj"
    with pytest.raises(ValueError, match="does not divide"):
        skipzero_shard({g + k: v for k, v in t.items()}, {g: geo}, 0, 5)
    o = "model.layers.0.mlp.switch_mlp.gate_up_proj"
    with pytest.raises(ValueError, match="no tensor split rule"):
        skipzero_shard({o + k: v for k, v in t.items()}, {o: geo}, 0, 2)
    with pytest.raises(ValueError, match="bad rank"):
        skipzero_shard({g + k: v for k, v in t.items()}, {g: geo}, 2, 2)


def test_load_artifact_rank_shards(tmp_path):
    """load_artifact(shard=(rank, n)) and the config's vq_skipzero.shard:
    the skipzero up_proj of the fixture comes back with the rank's 64 of its
    128 rows per expert, row tables that expand to the slices of the
    unsplit one; every other module is built whole."""
    from vqlab_amd import artifact
    cfg, mods = af.write(tmp_path, "sz_pack")
    full = artifact.load_artifact(tmp_path, device="cpu")
    p = next(iter(cfg["vq_skipzero"]["modules"]))
    rt_full = full.modules[p].row_table.numpy()
    for rank in range(2):
        a = artifact.load_artifact(tmp_path, device="cpu", shard=(rank, 2))
        m = a.modules[p]
        assert m.output_dims == 64 and m.row_table.shape == (2, 64)
        want = (rt_full[:, rank * 64:(rank + 1) * 64] >= 0)
        assert np.array_equal(m.row_table.numpy() >= 0, want)
        cf = _np(full.modules[p].codes)
        cr = _np(m.codes)
        rt = m.row_table.numpy()
        sl = rt_full[:, rank * 64:(rank + 1) * 64]
        assert np.array_equal(cr[rt[want]], cf[sl[want]])
        for q, mod in a.modules.items():
            if q != p and hasattr(mod, "output_dims"):
                assert mod.output_dims == full.modules[q].output_dims
    c2 = json.loads((tmp_path / "config.json").read_text())
    c2["vq_skipzero"]["shard"] = {"rank": 1, "n": 2}
    (tmp_path / "config.json").write_text(json.dumps(c2))
    b = artifact.load_artifact(tmp_path, device="cpu")
    assert b.modules[p].output_dims == 64
    assert torch.equal(b.modules[p].row_table,
                       artifact.load_artifact(tmp_path, device="cpu", shard=(1, 2)).modules[p].row_table)
