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
