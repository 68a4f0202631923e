"""Tensor-parallel split of skipzero modules through the kernels
(artifact.skipzero_shard, the reference's vq_switch.skipzero_shard,
vq_switch.py:5112-5147), after the reference's tests/test_sz_shard.py:
gate / up split on output rows -- the ranks' outputs, concatenated, are
byte-equal to the unsplit module's; down_proj splits on its input axis --
the ranks' outputs, summed, are byte-equal to the expanded module cut and
summed the same way. d2, d4 and d8, decode (fused GEMV) and prefill
(grouped GEMM) pair counts, 70 % dead rows."""
import numpy as np
import pytest

from oracle import vq_oracle as vo

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

GEOM = {2: 1024, 4: 2048, 8: 16384}          # d -> K


def _ondisk(E, OUT, IN, D, dead, seed):
    r = np.random.default_rng(seed)
    K, G = GEOM[D], 64
    bits = vo.bits_for_k(K)
    codes = r.integers(0, K, (E, OUT, IN // D)).astype(np.uint16)
    cb = (r.standard_normal((K, D)) * 0.05).astype(np.float16)
    sc = (r.standard_normal((E, OUT, IN // G)) * 0.1 + 1).astype(np.float16)
    live = r.random((E, OUT)) >= dead
    live[1, :] = False
    live[2, :] = True
    codes[~live] = 0
    sc[~live] = 0
    full = vo.pack(codes, bits)
    sz = vo.skipzero_compact(full, sc)
    t = {".sz_codes": torch.from_numpy(sz["sz_codes"].view(np.int32)).cuda(),
         ".sz_scales": torch.from_numpy(sz["sz_scales"]).cuda(),
         ".sz_rowmask": torch.from_numpy(sz["sz_rowmask"]),
         ".sz_shape": torch.from_numpy(sz["sz_shape"])}
    return full, sc, t, torch.from_numpy(cb).cuda(), bits, live


def _mod(codes, cb, sc, bits, IN, rt=None):
    from vqlab_amd.vq_switch import VQSwitchLinear
    return VQSwitchLinear(codes, cb, sc, group_size=64, pack_bits=bits, in_features=IN,
                          row_table=rt)


def _xi(T, top, E, IN, seed):
    r = np.random.default_rng(seed)
    x = torch.from_numpy(r.standard_normal((T, 1, 1, IN)).astype(np.float32)).to("cuda", torch.bfloat16)
    idx = torch.from_numpy(r.integers(0, E, (T, top)).astype(np.int32)).cuda()
    return x, idx


def _bits(y):
    return y.cpu().contiguous().view(torch.int16).numpy()


@pytest.mark.parametrize("D", [2, 4, 8])
@pytest.mark.parametrize("OUT,n", [(96, 2), (96, 4), (102, 2)])
@pytest.mark.parametrize("T,top", [(1, 8), (3, 10), (80, 10)])
def test_row_split_concat_byte_equal(D, OUT, n, T, top):
    from vqlab_amd.vq_switch import skipzero_shard, skipzero_weights
    print(f"row split d={D} OUT={OUT} n={n} T={T} top={top}", flush=True)
    E, IN = 8, 512
    p = "model.layers.3.mlp.switch_mlp.gate_proj"
    _, _, t, cb, bits, live = _ondisk(E, OUT, IN, D, 0.7, seed=D * 7 + n)
    w = {p + k: v for k, v in t.items()}
    mods = {p: {"experts": E, "out": OUT, "live_rows": int(live.sum())}}
    x, idx = _xi(T, top, E, IN, seed=T)
    u = skipzero_weights(dict(w), mods)
    ref = _mod(u[p + ".codes"], cb, u[p + ".vq_scales"], bits, IN, u[p + ".row_table"].cuda())(x, idx)
    parts = []
    for rank in range(n):
        wr, mr = skipzero_shard(dict(w), mods, rank, n)
        c = skipzero_weights(wr, mr)
        m = _mod(c[p + ".codes"], cb, c[p + ".vq_scales"], bits, IN, c[p + ".row_table"].cuda())
        assert m.output_dims == OUT // n
        parts.append(m(x, idx))
    got = torch.cat(parts, dim=-1)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(ref), _bits(got))


@pytest.mark.parametrize("D", [2, 4, 8])
@pytest.mark.parametrize("n", [2, 4])
@pytest.mark.parametrize("T,top", [(1, 8), (80, 10)])
def test_down_input_split_sum_byte_equal(D, n, T, top):
    from vqlab_amd.vq_switch import skipzero_shard, skipzero_weights
    print(f"down input split d={D} n={n} T={T} top={top}", flush=True)
    E, OUT, IN = 8, 97, 1024
    p = "model.layers.3.mlp.switch_mlp.down_proj"
    full, sc, t, cb, bits, live = _ondisk(E, OUT, IN, D, 0.7, seed=D + n)
    w = {p + k: v for k, v in t.items()}
    mods = {p: {"experts": E, "out": OUT, "live_rows": int(live.sum()), "in": IN, "dim": D,
                "group": 64, "pack_bits": bits, "k": GEOM[D]}}
    wr, mr = skipzero_shard(dict(w), mods, 1, n)
    assert mr[p] == mods[p] and all(wr[k] is w[k] for k in w)
    c = skipzero_weights(w, mods)
    cs, ss, rt = c[p + ".codes"], c[p + ".vq_scales"], c[p + ".row_table"].cuda()
    fc = torch.from_numpy(full.view(np.int32)).cuda()
    fs = torch.from_numpy(sc).cuda()
    Wd, NG, INr = cs.shape[-1] // n, ss.shape[-1] // n, IN // n
    x, idx = _xi(T, top, E, IN, seed=T + 1)
    ysz = yfull = None
    for r in range(n):
        xr = x[..., r * INr:(r + 1) * INr].contiguous()
        a = _mod(cs[:, r * Wd:(r + 1) * Wd].contiguous(), cb, ss[:, r * NG:(r + 1) * NG].contiguous(),
                 bits, INr, rt)(xr, idx)
        b = _mod(fc[..., r * Wd:(r + 1) * Wd].contiguous(), cb,
                 fs[..., r * NG:(r + 1) * NG].contiguous(), bits, INr)(xr, idx)
        ysz = a if ysz is None else ysz + a
        yfull = b if yfull is None else yfull + b
    torch.cuda.synchronize()
    assert np.array_equal(_bits(ysz), _bits(yfull))
