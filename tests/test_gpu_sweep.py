"""Seeded random geometries through every linear entry point and the MoE
layer, against the oracle.

The parametrised tests elsewhere pin the BASELINE shapes and the edge cases
named one by one; this sweep draws the module format at random -- d 2 / 4 / 8,
K log-uniform in [2, 65536] (powers of two and not), packed (K = 2^bits) or
byte codes, scale groups of 8..256 columns or one per row, IN of one group up to 2048,
OUT from 1, up to 6 experts, 1-4 tokens, fp16 / bf16 / fp32 activations (a
third of them at an unaligned base) and skipzero row tables -- so that every kernel instance the host can pick
(fast or generic GEMV, LDS or L2 tables, the register-decode segment kernel,
decode-then-GEMM with padded and staged operands) meets formats no
hand-written case names. Bars: bit-exact for the dequantised weight, rtol
2e-2 / atol 1e-3 of the float64 oracle elsewhere, with the operand rounding
each path documents (fp16 x for the fused and segment kernels, the
reference's bf16 weight for bf16 x in the dense GEMM).
"""
import numpy as np
import pytest

from oracle import vq_oracle as vo
from vq_cases import assert_close, make_module, skipzero, to_device

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

_DT = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}


def _draw_linear(n, seed):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        D = int(rng.choice([2, 4, 8]))
        K = int(min(65536, max(2, round(float(np.exp(rng.uniform(np.log(2), np.log(65536))))))))
        if rng.random() < 0.4:
            K = 1 << max(1, int(np.log2(K)))
        packed = bool(rng.random() < 0.6) and K & (K - 1) == 0   # packing needs K = 2^bits
        G = int(rng.choice([g for g in (8, 16, 32, 64, 128, 256) if g % D == 0]))
        IN = G * int(rng.integers(1, 2048 // G + 1))
        if rng.random() < 0.15:
            G = IN                                   # one scale per row
        OUT = int(rng.integers(1, 400))
        E = int(rng.integers(1, 7))
        T = int(rng.integers(1, 5))
        k = int(rng.integers(1, min(E, 4) + 1))
        xdt = str(rng.choice(["f16", "bf16", "f32"]))
        dead = 0.3 if rng.random() < 0.25 else 0.0
        cases.append((i, D, K, packed, G, IN, OUT, E, T, k, xdt, dead))
    return cases


_LIN = _draw_linear(64, 20261202)
_LIN_IDS = [f"{c[0]}-d{c[1]}K{c[2]}{'p' if c[3] else 'u'}G{c[4]}IN{c[5]}OUT{c[6]}E{c[7]}{c[10]}"
            + ("sz" if c[11] else "") for c in _LIN]


def _module(case):
    i, D, K, packed, G, IN, OUT, E, T, k, xdt, dead = case
    rng = np.random.default_rng(1000 + i)
    m = make_module(rng, E, OUT, IN, D, K, G=G, packed=packed, dead_frac=dead)
    return rng, m


def _x(rng, N, IN, xdt, shift=0):
    """N(0, 1) activations; shift > 0 places the rows `shift` elements into a
    larger buffer, so x's base is not 16-byte aligned (the staging paths for
    unaligned rows)."""
    v = torch.from_numpy(rng.standard_normal((N, IN)).astype(np.float32)).to("cuda", _DT[xdt])
    if not shift:
        return v
    buf = torch.zeros(N * IN + shift, dtype=v.dtype, device="cuda")
    buf[shift:] = v.reshape(-1)
    return buf[shift:].view(N, IN)


def _shift(case):
    """Every third case takes x at an element offset of 1-3."""
    return case[0] % 3 if case[0] % 3 else 0


def _np(t):
    return t.float().cpu().numpy()


def _x16(x):
    return x.to(torch.float16).float().cpu().numpy()


def _route(rng, T, E, k):
    return np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).reshape(-1).astype(np.int32)


def _compact(m):
    """Skipzero compact codes / scales / row table on the device."""
    sz, rt = skipzero(m)
    c = sz["sz_codes"]
    c = c.view(np.int32) if c.dtype == np.uint32 else (c.view(np.int16) if c.dtype == np.uint16 else c)
    return (torch.from_numpy(np.ascontiguousarray(c)).cuda(), torch.from_numpy(sz["sz_scales"]).cuda(),
            torch.from_numpy(rt).cuda(), rt)


@pytest.mark.parametrize("case", _LIN, ids=_LIN_IDS)
def test_sweep_dequant_bit_exact(case):
    from vqlab_amd import vq_switch as VS
    print(f"sweep dequant {case}", flush=True)
    rng, m = _module(case)
    _, D, K, packed, G, IN, OUT, E = case[:8]
    codes, cb, sc = to_device(m)
    got = VS.wdec_decode(codes, cb, sc, E * OUT, IN, G, m["pack_bits"])
    want = vo.dequant(m["codes"].reshape(E * OUT, -1), m["codebook"], m["scales"].reshape(E * OUT, -1), G)
    assert np.array_equal(got.cpu().numpy().view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("case", _LIN, ids=_LIN_IDS)
def test_sweep_expert_gemv(case):
    from vqlab_amd import vq_switch as VS
    print(f"sweep expert gemv {case}", flush=True)
    rng, m = _module(case)
    _, D, K, packed, G, IN, OUT, E, T, k, xdt, dead = case
    codes, cb, sc = to_device(m)
    ids = _route(rng, T, E, k)
    x = _x(rng, T, IN, xdt, _shift(case))
    e = torch.from_numpy(ids).cuda()
    y = VS._fused(x, e, codes, cb, sc, pack_bits=m["pack_bits"], xkrep=k)
    assert y.shape == (T * k, OUT) and y.dtype == x.dtype
    ref = vo.expert_gemv(_x16(x), ids, m["codes"], m["codebook"], m["scales"], G, xkrep=k)
    assert_close(_np(y), ref, what=f"expert gemv {case}")
    if dead:
        zc, zs, rtd, rt = _compact(m)
        yc = VS._fused(x, e, zc, cb, zs, pack_bits=m["pack_bits"], xkrep=k, rowtbl=rtd,
                       in_features=IN)
        assert torch.equal(yc, y)


@pytest.mark.parametrize("case", _LIN, ids=_LIN_IDS)
def test_sweep_dense_gemv(case):
    from vqlab_amd import vq_switch as VS
    print(f"sweep dense gemv {case}", flush=True)
    rng, m = _module(case)
    _, D, K, packed, G, IN, OUT, E, T, k, xdt, dead = case
    codes, cb, sc = to_device(m)
    x = _x(rng, T, IN, xdt, _shift(case))
    y = VS._dense_fused(x, codes[0], cb, sc[0], pack_bits=m["pack_bits"], in_features=IN)
    assert y.shape == (T, OUT) and y.dtype == x.dtype
    w = vo.dequant(m["codes"][0], m["codebook"], m["scales"][0], G)
    assert_close(_np(y), vo.decode_matmul(_x16(x), w), what=f"dense gemv {case}")


@pytest.mark.parametrize("case", _LIN, ids=_LIN_IDS)
def test_sweep_grouped_gemm(case):
    from vqlab_amd import vq_switch as VS
    print(f"sweep grouped gemm {case}", flush=True)
    rng, m = _module(case)
    _, D, K, packed, G, IN, OUT, E, T, k, xdt, dead = case
    codes, cb, sc = to_device(m)
    # a prefill-sized routing over the same experts: 3..40 tokens
    Tg = int(rng.integers(3, 41))
    ids = _route(rng, Tg, E, k)
    x = _x(rng, Tg, IN, xdt, _shift(case))
    e = torch.from_numpy(ids).cuda()
    y = VS._gemmseg(x, e, codes, cb, sc, m["pack_bits"], IN, k)
    assert y.shape == (Tg * k, OUT) and y.dtype == x.dtype
    ref = vo.expert_gemv(_x16(x), ids, m["codes"], m["codebook"], m["scales"], G, xkrep=k)
    assert_close(_np(y), ref, what=f"grouped gemm {case}")
    if dead:
        zc, zs, rtd, rt = _compact(m)
        yc = VS._gemmseg(x, e, zc, cb, zs, m["pack_bits"], IN, k, rowtbl=rtd)
        assert torch.equal(yc, y)


@pytest.mark.parametrize("case", _LIN, ids=_LIN_IDS)
def test_sweep_dense_gemm(case):
    from vqlab_amd import vq_dense as VD
    print(f"sweep dense gemm {case}", flush=True)
    rng, m = _module(case)
    _, D, K, packed, G, IN, OUT, E, T, k, xdt, dead = case
    codes, cb, sc = to_device(m)
    N = int(rng.integers(65, 200))              # above the register-decode cutoff
    x = _x(rng, N, IN, xdt, _shift(case))
    y = VD._decode_matmul(x, codes[0], cb, sc[0], G, OUT, IN, m["pack_bits"])
    assert y.shape == (N, OUT) and y.dtype == x.dtype
    w = vo.dequant(m["codes"][0], m["codebook"], m["scales"][0], G)
    # the reference's `xf @ w.T.astype(xf.dtype)`: bf16 x meets W rounded to bf16
    wr = vo.bf16_values(w) if xdt == "bf16" else w
    assert_close(_np(y), vo.decode_matmul(_np(x), wr), what=f"dense gemm {case}")


@pytest.mark.parametrize("case", _LIN, ids=_LIN_IDS)
def test_sweep_switch_apply_rounding(case):
    """vqk_switch_apply with bf16 x, on whichever path its options pick: with
    the defaults its rows are that path's fp32 rows rounded to fp16 and then
    to bf16 (the reference's default decode arithmetic); with the bf16-I/O
    options they are the fp32 rows rounded once to bf16, the GEMV keeping x
    exact on the float-staged formats (unpacked d4 K <= 1024, d8 K > 1024)."""
    import ctypes
    from vqlab_amd import _lib as L, _torch as Tt, vq_switch as VS
    print(f"sweep switch_apply {case}", flush=True)
    rng, m = _module(case)
    _, D, K, packed, G, IN, OUT, E, T, k, xdt, dead = case
    codes, cb, sc = to_device(m)
    pb = m["pack_bits"]
    ids = _route(rng, T, E, k)
    x = _x(rng, T, IN, "bf16", _shift(case))
    e = torch.from_numpy(ids).cuda()
    bits = lambda t: t.view(torch.int16)
    dflt, bio = L.options(), L.options(decode_bf16io=1, prefill_bf16io=1)
    yd = VS._switch_apply(x, e, codes, cb, sc, pb, IN, k, opts=dflt)
    y32 = VS._switch_apply(x, e, codes, cb, sc, pb, IN, k, out_dtype=torch.float32, opts=dflt)
    assert torch.equal(bits(yd), bits(y32.to(torch.float16).to(torch.bfloat16)))
    yio = VS._switch_apply(x, e, codes, cb, sc, pb, IN, k, opts=bio)
    yk = VS._switch_apply(x, e, codes, cb, sc, pb, IN, k, out_dtype=torch.float32, opts=bio)
    assert torch.equal(bits(yio), bits(yk.to(torch.bfloat16)))
    # which path ran: a workspace means the grouped GEMM, which narrows x to fp16
    keep = []
    w = Tt.weights(codes, cb, sc, G, pb, IN, keep=keep)
    ws = ctypes.c_size_t()
    L.check(L.lib().vqk_switch_apply_workspace(ctypes.byref(w), T * k, ctypes.byref(bio), ctypes.byref(ws)))
    exact_x = ws.value == 0 and VS._float_staged(cb, pb)
    ref = vo.expert_gemv(_np(x) if exact_x else _x16(x), ids, m["codes"], m["codebook"], m["scales"], G,
                         xkrep=k, weights="exact")
    assert_close(_np(yk), ref, what=f"switch_apply bf16io {case}")


def _draw_layers(n, seed):
    """Layer geometries inside the fused kernels' block limits (NSUB a multiple
    of 32 codes, (top_k + shared) x down blocks <= 64); a format the fused
    layer has no instance for raises NotImplementedError, and the composed
    path, which serves it then, is checked either way."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        D = int(rng.choice([2, 4, 8]))
        K = int(rng.choice([16, 256, 300, 1024, 4096, 5000, 16384]))
        H = 256 * int(rng.integers(1, 9))
        I = 256 * int(rng.integers(1, 4))
        shared = bool(rng.random() < 0.4)
        kmax = max(1, min(8, 64 // (I // (32 * D)) - int(shared)))
        k = int(rng.integers(1, kmax + 1))
        E = int(rng.integers(k, 65))
        T = int(rng.integers(1, 6))
        cases.append((i, E, H, I, D, K, k, shared, bool(rng.random() < 0.7), T))
    return cases


def _draw_batched_layers(n, seed):
    """Batched calls (8-48 tokens: 16-384 routed pairs, the fused, sliced and
    grouped compositions), tables of every size, experts up to 32 of H up to
    1024 x I up to 512."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        D = int(rng.choice([2, 4, 8]))
        K = int(rng.choice([16, 256, 1000, 4096, 16384]))
        H = 256 * int(rng.integers(1, 5))
        I = 256 * int(rng.integers(1, 3))
        shared = bool(rng.random() < 0.5)
        k = int(rng.integers(1, 9))
        E = int(rng.integers(max(k, 4), 33))
        T = int(rng.integers(8, 49))
        cases.append((100 + i, E, H, I, D, K, k, shared, bool(rng.random() < 0.7), T))
    return cases


_LAYERS = _draw_layers(12, 20261203) + _draw_batched_layers(6, 20261204)


@pytest.mark.parametrize("geom", _LAYERS,
                         ids=[f"{g[0]}-d{g[4]}K{g[5]}E{g[1]}H{g[2]}I{g[3]}k{g[6]}T{g[9]}"
                              + ("s" if g[7] else "") for g in _LAYERS])
def test_sweep_moe_layer(geom):
    """The layer call (routing, gate/up, SwiGLU, down, combine, on whichever
    path the plan picks) and the composed per-projection path over random
    layer geometries."""
    from vqlab_amd import moe
    i, E, H, I, D, K, k, shared, norm, T = geom
    print(f"sweep moe layer {geom}", flush=True)
    rng = np.random.default_rng(2000 + i)
    pk = K & (K - 1) == 0
    projs = {n: make_module(rng, E, o, j, D, K, packed=pk) for n, (o, j) in
             (("gate", (I, H)), ("up", (I, H)), ("down", (H, I)))}
    sh = shv = None
    if shared:
        sh = {n: make_module(rng, 1, o, j, D, K, packed=pk) for n, (o, j) in
              (("gate", (I, H)), ("up", (I, H)), ("down", (H, I)))}
        shv = (rng.standard_normal(H) * 0.02).astype(np.float32)
    dev = lambda ms: {n: to_device(mm) + (mm["pack_bits"],) for n, mm in ms.items()}
    blk = moe.VQSparseMoeBlock.from_modules(
        dev(projs), top_k=k, in_features={"gate": H, "up": H, "down": I},
        shared=dev(sh) if shared else None,
        shared_gate=torch.from_numpy(shv).to("cuda", torch.bfloat16) if shared else None,
        norm_topk_prob=norm)
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to("cuda", torch.bfloat16)
    lg = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32)).cuda()
    try:
        y, ids, w = blk.fused(x, lg, return_route=True)
    except NotImplementedError as ex:
        print(f"  fused layer refused: {ex}", flush=True)
        y = None
    spec = lambda mm: {"codes": mm["codes"], "codebook": mm["codebook"], "scales": mm["scales"],
                       "group": 64}
    ref, rids, rw = vo.moe_layer(
        x.float().cpu().numpy(), lg.cpu().numpy(), spec(projs["gate"]), spec(projs["up"]),
        spec(projs["down"]), k, norm=norm,
        shared={n: spec(mm) for n, mm in sh.items()} if shared else None,
        shared_gate=torch.from_numpy(shv).to(torch.bfloat16).float().numpy() if shared else None,
        h_round=np.float16)
    if y is not None:
        assert np.array_equal(ids.cpu().numpy(), rids)
        assert np.allclose(w.cpu().numpy(), rw, rtol=1e-5, atol=1e-6)
        assert_close(y.float().cpu().numpy(), ref, what=f"moe layer {geom}")
    yc = blk.composed(x, lg)
    assert_close(yc.float().cpu().numpy(), ref, what=f"composed {geom}")
