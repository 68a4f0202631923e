"""Fused MoE decode layer (routing + SwitchGLU + combine) against the oracle.

Routing must select exactly the oracle's experts (continuous logits: no
ties); weights agree to fp32 rounding; outputs are within rtol 2e-2 /
atol 1e-3 of the float64 oracle with the SwiGLU intermediate rounded to
fp16, the activation dtype down_proj receives.
"""
import numpy as np
import pytest

from oracle import vq_oracle as vo
from vq_cases import assert_close, make_module, to_device

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _spec(m):
    return {"codes": m["codes"], "codebook": m["codebook"], "scales": m["scales"], "group": 64}


def _block(rng, E, H, I, D, K, k, shared=False, norm=True):
    from vqlab_amd import moe
    projs = {n: make_module(rng, E, o, i, D, K) for n, (o, i) in
             (("gate", (I, H)), ("up", (I, H)), ("down", (H, I)))}
    sh = shv = None
    if shared:
        sh = {n: make_module(rng, 1, o, i, D, K) for n, (o, i) in
              (("gate", (I, H)), ("up", (I, H)), ("down", (H, I)))}
        shv = (rng.standard_normal(H) * 0.02).astype(np.float32)
    dev = lambda ms: {n: to_device(m) + (m["pack_bits"],) for n, m in ms.items()}
    blk = moe.VQSparseMoeBlock.from_modules(
        dev(projs), top_k=k, in_features={"gate": H, "up": H, "down": I},
        shared=dev(sh) if shared else None,
        shared_gate=torch.from_numpy(shv).to("cuda", torch.bfloat16) if shared else None,
        norm_topk_prob=norm)
    return blk, projs, sh, shv


def _check(blk, projs, sh, shv, rng, T, E, H, k, norm=True):
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to("cuda", torch.bfloat16)
    lg = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32)).cuda()
    y, ids, w = blk.fused(x, lg, return_route=True)
    torch.cuda.synchronize()
    shared = None
    sgv = None
    if sh is not None:
        shared = {n: _spec(m) for n, m in sh.items()}
        sgv = torch.from_numpy(shv).to(torch.bfloat16).float().numpy()
    ref, rids, rw = vo.moe_layer(x.float().cpu().numpy(), lg.cpu().numpy(), _spec(projs["gate"]),
                                 _spec(projs["up"]), _spec(projs["down"]), k, norm=norm,
                                 shared=shared, shared_gate=sgv, h_round=np.float16)
    assert np.array_equal(ids.cpu().numpy(), rids)
    assert np.allclose(w.cpu().numpy(), rw, rtol=1e-5, atol=1e-6)
    assert_close(y.float().cpu().numpy(), ref, what=f"moe T={T}")
    # the composed path (per-projection kernels + torch routing) agrees
    yc = blk.composed(x, lg)
    assert_close(yc.float().cpu().numpy(), ref, what=f"composed T={T}")
    return y


def test_moe_layer_c2_shape():
    """Qwen3.6-35B-A3B-shaped layer: H 2048, 256 experts of I 512, top-8,
    d4 K4096 12-bit packed."""
    print("moe c2 shape", flush=True)
    rng = np.random.default_rng(2)
    blk, projs, sh, shv = _block(rng, 256, 2048, 512, 4, 4096, 8)
    _check(blk, projs, sh, shv, rng, 1, 256, 2048, 8)


@pytest.mark.parametrize("T", [1, 2])
def test_moe_layer_multi_step_tiles(T):
    """H 4096, I 1024, top-7 + a shared expert, d4 K4096: each gate/up
    workgroup walks several row steps (2 at T=1, 4 at T=2) and its gate and up
    values meet in LDS for every one of them."""
    print(f"moe multi-step T={T}", flush=True)
    rng = np.random.default_rng(40 + T)
    blk, projs, sh, shv = _block(rng, 16, 4096, 1024, 4, 4096, 7, shared=True)
    _check(blk, projs, sh, shv, rng, T, 16, 4096, 7)


@pytest.mark.parametrize("T", [1, 3])
def test_moe_layer_d8_table_in_lds(T):
    """d8 K4096 (12-bit, a 64 KB table per projection): the gate/up kernel
    reads x from LDS per code at this width."""
    print(f"moe d8 K4096 T={T}", flush=True)
    rng = np.random.default_rng(50 + T)
    blk, projs, sh, shv = _block(rng, 32, 1024, 512, 8, 4096, 4, shared=True)
    _check(blk, projs, sh, shv, rng, T, 32, 1024, 4)


# (E, H, I, D, K, k, shared, norm, T): widths 2..14 bits, tables in and beyond
# LDS, ragged row counts against the workgroup tiles, 1-3 tokens
_GEOMS = [
    (24, 128, 192, 2, 256, 3, False, True, 1),
    (24, 640, 320, 2, 1024, 4, True, False, 2),
    (32, 768, 384, 4, 512, 5, False, True, 3),
    (16, 1536, 384, 4, 4096, 6, True, True, 1),
    (40, 1024, 640, 4, 2048, 2, False, False, 2),
    (16, 512, 256, 8, 256, 3, True, True, 2),
    (20, 1024, 512, 8, 4096, 4, False, True, 1),
    (12, 1024, 256, 8, 16384, 2, True, False, 1),
    (12, 512, 128, 4, 16384, 3, False, True, 3),
]


@pytest.mark.parametrize("geom", _GEOMS, ids=[f"d{g[3]}K{g[4]}E{g[0]}T{g[8]}" for g in _GEOMS])
def test_moe_layer_geometries(geom):
    """The fused layer over assorted geometries against the oracle."""
    E, H, I, D, K, k, shared, norm, T = geom
    print(f"moe geometry {geom}", flush=True)
    rng = np.random.default_rng(sum(geom[:6]))
    blk, projs, sh, shv = _block(rng, E, H, I, D, K, k, shared=shared, norm=norm)
    _check(blk, projs, sh, shv, rng, T, E, H, k, norm=norm)


@pytest.mark.parametrize("T", [1, 4])
def test_moe_layer_c3_shape_shared(T):
    """Qwen3.5-397B-A17B row shapes: H 4096, I 1024, d8 K16384 14-bit,
    top-10 + a shared expert (64 experts instead of 512)."""
    print(f"moe c3 shape T={T}", flush=True)
    rng = np.random.default_rng(3 + T)
    blk, projs, sh, shv = _block(rng, 64, 4096, 1024, 8, 16384, 10, shared=True)
    _check(blk, projs, sh, shv, rng, T, 64, 4096, 10)


def test_moe_layer_repeated_calls_one_workspace():
    """Many T == 1 calls in a row on one workspace keep giving the oracle's
    answer (the routing and SwiGLU buffers are rewritten every call)."""
    print("moe repeated calls", flush=True)
    rng = np.random.default_rng(7)
    E, H, I, k = 64, 1024, 256, 6
    blk, projs, sh, shv = _block(rng, E, H, I, 4, 4096, k)
    x = torch.from_numpy(rng.standard_normal((1, H)).astype(np.float32)).to("cuda", torch.bfloat16)
    ys = []
    for i in range(6):
        lg = torch.from_numpy(rng.standard_normal((1, E)).astype(np.float32)).cuda()
        ys.append((blk.fused(x, lg), lg))
    torch.cuda.synchronize()
    for y, lg in ys:
        ref, _, _ = vo.moe_layer(x.float().cpu().numpy(), lg.cpu().numpy(), _spec(projs["gate"]),
                                 _spec(projs["up"]), _spec(projs["down"]), k, h_round=np.float16)
        assert_close(y.float().cpu().numpy(), ref, what="repeat")


def test_moe_layer_unnormalised_d2():
    print("moe d2 norm=False", flush=True)
    rng = np.random.default_rng(4)
    blk, projs, sh, shv = _block(rng, 32, 1024, 256, 2, 512, 4, norm=False)
    _check(blk, projs, sh, shv, rng, 2, 32, 1024, 4, norm=False)


def test_moe_layer_workspace_too_small():
    import ctypes
    from vqlab_amd import _lib as L, _torch as Tt
    rng = np.random.default_rng(5)
    blk, *_ = _block(rng, 8, 256, 128, 4, 256, 2)
    keep = []
    d = blk._fused_desc(keep)
    x = torch.zeros((1, 256), dtype=torch.bfloat16, device="cuda")
    lg = torch.zeros((1, 8), dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    ws = torch.empty(16, dtype=torch.uint8, device="cuda")
    rc = L.lib().vqk_moe_decode_layer(ctypes.byref(d), Tt.ptr(x), L.VQK_BF16, 1, Tt.ptr(lg),
                                      Tt.ptr(y), L.VQK_BF16, None, None, Tt.ptr(ws), 16,
                                      Tt.stream())
    assert rc == L.VQK_ENOSPACE


def test_routing_ties_pick_lower_ids():
    """Tied logits: the kernel's argmax takes the lowest expert id first, the
    oracle's stable descending sort does the same."""
    print("routing ties", flush=True)
    rng = np.random.default_rng(6)
    blk, projs, sh, shv = _block(rng, 64, 256, 128, 4, 256, 6)
    x = torch.from_numpy(rng.standard_normal((4, 256)).astype(np.float32)).to("cuda", torch.bfloat16)
    lg = np.round(rng.standard_normal((4, 64)) * 2) / 2           # many exact ties
    lg[1, :] = 0.0                                                  # all tied
    lg[2, 10:] = -np.inf                                            # only 10 finite
    lg[3, :] = -1.0                                                 # -0 and +0 tie (equal floats)
    lg[3, rng.permutation(64)[:12]] = 0.0
    lg[3, rng.permutation(64)[:12]] = -0.0
    lgt = torch.from_numpy(lg.astype(np.float32)).cuda()
    _, ids, w = blk.fused(x, lgt, return_route=True)
    rids, rw = vo.route(lg.astype(np.float32), 6)
    assert np.array_equal(ids.cpu().numpy(), rids)
    assert np.allclose(w.cpu().numpy(), rw, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("D,K,T,shared,E", [(8, 16384, 8, True, 32), (8, 16384, 16, False, 32),
                                            (4, 4096, 12, True, 32), (2, 512, 40, False, 32),
                                            (8, 16384, 8, True, 64), (8, 16384, 12, False, 48),
                                            (8, 16384, 8, False, 96)])
def test_moe_layer_batched_grouped_path(D, K, T, shared, E):
    """T * top_k >= 64 pairs: the layer runs as one routing + one sort +
    grouped matrix-core GEMMs (SwiGLU built while down's input is staged) +
    the weighted combine; same oracle, same bar. With <= 2 pairs per expert
    (the last three cases) the d8 tables take 4-row tiles; the last has fewer
    pairs than experts (64 over 96), grouped only because of that path."""
    print(f"moe batched grouped D={D} K={K} T={T} shared={shared} E={E}", flush=True)
    rng = np.random.default_rng(20 + T + D + (E if E != 32 else 0))
    H, I, k = 1024, 256, 8
    blk, projs, sh, shv = _block(rng, E, H, I, D, K, k, shared=shared)
    _check(blk, projs, sh, shv, rng, T, E, H, k)


def test_moe_layer_batched_shared_ksplit():
    """Batched grouped layer whose shared expert's gate / up split K (H=2048:
    two supersteps, so two fp32 partials that the shared down adds while it
    stages silu(g) * u); same oracle, same bar."""
    print("moe batched shared K split", flush=True)
    rng = np.random.default_rng(47)
    E, H, I, k, T = 64, 2048, 256, 8, 8
    blk, projs, sh, shv = _block(rng, E, H, I, 8, 16384, k, shared=True)
    _check(blk, projs, sh, shv, rng, T, E, H, k)


@pytest.mark.parametrize("E,T", [(32, 16), (64, 8)])
def test_moe_layer_batched_skipzero(E, T):
    """The grouped layer over compact skipzero experts (20% dead rows): dead
    rows contribute exact zeros, as in the expanded oracle. E=64, T=8: one
    pair per expert on average, the config-4 path (4-row tiles, persistent
    segment kernel)."""
    from vq_cases import skipzero
    from vqlab_amd.vq_switch import VQSwitchLinear
    print(f"moe batched skipzero E={E} T={T}", flush=True)
    rng = np.random.default_rng(31 + E)
    H, I, k = 1024, 256, 8
    blk, projs, _, _ = _block(rng, E, H, I, 8, 16384, k)
    for name, (o, i) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
        m = make_module(rng, E, o, i, 8, 16384, dead_frac=0.2)
        projs[name] = m
        sz, rt = skipzero(m)
        cb = torch.from_numpy(m["codebook"]).cuda()
        mod = VQSwitchLinear(torch.from_numpy(sz["sz_codes"].view(np.int32)).cuda(), cb,
                             torch.from_numpy(sz["sz_scales"]).cuda(), pack_bits=m["pack_bits"],
                             in_features=i, row_table=torch.from_numpy(rt).cuda())
        setattr(blk.switch_mlp, name + "_proj", mod)
    _check(blk, projs, None, None, rng, T, E, H, k)


@pytest.mark.parametrize("D,K,shared", [(4, 16384, True), (2, 65536, False), (8, 8192, True)])
def test_moe_layer_decode_tables_beyond_lds(D, K, shared):
    """Decode (T = 1, 2) with codebooks larger than the LDS-resident limit:
    gate and up in separate workgroups, each with the first 128 KB of its
    table in LDS (all of a d4 K16384 table) and the rest read from L2."""
    print(f"moe decode big tables D={D} K={K} shared={shared}", flush=True)
    rng = np.random.default_rng(40 + D)
    E, H, I, k = 32, 1024, 512, 6
    blk, projs, sh, shv = _block(rng, E, H, I, D, K, k, shared=shared)
    for T in (1, 2):
        _check(blk, projs, sh, shv, rng, T, E, H, k)


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy()


def _xl(rng, T, H, E):
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to("cuda", torch.bfloat16)
    lg = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32)).cuda()
    return x, lg


@pytest.mark.parametrize("fill", ["random", "zeros", "ones"])
def test_moe_one_launch_matches_two_launches(fill):
    """A T = 1 call of a layer whose tables fit LDS runs as one launch (the
    down workgroups route for themselves and take the SwiGLU rows as tagged
    64-bit words through the workspace header); T = 2 runs the two kernels,
    and so does T = 1 with the one launch switched off. The same token gives
    the same bits all three ways, call after call on one workspace whose
    scratch part holds random bytes, zeros or all ones (the header starts
    zeroed, as the contract asks). In between, T = 2 calls whose second token
    is all zeros write zero SwiGLU rows across the scratch part: they must not
    disturb the following one-launch calls."""
    from vq_cases import PATH_FUSED, PATH_ONE_LAUNCH, moe_path, two_kernels
    print(f"moe one launch vs two launches, scratch {fill}", flush=True)
    rng = np.random.default_rng(11)
    E, H, I, k = 256, 2048, 512, 8
    blk, projs, sh, shv = _block(rng, E, H, I, 4, 4096, k)
    assert moe_path(blk, 1) == PATH_ONE_LAUNCH and moe_path(blk, 2) == PATH_FUSED
    with two_kernels():
        assert moe_path(blk, 1) == PATH_FUSED
    x, lg = _xl(rng, 2, H, E)
    blk.fused(x, lg)
    if fill == "random":
        g = torch.Generator(device="cuda").manual_seed(5)
        blk._ws.copy_(torch.randint(0, 256, blk._ws.shape, dtype=torch.uint8, device="cuda", generator=g))
    else:
        blk._ws.fill_(0 if fill == "zeros" else 255)
    blk.reset()
    for i in range(5):
        x, lg = _xl(rng, 2, H, E)
        y1 = blk.fused(x[:1], lg[:1])
        y2 = blk.fused(x, lg)
        with two_kernels():
            yk = blk.fused(x[:1], lg[:1])
        xz = x.clone()
        xz[1] = 0
        blk.fused(xz, lg)
        y1b = blk.fused(x[:1], lg[:1])
        torch.cuda.synchronize()
        assert np.array_equal(_bits(y1[0]), _bits(y2[0])), f"call {i}: one launch vs T=2"
        assert np.array_equal(_bits(y1), _bits(yk)), f"call {i}: one launch vs two kernels"
        assert np.array_equal(_bits(y1b), _bits(y1)), f"call {i}: after a zero-row T=2 call"
        if i == 0:
            ref, _, _ = vo.moe_layer(x[:1].float().cpu().numpy(), lg[:1].cpu().numpy(),
                                     _spec(projs["gate"]), _spec(projs["up"]), _spec(projs["down"]),
                                     k, h_round=np.float16)
            assert_close(y1.float().cpu().numpy(), ref, what="one launch")
    blk.status()


def test_moe_one_launch_graph_replays():
    """The one-launch layer captured in a HIP graph: every replay (new inputs
    copied in, eager calls on the same workspace in between) gives the eager
    call's bits; the call number it keeps in the workspace advances inside the
    graph too."""
    print("moe one launch graph replays", flush=True)
    rng = np.random.default_rng(12)
    E, H, I, k = 64, 1024, 256, 6
    blk, projs, sh, shv = _block(rng, E, H, I, 4, 4096, k)
    x = torch.from_numpy(rng.standard_normal((1, H)).astype(np.float32)).to("cuda", torch.bfloat16)
    lg = torch.from_numpy(rng.standard_normal((1, E)).astype(np.float32)).cuda()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        blk.fused(x, lg)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y = blk.fused(x, lg)
    for rep in range(4):
        x.copy_(torch.from_numpy(rng.standard_normal((1, H)).astype(np.float32)).to("cuda", torch.bfloat16))
        lg.copy_(torch.from_numpy(rng.standard_normal((1, E)).astype(np.float32)).cuda())
        graph.replay()
        torch.cuda.synchronize()
        yr = y.clone()
        ye = blk.fused(x, lg)
        torch.cuda.synchronize()
        assert np.array_equal(_bits(yr), _bits(ye)), f"replay {rep}"
        ref, _, _ = vo.moe_layer(x.float().cpu().numpy(), lg.cpu().numpy(), _spec(projs["gate"]),
                                 _spec(projs["up"]), _spec(projs["down"]), k, h_round=np.float16)
        assert_close(yr.float().cpu().numpy(), ref, what=f"replay {rep}")


_L1_GEOMS = [
    (24, 128, 384, 4, 1024, 3, False),
    (200, 640, 320, 2, 4096, 6, True),
    (256, 1024, 256, 4, 256, 8, False),
    (48, 512, 448, 2, 512, 5, True),
]


@pytest.mark.parametrize("geom", _L1_GEOMS, ids=[f"d{g[3]}K{g[4]}E{g[0]}I{g[2]}" for g in _L1_GEOMS])
def test_moe_one_launch_geometries(geom):
    """The one-launch layer (batch 1) over assorted geometries -- E not a
    power of two, I not a multiple of the gate/up row tile, unnormalised
    routing, d2 and d4 at 8 to 12 bits -- against the oracle and bit for bit
    against the two kernels (the same token inside a T = 2 call)."""
    from vq_cases import PATH_ONE_LAUNCH, moe_path, two_kernels
    E, H, I, D, K, k, norm = geom
    print(f"moe one launch geometry {geom}", flush=True)
    rng = np.random.default_rng(sum(geom[:6]) + 100)
    blk, projs, sh, shv = _block(rng, E, H, I, D, K, k, norm=norm)
    assert moe_path(blk, 1) == PATH_ONE_LAUNCH and moe_path(blk, 2) != PATH_ONE_LAUNCH
    x, lg = _xl(rng, 2, H, E)
    y1 = blk.fused(x[:1], lg[:1])
    y2 = blk.fused(x, lg)
    with two_kernels():
        yk = blk.fused(x[:1], lg[:1])
    torch.cuda.synchronize()
    assert np.array_equal(_bits(y1[0]), _bits(y2[0]))
    assert np.array_equal(_bits(y1), _bits(yk))
    ref, _, _ = vo.moe_layer(x[:1].float().cpu().numpy(), lg[:1].cpu().numpy(), _spec(projs["gate"]),
                             _spec(projs["up"]), _spec(projs["down"]), k, norm=norm, h_round=np.float16)
    assert_close(y1.float().cpu().numpy(), ref, what=f"one launch {geom}")


_L1_SHARED_GEOMS = [
    (128, 2048, 512, 4, 4096, 6, True),
    (48, 512, 448, 2, 512, 5, False),
    (24, 128, 384, 4, 1024, 3, True),
]


@pytest.mark.parametrize("geom", _L1_SHARED_GEOMS,
                         ids=[f"d{g[3]}K{g[4]}E{g[0]}I{g[2]}" for g in _L1_SHARED_GEOMS])
def test_moe_one_launch_shared_expert(geom):
    """A layer with a shared expert at batch 1 runs as one launch too: the
    shared pair's gate / up rows go through the hand-off like the routed
    pairs', its down table sits beside the routed one in the down
    workgroups' LDS, and each down workgroup takes the shared gate
    sigmoid(x . v) itself. Call after call on one workspace, the output is
    the two kernels' bits (the same token alone with the one launch switched
    off, and inside a T = 2 call) and within the oracle's bar."""
    from vq_cases import PATH_ONE_LAUNCH, moe_path, two_kernels
    E, H, I, D, K, k, norm = geom
    print(f"moe one launch with a shared expert {geom}", flush=True)
    rng = np.random.default_rng(sum(geom[:6]) + 300)
    blk, projs, sh, shv = _block(rng, E, H, I, D, K, k, shared=True, norm=norm)
    assert moe_path(blk, 1) == PATH_ONE_LAUNCH and moe_path(blk, 2) != PATH_ONE_LAUNCH
    shared = {n: _spec(m) for n, m in sh.items()}
    sgv = torch.from_numpy(shv).to(torch.bfloat16).float().numpy()
    for i in range(3):
        x, lg = _xl(rng, 2, H, E)
        y1 = blk.fused(x[:1], lg[:1])
        y2 = blk.fused(x, lg)
        with two_kernels():
            yk = blk.fused(x[:1], lg[:1])
        torch.cuda.synchronize()
        assert np.array_equal(_bits(y1[0]), _bits(y2[0])), f"call {i}: one launch vs T=2"
        assert np.array_equal(_bits(y1), _bits(yk)), f"call {i}: one launch vs two kernels"
        ref, _, _ = vo.moe_layer(x[:1].float().cpu().numpy(), lg[:1].cpu().numpy(), _spec(projs["gate"]),
                                 _spec(projs["up"]), _spec(projs["down"]), k, norm=norm,
                                 shared=shared, shared_gate=sgv, h_round=np.float16)
        assert_close(y1.float().cpu().numpy(), ref, what=f"one launch shared {geom} call {i}")
    blk.status()


def _share(ws_size, *blks):
    ws = torch.zeros(ws_size, dtype=torch.uint8, device="cuda")
    for b in blks:
        b._ws = ws
    return ws


def test_moe_one_launch_geometries_share_a_workspace():
    """Two one-launch geometries (different grids, word counts and row
    tiles) alternate on ONE workspace: the call number and the hand-off words
    sit at fixed header offsets and the tags name the word's header index, so
    neither geometry's words can pass for the other's. Every call is bit for
    bit the two-kernel form of the same token."""
    from vq_cases import PATH_ONE_LAUNCH, moe_path, two_kernels
    print("moe one launch: two geometries on one workspace", flush=True)
    rng = np.random.default_rng(31)
    ga = (256, 2048, 512, 4, 4096, 8)
    gb = (64, 1024, 256, 4, 256, 6)
    ba, pa, _, _ = _block(rng, *ga)
    bb, pb, _, _ = _block(rng, *gb)
    assert moe_path(ba, 1) == PATH_ONE_LAUNCH and moe_path(bb, 1) == PATH_ONE_LAUNCH
    _share(1 << 20, ba, bb)
    for i in range(4):
        for blk, g in ((ba, ga), (bb, gb), (bb, gb), (ba, ga)):
            E, H = g[0], g[1]
            x, lg = _xl(rng, 1, H, E)
            y = blk.fused(x, lg)
            with two_kernels():
                yk = blk.fused(x, lg)
            torch.cuda.synchronize()
            assert np.array_equal(_bits(y), _bits(yk)), f"round {i} geometry {g}"
    ba.status()


@pytest.mark.parametrize("shared", [False, True], ids=["routed", "shared"])
def test_moe_one_launch_gives_up_loudly(shared):
    """A one-launch wait that runs out never computes through: the
    affected rows come out NaN and the header's error word is set (all
    kernels still end normally -- the give-up is forced from the host with a
    zero wait bound). Later one-launch calls on that workspace give NaN rows
    until reset; vqk_moe_layer_status reports it; after reset the layer
    gives the two-kernel form's bits again. With and without a shared
    expert (its words travel with the routed ones)."""
    from vq_cases import PATH_ONE_LAUNCH, l1_spins, moe_path, two_kernels
    print(f"moe one launch: forced give-up, shared={shared}", flush=True)
    rng = np.random.default_rng(32)
    E, H, I, D, K, k = 64, 1024, 256, 4, 256, 6
    blk, projs, _, _ = _block(rng, E, H, I, D, K, k, shared=shared)
    assert moe_path(blk, 1) == PATH_ONE_LAUNCH
    x, lg = _xl(rng, 1, H, E)
    y0 = blk.fused(x, lg)
    blk.status()
    with l1_spins(0):
        yg = blk.fused(x, lg)
        torch.cuda.synchronize()
    assert bool(torch.isnan(yg.float()).all()), "every down workgroup gave up: all rows NaN"
    with pytest.raises(RuntimeError, match="ran out"):
        blk.status()
    ys = blk.fused(x, lg)                       # sticky: still NaN, no wait
    torch.cuda.synchronize()
    assert bool(torch.isnan(ys.float()).all())
    with two_kernels():                         # the other paths never read the header
        yk = blk.fused(x, lg)
        torch.cuda.synchronize()
    assert np.array_equal(_bits(yk), _bits(y0))
    blk.reset()
    yr = blk.fused(x, lg)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(yr), _bits(y0))
    blk.status()


_T1_LOGITS = ["ties", "all_equal", "ten_finite", "signed_zeros", "nan_mix", "few_valid"]


@pytest.mark.parametrize("shared", [False, True], ids=["routed", "shared"])
@pytest.mark.parametrize("case", _T1_LOGITS)
def test_moe_one_launch_special_logits(case, shared):
    """Batch-1 routing inside the one-launch layer (every workgroup routes the
    token itself) on tied, all-equal, -inf, +-0 and NaN logits, with and
    without a shared expert: the same experts and weights as the oracle (ties
    to the lower id; NaN never chosen, a selection left without a non-NaN
    logit is id -1 / weight 0, the shared expert still added), outputs within
    the bar, and bit for bit the two-kernel form."""
    from vq_cases import PATH_ONE_LAUNCH, moe_path, two_kernels
    print(f"moe one launch special logits {case} shared={shared}", flush=True)
    rng = np.random.default_rng(33)
    E, H, I, D, K, k = 64, 1024, 256, 4, 256, 6
    blk, projs, sh, shv = _block(rng, E, H, I, D, K, k, shared=shared)
    assert moe_path(blk, 1) == PATH_ONE_LAUNCH
    lg = (np.round(rng.standard_normal(E) * 2) / 2).astype(np.float32)
    if case == "all_equal":
        lg[:] = 0.0
    elif case == "ten_finite":
        lg[10:] = -np.inf
    elif case == "signed_zeros":
        lg[:] = -1.0
        lg[rng.permutation(E)[:12]] = 0.0
        lg[rng.permutation(E)[:12]] = -0.0
    elif case == "nan_mix":
        lg[rng.permutation(E)[:20]] = np.nan
    elif case == "few_valid":
        lg[:] = np.nan
        lg[[5, 40, 17, 33]] = [0.25, -0.5, 0.25, 1.0]
    x = torch.from_numpy(rng.standard_normal((1, H)).astype(np.float32)).to("cuda", torch.bfloat16)
    lgt = torch.from_numpy(lg[None]).cuda()
    y, ids, w = blk.fused(x, lgt, return_route=True)
    with two_kernels():
        yk = blk.fused(x, lgt)
    torch.cuda.synchronize()
    rids, rw = vo.route(lg[None], k)
    assert np.array_equal(ids.cpu().numpy(), rids), (ids.cpu().numpy(), rids)
    assert np.allclose(w.cpu().numpy(), rw, rtol=1e-5, atol=1e-6)
    assert np.array_equal(_bits(y), _bits(yk))
    shs = {n: _spec(m) for n, m in sh.items()} if shared else None
    sgv = torch.from_numpy(shv).to(torch.bfloat16).float().numpy() if shared else None
    ref, _, _ = vo.moe_layer(x.float().cpu().numpy(), lg[None], _spec(projs["gate"]),
                             _spec(projs["up"]), _spec(projs["down"]), k, shared=shs, shared_gate=sgv,
                             h_round=np.float16)
    assert_close(y.float().cpu().numpy(), ref, what=f"special logits {case} shared={shared}")


def test_empty_batches():
    """No tokens in: every module returns an empty result of the right shape
    and launches nothing (empty tensors have NULL pointers)."""
    from vqlab_amd.vq_dense import VQLinear
    rng = np.random.default_rng(61)
    E, H, I, k = 16, 256, 128, 4
    blk, projs, _, _ = _block(rng, E, H, I, 4, 1024, k, shared=True)
    x = torch.zeros((0, H), dtype=torch.bfloat16, device="cuda")
    lg = torch.zeros((0, E), dtype=torch.float32, device="cuda")
    y, ids, w = blk.fused(x, lg, return_route=True)
    assert y.shape == (0, H) and ids.shape == (0, k) and w.shape == (0, k)
    assert blk.composed(x, lg).shape == (0, H)
    g = blk.switch_mlp.gate_proj
    yg = g(x[:, None, None, :], torch.zeros((0, k), dtype=torch.int32, device="cuda"))
    assert yg.shape == (0, k, 1, I)
    m = projs["down"]
    codes, cb, sc = to_device(m)
    lin = VQLinear(codes[0], cb, sc[0], group_size=64, pack_bits=m["pack_bits"], in_features=I)
    assert lin(torch.zeros((0, I), dtype=torch.bfloat16, device="cuda")).shape == (0, H)
    torch.cuda.synchronize()


def test_batched_layer_from_two_host_threads():
    """The batched (grouped) layer forks its shared expert and routed up
    projection onto a second per-device stream with events: two host threads,
    each calling its own block (own workspace) on its own stream 12 times,
    get the bits of the same calls made one after another."""
    import threading
    from vq_cases import PATH_GROUPED, hooks
    import ctypes
    print("batched layer from two host threads", flush=True)
    rng = np.random.default_rng(77)
    E, H, I, D, K, k, T = 32, 1024, 512, 4, 4096, 4, 24
    blk, projs, sh, shv = _block(rng, E, H, I, D, K, k, shared=True)
    blk2, _, _, _ = _block(np.random.default_rng(77), E, H, I, D, K, k, shared=True)
    keep = []
    path = ctypes.c_int32()
    assert hooks().vqk__test_moe_path(ctypes.byref(blk._fused_desc(keep)), T, ctypes.byref(path)) == 0
    assert path.value == PATH_GROUPED
    xs = [torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to("cuda", torch.bfloat16)
          for _ in range(2)]
    lgs = [torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32)).cuda() for _ in range(2)]
    blocks = [blk, blk2]
    ref = [blocks[i].fused(xs[i], lgs[i]).clone() for i in range(2)]
    torch.cuda.synchronize()
    outs = [[], []]
    errs = []

    def worker(i):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                for _ in range(12):
                    outs[i].append(blocks[i].fused(xs[i], lgs[i]))
            s.synchronize()
        except Exception as ex:          # reported below, in the test's thread
            errs.append(ex)
    th = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    torch.cuda.synchronize()
    assert not errs, errs
    for i in range(2):
        assert len(outs[i]) == 12
        for y in outs[i]:
            assert torch.equal(y.view(torch.int16), ref[i].view(torch.int16))
    ref0, _, _ = vo.moe_layer(xs[0].float().cpu().numpy(), lgs[0].cpu().numpy(), _spec(projs["gate"]),
                              _spec(projs["up"]), _spec(projs["down"]), k, h_round=np.float16,
                              shared={n: _spec(m) for n, m in sh.items()},
                              shared_gate=torch.from_numpy(shv).to(torch.bfloat16).float().numpy())
    assert_close(ref[0].float().cpu().numpy(), ref0, what="two threads")
