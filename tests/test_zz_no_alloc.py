"""vqk_moe_decode_layer_noalloc (the entry point that allocates nothing)
against vqk_moe_decode_layer with a caller workspace, through the C ABI.

Two calls in a row on the shared scratch array, the second with fewer tokens,
on the fused decode path and on the batched grouped path; each must give
bit-identical outputs and routing to the workspace entry point on the same
inputs (same kernels, same arithmetic), and be within rtol 2e-2 / atol 1e-3
of the oracle. A layer call whose workspace exceeds the array is refused
before any launch.
"""
import ctypes

import numpy as np
import pytest

from oracle import vq_oracle as vo
from vq_cases import assert_close, make_module, to_device

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _block(rng, E, H, I, D, K, k, shared):
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
        shared_gate=torch.from_numpy(shv).to("cuda", torch.bfloat16) if shared else None)
    return blk, projs, sh, shv


def _spec(m):
    return {"codes": m["codes"], "codebook": m["codebook"], "scales": m["scales"], "group": 64}


def _call(L, Tt, d, x, lg, T, k, workspace):
    """One layer call through the C ABI: with a fresh workspace, or (None)
    through the no-allocation entry point."""
    H = x.shape[1]
    y = torch.full((T, H), float("nan"), dtype=torch.bfloat16, device="cuda")
    ids = torch.full((T, k), -7, dtype=torch.int32, device="cuda")
    w = torch.full((T, k), float("nan"), dtype=torch.float32, device="cuda")
    if workspace is None:
        rc = L.lib().vqk_moe_decode_layer_noalloc(
            ctypes.byref(d), Tt.ptr(x), L.VQK_BF16, T, Tt.ptr(lg), Tt.ptr(y), L.VQK_BF16,
            Tt.ptr(ids), Tt.ptr(w), Tt.stream())
    else:
        rc = L.lib().vqk_moe_decode_layer(
            ctypes.byref(d), Tt.ptr(x), L.VQK_BF16, T, Tt.ptr(lg), Tt.ptr(y), L.VQK_BF16,
            Tt.ptr(ids), Tt.ptr(w), Tt.ptr(workspace), workspace.numel(), Tt.stream())
    L.check(rc, "layer call")
    return y, ids, w


@pytest.mark.parametrize("case", [
    # (E, H, I, D, K, k, shared, T first, T second): fused decode path
    (64, 1024, 256, 4, 4096, 8, False, 3, 1),
    # grouped path (T * k >= 64 pairs), d8 table beyond LDS, shared expert
    (32, 1024, 256, 8, 16384, 8, True, 16, 9),
])
def test_noalloc_matches_workspace_entry(case):
    from vqlab_amd import _lib as L, _torch as Tt
    E, H, I, D, K, k, shared, T1, T2 = case
    print(f"noalloc {case}", flush=True)
    rng = np.random.default_rng(E + H + T1)
    blk, projs, sh, shv = _block(rng, E, H, I, D, K, k, shared)
    keep = []
    d = blk._fused_desc(keep)
    for T in (T1, T2):
        x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to("cuda", torch.bfloat16)
        lg = torch.from_numpy(rng.standard_normal((T, E)).astype(np.float32)).cuda()
        need = ctypes.c_size_t()
        L.check(L.lib().vqk_moe_decode_layer_workspace(ctypes.byref(d), T, ctypes.byref(need)))
        assert need.value <= L.VQK_NOALLOC_SCRATCH_BYTES
        ws = torch.zeros(max(1, need.value), dtype=torch.uint8, device="cuda")
        y0, i0, w0 = _call(L, Tt, d, x, lg, T, k, ws)
        y1, i1, w1 = _call(L, Tt, d, x, lg, T, k, None)
        torch.cuda.synchronize()
        assert torch.equal(i1, i0) and torch.equal(w1, w0), f"routing T={T}"
        assert torch.equal(y1.view(torch.int16), y0.view(torch.int16)), f"outputs T={T}"
        shared_spec = {n: _spec(m) for n, m in sh.items()} if shared else None
        sgv = torch.from_numpy(shv).to(torch.bfloat16).float().numpy() if shared else None
        ref, rid, _ = vo.moe_layer(x.float().cpu().numpy(), lg.cpu().numpy(),
                                   _spec(projs["gate"]), _spec(projs["up"]), _spec(projs["down"]),
                                   k, shared=shared_spec, shared_gate=sgv, h_round=np.float16)
        assert np.array_equal(i1.cpu().numpy(), rid)
        assert_close(y1.float().cpu().numpy(), ref, what=f"noalloc T={T}")


def test_noalloc_one_launch_geometries_alternate():
    """The scratch array is shared by every layer: three one-launch geometries
    (one with a shared expert) alternating through
    vqk_moe_decode_layer_noalloc (the call number and the hand-off words at
    fixed header offsets, tags naming the word's header index) give, call
    after call, the bits of the two-kernel form through a caller workspace;
    the scratch header reports no error afterwards."""
    from vqlab_amd import _lib as L, _torch as Tt
    from vq_cases import PATH_ONE_LAUNCH, moe_path, two_kernels
    print("noalloc: two one-launch geometries alternate", flush=True)
    rng = np.random.default_rng(77)
    geoms = [(256, 2048, 512, 4, 4096, 8, False), (64, 1024, 256, 4, 256, 6, False),
             (128, 1024, 256, 4, 1024, 6, True)]
    blks = []
    for g in geoms:
        blk, *_ = _block(rng, *g)
        assert moe_path(blk, 1) == PATH_ONE_LAUNCH
        keep = []
        blks.append((blk, blk._fused_desc(keep), keep, g))
    for rnd in range(3):
        for blk, d, _, g in blks + blks[::-1]:
            E, H, k = g[0], g[1], g[5]
            x = torch.from_numpy(rng.standard_normal((1, H)).astype(np.float32)).to("cuda", torch.bfloat16)
            lg = torch.from_numpy(rng.standard_normal((1, E)).astype(np.float32)).cuda()
            y1, i1, w1 = _call(L, Tt, d, x, lg, 1, k, None)
            need = ctypes.c_size_t()
            L.check(L.lib().vqk_moe_decode_layer_workspace(ctypes.byref(d), 1, ctypes.byref(need)))
            ws = torch.zeros(need.value, dtype=torch.uint8, device="cuda")
            with two_kernels():
                y0, i0, w0 = _call(L, Tt, d, x, lg, 1, k, ws)
            torch.cuda.synchronize()
            assert torch.equal(i1, i0) and torch.equal(w1, w0), f"routing round {rnd} {g}"
            assert torch.equal(y1.view(torch.int16), y0.view(torch.int16)), f"outputs round {rnd} {g}"
    L.check(L.lib().vqk_moe_layer_status(None, Tt.stream()), "noalloc scratch status")


def test_noalloc_refuses_oversized_call():
    """A call whose workspace exceeds the scratch array returns VQK_ENOSPACE
    before anything is launched (the output stays untouched)."""
    from vqlab_amd import _lib as L, _torch as Tt
    rng = np.random.default_rng(9)
    E, H, I, k = 16, 4096, 128, 4
    blk, *_ = _block(rng, E, H, I, 4, 256, k, False)
    keep = []
    d = blk._fused_desc(keep)
    T = 1
    need = ctypes.c_size_t()
    while True:
        L.check(L.lib().vqk_moe_decode_layer_workspace(ctypes.byref(d), T, ctypes.byref(need)))
        if need.value > L.VQK_NOALLOC_SCRATCH_BYTES:
            break
        T *= 2
    x = torch.zeros((T, H), dtype=torch.bfloat16, device="cuda")
    lg = torch.zeros((T, E), dtype=torch.float32, device="cuda")
    y = torch.full((T, H), 3.0, dtype=torch.bfloat16, device="cuda")
    rc = L.lib().vqk_moe_decode_layer_noalloc(ctypes.byref(d), Tt.ptr(x), L.VQK_BF16, T,
                                              Tt.ptr(lg), Tt.ptr(y), L.VQK_BF16, None, None,
                                              Tt.stream())
    assert rc == L.VQK_ENOSPACE
    assert "scratch" in L.last_error()
    torch.cuda.synchronize()
    assert bool((y.float() == 3.0).all())
