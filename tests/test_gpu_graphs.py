"""Every entry point captured in a HIP graph: each replay, with new inputs
copied in and eager calls on the same tensors in between, gives the bits of
an eager call on those inputs.

Graph capture is how a serving loop launches these kernels without host
overhead; a kernel that kept state between calls (a counter, a sort buffer, a
split-K partial) or relied on memory cleared outside its own launches would
pass eager tests and fail here. Every path below is deterministic (no atomics
in any sum), so the bar is bit equality.
"""
import numpy as np
import pytest

from vq_cases import PATH_FUSED, PATH_GROUPED, PATH_ONE_LAUNCH, hooks, make_module, to_device

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _rand_(t, rng):
    """Refill t in place with N(0, 1) values (host draw, one copy)."""
    t.copy_(torch.from_numpy(rng.standard_normal(tuple(t.shape)).astype(np.float32)).to(t.device, t.dtype))


def _replays(fn, refill, reps=4):
    """Capture fn() once, then for each replay: refill the inputs, replay,
    synchronise, and compare with an eager fn() on the same inputs."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()                                     # workspaces allocated outside the capture
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    outs = out if isinstance(out, tuple) else (out,)
    for rep in range(reps):
        refill(rep)
        graph.replay()
        torch.cuda.synchronize()
        got = [o.clone() for o in outs]
        want = fn()
        want = want if isinstance(want, tuple) else (want,)
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(got, want)):
            assert torch.equal(a.view(torch.uint8) if a.is_floating_point() else a,
                               b.view(torch.uint8) if b.is_floating_point() else b), \
                f"replay {rep}, output {i}"


def test_graph_dense_gemv():
    from vqlab_amd import vq_switch as VS
    print("graph: dense gemv", flush=True)
    rng = np.random.default_rng(61)
    m = make_module(rng, 1, 512, 1024, 2, 256, packed=False)
    codes, cb, sc = to_device(m)
    x = torch.empty((2, 1024), dtype=torch.bfloat16, device="cuda")
    _rand_(x, rng)
    _replays(lambda: VS._dense_fused(x, codes[0], cb, sc[0], pack_bits=0), lambda r: _rand_(x, rng))


def test_graph_expert_gemv_new_routing():
    from vqlab_amd import vq_switch as VS
    print("graph: expert gemv", flush=True)
    rng = np.random.default_rng(62)
    E, T, k = 8, 2, 3
    m = make_module(rng, E, 512, 2048, 4, 4096)
    codes, cb, sc = to_device(m)
    x = torch.empty((T, 2048), dtype=torch.bfloat16, device="cuda")
    e = torch.empty(T * k, dtype=torch.int32, device="cuda")

    def refill(r):
        _rand_(x, rng)
        e.copy_(torch.from_numpy(np.concatenate([rng.choice(E, k, replace=False) for _ in range(T)])
                                 .astype(np.int32)).cuda())
    refill(-1)
    _replays(lambda: VS._fused(x, e, codes, cb, sc, pack_bits=12, xkrep=k), refill)


def test_graph_grouped_gemm_new_routing():
    """The device sort (counts, offsets, tile records in the workspace) runs
    inside the graph: every replay routes anew."""
    from vqlab_amd import vq_switch as VS
    print("graph: grouped gemm", flush=True)
    rng = np.random.default_rng(63)
    E, T, k = 16, 40, 3
    m = make_module(rng, E, 384, 1024, 8, 4096)
    codes, cb, sc = to_device(m)
    x = torch.empty((T, 1024), dtype=torch.bfloat16, device="cuda")
    e = torch.empty(T * k, dtype=torch.int32, device="cuda")

    def refill(r):
        _rand_(x, rng)
        if r % 2:   # skewed: every token on experts 0 and 1 plus one other
            ids = np.concatenate([[0, 1, 2 + int(rng.integers(E - 2))] for _ in range(T)])
        else:
            ids = np.concatenate([rng.choice(E, k, replace=False) for _ in range(T)])
        e.copy_(torch.from_numpy(np.asarray(ids, np.int32)).cuda())
    refill(-1)
    _replays(lambda: VS._gemmseg(x, e, codes, cb, sc, 12, 1024, k), refill)


def test_graph_dense_gemm_split_k_tail():
    """Decode-then-GEMM with a split-K tail (257 tiles of 256 x 256): the
    panel dequant, the fp32 partials and their fixed-order sum, per replay."""
    from vqlab_amd import vq_dense as VD
    print("graph: dense gemm split-K tail", flush=True)
    rng = np.random.default_rng(64)
    N, OUT, IN, K = 256, 257 * 256, 1024, 4096
    g = torch.Generator(device="cuda")
    g.manual_seed(64)
    codes = torch.randint(0, K, (OUT, IN // 4), dtype=torch.int32, device="cuda", generator=g).to(torch.int16)
    cb = (torch.randn((K, 4), device="cuda", generator=g) * 0.02).to(torch.float16)
    sc = (torch.rand((OUT, IN // 64), device="cuda", generator=g) + 0.5).to(torch.float16)
    x = torch.empty((N, IN), dtype=torch.bfloat16, device="cuda")
    _rand_(x, rng)
    _replays(lambda: VD._decode_matmul(x, codes, cb, sc, 64, OUT, IN, 0), lambda r: _rand_(x, rng), reps=3)


def _block(rng, E, H, I, D, K, k, shared):
    from vqlab_amd import moe
    projs = {n: make_module(rng, E, o, i, D, K) for n, (o, i) in
             (("gate", (I, H)), ("up", (I, H)), ("down", (H, I)))}
    dev = lambda ms: {n: to_device(mm) + (mm["pack_bits"],) for n, mm in ms.items()}
    sh = {n: make_module(rng, 1, o, i, D, K) for n, (o, i) in
          (("gate", (I, H)), ("up", (I, H)), ("down", (H, I)))} if shared else None
    sgv = torch.from_numpy((rng.standard_normal(H) * 0.02).astype(np.float32)).to("cuda", torch.bfloat16)
    return moe.VQSparseMoeBlock.from_modules(
        dev(projs), top_k=k, in_features={"gate": H, "up": H, "down": I},
        shared=dev(sh) if shared else None, shared_gate=sgv if shared else None)


@pytest.mark.parametrize("T,path,shared", [(1, PATH_ONE_LAUNCH, False), (1, PATH_ONE_LAUNCH, True),
                                           (3, PATH_FUSED, False), (24, PATH_GROUPED, True)])
def test_graph_moe_layer(T, path, shared):
    """The layer at T = 1 (one launch, with and without a shared expert),
    T = 3 (two fused kernels) and T = 24 with a shared expert (96 routed
    pairs: device sort, grouped gate/up/down, split-K shared expert,
    combine): routing and outputs per replay."""
    import ctypes
    print(f"graph: moe layer T={T} shared={shared}", flush=True)
    rng = np.random.default_rng(65 + T + 7 * shared)
    E, H, I, k = 32, 1024, 512, 4
    blk = _block(rng, E, H, I, 4, 4096, k, shared=shared)
    keep = []
    got = ctypes.c_int32()
    assert hooks().vqk__test_moe_path(ctypes.byref(blk._fused_desc(keep)), T, ctypes.byref(got)) == 0
    assert got.value == path, (T, got.value)
    x = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    lg = torch.empty((T, E), dtype=torch.float32, device="cuda")

    def refill(r):
        _rand_(x, rng)
        _rand_(lg, rng)
    refill(-1)
    _replays(lambda: blk.fused(x, lg, return_route=True), refill)


_FIRST_CAPTURED = r"""
import sys
sys.path.insert(0, sys.argv[1]); sys.path.insert(0, sys.argv[1] + '/tests')
import numpy as np, torch
from test_gpu_graphs import _block, _rand_
rng = np.random.default_rng(91)
T, E = 24, 32
blk = _block(rng, E, 1024, 512, 4, 4096, 4, shared=True)
x = torch.empty((T, 1024), dtype=torch.bfloat16, device='cuda')
lg = torch.empty((T, E), dtype=torch.float32, device='cuda')
_rand_(x, rng); _rand_(lg, rng)
# the block's workspace comes from an allocation outside the capture
blk._ws = torch.zeros(1 << 26, dtype=torch.uint8, device='cuda')
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    y = blk.fused(x, lg)            # the process's first batched call: captured
for rep in range(3):
    _rand_(x, rng); _rand_(lg, rng)
    g.replay(); torch.cuda.synchronize()
    got = y.clone()
    want = blk.fused(x, lg)         # eager: creates the second stream now
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16)), rep
print('FIRST_CAPTURED_OK')
"""


def test_graph_first_batched_call_captured():
    """A process whose first batched layer call is made inside a graph
    capture: the library does not create its second stream during the
    capture (that call runs on the caller's stream alone), and the replays
    give the bits of eager calls made afterwards on the second stream.
    Runs in a fresh process, since the second stream lives per process."""
    import pathlib
    import subprocess
    import sys
    print("graph: first batched call captured (subprocess)", flush=True)
    root = str(pathlib.Path(__file__).resolve().parents[1])
    r = subprocess.run([sys.executable, "-c", _FIRST_CAPTURED, root], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0 and "FIRST_CAPTURED_OK" in r.stdout, (r.stdout[-2000:], r.stderr[-2000:])
