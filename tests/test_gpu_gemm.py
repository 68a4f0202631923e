"""Matrix-core paths against the oracle, through the C ABI.

vqk_dense_gemm (_decode_matmul, vq_dense.py:262-312) and vqk_grouped_gemm
(_gemmseg_prefill, vq_switch.py:4569-4722): outputs within rtol 2e-2 /
atol 1e-3 of the float64 decode-then-matmul oracle. The register-decode
segment kernels (dense N <= 64, grouped) take x rounded to fp16. Above 64
rows (or when the segment kernel refuses the shape) the dense GEMM is the
reference's own arithmetic, `xf @ w.T.astype(xf.dtype)` (vq_dense.py:288,
294): bf16 x against W cast to bf16, fp16 x against the fp16 W, fp32 x
against the fp16 W through the split bf16 form -- and the oracle rounds W
the same way. The device-side sort must build the oracle's tile metadata
(tile_meta, vq_switch.py:4590-4610) exactly.
"""
import ctypes

import numpy as np
import pytest

from oracle import vq_oracle as vo
from vq_cases import assert_close, make_module, skipzero, to_device

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _np(t):
    return t.float().cpu().numpy()


def _x(rng, N, IN, dt=torch.bfloat16):
    return torch.from_numpy(rng.standard_normal((N, IN)).astype(np.float32)).to("cuda", dt)


def _x16(x):
    """The fp16 operand the matrix cores see, as float32 on the host."""
    return x.to(torch.float16).float().cpu().numpy()


# -------------------------------------------------------------- dense GEMM
@pytest.mark.parametrize("case", [
    # (N, OUT, IN, D, K, G, packed)
    (33, 512, 1024, 2, 256, 64, False),        # just above the GEMV cutoff; c1 format
    (256, 640, 2048, 4, 4096, 64, True),       # c2 format, OUT not a multiple of 128
    (300, 384, 1024, 8, 16384, 64, True),      # d8 K16384: codebook gathered from L2
    (130, 256, 640, 8, 65536, 64, False),      # c5 format (uint16 codes), NSUB 80
    (64, 200, 96, 4, 1000, 32, False),         # IN not a multiple of 64, K not a power of 2
    (129, 128, 512, 2, 512, 128, True),        # a scale group spans two 64-column steps
])
def test_dense_gemm(case):
    from vqlab_amd import vq_dense as VD
    N, OUT, IN, D, K, G, packed = case
    print(f"dense gemm {case}", flush=True)
    rng = np.random.default_rng(N + OUT + IN)
    m = make_module(rng, 1, OUT, IN, D, K, G=G, packed=packed)
    codes, cb, sc = to_device(m)
    x = _x(rng, N, IN)
    y = VD._decode_matmul(x, codes[0], cb, sc[0], G, OUT, IN, m["pack_bits"])
    assert y.shape == (N, OUT) and y.dtype == x.dtype
    w = vo.dequant(m["codes"][0], m["codebook"], m["scales"][0], G)
    if N > 64 or (IN // D) % 32:    # decode-then-GEMM: the reference's bf16 operands
        ref = vo.decode_matmul(_np(x), vo.bf16_values(w))
    else:                           # register-decode segment kernel: fp16 operands
        ref = vo.decode_matmul(_x16(x), w)
    assert_close(_np(y), ref, what=f"dense gemm {case}")


@pytest.mark.parametrize("xdt", [torch.float16, torch.float32])
def test_dense_gemm_dtypes_and_linear(xdt):
    """VQLinear routes N > the GEMV cutoff to the GEMM; both agree with the
    oracle on the same module, in fp16 and fp32 activations (the GEMM keeps
    fp32 x to 16 significant bits, the GEMV narrows it to fp16)."""
    from vqlab_amd import vq_dense as VD
    rng = np.random.default_rng(21)
    m = make_module(rng, 1, 512, 2048, 4, 4096)
    codes, cb, sc = to_device(m)
    lin = VD.VQLinear(codes[0], cb, sc[0], group_size=64, pack_bits=12, in_features=2048)
    x = _x(rng, 200, 2048, xdt)
    y = lin(x[None])
    assert y.shape == (1, 200, 512) and y.dtype == xdt
    w = vo.dequant(m["codes"][0], m["codebook"], m["scales"][0], 64)
    ref = vo.decode_matmul(_np(x), w)
    assert_close(_np(y[0]), ref, what=f"VQLinear {xdt}")
    y8 = lin(x[:8])                                   # the GEMV side of the cutoff
    assert_close(_np(y8), vo.decode_matmul(_x16(x[:8]), w), what="VQLinear gemv side")


def test_dense_gemm_empty_and_refusals():
    from vqlab_amd import _lib as L, _torch as Tt
    rng = np.random.default_rng(22)
    m = make_module(rng, 2, 128, 256, 4, 256)
    codes, cb, sc = to_device(m)
    keep = []
    w = Tt.weights(codes, cb, sc, 64, 8, 256, keep=keep)
    y = torch.empty((1, 128), dtype=torch.bfloat16, device="cuda")
    x = torch.zeros((1, 256), dtype=torch.bfloat16, device="cuda")
    # two experts: the dense GEMM takes exactly one linear
    assert L.lib().vqk_dense_gemm(ctypes.byref(w), Tt.ptr(x), L.VQK_BF16, 1, Tt.ptr(y),
                                  L.VQK_BF16, None, 0, Tt.stream()) == L.VQK_EINVAL
    w1 = Tt.weights(codes[0], cb, sc[0], 64, 8, 256, keep=keep)
    assert L.lib().vqk_dense_gemm(ctypes.byref(w1), Tt.ptr(x), L.VQK_BF16, 0, Tt.ptr(y),
                                  L.VQK_BF16, None, 0, Tt.stream()) == L.VQK_OK
    # above 64 rows the decode-then-GEMM path wants the staged x (up to
    # fp32's split rows) + >= 128 weight rows; none at all is refused too
    xb = torch.zeros((100, 256), dtype=torch.bfloat16, device="cuda")
    yb = torch.empty((100, 128), dtype=torch.bfloat16, device="cuda")
    ws = ctypes.c_size_t()
    L.check(L.lib().vqk_dense_gemm_workspace(ctypes.byref(w1), 100, ctypes.byref(ws)))
    assert ws.value >= 100 * 3 * 256 * 2 + 128 * 3 * 256 * 2
    small = torch.empty(1024, dtype=torch.uint8, device="cuda")
    assert L.lib().vqk_dense_gemm(ctypes.byref(w1), Tt.ptr(xb), L.VQK_BF16, 100, Tt.ptr(yb),
                                  L.VQK_BF16, Tt.ptr(small), 1024, Tt.stream()) == L.VQK_ENOSPACE
    assert L.lib().vqk_dense_gemm(ctypes.byref(w1), Tt.ptr(xb), L.VQK_BF16, 100, Tt.ptr(yb),
                                  L.VQK_BF16, None, 0, Tt.stream()) == L.VQK_ENOSPACE
    # a workspace that is not 16-byte aligned is refused before any launch
    big = torch.empty(ws.value + 16, dtype=torch.uint8, device="cuda")
    assert L.lib().vqk_dense_gemm(ctypes.byref(w1), Tt.ptr(xb), L.VQK_BF16, 100, Tt.ptr(yb),
                                  L.VQK_BF16, ctypes.c_void_p(big.data_ptr() + 4), ws.value,
                                  Tt.stream()) == L.VQK_EINVAL


@pytest.mark.parametrize("panel_rows", [128, 256, 1024])
def test_dense_gemm_panels(panel_rows):
    """Workspaces smaller than the whole weight decode it in panels of whole
    128-row multiples; every panel size agrees with the oracle."""
    from vqlab_amd import _lib as L, _torch as Tt
    print(f"dense gemm panels {panel_rows}", flush=True)
    rng = np.random.default_rng(27)
    N, OUT, IN = 300, 700, 1024
    m = make_module(rng, 1, OUT, IN, 4, 4096)
    codes, cb, sc = to_device(m)
    keep = []
    w = Tt.weights(codes[0], cb, sc[0], 64, 12, IN, keep=keep)
    x = _x(rng, N, IN)
    y = torch.empty((N, OUT), dtype=torch.float32, device="cuda")
    nb = panel_rows * IN * 2
    work = torch.empty(nb, dtype=torch.uint8, device="cuda")
    L.check(L.lib().vqk_dense_gemm(ctypes.byref(w), Tt.ptr(x), L.VQK_BF16, N, Tt.ptr(y),
                                   L.VQK_F32, Tt.ptr(work), nb, Tt.stream()))
    wd = vo.dequant(m["codes"][0], m["codebook"], m["scales"][0], 64)
    assert_close(_np(y), vo.decode_matmul(_np(x), vo.bf16_values(wd)), what=f"panels {panel_rows}")


@pytest.mark.parametrize("xdt,IN,offset", [
    (torch.float32, 1000, 0),      # split bf16 operands, rows padded to the k step
    (torch.bfloat16, 1000, 0),     # bf16 rows padded (x staged)
    (torch.float16, 1024, 1),      # x misaligned by one element (x staged)
    (torch.float32, 1024, 3),      # misaligned fp32 x through the split form
])
def test_dense_gemm_staged_x(xdt, IN, offset):
    """x that the GEMM cannot read in place (fp32, IN not a multiple of 64,
    misaligned) is staged into the workspace: same arithmetic, same bar."""
    from vqlab_amd import _lib as L, _torch as Tt
    print(f"dense gemm staged x {xdt} IN {IN} offset {offset}", flush=True)
    rng = np.random.default_rng(31 + IN + offset)
    N, OUT = 200, 384
    G = 64 if IN % 64 == 0 else 40
    m = make_module(rng, 1, OUT, IN, 4, 4096, G=G, packed=False)
    codes, cb, sc = to_device(m)
    keep = []
    w = Tt.weights(codes[0], cb, sc[0], G, 0, IN, keep=keep)
    base = _x(rng, N * IN + offset, 1, xdt).reshape(-1)
    x = base[offset:].reshape(N, IN)
    y = torch.empty((N, OUT), dtype=torch.float32, device="cuda")
    ws = ctypes.c_size_t()
    L.check(L.lib().vqk_dense_gemm_workspace(ctypes.byref(w), N, ctypes.byref(ws)))
    work = torch.empty(ws.value, dtype=torch.uint8, device="cuda")
    L.check(L.lib().vqk_dense_gemm(ctypes.byref(w), Tt.ptr(x), Tt.ACT_TYPES[xdt], N, Tt.ptr(y),
                                   L.VQK_F32, Tt.ptr(work), ws.value, Tt.stream()))
    wd = vo.dequant(m["codes"][0], m["codebook"], m["scales"][0], G)
    wr = vo.bf16_values(wd) if xdt == torch.bfloat16 else wd
    assert_close(_np(y), vo.decode_matmul(_np(x), wr), what=f"staged x {xdt} {IN} {offset}")


def test_dense_gemm_split_k_tail():
    """257 output tiles of 256 x 256 on 256 CUs: one whole round, then the
    last tile's K split 8 ways into fp32 partials summed in a fixed order.
    Sampled columns (first, last, across the tail tile) against the oracle,
    and a second call gives the same bits (the sum order is fixed)."""
    from vqlab_amd import vq_dense as VD
    print("dense gemm split-K tail", flush=True)
    rng = np.random.default_rng(35)
    N, OUT, IN, K = 256, 257 * 256, 1024, 4096
    g = torch.Generator(device="cuda")
    g.manual_seed(35)
    codes = torch.randint(0, K, (OUT, IN // 4), dtype=torch.int32, device="cuda",
                          generator=g).to(torch.int16)
    cb = (torch.randn((K, 4), device="cuda", generator=g) * 0.02).to(torch.float16)
    sc = (torch.rand((OUT, IN // 64), device="cuda", generator=g) + 0.5).to(torch.float16)
    x = _x(rng, N, IN)
    y = VD._decode_matmul(x, codes, cb, sc, 64, OUT, IN, 0)
    y2 = VD._decode_matmul(x, codes, cb, sc, 64, OUT, IN, 0)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    cols = np.unique(np.concatenate([rng.choice(OUT, 48, replace=False), [0, OUT - 1],
                                     np.arange(OUT - 256, OUT, 9)]))
    ci = torch.from_numpy(cols).cuda()
    w = vo.dequant(codes.index_select(0, ci).cpu().numpy().view(np.uint16), cb.cpu().numpy(),
                   sc.index_select(0, ci).cpu().numpy(), 64)
    ref = vo.decode_matmul(_np(x), vo.bf16_values(w))
    assert_close(_np(y)[:, cols], ref, what="split-K tail")


def test_dense_gemm_bf16_beyond_fp16_range():
    """bf16 activations beyond fp16's range stay finite: the GEMM takes bf16
    operands, never a narrowing of x to fp16 (vq_dense.py:294)."""
    from vqlab_amd import vq_dense as VD
    rng = np.random.default_rng(33)
    N, OUT, IN = 96, 256, 512
    m = make_module(rng, 1, OUT, IN, 4, 4096)
    codes, cb, sc = to_device(m)
    x = _x(rng, N, IN) * 1e6                         # |x| far above 65504
    y = VD._decode_matmul(x, codes[0], cb, sc[0], 64, OUT, IN, m["pack_bits"])
    assert torch.isfinite(y).all()
    w = vo.dequant(m["codes"][0], m["codebook"], m["scales"][0], 64)
    assert_close(_np(y), vo.decode_matmul(_np(x), vo.bf16_values(w)), what="bf16 beyond fp16 range")


# ------------------------------------------------------------ grouped GEMM
def _routes(rng, T, k, E, lo=1, hi=8):
    """Top-k ids per token (distinct within a token) drawn so that each
    touched expert receives between lo and hi tokens where the draw allows."""
    ids = np.zeros((T, k), np.int64)
    load = np.zeros(E, np.int64)
    for t in range(T):
        w = np.where(load < hi, 1.0, 1e-6) * (1.0 + 4.0 * (load > 0) * (load < lo + 1))
        ids[t] = rng.choice(E, k, replace=False, p=w / w.sum())
        load[ids[t]] += 1
    return ids


@pytest.mark.parametrize("shape", [
    # (T, k, E, OUT, IN, D, K): c4 rows (c3 layer, fewer experts), c2 rows
    (64, 10, 40, 1024, 4096, 8, 16384),
    (16, 10, 48, 4096, 1024, 8, 16384),
    (64, 8, 32, 512, 2048, 4, 4096),
    (40, 4, 16, 2048, 512, 4, 4096),
])
def test_grouped_gemm_shapes(shape):
    from vqlab_amd import vq_switch as VS
    T, k, E, OUT, IN, D, K = shape
    print(f"grouped gemm {shape}", flush=True)
    rng = np.random.default_rng(sum(shape))
    m = make_module(rng, E, OUT, IN, D, K)
    codes, cb, sc = to_device(m)
    ids = _routes(rng, T, k, E).reshape(-1)
    x = _x(rng, T, IN)
    e = torch.from_numpy(ids.astype(np.int32)).cuda()
    y = VS._gemmseg(x, e, codes, cb, sc, m["pack_bits"], IN, k)
    assert y.shape == (T * k, OUT)
    ref = vo.expert_gemv(_x16(x), ids, m["codes"], m["codebook"], m["scales"], 64, xkrep=k)
    assert_close(_np(y), ref, what=f"grouped {shape}")
    # the GEMV on the same pairs agrees to the same bar
    yg = VS._fused(x, e, codes, cb, sc, pack_bits=m["pack_bits"], xkrep=k)
    assert_close(_np(y), _np(yg), rtol=2e-2, atol=2e-3, what="grouped vs gemv")


@pytest.mark.parametrize("shape", [
    # (T, k, E, OUT, IN, D, K): tables past the LDS-resident part (their
    # other entries gathered from L2), fp32 output as the MoE layer uses it
    (64, 10, 40, 1024, 4096, 8, 16384),
    (16, 10, 48, 4096, 1024, 8, 16384),
    (16, 10, 64, 4096, 512, 8, 16384),        # half a superstep per row
    (24, 6, 20, 4000, 1024, 8, 32768),        # OUT not a multiple of 128
    (32, 8, 24, 2560, 1024, 4, 32768),
    (32, 8, 24, 2048, 512, 2, 65536),
    # <= 2 pairs per expert on average: d8 tables take 4-row tiles
    (8, 10, 64, 1024, 4096, 8, 16384),
    (12, 6, 40, 1000, 512, 8, 32768),
    (8, 8, 40, 512, 1024, 8, 65536),
])
def test_grouped_gemm_fp32_out_large_tables(shape):
    """fp32 output with a table beyond LDS, against the oracle; the bf16
    output of the same call agrees."""
    from vqlab_amd import vq_switch as VS
    T, k, E, OUT, IN, D, K = shape
    print(f"grouped gemm fp32 out {shape}", flush=True)
    rng = np.random.default_rng(sum(shape) + 7)
    m = make_module(rng, E, OUT, IN, D, K)
    codes, cb, sc = to_device(m)
    ids = _routes(rng, T, k, E).reshape(-1)
    x = _x(rng, T, IN)
    e = torch.from_numpy(ids.astype(np.int32)).cuda()
    y = VS._gemmseg(x, e, codes, cb, sc, m["pack_bits"], IN, k, out_dtype=torch.float32)
    assert y.dtype == torch.float32 and y.shape == (T * k, OUT)
    ref = vo.expert_gemv(_x16(x), ids, m["codes"], m["codebook"], m["scales"], 64, xkrep=k)
    assert_close(_np(y), ref, what=f"fp32 out {shape}")
    yb = VS._gemmseg(x, e, codes, cb, sc, m["pack_bits"], IN, k)
    assert_close(_np(yb), _np(y), rtol=2e-2, atol=2e-3, what="bf16 vs fp32 out")


def test_grouped_gemm_fp32_out_skipzero():
    """fp32 output over compact skipzero rows: dead rows are exact zeros."""
    from vqlab_amd import vq_switch as VS
    print("grouped gemm fp32 out skipzero", flush=True)
    rng = np.random.default_rng(29)
    E, OUT, IN, T, k = 32, 2048, 1024, 16, 10
    m = make_module(rng, E, OUT, IN, 8, 16384, dead_frac=0.2)
    codes, cb, sc = to_device(m)
    sz, rt = skipzero(m)
    zc = torch.from_numpy(sz["sz_codes"].view(np.int32)).cuda()
    zs = torch.from_numpy(sz["sz_scales"]).cuda()
    rtd = torch.from_numpy(rt).cuda()
    ids = _routes(rng, T, k, E).reshape(-1)
    x = _x(rng, T, IN)
    e = torch.from_numpy(ids.astype(np.int32)).cuda()
    yc = VS._gemmseg(x, e, zc, cb, zs, 14, IN, k, rtd, out_dtype=torch.float32)
    dead = rt[ids] < 0
    assert dead.any() and (_np(yc)[dead] == 0).all()
    ref = vo.expert_gemv(_x16(x), ids, m["codes"], m["codebook"], m["scales"], 64, xkrep=k)
    assert_close(_np(yc), ref, what="fp32 out skipzero")


def test_grouped_gemm_skipzero_mtp_verify():
    """The c4 case: MTP verify on the c3 layer format, 20 % of rows dead,
    stored compact with a row table; dead rows give exact zeros."""
    from vqlab_amd import vq_switch as VS
    print("grouped gemm skipzero", flush=True)
    rng = np.random.default_rng(23)
    E, OUT, IN, T, k = 32, 1024, 4096, 16, 10
    m = make_module(rng, E, OUT, IN, 8, 16384, dead_frac=0.2)
    codes, cb, sc = to_device(m)
    sz, rt = skipzero(m)
    zc = torch.from_numpy(sz["sz_codes"].view(np.int32)).cuda()
    zs = torch.from_numpy(sz["sz_scales"]).cuda()
    rtd = torch.from_numpy(rt).cuda()
    ids = _routes(rng, T, k, E).reshape(-1)
    x = _x(rng, T, IN)
    e = torch.from_numpy(ids.astype(np.int32)).cuda()
    yc = VS._gemmseg(x, e, zc, cb, zs, 14, IN, k, rtd)
    ye = VS._gemmseg(x, e, codes, cb, sc, 14, IN, k)
    dead = rt[ids] < 0
    assert dead.any() and (_np(yc)[dead] == 0).all()
    assert torch.equal(yc[torch.from_numpy(~dead).cuda()], ye[torch.from_numpy(~dead).cuda()])
    ref = vo.expert_gemv(_x16(x), ids, m["codes"], m["codebook"], m["scales"], 64, xkrep=k)
    assert_close(_np(yc), ref, what="skipzero grouped")


def test_grouped_gemm_sort_builds_oracle_tiles():
    """Workspace after a call: order[] groups the pairs by expert exactly as
    the oracle's stable argsort does (as sets within each segment) and the
    tile records equal tile_meta(), including an id outside [0, E), whose
    rows come out as zeros."""
    from vqlab_amd import _lib as L, _torch as Tt
    print("grouped gemm sort", flush=True)
    rng = np.random.default_rng(24)
    E, OUT, IN, N = 40, 256, 512, 700
    m = make_module(rng, E, OUT, IN, 4, 256, packed=False)
    codes, cb, sc = to_device(m)
    ids = rng.integers(0, E, N).astype(np.int64)
    ids[rng.integers(0, E, N) < 4] = 7                 # one expert with > 32 rows
    ids[5] = E + 3                                      # outside [0, E)
    x = _x(rng, N, IN, torch.float16)
    e = torch.from_numpy(ids.astype(np.int32)).cuda()
    keep = []
    w = Tt.weights(codes, cb, sc, 64, 0, IN, keep=keep)
    ws = ctypes.c_size_t()
    L.check(L.lib().vqk_grouped_gemm_workspace(ctypes.byref(w), N, ctypes.byref(ws)))
    work = torch.zeros(ws.value, dtype=torch.uint8, device="cuda")
    y = torch.empty((N, OUT), dtype=torch.float32, device="cuda")
    L.check(L.lib().vqk_grouped_gemm(ctypes.byref(w), Tt.ptr(x), L.VQK_F16, N, Tt.ptr(e), N, 1,
                                     Tt.ptr(y), L.VQK_F32, Tt.ptr(work), ws.value, Tt.stream()))
    torch.cuda.synchronize()
    wb = work.cpu().numpy()
    al = lambda v: (v + 255) & ~255
    mt = (N + 15) // 16 + min(N, E + 1)                 # tiles of <= 16 rows
    room = (N + 3) // 4 + min(N, E + 1)                 # record room: 4-row tiles
    order = wb[:4 * N].view(np.int32)
    tm = wb[al(4 * N):al(4 * N) + 12 * mt].view(np.int32).reshape(mt, 3)
    nt = int(wb[al(4 * N) + al(12 * room):][:4].view(np.int32)[0])
    valid = ids < E
    ro, _, _, rs = vo.sort_routing(np.where(valid, ids, E), 1)
    ref_tm = vo.tile_meta(rs[rs < E], E, 16)
    assert nt == len(ref_tm) + 1                        # + one tile for the bad id
    assert np.array_equal(tm[:len(ref_tm)], ref_tm)
    assert tuple(tm[len(ref_tm)]) == (-1, N - 1, 1)
    starts = np.concatenate([[0], np.cumsum(np.bincount(rs, minlength=E + 1))])
    for ex in range(E + 1):                          # one segment per expert (+ bad ids)
        a, b = starts[ex], starts[ex + 1]
        assert sorted(order[a:b]) == sorted(ro[a:b])
    yn = _np(y)
    assert (yn[5] == 0).all()
    ref = vo.expert_gemv(x.float().cpu().numpy()[valid], ids[valid], m["codes"], m["codebook"],
                         m["scales"], 64)
    assert_close(yn[valid], ref, what="sort case")


def _narrow_rows(ids, E):
    """The device sort's choice for narrow tiles (restated): 8-row tiles when
    they cut the tile count by more than 1/21, else 4 (ids outside [0, E) in
    one bucket of their own)."""
    cnt = np.bincount(np.where((ids >= 0) & (ids < E), ids, E), minlength=E + 1)
    t4, t8 = int(((cnt + 3) // 4).sum()), int(((cnt + 7) // 8).sum())
    return 8 if 21 * t8 < 20 * t4 else 4


def _sort_records(work, N, E):
    """(tile records, tile count, tile rows chosen) from a grouped call's
    workspace: order [N] int32, records [room][3], then the count and the
    rows (256-byte aligned sections; room for 4-row tiles)."""
    wb = work.cpu().numpy()
    al = lambda v: (v + 255) & ~255
    room = (N + 3) // 4 + min(N, E + 1)
    tm = wb[al(4 * N):al(4 * N) + 12 * room].view(np.int32).reshape(-1, 3)
    nt, rows = (int(v) for v in wb[al(4 * N) + al(12 * room):][:8].view(np.int32))
    return tm[:nt], nt, rows


def test_grouped_gemm_narrow_tiles():
    """A d8 K16384 routing with <= 2 pairs per expert on average sorts into
    tiles of <= 4 rows (the oracle's tile_meta at 4), one expert on every
    token spanning several tiles, a skipzero row table on the same routing;
    fp32 outputs against the oracle, dead rows exact zeros."""
    from vqlab_amd import _lib as L, _torch as Tt, vq_switch as VS
    from vq_cases import skipzero
    print("grouped gemm narrow tiles", flush=True)
    rng = np.random.default_rng(41)
    E, OUT, IN, T, k = 64, 640, 1024, 11, 10              # N = 110 <= 2 E
    m = make_module(rng, E, OUT, IN, 8, 16384, dead_frac=0.2)
    codes, cb, sc = to_device(m)
    ids = _routes(rng, T, k, E)
    for t in range(T):                                  # expert 5 on every token
        if 5 not in ids[t]:
            ids[t, 0] = 5
    assert all(len(np.unique(r)) == k for r in ids)
    ids = ids.reshape(-1)
    assert (ids == 5).sum() == T
    N = T * k
    x = _x(rng, T, IN)
    e = torch.from_numpy(ids.astype(np.int32)).cuda()
    keep = []
    w = Tt.weights(codes, cb, sc, 64, m["pack_bits"], IN, keep=keep)
    ws = ctypes.c_size_t()
    L.check(L.lib().vqk_grouped_gemm_workspace(ctypes.byref(w), N, ctypes.byref(ws)))
    work = torch.zeros(ws.value, dtype=torch.uint8, device="cuda")
    y = torch.empty((N, OUT), dtype=torch.float32, device="cuda")
    L.check(L.lib().vqk_grouped_gemm(ctypes.byref(w), Tt.ptr(x), L.VQK_BF16, T, Tt.ptr(e), N, k,
                                     Tt.ptr(y), L.VQK_F32, Tt.ptr(work), ws.value, Tt.stream()))
    torch.cuda.synchronize()
    _, _, _, rs = vo.sort_routing(ids, 1)
    ref_tm = vo.tile_meta(rs, E, 4)
    tm, nt, rows = _sort_records(work, N, E)
    assert rows == 4 == _narrow_rows(ids, E)
    assert nt == len(ref_tm) and np.array_equal(tm, ref_tm)
    assert (ref_tm[ref_tm[:, 0] == 5][:, 2] == [4, 4, 3]).all()
    ref = vo.expert_gemv(_x16(x), ids, m["codes"], m["codebook"], m["scales"], 64, xkrep=k)
    assert_close(_np(y), ref, what="narrow tiles")
    sz, rt = skipzero(m)
    zc = torch.from_numpy(sz["sz_codes"].view(np.int32)).cuda()
    zs = torch.from_numpy(sz["sz_scales"]).cuda()
    yc = VS._gemmseg(x, e, zc, cb, zs, m["pack_bits"], IN, k, torch.from_numpy(rt).cuda(),
                     out_dtype=torch.float32)
    dead = rt[ids] < 0
    assert dead.any() and (_np(yc)[dead] == 0).all()
    assert torch.equal(yc[torch.from_numpy(~dead).cuda()], y[torch.from_numpy(~dead).cuda()])


@pytest.mark.parametrize("skew", ["capped", "mixed"])
def test_grouped_gemm_narrow_tiles_of_eight(skew):
    """Routings that put 5-8 pairs on most touched experts ("capped", as an
    MTP verify batch drawn with 1..8 tokens per expert) make the sort choose
    8-row tiles (one decode of each expert's rows instead of two); "mixed"
    adds a tail of single-pair experts and one expert on every token (tiles of
    8, 8, ..., rest). Tile records equal the oracle's tile_meta at the chosen
    size, the choice equals the restated rule, outputs match the oracle, and a
    skipzero row table on the same routing gives the same live rows."""
    from vqlab_amd import _lib as L, _torch as Tt, vq_switch as VS
    from vq_cases import skipzero
    print(f"grouped gemm 8-row tiles {skew}", flush=True)
    rng = np.random.default_rng(52 if skew == "capped" else 53)
    E, OUT, IN, T, k = 160, 640, 1024, 40, 8               # N = 320 <= 2 E: narrow
    m = make_module(rng, E, OUT, IN, 8, 16384, dead_frac=0.2)
    codes, cb, sc = to_device(m)
    if skew == "capped":
        ids = _routes(rng, T, k, E, lo=5, hi=8)
    else:
        ids = _routes(rng, T, k, E, lo=4, hi=8)
        for t in range(T):                               # expert 7 on every token
            if 7 not in ids[t]:
                ids[t, 1] = 7
    assert all(len(np.unique(r)) == k for r in ids)
    ids = ids.reshape(-1)
    N = T * k
    assert N <= 2 * E and _narrow_rows(ids, E) == 8     # narrow tiles, and 8 rows pay
    x = _x(rng, T, IN)
    e = torch.from_numpy(ids.astype(np.int32)).cuda()
    keep = []
    w = Tt.weights(codes, cb, sc, 64, m["pack_bits"], IN, keep=keep)
    ws = ctypes.c_size_t()
    L.check(L.lib().vqk_grouped_gemm_workspace(ctypes.byref(w), N, ctypes.byref(ws)))
    work = torch.zeros(ws.value, dtype=torch.uint8, device="cuda")
    y = torch.empty((N, OUT), dtype=torch.float32, device="cuda")
    L.check(L.lib().vqk_grouped_gemm(ctypes.byref(w), Tt.ptr(x), L.VQK_BF16, T, Tt.ptr(e), N, k,
                                     Tt.ptr(y), L.VQK_F32, Tt.ptr(work), ws.value, Tt.stream()))
    torch.cuda.synchronize()
    _, _, _, rs = vo.sort_routing(ids, 1)
    ref_tm = vo.tile_meta(rs, E, 8)
    tm, nt, rows = _sort_records(work, N, E)
    assert rows == 8
    assert nt == len(ref_tm) and np.array_equal(tm, ref_tm)
    assert ref_tm[:, 2].max() > 4 and len(ref_tm) < len(vo.tile_meta(rs, E, 4))
    if skew == "mixed":
        assert (ref_tm[ref_tm[:, 0] == 7][:, 2] == [8] * (T // 8) + ([T % 8] if T % 8 else [])).all()
    ref = vo.expert_gemv(_x16(x), ids, m["codes"], m["codebook"], m["scales"], 64, xkrep=k)
    assert_close(_np(y), ref, what=f"8-row tiles {skew}")
    sz, rt = skipzero(m)
    zc = torch.from_numpy(sz["sz_codes"].view(np.int32)).cuda()
    zs = torch.from_numpy(sz["sz_scales"]).cuda()
    yc = VS._gemmseg(x, e, zc, cb, zs, m["pack_bits"], IN, k, torch.from_numpy(rt).cuda(),
                     out_dtype=torch.float32)
    dead = rt[ids] < 0
    assert dead.any() and (_np(yc)[dead] == 0).all()
    assert torch.equal(yc[torch.from_numpy(~dead).cuda()], y[torch.from_numpy(~dead).cuda()])


def test_grouped_gemm_errors():
    from vqlab_amd import _lib as L, _torch as Tt
    rng = np.random.default_rng(25)
    m = make_module(rng, 4, 128, 256, 4, 256)
    codes, cb, sc = to_device(m)
    keep = []
    w = Tt.weights(codes, cb, sc, 64, 8, 256, keep=keep)
    x = torch.zeros((4, 256), dtype=torch.bfloat16, device="cuda")
    e = torch.zeros(8, dtype=torch.int32, device="cuda")
    y = torch.empty((8, 128), dtype=torch.bfloat16, device="cuda")
    ws = ctypes.c_size_t()
    L.check(L.lib().vqk_grouped_gemm_workspace(ctypes.byref(w), 8, ctypes.byref(ws)))
    work = torch.empty(ws.value, dtype=torch.uint8, device="cuda")
    lib = L.lib()
    assert lib.vqk_grouped_gemm(ctypes.byref(w), Tt.ptr(x), L.VQK_BF16, 4, Tt.ptr(e), 8, 2,
                                Tt.ptr(y), L.VQK_BF16, Tt.ptr(work), ws.value - 1,
                                Tt.stream()) == L.VQK_ENOSPACE
    assert lib.vqk_grouped_gemm(ctypes.byref(w), Tt.ptr(x), L.VQK_BF16, 4, Tt.ptr(e), 8, 3,
                                Tt.ptr(y), L.VQK_BF16, Tt.ptr(work), ws.value,
                                Tt.stream()) == L.VQK_EINVAL
    # a workspace that is not 16-byte aligned is refused before any launch
    big = torch.empty(ws.value + 16, dtype=torch.uint8, device="cuda")
    assert lib.vqk_grouped_gemm(ctypes.byref(w), Tt.ptr(x), L.VQK_BF16, 4, Tt.ptr(e), 8, 2,
                                Tt.ptr(y), L.VQK_BF16, ctypes.c_void_p(big.data_ptr() + 8),
                                ws.value, Tt.stream()) == L.VQK_EINVAL
    assert lib.vqk_grouped_gemm(ctypes.byref(w), Tt.ptr(x), L.VQK_BF16, 4, Tt.ptr(e), 8, 2,
                                Tt.ptr(y), L.VQK_BF16, Tt.ptr(work), ws.value,
                                Tt.stream()) == L.VQK_OK


def test_switch_linear_prefill_takes_grouped_gemm():
    """N > VQ_FUSED_MAX_N pairs: VQSwitchLinear runs the grouped GEMM."""
    from vqlab_amd import vq_switch as VS
    print("switch linear prefill", flush=True)
    rng = np.random.default_rng(26)
    E, OUT, IN, T, k = 16, 256, 1024, 80, 8
    m = make_module(rng, E, OUT, IN, 4, 4096)
    codes, cb, sc = to_device(m)
    mod = VS.VQSwitchLinear(codes, cb, sc, pack_bits=12, in_features=IN)
    assert VS.gemmseg_fits(4, 4096, 64, 12, IN)
    ids = _routes(rng, T, k, E)
    x = _x(rng, T, IN)
    idx = torch.from_numpy(ids.astype(np.int32)).cuda()
    y = mod(x[:, None, None, :], idx)
    assert y.shape == (T, k, 1, OUT)
    ref = vo.expert_gemv(_x16(x), ids.reshape(-1), m["codes"], m["codebook"], m["scales"], 64,
                         xkrep=k)
    assert_close(_np(y).reshape(T * k, OUT), ref, what="prefill module")
