"""Parity of the HIP kernels with the CPU oracle, through the C ABI.

Bit-exact: unpack, pack, dequantised weights (uint16 patterns). Tolerance
(rtol 2e-2, atol 1e-3 against the float64 decode-then-matmul oracle, the
north star's bar): the fused GEMVs. Shapes are the BASELINE.json configs'
row shapes (fewer experts where the expert count does not change what a
kernel computes), plus ragged / unaligned / skipzero / dtype edge cases.
"""
import numpy as np
import pytest

from oracle import vq_oracle as vo
from vq_cases import assert_close, make_module, skipzero, to_device

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _u16(t):
    return t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _np(t):
    return t.float().cpu().numpy()


# ------------------------------------------------------------ pack / unpack
@pytest.mark.parametrize("bits", list(range(1, 17)))
def test_unpack_pack_device(bits):
    from vqlab_amd import vq_pack
    rng = np.random.default_rng(100 + bits)
    for nsub in (32, 80, 512):
        print(f"unpack/pack bits={bits} nsub={nsub}", flush=True)
        codes = rng.integers(0, 1 << bits, (3, 5, nsub)).astype(np.uint16)
        packed = vo.pack(codes, bits)
        dp = torch.from_numpy(packed.view(np.int32)).cuda()
        got = vq_pack.unpack(dp, nsub, bits)
        torch.cuda.synchronize()
        g = got.cpu().numpy()
        g = g.view(np.uint16) if bits > 8 else g
        assert np.array_equal(g, codes)
        dc = torch.from_numpy(codes.view(np.int16)).cuda()
        rp = vq_pack.pack(dc, bits)
        assert np.array_equal(rp.cpu().numpy().view(np.uint32), packed)


def test_device_pack_matches_reference_golden():
    from golden import writer_fixture as wf
    from vqlab_amd import vq_pack
    gold = wf.golden()["pack"]["tensors"]
    for m, t in wf.vq_tensors().items():
        dc = torch.from_numpy(t["codes"].astype(np.int16)).cuda()
        got = vq_pack.pack(dc, 4).cpu().numpy().view(np.uint32)
        assert wf.sha16(got) == gold[m + ".codes"]["sha"], m


def test_codepack_device_round_trip():
    from vqlab_amd import codepack
    rng = np.random.default_rng(19)
    for k, bits in ((512, 9), (4096, 12), (16384, 14)):
        print(f"codepack device K={k}", flush=True)
        codes = rng.integers(0, k, (3, 4, 64)).astype(np.uint16)
        packed, b = codepack.pack_codes("m", torch.from_numpy(codes.view(np.int16)).cuda(), k)
        assert b == bits
        assert np.array_equal(packed.cpu().numpy().view(np.uint32), vo.pack(codes, bits))


# ----------------------------------------------------------------- dequant
@pytest.mark.parametrize("D", [2, 4, 8])
@pytest.mark.parametrize("K,packed", [(16, True), (256, False), (512, True), (4096, True),
                                      (16384, True), (65536, False), (1000, False)])
def test_wdec_bit_exact(D, K, packed):
    from vqlab_amd import vq_switch as VS
    print(f"wdec D={D} K={K} packed={packed}", flush=True)
    rng = np.random.default_rng(D * 7 + K)
    m = make_module(rng, 2, 24, 256, D, K, packed=packed and K & (K - 1) == 0)
    # special values: subnormal and negative-zero codebook rows, inf / nan / zero scales
    m["codebook"][0] = np.float16(2.0 ** -20)
    m["codebook"][1] = -0.0
    m["scales"][0, 0, 0] = np.inf
    m["scales"][0, 1, 1] = np.nan
    m["scales"][1, 2, :] = 0
    m["codes"][0, :3, :3] = [0, 1, 0]
    if m["pack_bits"]:
        m["stored"] = vo.pack(m["codes"], m["pack_bits"])
    else:
        m["stored"] = m["codes"].astype(np.uint8) if K <= 256 else m["codes"]
    codes, cb, sc = to_device(m)
    want = vo.dequant(m["codes"].reshape(48, -1), m["codebook"], m["scales"].reshape(48, -1), 64)
    got = VS.wdec_decode(codes, cb, sc, 48, 256, 64, m["pack_bits"])
    g, w = _u16(got), want.view(np.uint16)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got.float().cpu().numpy()), nan)
    assert np.array_equal(g[~nan], w[~nan])
    # a row slice: rows [r0, r0 + 10)
    part = VS.wdec_decode(codes, cb, sc, 10, 256, 64, m["pack_bits"], r0=30)
    assert np.array_equal(_u16(part), w[30:40])


@pytest.mark.parametrize("D", [2, 4, 8])
@pytest.mark.parametrize("rows,r0", [(1, 0), (3, 5), (7, 0), (13, 2), (48, 0)])
def test_wdec_special_products_ragged_rows(D, rows, r0):
    """Every fp16 product class the dequant can meet -- subnormal results and
    inputs, signed zeros, overflow to inf, RNE ties, inf / NaN / zero /
    subnormal scales -- at row counts that leave the last stride of rows
    partly filled and at row offsets: bit for bit (NaN positions by class)."""
    from vqlab_amd import vq_switch as VS
    print(f"wdec special products D={D} rows={rows} r0={r0}", flush=True)
    rng = np.random.default_rng(100 * D + rows + r0)
    K, IN, OUT = 16, 256, 64
    m = make_module(rng, 1, OUT, IN, D, K, packed=True)
    specials = np.array([2.0 ** -20, -0.0, 2.0 ** -24, 65504.0, -(2.0 ** -14), 1 + 2.0 ** -10,
                         0.5 + 2.0 ** -11, 3.0, -2.0 ** -23, 1.0, -1.5, 2.0 ** -14, 7.0, 0.0,
                         -65504.0, 2.0 ** -17], np.float16)
    cb = np.stack([np.roll(specials, i)[:K] for i in range(D)], axis=1)
    m["codebook"] = np.ascontiguousarray(cb.astype(np.float16))
    svals = np.array([np.inf, -np.inf, np.nan, 0.0, -0.0, 2.0 ** -24, 1.5, 1 + 2.0 ** -10,
                      1024.0, 0.75, 2.0 ** -10, 1.0], np.float16)
    m["scales"] = rng.choice(svals, m["scales"].shape).astype(np.float16)
    m["stored"] = vo.pack(m["codes"], m["pack_bits"])
    codes, cbd, sc = to_device(m)
    want = vo.dequant(m["codes"].reshape(OUT, -1), m["codebook"], m["scales"].reshape(OUT, -1),
                      64)[r0:r0 + rows]
    got = VS.wdec_decode(codes, cbd, sc, rows, IN, 64, m["pack_bits"], r0=r0)
    g, w = _u16(got), want.view(np.uint16)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got.float().cpu().numpy()), nan)
    assert np.array_equal(g[~nan], w[~nan])
    if rows < 13:
        return
    # the classes the case is meant to reach are all present
    wf = want[~nan].astype(np.float32)
    assert np.isinf(wf).any() and (wf == 0).any() and np.signbit(wf[wf == 0]).any()
    assert ((np.abs(wf) > 0) & (np.abs(wf) < 2.0 ** -14)).any()        # subnormal results


def test_decode_chunk_experts_and_skipzero():
    from vqlab_amd import vq_switch as VS
    rng = np.random.default_rng(5)
    m = make_module(rng, 6, 40, 512, 4, 4096, dead_frac=0.2)
    codes, cb, sc = to_device(m)
    eidx = torch.tensor([5, 0, 3, 3], dtype=torch.int32, device="cuda")
    got = VS._decode_chunk(codes, cb, sc, eidx, pack_bits=12, in_features=512)
    for i, e in enumerate([5, 0, 3, 3]):
        want = vo.dequant(m["codes"][e], m["codebook"], m["scales"][e], 64)
        assert np.array_equal(_u16(got[i]), want.view(np.uint16))
    sz, rt = skipzero(m)
    zc = torch.from_numpy(sz["sz_codes"].view(np.int32)).cuda()
    zs = torch.from_numpy(sz["sz_scales"]).cuda()
    rtd = torch.from_numpy(rt).cuda()
    got2 = VS._decode_chunk(zc, cb, zs, eidx, pack_bits=12, in_features=512, rowtbl=rtd)
    # live rows: byte for byte. Dead rows: +0 from the compact form; the
    # expanded form decodes fp16(0 * cb[0]), which is -0 where cb[0] < 0.
    live = (rt[[5, 0, 3, 3]] >= 0)
    assert np.array_equal(_u16(got2)[live], _u16(got)[live])
    assert (_u16(got2)[~live] == 0).all()
    assert (got[torch.from_numpy(~live).cuda()] == 0).all()


# -------------------------------------------------------------- dense GEMV
def _dense_case(rng, OUT, IN, D, K, G=64, packed=False, xdt=torch.bfloat16, N=1):
    m = make_module(rng, 1, OUT, IN, D, K, G=G, packed=packed)
    codes, cb, sc = to_device(m)
    x = torch.from_numpy(rng.standard_normal((N, IN)).astype(np.float32)).to("cuda", xdt)
    return m, codes[0], cb, sc[0], x


@pytest.mark.parametrize("case", [
    # (OUT, IN, D, K, G, packed): c1 is the first row
    (4096, 4096, 2, 256, 64, False),
    (512, 2048, 4, 4096, 64, True),
    (1024, 4096, 8, 16384, 64, True),
    (300, 1024, 8, 4096, 64, True),      # d8 K4096: 64 KB codebook table in LDS
    (96, 640, 8, 65536, 64, False),      # uint16 codes, NSUB 80: generic kernel
    (128, 512, 2, 512, 128, True),       # a group spans two blocks
    (64, 1024, 4, 256, 1024, False),     # one scale per row (G = IN)
    (70, 256, 4, 1000, 32, False),       # G=32 -> generic kernel, K not a power of 2
])
def test_dense_gemv(case):
    from vqlab_amd import vq_switch as VS
    OUT, IN, D, K, G, packed = case
    print(f"dense gemv {case}", flush=True)
    rng = np.random.default_rng(OUT + IN + D)
    m, codes, cb, sc, x = _dense_case(rng, OUT, IN, D, K, G, packed)
    y = VS._dense_fused(x, codes, cb, sc, pack_bits=m["pack_bits"], in_features=IN)
    assert y.dtype == x.dtype and y.shape == (1, OUT)
    w = vo.dequant(m["codes"][0], m["codebook"], m["scales"][0], G)
    ref = vo.decode_matmul(x.float().cpu().numpy(), w)
    assert_close(_np(y), ref, what=f"dense {case}")


@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16, torch.float32])
def test_dense_gemv_dtypes_and_batch(xdt):
    from vqlab_amd import vq_switch as VS
    rng = np.random.default_rng(3)
    m, codes, cb, sc, x = _dense_case(rng, 256, 2048, 4, 4096, packed=True, xdt=xdt, N=5)
    y = VS._dense_fused(x, codes, cb, sc, pack_bits=12, in_features=2048)
    assert y.dtype == xdt
    w = vo.dequant(m["codes"][0], m["codebook"], m["scales"][0], 64)
    assert_close(_np(y), vo.decode_matmul(x.float().cpu().numpy(), w), what=str(xdt))


# ------------------------------------------------------------ expert GEMV
@pytest.mark.parametrize("shape", [
    # (E, OUT, IN, D, K): c2 gate/up, c2 down, c3 gate/up, c3 down
    (16, 512, 2048, 4, 4096),
    (16, 2048, 512, 4, 4096),
    (12, 1024, 4096, 8, 16384),
    (12, 4096, 1024, 8, 16384),
])
def test_expert_gemv_baseline_shapes(shape):
    from vqlab_amd import vq_switch as VS
    E, OUT, IN, D, K = shape
    print(f"expert gemv {shape}", flush=True)
    rng = np.random.default_rng(sum(shape))
    m = make_module(rng, E, OUT, IN, D, K)
    codes, cb, sc = to_device(m)
    T, k = 2, 5
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).reshape(-1)
    x = torch.from_numpy(rng.standard_normal((T, IN)).astype(np.float32)).to("cuda", torch.bfloat16)
    eidx = torch.from_numpy(ids.astype(np.int32)).cuda()
    y = VS._fused(x, eidx, codes, cb, sc, pack_bits=m["pack_bits"], xkrep=k)
    ref = vo.expert_gemv(x.float().cpu().numpy(), ids, m["codes"], m["codebook"], m["scales"],
                         64, xkrep=k)
    assert_close(_np(y), ref, what=f"expert {shape}")
    # the historical contract (one x row per pair) computes the same bits
    xr = x.repeat_interleave(k, 0)
    y1 = VS._fused(xr, eidx, codes, cb, sc, pack_bits=m["pack_bits"])
    assert torch.equal(y1, y)


def test_expert_gemv_skipzero_equals_expanded():
    from vqlab_amd import vq_switch as VS
    rng = np.random.default_rng(9)
    m = make_module(rng, 8, 1024, 4096, 8, 16384, dead_frac=0.2)
    codes, cb, sc = to_device(m)
    sz, rt = skipzero(m)
    zc = torch.from_numpy(sz["sz_codes"].view(np.int32)).cuda()
    zs = torch.from_numpy(sz["sz_scales"]).cuda()
    rtd = torch.from_numpy(rt).cuda()
    ids = np.array([3, 7, 0, 3], np.int32)
    x = torch.from_numpy(rng.standard_normal((1, 4096)).astype(np.float32)).to("cuda", torch.bfloat16)
    e = torch.from_numpy(ids).cuda()
    ye = VS._fused(x, e, codes, cb, sc, pack_bits=14, xkrep=4)
    yc = VS._fused(x, e, zc, cb, zs, pack_bits=14, xkrep=4, rowtbl=rtd)
    assert torch.equal(ye, yc)
    dead = rt[ids] < 0
    assert (yc.float().cpu().numpy()[dead] == 0).all() and dead.any()
    ref = vo.expert_gemv(x.float().cpu().numpy(), ids, m["codes"], m["codebook"], m["scales"], 64,
                         xkrep=4)
    assert_close(_np(yc), ref, what="skipzero")


def test_expert_gemv_unpacked_and_bad_ids():
    from vqlab_amd import vq_switch as VS
    rng = np.random.default_rng(11)
    m = make_module(rng, 4, 256, 1024, 4, 256, packed=False)
    codes, cb, sc = to_device(m)
    x = torch.from_numpy(rng.standard_normal((3, 1024)).astype(np.float32)).to("cuda", torch.float16)
    ids = np.array([1, 3, 9], np.int32)            # 9 is outside [0, E): zeros, no fault
    y = VS._fused(x, torch.from_numpy(ids).cuda(), codes, cb, sc)
    ref = vo.expert_gemv(x.float().cpu().numpy(), ids[:2], m["codes"], m["codebook"],
                         m["scales"], 64)
    assert_close(_np(y[:2]), ref, what="u8 d4")
    assert (y[2] == 0).all()


def test_f32_to_bf16_conversion_bits():
    """The library's fp32 -> bf16 conversion (every bf16 output and weight)
    against the oracle's bit formulation: every sign and exponent with the
    mantissas at and around each rounding boundary (ties to even, carries into
    the exponent, the largest finite values, denormals), signalling and quiet
    NaN payloads, and 2^20 random patterns."""
    from vq_cases import hooks
    from vqlab_amd import _torch as TT
    rng = np.random.default_rng(5)
    se = (np.arange(512, dtype=np.uint32) << 23)
    mant = np.uint32([0, 1, 0x7FFF, 0x8000, 0x8001, 0xFFFF, 0x10000, 0x17FFF, 0x18000, 0x18001,
                      0x3FFFFF, 0x400000, 0x400001, 0x7F7FFF, 0x7F8000, 0x7FFFFF])
    mant = np.concatenate([mant, rng.integers(0, 1 << 23, 48, dtype=np.uint64).astype(np.uint32)])
    grid = (se[:, None] | mant[None, :]).reshape(-1)
    rand = rng.integers(0, 2**32, 1 << 20, dtype=np.uint64).astype(np.uint32)
    u = np.concatenate([grid, rand])
    x = torch.from_numpy(u.view(np.int32)).cuda().view(torch.float32)
    y = torch.empty(u.size, dtype=torch.int16, device="cuda")
    assert hooks().vqk__test_f32_to_bf16(x.data_ptr(), y.data_ptr(), u.size, TT.stream(x.device)) == 0
    got = y.cpu().numpy().view(np.uint16)
    want = vo.f32_to_bf16_bits(u)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, [(hex(int(u[i])), hex(int(got[i])), hex(int(want[i]))) for i in bad[:5]]


# ------------------------------------------------- wide x (VQK_X_KEEP, d=8)
def _wide_x(rng, IN):
    """Two bf16 token rows that fp16 staging cannot hold: row 0 reaches
    |x| = 4e5 (fp16 overflows above 65504), row 1 lies in fp16's subnormal
    range (1e-7 .. 1e-6, one to four significant bits left)."""
    sgn = np.where(rng.random((2, IN)) < 0.5, -1.0, 1.0)
    big = sgn[0] * np.exp(rng.uniform(0.0, np.log(4e5), IN))
    tiny = sgn[1] * np.exp(rng.uniform(np.log(1e-7), np.log(1e-6), IN))
    return torch.from_numpy(np.stack([big, tiny]).astype(np.float32)).to("cuda", torch.bfloat16)


def _float_staged(D, K, packed):
    """The reference's kernels that take bf16 x unrounded under
    VQ_DECODE_BF16IO: unpacked d4 with K <= 1024 (`_SRC_FUSED`,
    vq_switch.py:106-150, 3172-3175), d8 with K > 1024 (`_D8_TG_MAX_K`,
    2781; 153-237, 1316-1354, 1424-1660)."""
    return (D == 8 and K > 1024) or (D == 4 and not packed and K <= 1024)


@pytest.mark.parametrize("case", [
    # (D, E, OUT, IN, K, G, packed): c3 gate/up rows (14-bit table partly in
    # LDS, 4 scale groups per block); a 12-bit table in LDS with groups of two
    # blocks; 13 bits at 64 blocks per row (the fp16 kernels' LDS cannot hold
    # that table part and row: they take the generic kernel); d8 with a
    # 256-entry table (the reference's half-staged d8 kernel: the dispatch
    # rounds) on ragged unpacked rows (generic kernel); unpacked d4 with
    # uint16 and uint8 codes (the reference's float-staged d4 kernel); packed
    # ragged d4 (half-staged in the reference; generic wide-x kernel here)
    (8, 6, 1024, 4096, 16384, 64, True),
    (8, 4, 512, 2048, 4096, 512, True),
    (8, 3, 128, 16384, 8192, 64, True),
    (8, 3, 300, 1000, 256, 8, False),
    (4, 6, 512, 2048, 1024, 64, False),
    (4, 4, 256, 1024, 256, 64, False),
    (4, 3, 200, 1000, 1024, 8, True),
])
def test_expert_gemv_wide_x(case):
    """VQK_X_KEEP: bf16 x beyond fp16's range and below its normal range
    enters the GEMV unrounded, fp32 products with the widened table, as the
    reference's float-staged kernels take it under VQ_DECODE_BF16IO
    (vq_switch.py:4412-4417). Bar: |y - ref| <= 3e-5 * (|x| @ |W|^T) against
    the float64 fused formula (oracle weights="exact"), an fp32 accumulation
    bar that fp16 staging of either row misses (checked). The dispatch sets
    the flag exactly where the reference's kernel stages x as float."""
    import ctypes
    from vqlab_amd import _lib as L, _torch as TT, vq_switch as VS
    D, E, OUT, IN, K, G, packed = case
    print(f"wide x {case}", flush=True)
    rng = np.random.default_rng(sum(case[:6]))
    m = make_module(rng, E, OUT, IN, D, K, G=G, packed=packed)
    codes, cb, sc = to_device(m)
    x = _wide_x(rng, IN)
    k = 3
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(2)]).reshape(-1).astype(np.int32)
    eidx = torch.from_numpy(ids).cuda()
    xf = x.float().cpu().numpy()
    ref = vo.expert_gemv(xf, ids, m["codes"], m["codebook"], m["scales"], G, xkrep=k,
                         weights="exact")
    absref = vo.expert_gemv(np.abs(xf), ids, m["codes"], np.abs(m["codebook"]), m["scales"], G,
                            xkrep=k, weights="exact")
    bar = 3e-5 * absref
    keep = []
    w = TT.weights(codes, cb, sc, G, m["pack_bits"], IN if packed else None, keep=keep)

    def run(xt):
        y = torch.empty((2 * k, OUT), dtype=torch.float32, device="cuda")
        L.check(L.lib().vqk_moe_expert_gemv(ctypes.byref(w), TT.ptr(x), xt, 2, TT.ptr(eidx), 2 * k,
                                            k, TT.ptr(y), L.VQK_F32, TT.stream(x.device)), "wide x")
        return y

    yt = run(L.VQK_BF16 | L.VQK_X_KEEP)
    y = yt.cpu().numpy().astype(np.float64)
    err = np.abs(y - ref)
    i = np.unravel_index(np.argmax(err - bar), err.shape)
    assert np.isfinite(y).all() and (err <= bar).all(), (i, y[i], ref[i], bar[i])
    # the fp16-staged kernel misses the bar: row 0 overflows, row 1 loses bits
    y16t = run(L.VQK_BF16)
    y16 = y16t.cpu().numpy().astype(np.float64)
    assert not np.isfinite(y16[:k]).all()
    assert (np.abs(y16[k:] - ref[k:]) > bar[k:]).any()
    # the dispatch under decode_bf16io: the flag where the reference stages x
    # as float, fp16 staging elsewhere; the out_dtype form runs the same kernel
    o = L.options(decode_bf16io=1, crowded_grouped=0)
    yo = VS._switch_apply(x, eidx, codes, cb, sc, m["pack_bits"], IN, k, out_dtype=torch.float32,
                          opts=o)
    yb = VS._switch_apply(x, eidx, codes, cb, sc, m["pack_bits"], IN, k, opts=o)
    assert yb.dtype == torch.bfloat16
    if _float_staged(D, K, packed):
        assert torch.equal(yo, yt)
        assert (np.abs(_np(yb) - ref) <= bar + np.abs(ref) * 2.0 ** -8).all()
    else:
        assert torch.equal(yo.view(torch.int32), y16t.view(torch.int32))   # bits: row 0 holds NaN
        assert not np.isfinite(_np(yb)[:k]).all()


@pytest.mark.parametrize("N", [1, 4, 32])
def test_dense_linear_d8_takes_bf16_x_unrounded(N):
    """VQLinear at d8: the reference has no fused d8 dense kernel (dense_fits
    refuses d8, vq_switch.py:3290-3306) and multiplies in x's dtype at every N
    (vq_dense.py:288-294); the GEMV rows (N <= 32) take bf16 x unrounded too,
    so activations beyond fp16's range stay finite. Bar as above."""
    from vqlab_amd.vq_dense import VQLinear
    print(f"dense d8 N={N}", flush=True)
    rng = np.random.default_rng(70 + N)
    OUT, IN, K = 384, 2048, 4096
    m = make_module(rng, 1, OUT, IN, 8, K)
    codes, cb, sc = to_device(m)
    lin = VQLinear(codes[0], cb, sc[0], group_size=64, pack_bits=m["pack_bits"], in_features=IN)
    x = torch.cat([_wide_x(rng, IN) for _ in range((N + 1) // 2)])[:N]
    y = lin(x)
    assert y.dtype == torch.bfloat16
    xf = x.float().cpu().numpy()
    ref = vo.expert_gemv(xf, np.zeros(N, np.int64), m["codes"], m["codebook"], m["scales"], 64,
                         weights="exact")
    absref = vo.expert_gemv(np.abs(xf), np.zeros(N, np.int64), m["codes"], np.abs(m["codebook"]),
                            m["scales"], 64, weights="exact")
    assert torch.isfinite(y).all()
    assert (np.abs(_np(y) - ref) <= 3e-5 * absref + np.abs(ref) * 2.0 ** -8).all()


def test_switch_linear_module_and_errors():
    from vqlab_amd import vq_switch as VS
    rng = np.random.default_rng(12)
    m = make_module(rng, 8, 512, 2048, 4, 4096)
    codes, cb, sc = to_device(m)
    mod = VS.VQSwitchLinear(codes, cb, sc, pack_bits=12, in_features=2048)
    assert (mod.input_dims, mod.output_dims, mod.num_experts) == (2048, 512, 8)
    x = torch.from_numpy(rng.standard_normal((1, 1, 2048)).astype(np.float32)).to("cuda", torch.bfloat16)
    idx = torch.tensor([[[1, 4, 6, 2]]], dtype=torch.int32, device="cuda")
    y = mod(x[:, :, None, None, :], idx)
    assert y.shape == (1, 1, 4, 1, 512) and y.dtype == torch.bfloat16
    ref = vo.expert_gemv(x.float().cpu().numpy().reshape(1, -1), [1, 4, 6, 2], m["codes"],
                         m["codebook"], m["scales"], 64, xkrep=4)
    assert_close(_np(y).reshape(4, 512), ref, what="module")
    mod.codebook = cb[:2048]
    with pytest.raises(RuntimeError, match="sharded"):
        mod(x[:, :, None, None, :], idx)
    with pytest.raises(ValueError):
        VS._fused(x.reshape(1, -1), idx.reshape(-1), codes[:, :, :100], cb, sc, pack_bits=12)
    with pytest.raises(ValueError):
        VS.VQSwitchLinear(codes, cb, sc, pack_bits=12)
