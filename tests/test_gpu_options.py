"""Options and output rounding through the C ABI.

VQK_VIA_F16 (the reference's default decode arithmetic: fused kernels return
fp16 that the caller casts to x's dtype, vq_switch.py:5306-5308, 5423) must
give exactly the fp32 result rounded to fp16 and then to y's type, on every
entry point that writes activations. vqk_switch_apply / vqk_linear_apply
must run the same kernels as the direct entry points they dispatch to
(vq_switch.py:5284-5423, vq_dense.py:347-441), with the options deciding
path and rounding.
"""
import ctypes

import numpy as np
import pytest

from vq_cases import make_module, to_device

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _via(y32):
    """fp32 -> fp16 -> bf16, both round-to-nearest-even (torch's casts)."""
    return y32.to(torch.float16).to(torch.bfloat16)


def _x(rng, n, k):
    return torch.from_numpy(rng.standard_normal((n, k)).astype(np.float32)).to("cuda", torch.bfloat16)


@pytest.fixture(scope="module")
def mod():
    from vqlab_amd import _torch as Tt
    rng = np.random.default_rng(41)
    E, OUT, IN = 16, 384, 1024
    m = make_module(rng, E, OUT, IN, 4, 4096)
    codes, cb, sc = to_device(m)
    keep = []
    w = Tt.weights(codes, cb, sc, 64, m["pack_bits"], IN, keep=keep)
    w1 = Tt.weights(codes[0], cb, sc[0], 64, m["pack_bits"], IN, keep=keep)
    return {"w": w, "w1": w1, "keep": keep, "E": E, "OUT": OUT, "IN": IN, "rng": rng,
            "codes": codes, "cb": cb, "sc": sc, "bits": m["pack_bits"]}


def _run(fn, y_dtype, flag, shape):
    from vqlab_amd import _lib as L, _torch as Tt
    y = torch.empty(shape, dtype=y_dtype, device="cuda")
    fn(y, Tt.ACT_TYPES[y_dtype] | flag)
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("path", ["expert_gemv", "grouped_gemm", "dense_gemv", "dense_gemm"])
def test_via_f16_is_exactly_fp16_then_bf16(mod, path):
    from vqlab_amd import _lib as L, _torch as Tt
    print(f"VIA_F16 {path}", flush=True)
    lib, rng, OUT, IN, E = L.lib(), mod["rng"], mod["OUT"], mod["IN"], mod["E"]
    T, k = 24, 4
    x = _x(rng, T, IN)
    e = torch.from_numpy(rng.integers(0, E, T * k).astype(np.int32)).cuda()
    if path == "expert_gemv":
        shape = (T * k, OUT)
        fn = lambda y, yt: L.check(lib.vqk_moe_expert_gemv(ctypes.byref(mod["w"]), Tt.ptr(x), L.VQK_BF16,
                                                           T, Tt.ptr(e), T * k, k, Tt.ptr(y), yt,
                                                           Tt.stream()))
    elif path == "grouped_gemm":
        shape = (T * k, OUT)
        ws = ctypes.c_size_t()
        L.check(lib.vqk_grouped_gemm_workspace(ctypes.byref(mod["w"]), T * k, ctypes.byref(ws)))
        work = torch.empty(ws.value, dtype=torch.uint8, device="cuda")
        fn = lambda y, yt: L.check(lib.vqk_grouped_gemm(ctypes.byref(mod["w"]), Tt.ptr(x), L.VQK_BF16, T,
                                                        Tt.ptr(e), T * k, k, Tt.ptr(y), yt, Tt.ptr(work),
                                                        ws.value, Tt.stream()))
    elif path == "dense_gemv":
        shape = (4, OUT)
        fn = lambda y, yt: L.check(lib.vqk_dense_gemv(ctypes.byref(mod["w1"]), Tt.ptr(x), L.VQK_BF16, 4,
                                                      Tt.ptr(y), yt, Tt.stream()))
    else:
        x = _x(rng, 100, IN)
        shape = (100, OUT)
        ws = ctypes.c_size_t()
        L.check(lib.vqk_dense_gemm_workspace(ctypes.byref(mod["w1"]), 100, ctypes.byref(ws)))
        work = torch.empty(ws.value, dtype=torch.uint8, device="cuda")
        fn = lambda y, yt: L.check(lib.vqk_dense_gemm(ctypes.byref(mod["w1"]), Tt.ptr(x), L.VQK_BF16, 100,
                                                      Tt.ptr(y), yt, Tt.ptr(work), ws.value, Tt.stream()))
    y32 = _run(fn, torch.float32, 0, shape)
    yv = _run(fn, torch.bfloat16, L.VQK_VIA_F16, shape)
    yd = _run(fn, torch.bfloat16, 0, shape)
    assert torch.equal(yv.view(torch.int16), _via(y32).view(torch.int16))
    assert torch.equal(yd.view(torch.int16), y32.to(torch.bfloat16).view(torch.int16))
    yv32 = _run(fn, torch.float32, L.VQK_VIA_F16, shape)
    assert torch.equal(yv32, y32.to(torch.float16).float())
    # bits other than the flag are refused before launch
    y = torch.empty(shape, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        fn(y, L.VQK_BF16 | 0x200)


def test_switch_apply_paths_and_rounding(mod):
    from vqlab_amd import _lib as L, _torch as Tt
    print("switch apply", flush=True)
    lib, rng, OUT, IN, E = L.lib(), mod["rng"], mod["OUT"], mod["IN"], mod["E"]
    T, k = 6, 4
    x = _x(rng, T, IN)
    e = torch.from_numpy(rng.integers(0, E, T * k).astype(np.int32)).cuda()

    def apply(opts, y_dtype=torch.bfloat16):
        ws = ctypes.c_size_t()
        L.check(lib.vqk_switch_apply_workspace(ctypes.byref(mod["w"]), T * k, ctypes.byref(opts),
                                               ctypes.byref(ws)))
        work = torch.empty(max(1, ws.value), dtype=torch.uint8, device="cuda")
        y = torch.empty((T * k, OUT), dtype=y_dtype, device="cuda")
        L.check(lib.vqk_switch_apply(ctypes.byref(mod["w"]), Tt.ptr(x), L.VQK_BF16, T, Tt.ptr(e), T * k,
                                     k, Tt.ptr(y), Tt.ACT_TYPES[y_dtype], Tt.ptr(work), ws.value,
                                     ctypes.byref(opts), Tt.stream()))
        torch.cuda.synchronize()
        return y, ws.value

    def direct(grouped):
        y = torch.empty((T * k, OUT), dtype=torch.float32, device="cuda")
        if grouped:
            ws = ctypes.c_size_t()
            L.check(lib.vqk_grouped_gemm_workspace(ctypes.byref(mod["w"]), T * k, ctypes.byref(ws)))
            work = torch.empty(ws.value, dtype=torch.uint8, device="cuda")
            L.check(lib.vqk_grouped_gemm(ctypes.byref(mod["w"]), Tt.ptr(x), L.VQK_BF16, T, Tt.ptr(e),
                                         T * k, k, Tt.ptr(y), L.VQK_F32, Tt.ptr(work), ws.value,
                                         Tt.stream()))
        else:
            L.check(lib.vqk_moe_expert_gemv(ctypes.byref(mod["w"]), Tt.ptr(x), L.VQK_BF16, T, Tt.ptr(e),
                                            T * k, k, Tt.ptr(y), L.VQK_F32, Tt.stream()))
        torch.cuda.synchronize()
        return y

    gemv32, grp32 = direct(False), direct(True)
    y, ws = apply(L.options())                                  # 24 pairs: fused, via fp16
    assert ws == 0 and torch.equal(y.view(torch.int16), _via(gemv32).view(torch.int16))
    y, _ = apply(L.options(decode_bf16io=1))                    # fused, one rounding
    assert torch.equal(y.view(torch.int16), gemv32.to(torch.bfloat16).view(torch.int16))
    y, ws = apply(L.options(fused_max_n=8))                     # grouped, via fp16
    assert ws > 0 and torch.equal(y.view(torch.int16), _via(grp32).view(torch.int16))
    y, _ = apply(L.options(fused_max_n=8, prefill_bf16io=1))    # grouped, one rounding
    assert torch.equal(y.view(torch.int16), grp32.to(torch.bfloat16).view(torch.int16))
    # the wrapper: VQSwitchLinear with the module options (defaults here)
    from vqlab_amd import vq_switch as VS
    m = VS.VQSwitchLinear(mod["codes"], mod["cb"], mod["sc"], pack_bits=mod["bits"], in_features=IN)
    ym = m(x.reshape(T, 1, 1, IN), e.reshape(T, k))
    assert torch.equal(ym.reshape(T * k, OUT).view(torch.int16), _via(gemv32).view(torch.int16))


def test_linear_apply_paths(mod):
    from vqlab_amd import _lib as L, _torch as Tt
    from vqlab_amd import vq_dense as VD
    print("linear apply", flush=True)
    lib, rng, OUT, IN = L.lib(), mod["rng"], mod["OUT"], mod["IN"]
    for N in (8, 100):
        x = _x(rng, N, IN)
        yd = torch.empty((N, OUT), dtype=torch.bfloat16, device="cuda")
        if N <= 32 and lib.vqk_dense_fits(4096, IN, 64, 4):
            L.check(lib.vqk_dense_gemv(ctypes.byref(mod["w1"]), Tt.ptr(x), L.VQK_BF16, N, Tt.ptr(yd),
                                       L.VQK_BF16, Tt.stream()))
        else:
            ws = ctypes.c_size_t()
            L.check(lib.vqk_dense_gemm_workspace(ctypes.byref(mod["w1"]), N, ctypes.byref(ws)))
            work = torch.empty(ws.value, dtype=torch.uint8, device="cuda")
            L.check(lib.vqk_dense_gemm(ctypes.byref(mod["w1"]), Tt.ptr(x), L.VQK_BF16, N, Tt.ptr(yd),
                                       L.VQK_BF16, Tt.ptr(work), ws.value, Tt.stream()))
        lin = VD.VQLinear(mod["codes"][0], mod["cb"], mod["sc"][0], group_size=64,
                          pack_bits=mod["bits"], in_features=IN)
        y = lin(x)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), yd.view(torch.int16)), N
