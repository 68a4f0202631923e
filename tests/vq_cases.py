"""Seeded synthetic VQ modules for the parity tests (numpy side; the oracle
consumes the unpacked codes, the kernels the stored form)."""
from __future__ import annotations

import numpy as np

from oracle import vq_oracle as vo


def make_module(rng, E, OUT, IN, D, K, G=64, packed=True, dead_frac=0.0, cb_std=0.02):
    """Codes uniform in [0, K), codebook ~N(0, cb_std) fp16, scales ~U(0.5,1.5)
    fp16 (BASELINE.json config conventions). packed=True stores log2(K)-bit
    words (any width); False stores uint8 (K <= 256) or uint16. dead_frac
    zeroes whole rows' scales (skipzero dead rows)."""
    nsub = IN // D
    codes = rng.integers(0, K, (E, OUT, nsub)).astype(np.uint16)
    cb = (rng.standard_normal((K, D)) * cb_std).astype(np.float16)
    sc = rng.uniform(0.5, 1.5, (E, OUT, IN // G)).astype(np.float16)
    if dead_frac:
        dead = rng.random((E, OUT)) < dead_frac
        sc[dead] = 0
        codes[dead] = 0
    if packed:
        bits = vo.bits_for_k(K) if K > 1 else 1
        stored = vo.pack(codes, bits)
        pack_bits = bits
    else:
        stored = codes.astype(np.uint8) if K <= 256 else codes
        pack_bits = 0
    return {"codes": codes, "stored": stored, "codebook": cb, "scales": sc, "pack_bits": pack_bits,
            "group": G, "E": E, "OUT": OUT, "IN": IN, "D": D, "K": K}


def to_device(m, dev="cuda"):
    import torch
    st = m["stored"]
    if st.dtype == np.uint32:
        codes = torch.from_numpy(st.view(np.int32)).to(dev)
    elif st.dtype == np.uint16:
        codes = torch.from_numpy(st.view(np.int16)).to(dev)
    else:
        codes = torch.from_numpy(st).to(dev)
    cb = torch.from_numpy(m["codebook"]).to(dev)
    sc = torch.from_numpy(m["scales"]).to(dev)
    return codes, cb, sc


def skipzero(m):
    """Compact form of m (dead rows dropped) + its row table."""
    sz = vo.skipzero_compact(m["stored"], m["scales"])
    rt = vo.skipzero_row_table(sz["sz_rowmask"], m["E"], m["OUT"])
    return sz, rt


def assert_close(y, ref, rtol=2e-2, atol=1e-3, what=""):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    assert y.shape == ref.shape, (y.shape, ref.shape)
    bad = ~np.isclose(y, ref, rtol=rtol, atol=atol)
    if bad.any():
        i = np.argwhere(bad)[0]
        raise AssertionError(f"{what}: {bad.sum()} of {bad.size} outside rtol={rtol} "
                             f"atol={atol}; first at {tuple(i)}: {y[tuple(i)]} vs {ref[tuple(i)]}")


def assert_rel_max(y, ref, tol=2e-2, what=""):
    """The reference's own acceptance metric (gate/kernel_accept.py:48-63):
    max |y - ref| / max(max |ref|, 1e-6) < tol. Used against the oracle's
    reference-rounding mode, whose bf16 intermediates put elements near zero
    outside any elementwise bar that exact arithmetic would meet."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    assert y.shape == ref.shape, (y.shape, ref.shape)
    rel = float(np.abs(y - ref).max() / max(float(np.abs(ref).max()), 1e-6)) if y.size else 0.0
    assert rel < tol, f"{what}: max-abs error {rel:.3e} of max |ref| (bar {tol})"


# ---------------------------------------------------------------- test hooks
_HOOKS = None


def hooks():
    """libvqk's test hooks (exported, deliberately not in include/vqk.h):
    vqk__test_l1_spins(n) -> previous bound of the one-launch layer's waits;
    vqk__test_l1_mode(m) -> previous mode (0 one launch where it applies,
    1 never); vqk__test_moe_path(desc*, T, int32*) -> status, the path a layer
    call takes (0 two fused kernels, 1 sliced GEMVs, 2 grouped, 3 one launch);
    vqk__test_f32_to_bf16(x*, y*, n, stream) -> status, the library's fp32 ->
    bf16 conversion applied to n device values."""
    global _HOOKS
    if _HOOKS is None:
        import ctypes
        from vqlab_amd import _lib as L
        lib = L.lib()
        for name, res, args in (("vqk__test_l1_spins", ctypes.c_int, [ctypes.c_int]),
                                ("vqk__test_l1_mode", ctypes.c_int, [ctypes.c_int]),
                                ("vqk__test_moe_path", ctypes.c_int32,
                                 [ctypes.POINTER(L.VQKMoeDesc), ctypes.c_int64,
                                  ctypes.POINTER(ctypes.c_int32)]),
                                ("vqk__test_f32_to_bf16", ctypes.c_int,
                                 [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                  ctypes.c_void_p])):
            f = getattr(lib, name)
            f.restype, f.argtypes = res, args
        _HOOKS = lib
    return _HOOKS


PATH_FUSED, PATH_SLICED, PATH_GROUPED, PATH_ONE_LAUNCH = range(4)


def moe_path(blk, T):
    """The path vqk_moe_decode_layer takes for block `blk` at T tokens."""
    import ctypes
    from vqlab_amd import _lib as L
    keep = []
    d = blk._fused_desc(keep)
    p = ctypes.c_int32(-1)
    L.check(hooks().vqk__test_moe_path(ctypes.byref(d), int(T), ctypes.byref(p)))
    return p.value


class two_kernels:
    """Context: every layer call planned inside takes the two-kernel form
    where it would have taken one launch."""

    def __enter__(self):
        self._prev = hooks().vqk__test_l1_mode(1)
        return self

    def __exit__(self, *exc):
        hooks().vqk__test_l1_mode(self._prev)
        return False


class l1_spins:
    """Context: the one-launch layer's waits give up after n rounds."""

    def __init__(self, n):
        self.n = n

    def __enter__(self):
        self._prev = hooks().vqk__test_l1_spins(self.n)
        return self

    def __exit__(self, *exc):
        hooks().vqk__test_l1_spins(self._prev)
        return False
