"""The C ABI without a GPU: libvqk.so loads, exports every function
include/vqk.h declares, and its host-side logic (widths, host pack/unpack,
predicates, row table, argument validation) agrees with the oracle. Nothing
here launches a kernel: every error path below is refused on the host."""
import ctypes
import pathlib
import re

import numpy as np
import pytest

from oracle import vq_oracle as vo

ROOT = pathlib.Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def L():
    from vqlab_amd import _lib
    return _lib


def _declared():
    txt = (ROOT / "include" / "vqk.h").read_text()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(vqk_\w+)\s*\(", txt)))


def test_exports_every_declared_symbol(L):
    lib = L.lib()
    names = _declared()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(L.SIGNATURES), set(names) ^ set(L.SIGNATURES)


def test_widths(L):
    from vqlab_amd import vq_pack
    for k in (2, 16, 256, 4096, 16384, 65536):
        assert vq_pack.bits_for_k(k) == vo.bits_for_k(k)
    with pytest.raises(AssertionError):
        vq_pack.bits_for_k(3000)
    for nsub, bits in ((512, 12), (128, 12), (512, 14), (128, 14), (80, 14), (640, 16)):
        assert vq_pack.words_per_row(nsub, bits) == vo.words_per_row(nsub, bits)
    b = ctypes.c_int32()
    for k, nsub, un in ((256, 512, 0), (4096, 512, 0), (4096, 80, 0), (4096, 80, 1), (65536, 64, 0)):
        assert L.lib().vqk_pack_bits_for(k, nsub, un, ctypes.byref(b)) == 0
        assert b.value == vo.pack_bits_for(k, nsub, bool(un))


@pytest.mark.parametrize("bits", list(range(1, 17)))
def test_host_pack_unpack_vs_oracle(L, bits):
    from vqlab_amd import vq_pack
    rng = np.random.default_rng(bits)
    for nsub in (32, 80, 96):
        codes = rng.integers(0, 1 << bits, (2, 3, nsub)).astype(np.uint16)
        p = vq_pack.pack(codes, bits)
        assert np.array_equal(p, vo.pack(codes, bits))
        u = vq_pack.unpack(p, nsub, bits)
        assert u.dtype == (np.uint8 if bits <= 8 else np.uint16)
        assert np.array_equal(u, codes)
    with pytest.raises(AssertionError):
        vq_pack.pack(np.full((1, 1, 32), 1 << bits, np.uint32), bits)


def test_codepack_rule_and_round_trip(L, monkeypatch):
    """codepack.pack_codes (codepack.py:33-52) on the reference's own
    fit-pack geometry (tests/test_fit_pack.py:22, 79-99): gate d4 K512 packs
    to 9-bit uint32 words, up d4 K256 stays byte-aligned; a packer whose
    output does not round-trip stops the process."""
    from vqlab_amd import codepack, vq_pack
    rng = np.random.default_rng(9)
    E, I, NSUB = 2, 8, 128 // 4
    gate = rng.integers(0, 512, (E, I, NSUB)).astype(np.uint16)
    up = rng.integers(0, 256, (E, I, NSUB)).astype(np.uint8)
    pg, bg = codepack.pack_codes("gate_proj", gate, 512)
    assert bg == 9 and pg.dtype == np.uint32
    assert np.array_equal(pg, vo.pack(gate, 9))
    pu, bu = codepack.pack_codes("up_proj", up, 256)
    assert bu == 0 and pu is up
    odd = rng.integers(0, 512, (1, 2, 40)).astype(np.uint16)       # NSUB % 32 != 0
    assert codepack.pack_codes("x", odd, 512)[1] == 0
    assert codepack.pack_codes("x", odd, 512, pack_unaligned=True)[1] == 9
    for k, nsub, un in ((256, 512, 0), (4096, 512, 0), (4096, 80, 0), (4096, 80, 1), (65536, 64, 0)):
        assert codepack.pack_bits_for(k, nsub, bool(un)) == vo.pack_bits_for(k, nsub, bool(un))
    real = vq_pack.unpack
    monkeypatch.setattr(vq_pack, "unpack", lambda p, n, b: real(p, n, b) ^ 1)
    with pytest.raises(SystemExit):
        codepack.pack_codes("gate_proj", gate, 512)


def test_host_pack_matches_reference_golden(L):
    from golden import writer_fixture as wf
    from vqlab_amd import vq_pack
    gold = wf.golden()["pack"]["tensors"]
    for m, t in wf.vq_tensors().items():
        assert wf.sha16(vq_pack.pack(t["codes"], 4)) == gold[m + ".codes"]["sha"]


def test_row_table_host_vs_oracle(L):
    from vqlab_amd import vq_switch as VS
    rng = np.random.default_rng(2)
    E, OUT = 7, 45
    live = rng.random((E, OUT)) > 0.3
    rm = np.packbits(live, axis=-1, bitorder="little")
    t = VS.skipzero_row_table(rm, E, OUT).numpy()
    assert np.array_equal(t, vo.skipzero_row_table(rm, E, OUT))


def test_predicates(L):
    from vqlab_amd import vq_switch as VS
    assert VS.dense_fits(256, 4096, 64, 2) and VS.dense_fits(65536, 5120, 64, 8)
    assert not VS.dense_fits(256, 4096, 64, 3)
    assert not VS.dense_fits(256, 4096, 48, 8)      # 48 does not divide IN
    assert not VS.dense_fits(256, 4096, 4, 8)       # a group smaller than one subvector
    assert VS.wdec_fits(4, 512, 64, 12) and not VS.wdec_fits(3, 512, 64, 12)
    # the grouped GEMM: d 2/4/8, up to 16-bit codes (0 = unpacked), any K
    # that 16 bits index, IN a whole number of scale groups
    assert VS.gemmseg_fits(8, 16384, 64, 14, 4096) and VS.gemmseg_fits(2, 256, 64, 0, 2048)
    assert VS.gemmseg_fits(8, 65536, 64, 16, 640)
    assert not VS.gemmseg_fits(3, 4096, 64, 12, 2048)
    assert not VS.gemmseg_fits(4, 4096, 64, 17, 2048)
    assert not VS.gemmseg_fits(4, 4096, 48, 12, 2048)  # 48 does not divide IN


def _w(L, **kw):
    w = L.VQKWeights()
    w.codes, w.codebook, w.scales = 16, 16, 16       # never dereferenced: refused first
    w.code_type, w.pack_bits, w.K, w.D, w.group = L.VQK_U32, 12, 4096, 4, 64
    w.E, w.OUT, w.IN = 1, 8, 256
    w.code_cols = vo.words_per_row(64, 12)
    for k, v in kw.items():
        setattr(w, k, v)
    return w


@pytest.mark.parametrize("N,E", [(640, 512), (64, 96), (700, 40), (1, 1)])
def test_grouped_workspace_layout(L, N, E):
    """vqk_grouped_gemm_workspace (host only): the pair order, room for the
    tile records of the smallest tiles the sort builds (4 rows: the sparse
    routings over d8 tables beyond LDS; ceil(N/4) + min(N, E + 1) records of
    3 int32), the tile count -- each 256-byte aligned, as the GPU tests read
    the sort's output back."""
    w = _w(L, D=8, K=16384, pack_bits=14, E=E, OUT=1024, IN=4096,
           code_cols=vo.words_per_row(512, 14))
    ws = ctypes.c_size_t()
    assert L.lib().vqk_grouped_gemm_workspace(ctypes.byref(w), N, ctypes.byref(ws)) == L.VQK_OK
    al = lambda v: (v + 255) & ~255
    room = (N + 3) // 4 + min(N, E + 1)
    assert ws.value == al(4 * N) + al(12 * room) + 256


@pytest.mark.parametrize("kw,rc", [
    ({"D": 3}, 1),                          # NotImplementedError: no kernel for d=3
    ({"code_cols": 5}, 2),                  # ValueError: WPR mismatch
    ({"k_expect": 2048}, 3),                # RuntimeError: sharded codebook
    ({"pack_bits": 17}, 1),
    ({"code_type": 3, "pack_bits": 0, "code_cols": 64}, 2),   # uint8 codes, K=4096
    ({"group": 48}, 2),                     # 48 does not divide IN=256
    ({"group": 6, "IN": 240, "code_cols": vo.words_per_row(60, 12)}, 1),  # G % D != 0
])
def test_validation_refuses_before_launch(L, kw, rc):
    w = _w(L, **kw)
    got = L.lib().vqk_dense_gemv(ctypes.byref(w), ctypes.c_void_p(16), L.VQK_BF16, 1,
                                 ctypes.c_void_p(16), L.VQK_BF16, None)
    assert got == rc, L.last_error()
    assert L.last_error()


def test_status_maps_to_reference_exceptions(L):
    with pytest.raises(NotImplementedError):
        L.check(L.VQK_ENOTIMPL)
    with pytest.raises(ValueError):
        L.check(L.VQK_EINVAL)
    with pytest.raises(RuntimeError):
        L.check(L.VQK_ESHARDED)


def test_gemv_argument_errors(L):
    w = _w(L)
    lib = L.lib()
    # N != T * xkrep
    assert lib.vqk_moe_expert_gemv(ctypes.byref(w), ctypes.c_void_p(16), L.VQK_BF16, 2,
                                   ctypes.c_void_p(16), 5, 2, ctypes.c_void_p(16), L.VQK_BF16,
                                   None) == L.VQK_EINVAL
    # bad activation type
    assert lib.vqk_dense_gemv(ctypes.byref(w), ctypes.c_void_p(16), 7, 1, ctypes.c_void_p(16),
                              L.VQK_BF16, None) == L.VQK_EINVAL
    # dense takes E == 1
    w2 = _w(L, E=2)
    assert lib.vqk_dense_gemv(ctypes.byref(w2), ctypes.c_void_p(16), L.VQK_BF16, 1,
                              ctypes.c_void_p(16), L.VQK_BF16, None) == L.VQK_EINVAL


def _emb(L, **kw):
    w = L.VQKWeights()
    w.codes, w.codebook, w.scales = 16, 16, 16       # never dereferenced: refused first
    w.code_type, w.pack_bits, w.K, w.D, w.group = L.VQK_U8, 11, 2048, 4, 32
    w.E, w.OUT, w.IN = 1, 100, 160
    w.code_cols = 55                                  # 40 codes x 11 bits = 55 bytes
    for k, v in kw.items():
        setattr(w, k, v)
    return w


@pytest.mark.parametrize("kw,rc", [
    ({"D": 0}, 1),                                    # no subvector dim
    ({"D": 32, "IN": 160, "group": 32}, 1),           # d beyond 16
    ({"E": 2}, 2),                                    # a table is one matrix
    ({"code_cols": 54}, 2),                           # byte stream too short for 40 x 11 bits
    ({"K": 4096}, 2),                                 # K does not fit 11-bit codes
    ({"code_type": 4}, 2),                            # packed rows are bytes or u32 words
    ({"pack_bits": 0, "code_cols": 40}, 2),           # uint8 codes, K=2048
    ({"pack_bits": 0, "code_type": 4, "code_cols": 41}, 2),   # NSUB mismatch
    ({"code_type": 5, "code_cols": 10}, 2),           # u32 words: WPR(40, 11) = 22
    ({"group": 48}, 2),                               # 48 does not divide 160
    ({"row_table": 16, "n_live": 4}, 1),              # no skipzero tables for embeddings
    ({"k_expect": 4096}, 3),                          # sharded codebook
])
def test_embed_validation_refuses_before_launch(L, kw, rc):
    w = _emb(L, **kw)
    got = L.lib().vqk_embed_gather(ctypes.byref(w), ctypes.c_void_p(16), L.VQK_I64, 3,
                                   ctypes.c_void_p(16), L.VQK_BF16, None)
    assert got == rc, L.last_error()
    assert L.last_error()


def test_embed_argument_errors(L):
    w = _emb(L)
    lib = L.lib()
    for id_type, out_type, n in ((L.VQK_F32, L.VQK_BF16, 3), (L.VQK_I32, L.VQK_U8, 3),
                                 (L.VQK_I32, L.VQK_BF16, -1)):
        assert lib.vqk_embed_gather(ctypes.byref(w), ctypes.c_void_p(16), id_type, n,
                                    ctypes.c_void_p(16), out_type, None) == L.VQK_EINVAL
    # nothing to gather: valid and no launch
    assert lib.vqk_embed_gather(ctypes.byref(w), None, L.VQK_I32, 0, None, L.VQK_F16,
                                None) == L.VQK_OK


def _staged_pieces(K, D, CBN, NT):
    """The 16-byte pieces stage_codebook_fixed<D, CBN, NT> copies (vqk_gemv.h),
    restated: round r, wave w, lane l copies piece (r*NT/64 + w)*64 + l when
    it is below min(K*D*2/16, CBN*D*2/16)."""
    pieces = CBN * D * 2 // 16
    valid = min(K * D * 2 // 16, pieces)
    rounds = -(-pieces // NT)
    out = set()
    for r in range(rounds):
        for w in range(NT // 64):
            c = (r * (NT // 64) + w) * 64
            out.update(c + l for l in range(64) if c + l < valid)
    return out, pieces, valid


@pytest.mark.parametrize("D,BITS", [(2, 9), (4, 12), (4, 14), (8, 12), (8, 14), (8, 16), (2, 16)])
@pytest.mark.parametrize("NT", [256, 192])
def test_codebook_staging_stays_in_its_table(D, BITS, NT):
    """Every launch shape that stages a table (whole tables of 2^BITS entries
    up to 64 KB; the first 64 KB / 128 KB of larger ones) copies each valid
    piece exactly once and nothing past the LDS table, also when NT threads
    do not divide the table (the 192 staging threads of the fused layer)."""
    full = (1 << BITS) * D * 2 <= 64 * 1024
    for cbn_bytes in ([(1 << BITS) * D * 2] if full else [64 * 1024, 128 * 1024]):
        CBN = cbn_bytes // (2 * D)
        for K in {1 << BITS, (1 << BITS) - 8, 8}:
            got, pieces, valid = _staged_pieces(K, D, CBN, NT)
            assert got == set(range(valid)) and max(got, default=0) < pieces


def test_noalloc_scratch_size_matches_header(L):
    """The Python mirror of VQK_NOALLOC_SCRATCH_BYTES is the header's value."""
    txt = (ROOT / "include" / "vqk.h").read_text()
    m = re.search(r"#define\s+VQK_NOALLOC_SCRATCH_BYTES\s+\((\d+)u\s*<<\s*(\d+)\)", txt)
    assert m, "VQK_NOALLOC_SCRATCH_BYTES not found"
    assert int(m.group(1)) << int(m.group(2)) == L.VQK_NOALLOC_SCRATCH_BYTES


def test_options_defaults_and_env(L, monkeypatch):
    """vqk_options: the reference's dispatch defaults (VQ_FUSED_MAX_N 512,
    dense cutoff 32, fp16 outputs), and the VQ_* variables read only when
    vqk_options_from_env is asked to."""
    o = L.options()
    assert (o.fused_max_n, o.dense_fused_max_n, o.decode_bf16io, o.prefill_bf16io) == (512, 32, 0, 0)
    monkeypatch.setenv("VQ_FUSED_MAX_N", "77")
    monkeypatch.setenv("VQ_DENSE_FUSED_MAX_N", "5")
    monkeypatch.setenv("VQ_DECODE_BF16IO", "1")
    monkeypatch.setenv("VQ_GEMMSEG_BF16IO", "0")
    e = L.options(from_env=True)
    assert (e.fused_max_n, e.dense_fused_max_n, e.decode_bf16io, e.prefill_bf16io) == (77, 5, 1, 0)
    assert L.options().fused_max_n == 512            # defaults ignore the environment
    monkeypatch.setenv("VQ_FUSED_MAX_N", "not a number")
    assert L.options(from_env=True).fused_max_n == 512


def test_apply_workspace_follows_dispatch(L):
    """vqk_switch_apply_workspace is 0 where the fused GEMV runs (few pairs)
    and the grouped GEMM's size where it does not (many pairs, or pairs
    crowding onto few experts); vqk_linear_apply_workspace likewise."""
    import ctypes
    import numpy as np
    w = L.VQKWeights()
    w.codes, w.code_cols, w.code_type, w.pack_bits = 1 << 20, 16 * 12, L.VQK_U32, 12
    w.codebook, w.K, w.D, w.group = 1 << 24, 4096, 4, 64
    w.scales, w.E, w.OUT, w.IN = 1 << 28, 512, 256, 2048
    ws, g = ctypes.c_size_t(), ctypes.c_size_t()
    o = L.options()
    # E = 512: VQ_FUSED_MAX_N decides; E = 64: 128 pairs crowd (N >= 2E)
    for E, N, grouped in [(512, 8, False), (512, 512, False), (512, 513, True), (64, 100, False),
                          (64, 128, True)]:
        w.E = E
        L.check(L.lib().vqk_switch_apply_workspace(ctypes.byref(w), N, ctypes.byref(o), ctypes.byref(ws)))
        L.check(L.lib().vqk_grouped_gemm_workspace(ctypes.byref(w), N, ctypes.byref(g)))
        assert ws.value == (g.value if grouped else 0), (N, ws.value)
    small = L.options(fused_max_n=4)
    L.check(L.lib().vqk_switch_apply_workspace(ctypes.byref(w), 8, ctypes.byref(small), ctypes.byref(ws)))
    assert ws.value > 0
    w.E = 1
    for N, fused in [(1, True), (32, True), (65, False)]:        # 33..64: segment kernel, no workspace
        L.check(L.lib().vqk_linear_apply_workspace(ctypes.byref(w), N, ctypes.byref(o), ctypes.byref(ws)))
        assert (ws.value == 0) == fused, (N, ws.value)
    assert np.int64(L.VQK_VIA_F16) == 0x100


def test_moe_header_constant_and_paths(L):
    """The Python mirror of VQK_MOE_HEADER_BYTES is the header's value; the
    layer's workspace starts with that header at every T; the one-launch form
    is planned for batch 1 only (config-2 shape: T = 1 one launch, T = 2 the
    two fused kernels), and the test hook switches it off. Host only: plans,
    no launches."""
    import ctypes
    import sys
    sys.path.insert(0, str(ROOT / "tests"))
    from vq_cases import PATH_FUSED, PATH_GROUPED, PATH_ONE_LAUNCH, hooks
    txt = (ROOT / "include" / "vqk.h").read_text()
    m = re.search(r"#define\s+VQK_MOE_HEADER_BYTES\s+(\d+)u", txt)
    assert m and int(m.group(1)) == L.VQK_MOE_HEADER_BYTES
    for hook in ("vqk__test_l1_spins", "vqk__test_l1_mode", "vqk__test_moe_path"):
        assert hasattr(L.lib(), hook) and hook not in txt

    def proj(E, OUT, IN, base):
        w = L.VQKWeights()
        w.codes, w.code_cols, w.code_type, w.pack_bits = base, (IN // 4 + 31) // 32 * 12, L.VQK_U32, 12
        w.codebook, w.K, w.D, w.group = base + (1 << 26), 4096, 4, 64
        w.scales, w.E, w.OUT, w.IN = base + (1 << 27), E, OUT, IN
        return w
    E, H, I = 256, 2048, 512
    ws_ = [proj(E, I, H, 1 << 30), proj(E, I, H, 2 << 30), proj(E, H, I, 3 << 30)]
    d = L.VQKMoeDesc()
    d.gate, d.up, d.down = (ctypes.pointer(w) for w in ws_)
    d.top_k, d.norm_topk = 8, 1
    p, sz = ctypes.c_int32(), ctypes.c_size_t()
    for T, want in ((1, PATH_ONE_LAUNCH), (2, PATH_FUSED), (4, PATH_FUSED), (64, PATH_GROUPED)):
        L.check(hooks().vqk__test_moe_path(ctypes.byref(d), T, ctypes.byref(p)))
        assert p.value == want, (T, p.value)
        L.check(L.lib().vqk_moe_decode_layer_workspace(ctypes.byref(d), T, ctypes.byref(sz)))
        assert sz.value > L.VQK_MOE_HEADER_BYTES
    prev = hooks().vqk__test_l1_mode(1)
    try:
        L.check(hooks().vqk__test_moe_path(ctypes.byref(d), 1, ctypes.byref(p)))
        assert p.value == PATH_FUSED
    finally:
        hooks().vqk__test_l1_mode(prev)
    # with a shared expert (its own E = 1 projections and gate vector): batch
    # 1 is one launch while the grid fits two workgroups per CU -- top-6 of
    # 128 (7 pairs: 224 gate/up + 128 down workgroups) -- and two kernels
    # past it: top-8 (9 pairs, 64 lanes per down row: 288 + 256 > 2 x 256)
    sh = [proj(1, I, H, 4 << 30), proj(1, I, H, 5 << 30), proj(1, H, I, 6 << 30)]
    d.sh_gate, d.sh_up, d.sh_down = (ctypes.pointer(w) for w in sh)
    d.sh_gate_vec, d.sh_gate_vec_type = 7 << 30, L.VQK_BF16
    L.check(hooks().vqk__test_moe_path(ctypes.byref(d), 1, ctypes.byref(p)))
    assert p.value == PATH_FUSED, ("shared, 9 pairs", p.value)
    ws_[0].E = ws_[1].E = ws_[2].E = 128
    d.top_k = 6
    for T, want in ((1, PATH_ONE_LAUNCH), (2, PATH_FUSED), (64, PATH_GROUPED)):
        L.check(hooks().vqk__test_moe_path(ctypes.byref(d), T, ctypes.byref(p)))
        assert p.value == want, ("shared", T, p.value)


def test_options_crowded_rule_is_switchable(L):
    """crowded_grouped (an extension beyond the reference's dispatch) is on
    by default; off, only fused_max_n decides, as in the reference."""
    import ctypes
    w = L.VQKWeights()
    w.codes, w.code_cols, w.code_type, w.pack_bits = 1 << 20, 16 * 12, L.VQK_U32, 12
    w.codebook, w.K, w.D, w.group = 1 << 24, 4096, 4, 64
    w.scales, w.E, w.OUT, w.IN = 1 << 28, 64, 256, 2048
    assert L.options().crowded_grouped == 1
    ws = ctypes.c_size_t()
    for crowded, grouped in ((1, True), (0, False)):
        o = L.options(crowded_grouped=crowded)
        L.check(L.lib().vqk_switch_apply_workspace(ctypes.byref(w), 128, ctypes.byref(o), ctypes.byref(ws)))
        assert (ws.value > 0) == grouped


def test_wide_x_flag_is_d4_d8_gemv_only(L):
    """VQK_X_KEEP (x enters the d=4 / d=8 GEMV unrounded) has the header's
    value; a d=2 module, whose reference kernels all stage x as fp16, and the
    grouped GEMM refuse it before anything reaches a device."""
    import ctypes
    txt = (ROOT / "include" / "vqk.h").read_text()
    m = re.search(r"#define\s+VQK_X_KEEP\s+(0x[0-9a-fA-F]+)", txt)
    assert m and int(m.group(1), 16) == L.VQK_X_KEEP
    assert L.VQK_X_KEEP & (L.VQK_VIA_F16 | 0xff) == 0
    w = L.VQKWeights()
    w.codes, w.code_cols, w.code_type, w.pack_bits = 1 << 20, 16 * 12, L.VQK_U32, 12
    w.codebook, w.K, w.D, w.group = 1 << 24, 4096, 2, 64
    w.scales, w.E, w.OUT, w.IN = 1 << 28, 8, 256, 1024
    xt = L.VQK_BF16 | L.VQK_X_KEEP
    rc = L.lib().vqk_moe_expert_gemv(ctypes.byref(w), 1 << 32, xt, 1, 1 << 33, 1, 1, 1 << 34,
                                     L.VQK_F32, None)
    assert rc == L.VQK_EINVAL and "d=2" in L.last_error()
    w.E = 1
    rc = L.lib().vqk_dense_gemv(ctypes.byref(w), 1 << 32, xt, 0, 1 << 34, L.VQK_F32, None)
    assert rc == L.VQK_EINVAL and "d=2" in L.last_error()
    w.code_cols, w.D, w.IN = 16 * 12, 4, 2048
    ws = ctypes.c_size_t()
    L.check(L.lib().vqk_grouped_gemm_workspace(ctypes.byref(w), 64, ctypes.byref(ws)))
    rc = L.lib().vqk_grouped_gemm(ctypes.byref(w), 1 << 32, xt, 64, 1 << 33, 64, 1, 1 << 34,
                                  L.VQK_F32, 1 << 35, ws.value, None)
    assert rc == L.VQK_EINVAL and "type" in L.last_error()


def test_empty_calls_need_no_pointers(L):
    """A call with no rows, pairs or tokens returns VQK_OK without reading a
    pointer (an empty tensor's pointer is NULL) or touching a device: the
    GEMVs, the GEMMs, both dispatchers, the dequant and the MoE layer."""
    import ctypes
    w = L.VQKWeights()
    w.codes, w.code_cols, w.code_type, w.pack_bits = 1 << 20, 16 * 12, L.VQK_U32, 12
    w.codebook, w.K, w.D, w.group = 1 << 24, 4096, 4, 64
    w.scales, w.E, w.OUT, w.IN = 1 << 28, 8, 256, 2048
    lib, bf = L.lib(), L.VQK_BF16
    o = L.options()
    assert lib.vqk_moe_expert_gemv(ctypes.byref(w), None, bf, 0, None, 0, 1, None, bf, None) == L.VQK_OK
    assert lib.vqk_grouped_gemm(ctypes.byref(w), None, bf, 0, None, 0, 1, None, bf, None, 0,
                                None) == L.VQK_OK
    assert lib.vqk_switch_apply(ctypes.byref(w), None, bf, 0, None, 0, 1, None, bf, None, 0,
                                ctypes.byref(o), None) == L.VQK_OK
    assert lib.vqk_dequant(ctypes.byref(w), 0, 0, None, None) == L.VQK_OK
    assert lib.vqk_dequant_experts(ctypes.byref(w), None, 0, None, None) == L.VQK_OK
    w.E = 1
    assert lib.vqk_dense_gemv(ctypes.byref(w), None, bf, 0, None, bf, None) == L.VQK_OK
    assert lib.vqk_dense_gemm(ctypes.byref(w), None, bf, 0, None, bf, None, 0, None) == L.VQK_OK
    assert lib.vqk_linear_apply(ctypes.byref(w), None, bf, 0, None, bf, None, 0, ctypes.byref(o),
                                None) == L.VQK_OK
    # rows with NULL pointers are still refused
    assert lib.vqk_dense_gemv(ctypes.byref(w), None, bf, 1, None, bf, None) == L.VQK_EINVAL
    assert lib.vqk_dequant(ctypes.byref(w), 0, 1, None, None) == L.VQK_EINVAL

    def proj(E, OUT, IN, base):
        p = L.VQKWeights()
        p.codes, p.code_cols, p.code_type, p.pack_bits = base, (IN // 4 + 31) // 32 * 12, L.VQK_U32, 12
        p.codebook, p.K, p.D, p.group = base + (1 << 26), 4096, 4, 64
        p.scales, p.E, p.OUT, p.IN = base + (1 << 27), E, OUT, IN
        return p
    ws_ = [proj(256, 512, 2048, 1 << 30), proj(256, 512, 2048, 2 << 30), proj(256, 2048, 512, 3 << 30)]
    d = L.VQKMoeDesc()
    d.gate, d.up, d.down = (ctypes.pointer(p) for p in ws_)
    d.top_k, d.norm_topk = 8, 1
    assert lib.vqk_moe_decode_layer(ctypes.byref(d), None, bf, 0, None, None, bf, None, None, None,
                                    0, None) == L.VQK_OK
