"""The BASELINE configurations at their real shapes, against the oracle.

Weights are drawn on the device (uniform random packed words: every field is a
uniform code in [0, K)), as the benchmark builds them; the oracle receives
only the experts a call touches, copied to the host and unpacked there, so
each test stays within about a minute.

  c3  E=512, H=4096, I=1024, d8 K16384 14-bit, top-10 + shared expert, T = 1
      and 4, through vqk_moe_decode_layer (vq_switch.py:5284-5423,
      decode_ladder.py:107-125); plus routing-only checks at E = 512 and 1024
      (8 and 16 logits per lane) with tied, -inf and signed-zero logits.
  c4  the c3 layer as an MTP verify batch, T = 4, 16, 64, 20 % of the routed
      experts' rows dead and stored compact (skipzero row table), with the
      shared expert (vq_switch.py:4569-4722, 4958-5013).
  c5  dense prefill, x [2048, 5120] through 5120 -> 17408 and x [2048, 17408]
      through 17408 -> 5120, d8 K65536 uint16 codes (vq_dense.py:262-312);
      a sampled block of outputs is compared with the float64 oracle over
      bf16-rounded weights (the reference's `w.T.astype(xf.dtype)`).

MoE outputs are checked against both of the oracle's rounding modes: within
rtol 2e-2 / atol 1e-3 elementwise of the kernels' (SwiGLU intermediate rounded
to fp16 once, everything else float64), and within the reference's own bar,
max |y - ref| < 2e-2 * max |ref| (gate/kernel_accept.py:48-63), of the
reference's (every linear's output rounded to fp16 then bf16, SwiGLU in
bf16): that mode's own bf16 noise puts a few percent of the elements near
zero outside the elementwise bar even for exact arithmetic.
"""
import numpy as np
import pytest

from oracle import vq_oracle as vo
from vq_cases import assert_close, assert_rel_max

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

H3, E3, I3, K3, D3, BITS3, TOPK3 = 4096, 512, 1024, 16384, 8, 14, 10


class _HostExperts:
    """Host view of one device projection, expert by expert: load(e) gives
    the unpacked codes [OUT, NSUB] and fp16 scales [OUT, NGRP] of expert e,
    dead skipzero rows as code 0 with scale 0 (the expanded form). Only the
    experts the oracle asks for are copied, each once."""

    def __init__(self, proj, nsub, bits):
        self.p, self.nsub, self.bits = proj, nsub, bits
        self.OUT = proj.output_dims
        self.shape = (proj.num_experts, self.OUT, nsub)
        self._cache = {}

    def load(self, e):
        e = int(e)
        if e not in self._cache:
            p = self.p
            if p.row_table is None:
                words = p.codes[e].cpu().numpy().view(np.uint32)
                sc = p.vq_scales[e].cpu().numpy()
                codes = vo.unpack(words, self.nsub, self.bits)
            else:
                rt = p.row_table[e].cpu().numpy()
                live = rt >= 0
                codes = np.zeros((self.OUT, self.nsub), np.uint16)
                sc = np.zeros((self.OUT, p.vq_scales.shape[-1]), np.float16)
                if live.any():
                    rows = torch.from_numpy(rt[live].astype(np.int64)).to(p.codes.device)
                    words = p.codes.index_select(0, rows).cpu().numpy().view(np.uint32)
                    codes[live] = vo.unpack(words, self.nsub, self.bits)
                    sc[live] = p.vq_scales.index_select(0, rows).cpu().numpy()
            self._cache[e] = (codes, sc)
        return self._cache[e]


class _View:
    """`[e]` -> codes (part 0) or scales (part 1) of a _HostExperts."""

    def __init__(self, src, part):
        self.src, self.part, self.shape = src, part, src.shape

    def __getitem__(self, e):
        return self.src.load(e)[self.part]


def _host_spec(proj, d, bits):
    src = _HostExperts(proj, proj.input_dims // d, bits)
    return {"codes": _View(src, 0), "scales": _View(src, 1),
            "codebook": proj.codebook.cpu().numpy(), "group": 64}


def _proj(g, E, OUT, IN, d, K, bits, dead=0.0):
    """Random VQ projection on the device; with `dead`, that fraction of the
    (expert, row) rows is dead and the tensors are stored compact."""
    from vqlab_amd.vq_switch import VQSwitchLinear
    wpr = ((IN // d) + 31) // 32 * bits
    cb = (torch.randn((K, d), device="cuda", generator=g) * 0.02).to(torch.float16)
    if not dead:
        codes = torch.randint(-2**31, 2**31 - 1, (E, OUT, wpr), dtype=torch.int32,
                              device="cuda", generator=g)
        sc = (torch.rand((E, OUT, IN // 64), device="cuda", generator=g) + 0.5).to(torch.float16)
        return VQSwitchLinear(codes, cb, sc, pack_bits=bits, in_features=IN)
    live = torch.rand((E, OUT), device="cuda", generator=g) >= dead
    n_live = int(live.sum().item())
    rt = torch.full((E, OUT), -1, dtype=torch.int32, device="cuda")
    rt[live] = torch.arange(n_live, dtype=torch.int32, device="cuda")
    codes = torch.randint(-2**31, 2**31 - 1, (n_live, wpr), dtype=torch.int32, device="cuda",
                          generator=g)
    sc = (torch.rand((n_live, IN // 64), device="cuda", generator=g) + 0.5).to(torch.float16)
    return VQSwitchLinear(codes, cb, sc, pack_bits=bits, in_features=IN, row_table=rt)


def _c3_layer(seed, dead=0.0, shared=True, E=E3, H=H3, I=I3, d=D3, K=K3, bits=BITS3, k=TOPK3):
    from vqlab_amd.moe import VQSparseMoeBlock, VQSwitchGLU
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    mlp = VQSwitchGLU(*(_proj(g, E, o, i, d, K, bits, dead) for o, i in ((I, H), (I, H), (H, I))))
    sh = sgv = None
    if shared:
        sh = VQSwitchGLU(*(_proj(g, 1, o, i, d, K, bits) for o, i in ((I, H), (I, H), (H, I))))
        sgv = (torch.randn((H,), device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    return VQSparseMoeBlock(mlp, k, True, sh, sgv)


def _oracle_specs(blk, d=D3, bits=BITS3):
    """Host views of the block's projections, shared by both oracle runs."""
    m = blk.switch_mlp
    specs = [_host_spec(p, d, bits) for p in (m.gate_proj, m.up_proj, m.down_proj)]
    kw = {}
    if blk.shared_expert is not None:
        s = blk.shared_expert
        kw["shared"] = dict(zip(("gate", "up", "down"),
                                (_host_spec(p, d, bits)
                                 for p in (s.gate_proj, s.up_proj, s.down_proj))))
        kw["shared_gate"] = blk.shared_expert_gate.float().cpu().numpy()
    return specs, kw


def _check_layer(blk, T, seed, k=TOPK3, rows=None, E=E3, H=H3, routing="iid"):
    """One fused layer call on T tokens; the oracle checks tokens `rows`
    (all by default) in both rounding modes, and the routing exactly.
    routing "capped": logits whose top-k gives each touched expert 1..8 of
    the batch's tokens (bench.mtp_logits), else i.i.d. N(0, 1)."""
    rng = np.random.default_rng(seed)
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to("cuda", torch.bfloat16)
    if routing == "capped":
        from bench import mtp_logits
        lg = mtp_logits(rng, T, E, k)
    else:
        lg = rng.standard_normal((T, E)).astype(np.float32)
    y, ids, w = blk.fused(x, torch.from_numpy(lg).cuda(), return_route=True)
    torch.cuda.synchronize()
    rows = np.arange(T) if rows is None else np.asarray(rows)
    xh = x.float().cpu().numpy()[rows]
    yh = y.float().cpu().numpy()[rows]
    assert np.isfinite(y.float().cpu().numpy()).all()
    rid, rw = vo.route(lg[rows], k)
    assert np.array_equal(ids.cpu().numpy()[rows], rid)
    assert np.allclose(w.cpu().numpy()[rows], rw, rtol=1e-5, atol=1e-6)
    specs, kw = _oracle_specs(blk)
    ref_k, _, _ = vo.moe_layer(xh, lg[rows], *specs, k, h_round=np.float16, **kw)
    assert_close(yh, ref_k, what=f"T={T} kernel rounding")
    ref_r, _, _ = vo.moe_layer(xh, lg[rows], *specs, k, rounding="reference", **kw)
    assert_rel_max(yh, ref_r, what=f"T={T} reference rounding")


# ------------------------------------------------------------------ c3
@pytest.fixture(scope="module")
def c3_layer():
    blk = _c3_layer(303)
    yield blk
    del blk
    torch.cuda.empty_cache()


@pytest.mark.parametrize("T", [1, 4])
def test_c3_layer_full_shape(c3_layer, T):
    """Config 3 decode: the fused layer at E=512 (8 logits per lane in the
    routing), tables beyond LDS, the shared expert and its gate."""
    print(f"c3 full shape T={T}", flush=True)
    _check_layer(c3_layer, T, 3000 + T)


@pytest.mark.parametrize("E,k", [(512, 10), (1024, 8), (256, 16), (256, 20), (100, 8), (64, 9)])
def test_routing_many_experts_ties(E, k):
    """Routing with 8 (E=512) and 16 (E=1024) logits per lane: tied logits go
    to the lower expert id, -inf logits are chosen last, -0 and +0 tie. The
    threshold-and-rank top-k takes k <= 16 (16 its largest, 8-lane groups up
    to k = 8 and 4-lane groups above); k = 20 and the rows where more than 64
    keys reach the threshold (all tied) take the sequential selection; E = 100
    leaves padding slots in the lanes."""
    from vqlab_amd.moe import VQSparseMoeBlock, VQSwitchGLU
    print(f"routing E={E} k={k}", flush=True)
    g = torch.Generator(device="cuda")
    g.manual_seed(E)
    H, I, d, K, bits = 256, 128, 4, 256, 8
    mlp = VQSwitchGLU(*(_proj(g, E, o, i, d, K, bits) for o, i in ((I, H), (I, H), (H, I))))
    blk = VQSparseMoeBlock(mlp, k, True)
    rng = np.random.default_rng(E + 1)
    T = 6
    lg = np.round(rng.standard_normal((T, E)) * 2) / 2               # many exact ties
    lg[1, :] = 0.0                                                      # all tied
    lg[2, :] = -np.inf
    lg[2, rng.permutation(E)[: k // 2]] = 1.5                           # fewer finite than k
    lg[3, :] = -1.0
    lg[3, rng.permutation(E)[: 3 * k]] = 0.0                            # +0 / -0 ties
    lg[3, rng.permutation(E)[: 3 * k]] = -0.0
    lg[4] = rng.standard_normal(E)                                      # continuous
    lg[5, :] = 2.0
    lg[5, E - 1] = 3.0                                                  # the top id is the last
    x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to("cuda", torch.bfloat16)
    _, ids, w = blk.fused(x, torch.from_numpy(lg.astype(np.float32)).cuda(), return_route=True)
    rid, rw = vo.route(lg.astype(np.float32), k)
    assert np.array_equal(ids.cpu().numpy(), rid)
    assert np.allclose(w.cpu().numpy(), rw, rtol=1e-5, atol=1e-6)


# ------------------------------------------------------------------ c4
@pytest.fixture(scope="module")
def c4_layer():
    blk = _c3_layer(404, dead=0.2)
    yield blk
    del blk
    torch.cuda.empty_cache()


@pytest.mark.parametrize("T", [4, 16, 64])
def test_c4_verify_batch_full_shape(c4_layer, T):
    """Config 4: the MTP verify batch on the c3 layer with 20 % dead routed
    rows stored compact and the shared expert (K split in four slices at
    H=4096 on the grouped path). At T=64 the oracle checks 12 of the 64
    tokens (each token's output depends on its own experts only; the kernels
    still run the whole batch)."""
    print(f"c4 full shape T={T}", flush=True)
    rows = None if T <= 16 else [0, 1, 7, 13, 22, 31, 32, 40, 47, 55, 62, 63]
    _check_layer(c4_layer, T, 4000 + T, rows=rows)


@pytest.mark.parametrize("T", [16, 64])
def test_c4_verify_batch_capped_routing(c4_layer, T):
    """Config 4 on its MTP verify routing: each touched expert receives
    1..min(8, T) of the batch's tokens and no token repeats an expert (about
    34 touched experts at T = 16, 140 at T = 64, against ~370 for i.i.d.
    logits at T = 64), so the grouped tiles hold several rows each. The
    oracle checks 12 tokens at T = 64, all at T = 16."""
    print(f"c4 capped routing T={T}", flush=True)
    rows = None if T <= 16 else [0, 3, 9, 15, 20, 27, 33, 38, 44, 51, 57, 63]
    _check_layer(c4_layer, T, 4100 + T, rows=rows, routing="capped")


# ------------------------------------------------------------------ c5
@pytest.mark.parametrize("OUT,IN", [(17408, 5120), (5120, 17408)])
def test_c5_prefill_full_shape(OUT, IN):
    """Config 5: one dense VQ linear on 2048 tokens (d8, K65536, uint16 codes)
    through VQLinear's decode-then-GEMM path; 64 output columns x 96 tokens
    (spread over the whole output, including its last rows and columns) are
    compared with the oracle."""
    from vqlab_amd.vq_dense import VQLinear
    print(f"c5 full shape {OUT}x{IN}", flush=True)
    N, d, K = 2048, 8, 65536
    g = torch.Generator(device="cuda")
    g.manual_seed(OUT)
    codes = torch.randint(0, K, (OUT, IN // d), dtype=torch.int32, device="cuda",
                          generator=g).to(torch.int16)
    cb = (torch.randn((K, d), device="cuda", generator=g) * 0.02).to(torch.float16)
    sc = (torch.rand((OUT, IN // 64), device="cuda", generator=g) + 0.5).to(torch.float16)
    lin = VQLinear(codes, cb, sc, group_size=64, pack_bits=0)
    x = torch.randn((N, IN), device="cuda", generator=g).to(torch.bfloat16)
    y = lin(x)
    torch.cuda.synchronize()
    assert y.shape == (N, OUT) and y.dtype == torch.bfloat16
    assert torch.isfinite(y.float()).all().item()
    rng = np.random.default_rng(5)
    cols = np.unique(np.concatenate([rng.choice(OUT, 60, replace=False), [0, 1, OUT - 2, OUT - 1]]))
    toks = np.unique(np.concatenate([rng.choice(N, 92, replace=False), [0, 1, N - 2, N - 1]]))
    ci = torch.from_numpy(cols).cuda()
    w16 = vo.dequant(codes.index_select(0, ci).cpu().numpy().view(np.uint16), cb.cpu().numpy(),
                     sc.index_select(0, ci).cpu().numpy(), 64)
    xs = x.float().cpu().numpy()[toks]
    ref = vo.decode_matmul(xs, vo.bf16_values(w16))
    got = y.float().cpu().numpy()[np.ix_(toks, cols)]
    assert_close(got, ref, what=f"c5 {OUT}x{IN}")
