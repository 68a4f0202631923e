"""Benchmark of the VQ MoE decode layer on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
                    [--workload c1|c2|c3|c3b4|c4|c4t16|c4capped|c4t16capped|c5|gather|stream|launch]

Default workload: a Qwen3.6-35B-A3B-shaped MoE
decode layer -- hidden 2048, 256 experts of intermediate 512, top-8 softmax
router on N(0,1) logits, SwiGLU gate/up/down, VQ d=4, K=4096 (12-bit packed
indices), one fp16 codebook per projection, fp16 scales per 64 weights,
batch 1, bf16 activations. Weights are random (no checkpoints offline), in
8 distinct layers (2.6 GB) so every call streams its experts from HBM
rather than the 256 MB MALL.

A step is one decode token through the 8-layer stack: per layer, one fused
call (device routing + gate/up/SwiGLU + down/combine in one launch) with that
step's own logits. The timed steps are captured once in a HIP graph and
replayed; HIP events on the launch stream bracket the replay.

value = packed-weight GB/s: bytes of the codes and scales of the experts the
router touched, summed over every layer call, over
the timed wall time. roofline uses the layer call's total algorithmic bytes
(codes + scales + codebooks + activations) over its event-timed duration.
cpu_baseline: the reference's decode-then-matmul of the same layer on the
host cores (unpack -> fp16 dequant -> fp32 matvecs, numpy), timed on one
thread and on every usable core, on a bounded sample.

--workload c4 / c4t16: an MTP verify batch of T tokens
through the config-3 layer with 20% of the routed experts' rows dead and
stored compact (skipzero row table); the block runs its composed path
(device softmax/top-k, then each projection as ONE grouped call over the
T*k pairs: vqk_grouped_gemm above 512 pairs, the fused GEMV below).
value = packed GB/s of the live rows of the touched experts.

--workload c1 (the reference's CPU-runnable case): one
dense VQ GEMV per call (W 4096x4096, d=2, K=256, uint8 codes, x [1, 4096]
bf16) over 120 distinct weights (1.07 GB) so each call streams from HBM; value
= packed GB/s of codes + scales; cpu_baseline: the same GEMV as fp16 dequant +
fp32 matvec on the host, one thread and all cores.

--workload c5: dense VQ prefill, x [2048, 5120]
through VQLinear 5120->17408 then 17408->5120 (d8, K=65536 uint16 codes);
value = TFLOP/s of the two GEMMs, roofline against the fp16 MFMA peak.

--workload gather / stream / launch: measurement probes (libvqk test hooks
outside the ABI): the random 16-byte gather rate from an L2-resident table,
the fastest one-launch streaming read of config 1's weight bytes (the floor
of a GEMV that reads them in one launch), and the cost of one kernel boundary
(back-to-back launches of a kernel that reads 16 bytes, in a HIP graph: what
every call of a one-launch layer pays beyond its own work).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0

WORKLOADS = {
    # the reference's CPU-runnable case, on the GPU: one dense VQ GEMV per call
    "c1": dict(OUT=4096, IN=4096, d=2, K=256, G=64, layers=120, kind="dense_gemv",
               desc="Single dense VQ linear, decode GEMV: W 4096x4096, d=2, K=256, uint8 codes, "
                    "x [1, 4096] (BASELINE configs[0])"),
    # name: (H, E, I, top_k, shared, d, K, bits, T, layers)
    "c2": dict(H=2048, E=256, I=512, k=8, shared=False, d=4, K=4096, bits=12, T=1, layers=8,
               desc="Qwen3.6-35B-A3B-shaped MoE decode layer (BASELINE configs[1])"),
    "c3": dict(H=4096, E=512, I=1024, k=10, shared=True, d=8, K=16384, bits=14, T=1, layers=4,
               desc="Qwen3.5-397B-A17B-shaped MoE decode layer, B=1 (BASELINE configs[2])"),
    "c3b4": dict(H=4096, E=512, I=1024, k=10, shared=True, d=8, K=16384, bits=14, T=4, layers=4,
                 desc="Qwen3.5-397B-A17B-shaped MoE decode layer, B=4 (BASELINE configs[2])"),
    # batched paths: grouped expert GEMM (c4) and dense prefill GEMM (c5)
    "c4": dict(H=4096, E=512, I=1024, k=10, shared=True, d=8, K=16384, bits=14, T=64, layers=2,
               dead=0.2, kind="mtp",
               desc="MTP verify batch on the config-3 layer, T=64, 20% skipzero rows "
                    "(BASELINE configs[3])"),
    "c4t16": dict(H=4096, E=512, I=1024, k=10, shared=True, d=8, K=16384, bits=14, T=16,
                  layers=2, dead=0.2, kind="mtp",
                  desc="MTP verify batch on the config-3 layer, T=16, 20% skipzero rows "
                       "(BASELINE configs[3])"),
    # config 4 on capped routing, the MTP verify batch's: each touched expert
    # gets 1..min(8, T) of the batch's tokens, no token repeats an expert
    # (mtp_logits)
    "c4capped": dict(H=4096, E=512, I=1024, k=10, shared=True, d=8, K=16384, bits=14, T=64,
                     layers=2, dead=0.2, kind="mtp", routing="capped",
                     desc="MTP verify batch on the config-3 layer, T=64, 20% skipzero rows, "
                          "each touched expert 1..8 tokens (BASELINE configs[3])"),
    "c4t16capped": dict(H=4096, E=512, I=1024, k=10, shared=True, d=8, K=16384, bits=14, T=16,
                        layers=2, dead=0.2, kind="mtp", routing="capped",
                        desc="MTP verify batch on the config-3 layer, T=16, 20% skipzero rows, "
                             "each touched expert 1..8 tokens (BASELINE configs[3])"),
    # measurement probe: the random-gather rate of an L2-resident table
    "gather": dict(kind="gather",
                   desc="random 16-byte gathers from a 256 KB / 1 MB L2-resident table (probe)"),
    # measurement probe: one launch that only streams config 1's weight bytes
    "stream": dict(kind="stream", bytes=4096 * 2048 + 4096 * 64 * 2, layers=120,
                   desc="streaming read of config 1's codes + scales (8.9 MB) per launch, "
                        "120 rotating buffers (probe)"),
    # measurement probe: back-to-back launches that do (almost) nothing
    "launch": dict(kind="launch", launches=1000,
                   desc="1000 back-to-back launches of a 16-byte read in one HIP graph (probe)"),
    "c5": dict(N=2048, H=5120, F=17408, d=8, K=65536, kind="prefill",
               desc="Dense Qwen3.8-27B-shaped VQ prefill: 5120x17408 then 17408x5120, "
                    "x [2048, 5120] (BASELINE configs[4])"),
}
MFMA_F16_PEAK_TFS = 2500.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


L2_REQ_PER_CLK_PER_CU = 0.5      # 16 L2 channels per XCD, one request per clock each, 32 CUs
N_CUS = 256
PEAK_CLOCK_GHZ = 2.4


def measured_traffic(name, key="traffic_bytes_per_call"):
    """HBM bytes per call (or per step) from the committed counter profile of
    this workload (rocprofv3 FETCH_SIZE + WRITE_SIZE, copy-calibrated), or None."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(key + ":"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def make_layer(torch, dev, w, g):
    """Random VQ weights of one MoE layer on the device (generator g)."""
    from vqlab_amd.vq_switch import VQSwitchLinear
    from vqlab_amd.moe import VQSparseMoeBlock, VQSwitchGLU
    H, E, I, d, K, bits = w["H"], w["E"], w["I"], w["d"], w["K"], w["bits"]

    def proj(e, out, inn):
        nsub = inn // d
        wpr = (nsub + 31) // 32 * bits
        # uniform random words: every bits-wide field is a uniform code in [0, K)
        codes = torch.randint(-2**31, 2**31 - 1, (e, out, wpr), dtype=torch.int32, device=dev,
                              generator=g)
        cb = (torch.randn((K, d), device=dev, generator=g) * 0.02).to(torch.float16)
        sc = (torch.rand((e, out, inn // 64), device=dev, generator=g) + 0.5).to(torch.float16)
        return VQSwitchLinear(codes, cb, sc, pack_bits=bits, in_features=inn)

    mlp = VQSwitchGLU(proj(E, I, H), proj(E, I, H), proj(E, H, I))
    sh = sg = None
    if w["shared"]:
        sh = VQSwitchGLU(proj(1, I, H), proj(1, I, H), proj(1, H, I))
        sg = (torch.randn((H,), device=dev, generator=g) * 0.02).to(torch.bfloat16)
    return VQSparseMoeBlock(mlp, w["k"], True, sh, sg)


def expert_bytes(w):
    """Packed code + scale bytes of one expert's three projections."""
    H, I, d, bits = w["H"], w["I"], w["d"], w["bits"]
    gu = I * (((H // d) + 31) // 32 * bits * 4 + (H // 64) * 2)
    dn = H * (((I // d) + 31) // 32 * bits * 4 + (I // 64) * 2)
    return 2 * gu + dn


def mtp_logits(rng, T, E, k, cap=8):
    """Router logits [T, E] (fp32) whose top-k is an MTP verify batch's routing
    (config 4: experts receive 1..8 tokens each): experts are taken in random
    order, each with a uniform count of 1..min(cap, T) tokens, until the T*k
    pairs are placed;
    each expert's tokens are the least-loaded ones that still need experts
    (never a token twice), so every token gets exactly k distinct experts.
    Selected logits lie in [4, 5), the rest are N(0, 1) clipped below 3."""
    need = np.full(T, k)
    order = rng.permutation(E)
    pick = np.zeros((T, E), bool)
    left = T * k
    for e in order:
        if left == 0:
            break
        c = min(int(rng.integers(1, min(cap, T) + 1)), left, int((need > 0).sum()))
        cand = np.flatnonzero(need > 0)
        cand = cand[np.lexsort((rng.random(cand.size), -need[cand]))][:c]
        pick[cand, e] = True
        need[cand] -= 1
        left -= c
    if left:
        raise RuntimeError("mtp_logits: pairs left unplaced")
    lg = np.minimum(rng.standard_normal((T, E)), 3.0)
    lg[pick] = 4.0 + rng.random(int(pick.sum()))
    return lg.astype(np.float32)


# ------------------------------------------------------------ CPU baseline
def _cpu_env():
    """Host facts the CPU baseline is quoted with: usable cores, CPU model,
    numpy's BLAS (vendor, version, default threads)."""
    cores = len(os.sched_getaffinity(0))
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    blas = None
    try:
        from threadpoolctl import threadpool_info
        np.ones((64, 64)) @ np.ones((64, 64))            # loads the BLAS
        for i in threadpool_info():
            if i.get("user_api") == "blas":
                blas = {"vendor": i.get("internal_api"), "version": i.get("version"),
                        "threads": i.get("num_threads")}
                break
    except ImportError:
        pass
    return cores, model, blas


def _cpu_time(units, budget_s, workers):
    """Mean seconds per unit: units(i) -> list of independent zero-argument
    tasks (plus a finishing callable of their results). BLAS runs one thread;
    `workers` > 1 spreads each unit's tasks over a thread pool (numpy's
    gathers, conversions and matmuls release the GIL)."""
    import concurrent.futures as cf
    from threadpoolctl import threadpool_limits
    pool = cf.ThreadPoolExecutor(workers) if workers > 1 else None
    n, t0 = 0, time.perf_counter()
    try:
        with threadpool_limits(1):
            while n < 2 or (time.perf_counter() - t0 < budget_s and n < 4096):
                tasks, finish = units(n)
                res = list(pool.map(lambda f: f(), tasks)) if pool else [f() for f in tasks]
                finish(res)
                n += 1
    finally:
        if pool:
            pool.shutdown()
    return (time.perf_counter() - t0) / n, n


def _cpu_report(units, budget_s, per_unit, unit, what, sample):
    """Times `units` on one thread and on every usable core; the all-core run
    is the reported value, the one-thread run rides along."""
    cores, model, blas = _cpu_env()
    t1, n1 = _cpu_time(units, budget_s / 2, 1)
    tn, nn = _cpu_time(units, budget_s / 2, cores) if cores > 1 else (t1, n1)
    return {"value": round(per_unit / tn, 6), "unit": unit, "cores": cores, "kind": "port",
            "sample": f"{sample}; {nn} units on {cores} threads, {n1} on 1",
            "one_thread": {"value": round(per_unit / t1, 6), "cores": 1,
                           "us_per_unit": round(t1 * 1e6, 1)},
            "us_per_unit": round(tn * 1e6, 1), "what": what,
            "host": {"cpu_model": model, "usable_cores": cores, "numpy": np.__version__,
                     "blas": blas, "blas_threads_used": 1}}


def _f32_linear(codes, cb, sc, x32):
    """The reference's decode-then-matmul on the CPU (vq_dense.py:132-137,
    288-294): W = fp16(cb[codes] * s), cast to fp32, x @ W.T in fp32."""
    from oracle import vq_oracle as vo
    return x32 @ vo.dequant(codes, cb, sc, 64).astype(np.float32).T


def cpu_baseline(w, budget_s=16.0):
    """The MoE decode layer on the host: per token, softmax/top-k routing,
    then per routed expert unpack + fp16 dequant + fp32 matvecs of gate, up
    and down with SwiGLU between, and the weighted combine; the experts are
    the parallel tasks."""
    sys.path.insert(0, ROOT)
    from oracle import vq_oracle as vo
    H, I, d, K, bits, k = w["H"], w["I"], w["d"], w["K"], w["bits"], w["k"]
    rng = np.random.default_rng(7)
    pool = 2 * k          # experts generated for the sample; per-token work equals E's
    projs = {}
    for name, (o, i) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
        codes = rng.integers(0, K, (pool, o, i // d)).astype(np.uint16)
        projs[name] = {"packed": vo.pack(codes, bits), "nsub": i // d,
                       "codebook": (rng.standard_normal((K, d)) * 0.02).astype(np.float16),
                       "scales": rng.uniform(0.5, 1.5, (pool, o, i // 64)).astype(np.float16)}
    xs = rng.standard_normal((64, H)).astype(np.float32)
    lgs = rng.standard_normal((64, pool)).astype(np.float32)

    def lin(name, e, v):
        p = projs[name]
        codes = vo.unpack(p["packed"][e], p["nsub"], bits)
        return _f32_linear(codes, p["codebook"], p["scales"][e], v[None])[0]

    def expert(e, x):
        g, u = lin("gate", e, x), lin("up", e, x)
        return lin("down", e, (g / (1 + np.exp(-g)) * u).astype(np.float32))

    def units(n):
        x, lg = xs[n % 64], lgs[n % 64]
        ids, wt = vo.route(lg[None], k)
        tasks = [lambda e=int(e): expert(e, x) for e in ids[0]]
        return tasks, lambda ys: sum(float(a) * y for a, y in zip(wt[0], ys))

    return _cpu_report(units, budget_s, k * expert_bytes(w) / 1e9, "GB/s",
                       "MoE decode token-layer: routing + unpack, fp16 dequant and fp32 matvecs "
                       "of the routed experts (the reference's decode-then-matmul)",
                       f"token-layers of the benchmark's shape (H {H}, I {I}, top-{k}, d{d} "
                       f"K{K} {bits}-bit; an expert pool of {pool}, since per-token work does "
                       f"not depend on E)")


def cpu_prefill_baseline(w, budget_s=16.0):
    """Dense prefill on the host: fp16 dequant of weight rows + fp32 GEMM
    with a block of tokens; row blocks are the parallel tasks."""
    from oracle import vq_oracle as vo
    rng = np.random.default_rng(7)
    H, d, K = w["H"], w["d"], w["K"]
    rows, ntok, nblk = 64, 256, 8
    codes = rng.integers(0, K, (nblk, rows, H // d)).astype(np.uint16)
    cb = (rng.standard_normal((K, d)) * 0.02).astype(np.float16)
    sc = rng.uniform(0.5, 1.5, (nblk, rows, H // 64)).astype(np.float16)
    x = rng.standard_normal((ntok, H)).astype(np.float32)

    def units(n):
        return [lambda b=b: _f32_linear(codes[b], cb, sc[b], x) for b in range(nblk)], \
            lambda ys: None

    return _cpu_report(units, budget_s, 2.0 * nblk * rows * H * ntok / 1e12, "TFLOP/s",
                       "dense VQ prefill: fp16 dequant + fp32 GEMM (the reference's "
                       "decode-then-matmul)",
                       f"{nblk} x {rows} weight rows of the {H}-wide linear (d{d} K{K}) "
                       f"against {ntok} tokens per unit")


def cpu_gemv_baseline(w, budget_s=16.0):
    """Dense VQ GEMV on the host: fp16 dequant + fp32 matvec of the whole
    4096 x 4096 weight; 8 row blocks are the parallel tasks."""
    from oracle import vq_oracle as vo
    rng = np.random.default_rng(11)
    OUT, IN, d, K, G = w["OUT"], w["IN"], w["d"], w["K"], w["G"]
    codes = rng.integers(0, K, (OUT, IN // d)).astype(np.uint8)
    cb = (rng.standard_normal((K, d)) * 0.02).astype(np.float16)
    sc = rng.uniform(0.5, 1.5, (OUT, IN // G)).astype(np.float16)
    x = rng.standard_normal((1, IN)).astype(np.float32)
    blk = OUT // 8

    def units(n):
        return [lambda b=b: _f32_linear(codes[b * blk:(b + 1) * blk], cb,
                                        sc[b * blk:(b + 1) * blk], x) for b in range(8)], \
            lambda ys: None

    packed = OUT * (IN // d) + OUT * (IN // G) * 2
    return _cpu_report(units, budget_s, packed / 1e9, "GB/s",
                       "dense VQ GEMV: fp16 dequant + fp32 matvec",
                       f"calls of the full {OUT}x{IN} GEMV (d{d} K{K} uint8 codes)")


def _check_linear(torch, lin, x, y, cols, what):
    """Sampled output check outside the timed region: rows `cols` of the
    module decoded by libvqk's bit-exact dequant (itself pinned against the
    oracle by the tests), cast to x's dtype as the reference does
    (vq_dense.py:294), multiplied in fp32 by torch, against y's columns
    (rtol 2e-2 / atol 1e-3). The oracle is not used outside the CPU baseline."""
    from vqlab_amd.vq_switch import wdec_decode
    ci = torch.as_tensor(cols, device=y.device)
    w = torch.cat([wdec_decode(lin.codes, lin.codebook, lin.vq_scales, 1, lin.input_dims,
                               lin.group_size, lin.pack_bits, r0=int(c)) for c in cols])
    ref = x.float() @ w.to(x.dtype if x.dtype != torch.float32 else torch.float16).float().T
    got = y.float().index_select(-1, ci)
    if not torch.allclose(got, ref, rtol=2e-2, atol=1e-3):
        raise SystemExit(f"{what}: output differs from the dequant-then-matmul check")


def _graph_time(torch, step, warmup, steps, dev):
    """Warm up eagerly, capture `steps` calls of step(s) in one HIP graph,
    replay it between HIP events on the capture stream. -> (wall s, event ms)."""
    for s in range(warmup):
        step(s)
    torch.cuda.synchronize()
    cap = torch.cuda.Stream(device=dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cap):
        with torch.cuda.graph(graph, stream=cap):
            for s in range(warmup, warmup + steps):
                step(s)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    with torch.cuda.stream(cap):
        ev0.record(cap)
        graph.replay()
        ev1.record(cap)
    torch.cuda.synchronize()
    return time.perf_counter() - t0, ev0.elapsed_time(ev1)


def _skipzero_proj(torch, dev, g, e, out, inn, d, K, bits, dead):
    """Routed projection with `dead` of its rows all-zero, stored compact:
    codes [n_live, WPR] + scales [n_live, NGRP] + row table [e, out]."""
    from vqlab_amd.vq_switch import VQSwitchLinear
    wpr = ((inn // d) + 31) // 32 * bits
    live = torch.rand((e, out), device=dev, generator=g) >= dead
    n_live = int(live.sum().item())
    rt = torch.full((e, out), -1, dtype=torch.int32, device=dev)
    rt[live] = torch.arange(n_live, dtype=torch.int32, device=dev)
    codes = torch.randint(-2**31, 2**31 - 1, (n_live, wpr), dtype=torch.int32, device=dev,
                          generator=g)
    cb = (torch.randn((K, d), device=dev, generator=g) * 0.02).to(torch.float16)
    sc = (torch.rand((n_live, inn // 64), device=dev, generator=g) + 0.5).to(torch.float16)
    return VQSwitchLinear(codes, cb, sc, pack_bits=bits, in_features=inn, row_table=rt)


def run_mtp(torch, dev, a, w):
    """c4: MTP verify batch through the skipzero config-3 layer: one
    vqk_moe_decode_layer call per layer (routing, one sort, grouped GEMMs,
    combine on device), or with --mtp-path composed torch's routing and
    combine around per-projection grouped calls."""
    from vqlab_amd.moe import VQSparseMoeBlock, VQSwitchGLU
    from vqlab_amd.vq_switch import VQSwitchLinear
    g = torch.Generator(device=dev)
    g.manual_seed(1234)
    H, E, I, k, d, K, bits, T, L = (w[n] for n in ("H", "E", "I", "k", "d", "K", "bits", "T",
                                                    "layers"))
    log(f"building {L} layers of {w['desc']}")
    layers, live_rows = [], []
    for _ in range(L):
        gp, up, dn = (_skipzero_proj(torch, dev, g, E, o, i, d, K, bits, w["dead"])
                      for o, i in ((I, H), (I, H), (H, I)))
        live_rows.append([(p.row_table >= 0).sum(1).cpu().numpy() for p in (gp, up, dn)])

        def dense(o, i):
            wpr = ((i // d) + 31) // 32 * bits
            return VQSwitchLinear(
                torch.randint(-2**31, 2**31 - 1, (1, o, wpr), dtype=torch.int32, device=dev,
                              generator=g),
                (torch.randn((K, d), device=dev, generator=g) * 0.02).to(torch.float16),
                (torch.rand((1, o, i // 64), device=dev, generator=g) + 0.5).to(torch.float16),
                pack_bits=bits, in_features=i)
        sh = VQSwitchGLU(dense(I, H), dense(I, H), dense(H, I))
        sg = (torch.randn((H,), device=dev, generator=g) * 0.02).to(torch.bfloat16)
        layers.append(VQSparseMoeBlock(VQSwitchGLU(gp, up, dn), k, True, sh, sg))
    total = a.warmup + a.steps
    xs = [torch.randn((T, H), device=dev, generator=g).to(torch.bfloat16) for _ in range(L)]
    if w.get("routing") == "capped":
        rng = np.random.default_rng(4321)
        logits = torch.from_numpy(np.stack([np.stack([mtp_logits(rng, T, E, k) for _ in range(L)])
                                            for _ in range(total)])).to(dev)
    else:
        logits = torch.randn((total, L, T, E), device=dev, generator=g)
    ys = [None] * L

    def step(s):
        for l in range(L):
            if a.mtp_path == "composed":
                ys[l] = layers[l].composed(xs[l], logits[s, l])
            else:
                ys[l] = layers[l].fused(xs[l], logits[s, l])

    wall, ev_ms = _graph_time(torch, step, a.warmup, a.steps, dev)
    # bytes of the live rows of the experts each call touched (+ the shared expert)
    wpr_h, wpr_i = ((H // d) + 31) // 32 * bits, ((I // d) + 31) // 32 * bits
    row_gu, row_dn = wpr_h * 4 + (H // 64) * 2, wpr_i * 4 + (I // 64) * 2
    top = torch.topk(logits[a.warmup:].float(), k, dim=-1).indices.cpu().numpy()
    packed, flop, touched = 0, 0.0, 0
    for s in range(a.steps):
        for l in range(L):
            u = np.unique(top[s, l])
            lr = live_rows[l]
            touched += len(u)
            packed += int(lr[0][u].sum() + lr[1][u].sum()) * row_gu + int(lr[2][u].sum()) * row_dn
            # 2 FLOP per weight of each live row, once per routed pair
            e = top[s, l].ravel()
            flop += 2.0 * (float(lr[0][e].sum() + lr[1][e].sum()) * H + float(lr[2][e].sum()) * I)
    packed += a.steps * L * (2 * I * row_gu + H * row_dn)          # shared expert
    flop += a.steps * L * T * 2.0 * 3 * H * I
    calls = a.steps * L
    alg_per_call = packed / calls + 6 * K * d * 2 + T * (2 * H * 2 + E * 4)
    us_call = ev_ms * 1e3 / calls
    achieved = alg_per_call / (us_call * 1e-6) / 1e9
    value = packed / wall / 1e9
    tfs = flop / calls / (us_call * 1e-6) / 1e12
    cpu = None if a.no_cpu else cpu_baseline(dict(w, shared=False))
    return {
        "metric": "packed-weight GB/s (% of HBM peak) and µs/call for the MTP-verify MoE layer",
        "value": round(value, 2), "unit": "GB/s", "dtype": "fp16",
        "config": {"workload": w["desc"], "hidden": H, "experts": E, "intermediate": I,
                   "top_k": k, "shared_expert": True, "d": d, "K": K, "index_bits": bits,
                   "group": 64, "tokens": T, "dead_row_frac": w["dead"], "io_dtype": "bf16",
                   "layers_rotated": L, "routing": w.get("routing", "iid N(0,1) logits"),
                   "touched_experts_per_call": round(touched / calls, 1)},
        "us_per_call": round(wall * 1e6 / calls, 3),
        "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "mfma": {"achieved": round(tfs, 2), "peak": MFMA_F16_PEAK_TFS, "unit": "TFLOP/s",
                 "frac": round(tfs / MFMA_F16_PEAK_TFS, 4), "flop_per_call": int(flop / calls)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": (measured_traffic(f"mtp_verify_{a.workload}_traffic.md")
                                 if a.mtp_path == "fused" else None),
                     "traffic_source": "profiles/mtp_verify_<workload>_traffic.md",
                     "kernel": "k_seg_persist (routed gate/up/down) + k_seg_mfma (shared expert) + routing / sort / combine",
                     "path": a.mtp_path,
                     "alg_bytes_per_call": int(alg_per_call),
                     "us_per_call_events": round(us_call, 3)},
        "cpu_baseline": cpu,
    }, wall, calls


def run_dense_gemv(torch, dev, a, w):
    """c1: one dense VQ GEMV per call (VQLinear, N = 1 -> vqk_dense_gemv), over
    `layers` distinct weights (1.07 GB, four times the 256 MB MALL) so every call
    streams its weight from HBM."""
    from vqlab_amd.vq_dense import VQLinear
    g = torch.Generator(device=dev)
    g.manual_seed(1234)
    OUT, IN, d, K, G, L = (w[n] for n in ("OUT", "IN", "d", "K", "G", "layers"))
    log(f"building {L} linears of {w['desc']}")
    lins, xs = [], []
    for _ in range(L):
        codes = torch.randint(0, K, (OUT, IN // d), dtype=torch.int32, device=dev,
                              generator=g).to(torch.uint8)
        cb = (torch.randn((K, d), device=dev, generator=g) * 0.02).to(torch.float16)
        sc = (torch.rand((OUT, IN // G), device=dev, generator=g) + 0.5).to(torch.float16)
        lins.append(VQLinear(codes, cb, sc, group_size=G, pack_bits=0))
        xs.append(torch.randn((1, IN), device=dev, generator=g).to(torch.bfloat16))
    ys = [None] * L

    def step(s):
        for l in range(L):
            ys[l] = lins[l](xs[l])

    wall, ev_ms = _graph_time(torch, step, a.warmup, a.steps, dev)
    # sanity: the last call of linear 0 (x is narrowed to fp16 by the GEMV,
    # as the reference's fused kernels take it)
    _check_linear(torch, lins[0], xs[0].to(torch.float16), ys[0],
                  [0, 1, 777, 2048, OUT - 2, OUT - 1], "c1")
    calls = a.steps * L
    packed = OUT * (IN // d) + OUT * (IN // G) * 2                 # codes + scales
    alg = packed + K * d * 2 + IN * 2 + OUT * 2                     # + codebook, x, y
    us_call = ev_ms * 1e3 / calls
    cpu = None if a.no_cpu else cpu_gemv_baseline(w)
    return {
        "metric": "packed-weight GB/s (% of HBM peak) of the dense VQ decode GEMV",
        "value": round(packed * calls / wall / 1e9, 2), "unit": "GB/s", "dtype": "fp16",
        "config": {"workload": w["desc"], "out": OUT, "in": IN, "d": d, "K": K,
                   "index_bits": 8, "group": G, "batch": 1, "io_dtype": "bf16",
                   "weights_rotated": L},
        "us_per_call": round(us_call, 3),
        "roofline": {"bound": "hbm", "achieved": round(alg / (us_call * 1e-6) / 1e9, 2),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(alg / (us_call * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic("dense_gemv_c1_traffic.md"),
                     "traffic_source": "profiles/dense_gemv_c1_traffic.md",
                     "kernel": "k_gemv_fast<2, 8, 1> (vqk_dense_gemv)",
                     "alg_bytes_per_call": alg, "us_per_call_events": round(us_call, 3)},
        "cpu_baseline": cpu,
    }, wall, a.steps


def run_prefill(torch, dev, a, w):
    """c5: dense VQ prefill, two linears through VQLinear (vqk_dense_gemm)."""
    from vqlab_amd.vq_dense import VQLinear
    g = torch.Generator(device=dev)
    g.manual_seed(1234)
    N, H, F, d, K = (w[n] for n in ("N", "H", "F", "d", "K"))
    log(f"building {w['desc']}")

    def lin(o, i):
        codes = torch.randint(0, K, (o, i // d), dtype=torch.int32, device=dev,
                              generator=g).to(torch.int16)
        cb = (torch.randn((K, d), device=dev, generator=g) * 0.02).to(torch.float16)
        sc = (torch.rand((o, i // 64), device=dev, generator=g) + 0.5).to(torch.float16)
        return VQLinear(codes, cb, sc, group_size=64, pack_bits=0)
    l1, l2 = lin(F, H), lin(H, F)
    x = torch.randn((N, H), device=dev, generator=g).to(torch.bfloat16)
    out = [None, None]

    def step(s):
        out[0] = l1(x)
        out[1] = l2(out[0])

    wall, ev_ms = _graph_time(torch, step, a.warmup, a.steps, dev)
    # sanity: sampled output columns of both linears (first, last, spread)
    _check_linear(torch, l1, x, out[0], [0, 1, 4099, 9000, F - 2, F - 1], "c5 linear 1")
    _check_linear(torch, l2, out[0], out[1], [0, 1, 2500, H - 2, H - 1], "c5 linear 2")
    flop = 2.0 * 2 * N * H * F
    tfs = flop * a.steps / wall / 1e12
    ev_tfs = flop * a.steps / (ev_ms * 1e-3) / 1e12
    cpu = None if a.no_cpu else cpu_prefill_baseline(w)
    return {
        "metric": "TFLOP/s (% of fp16 MFMA peak) of the dense VQ prefill GEMMs",
        "value": round(tfs, 2), "unit": "TFLOP/s", "dtype": "bf16",   # bf16 GEMM, fp32 accumulate
        "config": {"workload": w["desc"], "tokens": N, "hidden": H, "ffn": F, "d": d, "K": K,
                   "index_bits": 16, "group": 64, "io_dtype": "bf16"},
        "us_per_step_events": round(ev_ms * 1e3 / a.steps, 2),
        "roofline": {"bound": "mfma", "achieved": round(ev_tfs, 2), "peak": MFMA_F16_PEAK_TFS,
                     "unit": "TFLOP/s", "frac": round(ev_tfs / MFMA_F16_PEAK_TFS, 4),
                     "traffic": measured_traffic("dense_prefill_c5_traffic.md",
                                                 "traffic_bytes_per_step"),
                     "traffic_source": "profiles/dense_prefill_c5_traffic.md (per step)",
                     "kernel": "vqk_dense_gemm (both linears)",
                     "flop_per_step": flop},
        "cpu_baseline": cpu,
    }, wall, a.steps


def run_layer(torch, dev, a, w):
    """c2 / c3 / c3b4: one fused MoE decode layer call (vqk_moe_decode_layer:
    routing, gate/up, SwiGLU, down, combine on device) per layer per step,
    over `layers` distinct random layers, captured in one HIP graph."""
    g = torch.Generator(device=dev)
    g.manual_seed(1234)
    L, T, E, H, k = w["layers"], w["T"], w["E"], w["H"], w["k"]
    log(f"building {L} layers of {w['desc']}")
    layers = [make_layer(torch, dev, w, g) for _ in range(L)]
    xs = [(torch.randn((T, H), device=dev, generator=g)).to(torch.bfloat16) for _ in range(L)]
    total = a.warmup + a.steps
    logits = torch.randn((total, L, T, E), device=dev, generator=g)
    ys = [torch.empty((T, H), dtype=torch.bfloat16, device=dev) for _ in range(L)]
    ids_all = torch.empty((total, L, T, k), dtype=torch.int32, device=dev)
    w_all = torch.empty((total, L, T, k), dtype=torch.float32, device=dev)

    import ctypes
    from vqlab_amd import _lib as LB, _torch as TT
    keeps, descs, wss = [], [], []
    for blk in layers:
        keep = []
        d = blk._fused_desc(keep)
        ws = ctypes.c_size_t()
        LB.check(LB.lib().vqk_moe_decode_layer_workspace(ctypes.byref(d), T, ctypes.byref(ws)))
        wbuf = torch.zeros(ws.value, dtype=torch.uint8, device=dev)   # header starts zeroed
        keeps.append(keep)
        descs.append(d)
        wss.append((wbuf, ws.value))

    def step(s, stream):
        for l in range(L):
            LB.check(LB.lib().vqk_moe_decode_layer(
                ctypes.byref(descs[l]), TT.ptr(xs[l]), LB.VQK_BF16, T, TT.ptr(logits[s, l]),
                TT.ptr(ys[l]), LB.VQK_BF16, TT.ptr(ids_all[s, l]), TT.ptr(w_all[s, l]),
                TT.ptr(wss[l][0]), wss[l][1], stream))

    # warmup eagerly (also raises the kernels' LDS limits before capture)
    st = TT.stream(dev)
    for s in range(a.warmup):
        step(s, st)
    torch.cuda.synchronize()
    cap = torch.cuda.Stream(device=dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(cap):
        with torch.cuda.graph(graph, stream=cap):
            cst = TT.stream(dev)
            for s in range(a.warmup, total):
                step(s, cst)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.cuda.stream(cap):
        ev0.record(cap)
        graph.replay()
        ev1.record(cap)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ev_ms = ev0.elapsed_time(ev1)

    # unique experts touched per layer call (token-expert pairs share weights)
    ids_t = ids_all[a.warmup:].cpu().numpy()                  # [steps, L, T, k]
    uniq = sum(len(np.unique(ids_t[s, l])) for s in range(a.steps) for l in range(L))
    shared_calls = a.steps * L if w["shared"] else 0
    packed_bytes = (uniq + shared_calls) * expert_bytes(w)
    calls = a.steps * L
    cb_bytes = 3 * w["K"] * w["d"] * 2 * (2 if w["shared"] else 1)
    act_bytes = (T * H * 2 + T * E * 4 + T * H * 2)            # x in, logits, y out
    alg_per_call = packed_bytes / calls + cb_bytes + act_bytes
    value = packed_bytes / wall / 1e9
    us_call = ev_ms * 1e3 / calls
    achieved = alg_per_call / (us_call * 1e-6) / 1e9

    # sanity: the routing the kernels used is the top-k of the logits (first
    # timed call; N(0,1) logits have no ties)
    rid = torch.topk(logits[a.warmup, 0].float(), k, dim=-1).indices.cpu().numpy()
    if not np.array_equal(ids_t[0, 0], rid):
        raise SystemExit("device routing differs from the logits' top-k")

    cpu = None if a.no_cpu else cpu_baseline(w)
    out = {
        "metric": "packed-weight GB/s (% of HBM peak) and µs/token for MoE VQ decode layer",
        "value": round(value, 2), "unit": "GB/s", "dtype": "fp16",
        "config": {"workload": w["desc"], "hidden": H, "experts": E, "intermediate": w["I"],
                   "top_k": k, "shared_expert": w["shared"], "d": w["d"], "K": w["K"],
                   "index_bits": w["bits"], "group": 64, "batch": T, "io_dtype": "bf16",
                   "layers_rotated": L,
                   "resident_weight_GB": round(L * (E + (1 if w["shared"] else 0))
                                               * expert_bytes(w) / 1e9, 3)},
        "us_per_token_layer": round(wall * 1e6 / calls, 3),
        "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(f"moe_layer_{a.workload}_traffic.md"),
                     "traffic_source": "profiles/moe_layer_<workload>_traffic.md (rocprofv3 "
                                       "FETCH_SIZE + WRITE_SIZE per dispatch, copy-calibrated)",
                     "kernel": ("k_moe_layer1 (the layer in one launch)" if T == 1 and not w["shared"]
                                and w["d"] in (2, 4) and 8 <= w["bits"] <= 12 and E <= 256
                                else "k_moe_up (or k_moe_up_split) + k_moe_down (one fused layer call)"),
                     "alg_bytes_per_call": int(alg_per_call), "us_per_call_events": round(us_call, 3)},
        "cpu_baseline": cpu,
    }
    # tables beyond LDS: the codes past the LDS part are gathered from L2, whose
    # 16 channels per XCD take one request per clock (0.5 per clock per CU);
    # the committed counter profile gives the L1 -> L2 read requests per call
    req = measured_traffic(f"moe_layer_{a.workload}_traffic.md", "l2_read_requests_per_call")
    cap = measured_traffic("moe_layer_c3_traffic.md", "l2_request_cap_per_us_per_cu")
    if req:
        floor_us = req / (L2_REQ_PER_CLK_PER_CU * N_CUS * PEAK_CLOCK_GHZ * 1e3)
        out["roofline"]["l2_request_floor"] = {
            "requests_per_call": req, "floor_us": round(floor_us, 2),
            "achieved_us": round(us_call, 3), "frac": round(floor_us / us_call, 4),
            "basis": f"{L2_REQ_PER_CLK_PER_CU} L2 requests per clock per CU x {N_CUS} CUs x "
                     f"{PEAK_CLOCK_GHZ} GHz (published peak clock)"}
        if cap:
            mfloor = req / (cap * N_CUS)
            out["roofline"]["l2_request_floor"].update({
                "measured_cap_floor_us": round(mfloor, 2),
                "measured_cap_frac": round(mfloor / us_call, 4),
                "measured_cap_basis": f"{cap} L1->L2 requests per us per CU, the gather probe's "
                                      "rate (bench.py --workload gather)"})
    return out, wall, calls


def _summary(name, body):
    """The per-workload figures of the default line's `workloads` object."""
    r = body["roofline"]
    out = {"workload": body["config"]["workload"],
           "us_per_call": r.get("us_per_call_events"),
           "value": body["value"], "unit": body["unit"],
           "roofline_frac": r["frac"], "roofline_unit": r["unit"],
           "achieved": r["achieved"], "traffic": r.get("traffic"),
           "alg_bytes_per_call": r.get("alg_bytes_per_call"), "kernel": r.get("kernel")}
    if "us_per_step_events" in body:
        out["us_per_step"] = body["us_per_step_events"]
    if "mfma" in body:
        out["mfma_frac"] = body["mfma"]["frac"]
        out["touched_experts_per_call"] = body["config"]["touched_experts_per_call"]
    if "l2_request_floor" in r:
        out["l2_request_floor"] = r["l2_request_floor"]
    return out


# every BASELINE config beside the headline: (workload, timed steps)
EXTRA_WORKLOADS = [("c1", 20), ("c3", 20), ("c3b4", 10), ("c4t16", 10), ("c4t16capped", 10),
                   ("c4", 8), ("c4capped", 8), ("c5", 5)]


def extra_workloads(torch, dev, a):
    """Each other configuration timed in this process with HIP events (a few
    steps each, no CPU baseline): µs per call, roofline fraction, traffic."""
    res = {}
    for name, steps in EXTRA_WORKLOADS:
        w = WORKLOADS[name]
        sub = argparse.Namespace(**vars(a))
        sub.workload, sub.steps, sub.warmup, sub.no_cpu, sub.mtp_path = name, steps, 3, True, "fused"
        t0 = time.perf_counter()
        try:
            body, _, _ = RUNNERS[w.get("kind", "layer")](torch, dev, sub, w)
            res[name] = _summary(name, body)
        except Exception as e:                      # reported, never hidden
            res[name] = {"error": f"{type(e).__name__}: {e}"}
        res[name]["seconds"] = round(time.perf_counter() - t0, 1)
        log(f"workload {name}: {res[name]}")
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return res


def run_gather(torch, dev, a, w):
    """The random-gather rate the hardware sustains from an L2-resident table
    (libvqk's vqk__probe_gather test hook): the codebook reads beyond the LDS
    part of the config-3 / config-4 kernels and the config-5 dequant. Reported
    as 16-byte gathers per us per CU at 4, 8 and 16 waves per CU."""
    import ctypes
    from vqlab_amd import _lib as LB, _torch as TT
    lib = LB.lib()
    lib.vqk__probe_gather.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    ncu = torch.cuda.get_device_properties(dev).multi_processor_count
    table = torch.randint(0, 2**31 - 1, (1 << 18,), dtype=torch.int32, device=dev)   # 1 MiB
    sink = torch.empty(ncu * 4 * 256, dtype=torch.int32, device=dev)
    st = TT.stream(dev)
    rows = []
    for kb in (256, 1024):
        for wpc in (4, 8, 16):
            for inflight in (1, 8):
                wgs, rounds = ncu * wpc // 4, 200
                LB.check(lib.vqk__probe_gather(TT.ptr(table), kb << 10, wgs, inflight, 4, TT.ptr(sink), st))
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                LB.check(lib.vqk__probe_gather(TT.ptr(table), kb << 10, wgs, inflight, rounds,
                                               TT.ptr(sink), st))
                e1.record()
                torch.cuda.synchronize()
                us = e0.elapsed_time(e1) * 1e3
                rate = wgs * 256 * rounds * inflight / us / ncu
                rows.append({"table_kb": kb, "waves_per_cu": wpc, "loads_in_flight": inflight,
                             "gathers_per_us_per_cu": round(rate, 1)})
                log(rows[-1])
    best = max(r["gathers_per_us_per_cu"] for r in rows if r["table_kb"] == 256)
    return {"metric": "random 16-byte gathers per us per CU from an L2-resident table",
            "value": best, "unit": "gathers/us/CU", "dtype": "u32",
            "config": {"workload": w["desc"], "cus": ncu},
            "rates": rows,
            "roofline": {"bound": "l2", "achieved": best, "peak": None, "unit": "gathers/us/CU",
                         "frac": None},
            "cpu_baseline": None}, 0.0, 1


def run_stream(torch, dev, a, w):
    """The fastest one-launch read of config 1's weight bytes (libvqk's
    vqk__probe_stream test hook: 16-byte loads, one word written per
    workgroup), launched back to back in a HIP graph over rotating buffers
    like the c1 workload: the floor of a decode GEMV that must read those
    bytes in one launch, at several grid sizes."""
    import ctypes
    from vqlab_amd import _lib as LB, _torch as TT
    lib = LB.lib()
    lib.vqk__probe_stream.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p,
                                      ctypes.c_void_p]
    nb, L = w["bytes"], w["layers"]
    bufs = [torch.randint(0, 2**31 - 1, (nb // 4,), dtype=torch.int32, device=dev) for _ in range(L)]
    sink = torch.empty(8192, dtype=torch.int32, device=dev)
    rows = []
    for wgs in (512, 1024, 2048, 4096, 8192):
        def step(s, wgs=wgs):
            st = TT.stream(dev)
            for b in bufs:
                LB.check(lib.vqk__probe_stream(TT.ptr(b), nb, wgs, TT.ptr(sink), st))
        steps = max(1, a.steps // 10)
        _, ev_ms = _graph_time(torch, step, 2, steps, dev)
        us = ev_ms * 1e3 / (steps * L)
        rows.append({"workgroups": wgs, "us_per_launch": round(us, 3), "GBps": round(nb / us / 1e3, 1)})
        log(rows[-1])
    best = min(rows, key=lambda r: r["us_per_launch"])
    return {"metric": "us per launch of a streaming read of config 1's weight bytes",
            "value": best["us_per_launch"], "unit": "us", "higher_is_better": False, "dtype": "u32",
            "config": {"workload": w["desc"], "bytes": nb, "buffers": L},
            "grids": rows,
            "roofline": {"bound": "hbm", "achieved": best["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(best["GBps"] / HBM_PEAK_GBS, 4)},
            "cpu_baseline": None}, 0.0, 1


def _launch_us(torch, dev, wgs, launches, reps=5):
    """µs per launch of vqk__probe_stream over one 16-byte buffer (one load,
    one word written per workgroup) at `wgs` workgroups, `launches` back to
    back on one stream, `reps` times over in one HIP graph."""
    import ctypes
    from vqlab_amd import _lib as LB, _torch as TT
    lib = LB.lib()
    lib.vqk__probe_stream.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_void_p,
                                      ctypes.c_void_p]
    buf = torch.zeros(4, dtype=torch.int32, device=dev)
    sink = torch.empty(max(wgs, 1), dtype=torch.int32, device=dev)

    def step(s):
        st = TT.stream(dev)
        for _ in range(launches):
            LB.check(lib.vqk__probe_stream(TT.ptr(buf), 16, wgs, TT.ptr(sink), st))
    _, ev_ms = _graph_time(torch, step, 2, reps, dev)
    return round(ev_ms * 1e3 / (reps * launches), 3)


def run_launch(torch, dev, a, w):
    """The kernel boundary: vqk__probe_stream over one 16-byte buffer,
    launched back to back on one stream in a HIP graph at several grid sizes.
    Each launch waits for the previous one to end, as a layer call waits for
    the layer before it, so the time per launch is what dispatch, the
    end-of-kernel release and the next start cost together (plus the probe's
    own load and store)."""
    L = w["launches"]
    rows = []
    for wgs in (1, 128, 384, 1024):
        rows.append({"workgroups": wgs, "us_per_launch": _launch_us(torch, dev, wgs, L)})
        log(rows[-1])
    best = min(rows, key=lambda r: r["us_per_launch"])
    return {"metric": "us per back-to-back launch of a kernel that reads 16 bytes",
            "value": best["us_per_launch"], "unit": "us", "higher_is_better": False, "dtype": "u32",
            "config": {"workload": w["desc"], "launches": L},
            "grids": rows, "roofline": None, "cpu_baseline": None}, 0.0, 1


RUNNERS = {"layer": run_layer, "mtp": run_mtp, "prefill": run_prefill, "dense_gemv": run_dense_gemv,
           "gather": run_gather, "stream": run_stream, "launch": run_launch}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="c2", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-workloads", action="store_true",
                    help="default workload only: skip the other configurations' figures")
    ap.add_argument("--mtp-path", default="fused", choices=("fused", "composed"),
                    help="c4 workloads: the layer entry point, or torch glue around grouped calls")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (each GPU would "
              "hold its own experts or row shards and run these kernels on its share).",
              file=sys.stderr)
        sys.exit(2)
    import torch
    sys.path.insert(0, ROOT)
    import vqlab_amd
    vqlab_amd.load()
    w = WORKLOADS[a.workload]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    body, wall, _ = RUNNERS[w.get("kind", "layer")](torch, dev, a, w)
    out = {"metric": body.pop("metric"), "value": body.pop("value"), "unit": body.pop("unit"),
           "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
           "ms_per_step": round(wall * 1e3 / a.steps, 5), "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": body.pop("dtype"),
           "data": "synthetic (random VQ weights, N(0,1) activations and router logits; "
                   "no checkpoints offline)"}
    out.update(body)
    if a.workload == "c2" and not a.no_workloads:
        out["workloads"] = extra_workloads(torch, dev, a)
        try:
            out["kernel_boundary"] = {
                "us_per_launch": _launch_us(torch, dev, 384, 1000), "workgroups": 384,
                "what": "back-to-back launches in a HIP graph of a kernel that loads 16 bytes and "
                        "stores one word per workgroup, at this layer's grid (--workload launch): "
                        "the part of each layer call that any dependent launch pays"}
        except Exception as e:                      # reported, never hidden
            out["kernel_boundary"] = {"error": f"{type(e).__name__}: {e}"}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
