"""Benchmark of the VQ MoE decode layer on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload c2|c3|c3b4|c1]

Default workload: a Qwen3.6-35B-A3B-shaped MoE
decode layer -- hidden 2048, 256 experts of intermediate 512, top-8 softmax
router on N(0,1) logits, SwiGLU gate/up/down, VQ d=4, K=4096 (12-bit packed
indices), one fp16 codebook per projection, fp16 scales per 64 weights,
batch 1, bf16 activations. Weights are random (no checkpoints offline), in
8 distinct layers (2.6 GB) so every call streams its experts from HBM
rather than the 256 MB MALL.

A step is one decode token through the 8-layer stack: per layer, one fused
call (device routing + gate/up/SwiGLU + down/combine, two kernels) with that
step's own logits. The timed steps are captured once in a HIP graph and
replayed; HIP events on the launch stream bracket the replay.

value = packed-weight GB/s: bytes of the codes and scales of the experts the
router touched (SURVEY 8(d) first term), summed over every layer call, over
the timed wall time. roofline uses the layer call's total algorithmic bytes
(codes + scales + codebooks + activations) over its event-timed duration.
cpu_baseline: the repository's numpy oracle of the same layer (unpack ->
fp16 dequant -> float64 matmuls), single-threaded, on a bounded sample.
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
    # name: (H, E, I, top_k, shared, d, K, bits, T, layers)
    "c2": dict(H=2048, E=256, I=512, k=8, shared=False, d=4, K=4096, bits=12, T=1, layers=8,
               desc="Qwen3.6-35B-A3B-shaped MoE decode layer (BASELINE configs[1])"),
    "c3": dict(H=4096, E=512, I=1024, k=10, shared=True, d=8, K=16384, bits=14, T=1, layers=4,
               desc="Qwen3.5-397B-A17B-shaped MoE decode layer, B=1 (BASELINE configs[2])"),
    "c3b4": dict(H=4096, E=512, I=1024, k=10, shared=True, d=8, K=16384, bits=14, T=4, layers=4,
                 desc="Qwen3.5-397B-A17B-shaped MoE decode layer, B=4 (BASELINE configs[2])"),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


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


def cpu_baseline(w, budget_s=12.0):
    """Numpy oracle of one token-layer (decode-then-matmul), single thread."""
    try:
        from threadpoolctl import threadpool_limits
    except ImportError:
        threadpool_limits = None
    sys.path.insert(0, ROOT)
    from oracle import vq_oracle as vo
    H, I, d, K, bits, k = w["H"], w["I"], w["d"], w["K"], w["bits"], w["k"]
    rng = np.random.default_rng(7)
    pool = 2 * k          # experts generated for the sample; per-token work equals E's
    projs = {}
    for name, (o, i) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
        codes = rng.integers(0, K, (pool, o, i // d)).astype(np.uint16)
        projs[name] = {"packed": vo.pack(codes, bits), "codebook":
                       (rng.standard_normal((K, d)) * 0.02).astype(np.float16),
                       "scales": rng.uniform(0.5, 1.5, (pool, o, i // 64)).astype(np.float16),
                       "group": 64, "nsub": i // d}
    xs = rng.standard_normal((64, H)).astype(np.float32)
    lgs = rng.standard_normal((64, pool)).astype(np.float32)

    def token_layer(x, lg):
        spec = {}
        ids, _ = vo.route(lg[None], k)
        for name, p in projs.items():
            codes = np.zeros(p["scales"].shape[:2] + (p["nsub"],), np.uint16)
            for e in ids[0]:                      # unpack only the touched experts
                codes[e] = vo.unpack(p["packed"][e:e + 1], p["nsub"], bits)[0]
            spec[name] = {"codes": codes, "codebook": p["codebook"], "scales": p["scales"],
                          "group": 64}
        return vo.moe_layer(x[None], lg[None], spec["gate"], spec["up"], spec["down"], k)[0]

    ctx = threadpool_limits(1) if threadpool_limits else None
    n, t0 = 0, time.perf_counter()
    try:
        if ctx:
            ctx.__enter__()
        while n < 64 and (n < 3 or time.perf_counter() - t0 < budget_s):
            token_layer(xs[n], lgs[n])
            n += 1
    finally:
        if ctx:
            ctx.__exit__(None, None, None)
    dt = (time.perf_counter() - t0) / n
    gbs = k * expert_bytes(w) / dt / 1e9
    return {"value": round(gbs, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "us_per_token_layer": round(dt * 1e6, 1),
            "sample": f"{n} token-layers of the same shape (numpy oracle: unpack + fp16 dequant "
                      f"of the {k} routed experts + float64 matmuls, 1 thread; expert pool "
                      f"{pool} since per-token work does not depend on E)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="c2", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(see DESIGN.md, 'How the path would shard').", file=sys.stderr)
        sys.exit(2)
    import torch
    sys.path.insert(0, ROOT)
    import vqlab_amd
    vqlab_amd.load()
    w = WORKLOADS[a.workload]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
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
        wbuf = torch.empty(ws.value, dtype=torch.uint8, device=dev)
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

    # sanity: the routing the kernels used is the oracle's (first timed call)
    from oracle import vq_oracle as vo
    rid, _ = vo.route(logits[a.warmup, 0].cpu().numpy(), k)
    assert np.array_equal(ids_t[0, 0], rid), "device routing differs from the oracle"

    cpu = None if a.no_cpu else cpu_baseline(w)
    out = {
        "metric": "packed-weight GB/s (% of HBM peak) and µs/token for MoE VQ decode layer",
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": a.steps,
        "warmup": a.warmup, "ms_per_step": round(wall * 1e3 / a.steps, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic (random VQ weights and N(0,1) router logits; no checkpoints offline)",
        "config": {"workload": w["desc"], "hidden": H, "experts": E, "intermediate": w["I"],
                   "top_k": k, "shared_expert": w["shared"], "d": w["d"], "K": w["K"],
                   "index_bits": w["bits"], "group": 64, "batch": T, "io_dtype": "bf16",
                   "layers_rotated": L,
                   "resident_weight_GB": round(L * (E + (1 if w["shared"] else 0))
                                               * expert_bytes(w) / 1e9, 3)},
        "us_per_token_layer": round(wall * 1e6 / calls, 3),
        "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "k_moe_up + k_moe_down (one fused layer call)",
                     "alg_bytes_per_call": int(alg_per_call), "us_per_call_events": round(us_call, 3)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
