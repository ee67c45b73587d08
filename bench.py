"""Benchmark of the gated-attention decode path on one MI355X.

Workload: split-KV flash-decoding, 1 query row, 24 Q / 4 KV heads, head_dim 256, bf16 KV
~ N(0,1) at KV lengths 4096 / 16384 / 32768. One "step" is one decode step's attention layers:
16 layer-calls (attn_decode = partials + gated combine), each on its own KV cache, captured in
one hipGraph and replayed. The KV buffers rotate over >= 512 MB so the 256 MB Infinity Cache
cannot serve repeated reads. Inputs are resident in HBM before timing starts.

Printed (one JSON line): value = microseconds per layer-call at KV 16384 (the shortest length
the >= 75 %-of-HBM target applies to), the sweep at every length, the roofline of the dominant
kernel (the split-KV partials kernel, timed with HIP events on its stream over a graph of its
own launches), and the CPU baseline (the reference's PyTorch attention path restated in
oracle/, on this host's cores, bounded sample).

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--lengths 4096,16384,32768]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HQ, HKV, D = 24, 4, 256
LAYERS = 16
ROTATE_BYTES = 512 * 2 ** 20
HBM_PEAK_GBS = 8000.0
HEADLINE_L = 16384
METRIC = "decode-attn µs/layer + achieved HBM GB/s (% of 8 TB/s) at KV 1k–128k"


def alg_bytes_layer(L: int, n: int = 1) -> int:
    """Algorithmic bytes of one decode layer-call: K+V once (4096 B per position for 4 KV heads
    x 256 dims x 2 tensors x 2 B) plus q, gate and out (12,288 B each per row)."""
    return 4096 * L + 36864 * n


def alg_bytes_partials(L: int, n: int = 1) -> int:
    """Algorithmic bytes of the split-KV partials kernel: K+V once plus the q rows."""
    return 4096 * L + 12288 * n


def build_if_missing():
    import importlib.util
    spec = importlib.util.spec_from_file_location("qe_build", ROOT / "qengine_amd" / "_build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    if not mod.built():
        mod.build()


class LayerSet:
    """LAYERS layer-calls on distinct KV caches of length L (one graph)."""

    def __init__(self, torch, C, L: int, ns: int, gen):
        dev = "cuda"
        BF = torch.bfloat16
        self.kc = [torch.randn(HKV, L, D, device=dev, generator=gen).to(BF) for _ in range(LAYERS)]
        self.vc = [torch.randn(HKV, L, D, device=dev, generator=gen).to(BF) for _ in range(LAYERS)]
        self.q = torch.randn(1, HQ * D, device=dev, generator=gen).to(BF)
        self.qg = torch.randn(1, HQ * 2 * D, device=dev, generator=gen).to(BF)
        self.out = torch.empty(1, HQ * D, dtype=BF, device=dev)
        self.po = torch.empty(1, HQ, ns, D, device=dev)
        self.pml = torch.empty(1, HQ, ns, 2, device=dev)
        self.pos = torch.tensor([L - 1], dtype=torch.int32, device=dev)
        self.C = C

    def decode_all(self):
        for k, v in zip(self.kc, self.vc):
            self.C.attn_decode(self.q, k, v, self.pos, self.qg, self.po, self.pml, self.out)

    def partials_all(self):
        for k, v in zip(self.kc, self.vc):
            self.C.attn_decode_partials(self.q, k, v, self.pos, self.qg, self.po, self.pml,
                                        self.out)

    def combine_all(self):
        """The combine alone, LAYERS times on the partials of the last layer-call."""
        for k, v in zip(self.kc, self.vc):
            self.C.attn_decode_combine(self.q, k, v, self.pos, self.qg, self.po, self.pml,
                                       self.out)


def fp8_codes(torch, shape, gen):
    """E4M3FN codes of N(0,1) values at scale 1/16 (code = RNE(16 x), saturated at 448)."""
    x = torch.randn(*shape, device="cuda", generator=gen) * 16
    return x.clamp_(-448, 448).to(torch.float8_e4m3fn)


class LayerSet8(LayerSet):
    """The same layer-calls on fp8 KV caches (scale 1/16, the bf16 legs' N(0,1) data quantized:
    the same values after dequantization): half the bytes per position."""

    def __init__(self, torch, C, L: int, ns: int, gen):
        dev = "cuda"
        BF = torch.bfloat16

        def codes():
            return fp8_codes(torch, (HKV, L, D), gen)
        self.kc = [codes() for _ in range(LAYERS)]
        self.vc = [codes() for _ in range(LAYERS)]
        self.q = torch.randn(1, HQ * D, device=dev, generator=gen).to(BF)
        self.qg = torch.randn(1, HQ * 2 * D, device=dev, generator=gen).to(BF)
        self.out = torch.empty(1, HQ * D, dtype=BF, device=dev)
        self.po = torch.empty(1, HQ, ns, D, device=dev)
        self.pml = torch.empty(1, HQ, ns, 2, device=dev)
        self.pos = torch.tensor([L - 1], dtype=torch.int32, device=dev)
        self.C = C

    def decode_all(self):
        for k, v in zip(self.kc, self.vc):
            self.C.attn_decode_fp8(self.q, k, v, self.pos, self.qg, self.po, self.pml, self.out,
                                   1 / 16, 1 / 16)

    def partials_all(self):
        for k, v in zip(self.kc, self.vc):
            self.C.attn_decode_fp8_partials(self.q, k, v, self.pos, self.qg, self.po, self.pml,
                                            self.out, 1 / 16, 1 / 16)


def bench_length_fp8(torch, C, qa, L: int, steps: int, warmup: int) -> dict:
    """fp8 KV decode at KV length L: layer-call and partials-only µs; bytes = 2048*L (+ q)."""
    ns = qa.default_splits(L, HKV, kv8=True)
    nsets = max(1, math.ceil(ROTATE_BYTES / (LAYERS * L * 2048)))
    gen = torch.Generator(device="cuda").manual_seed(L + 8)
    sets = [LayerSet8(torch, C, L, ns, gen) for _ in range(nsets)]
    full = [capture(torch, s.decode_all) for s in sets]
    part = [capture(torch, s.partials_all) for s in sets]
    us_layer = time_graphs(torch, full, steps, warmup).median * 1e3 / LAYERS
    us_part = time_graphs(torch, part, steps, warmup).median * 1e3 / LAYERS
    b_layer = 2048 * L + 36864
    b_part = 2048 * L + 12288
    del sets, full, part
    torch.cuda.empty_cache()
    return {"us_per_layer": round(us_layer, 3), "GBps": round(b_layer / (us_layer * 1e3), 1),
            "kv_rotation_MB": round(nsets * LAYERS * L * 2048 / 2 ** 20, 1),
            "partials_us": round(us_part, 3),
            "partials_GBps": round(b_part / (us_part * 1e3), 1),
            "partials_frac": round(b_part / (us_part * 1e3) / HBM_PEAK_GBS, 4)}


def capture(torch, fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm-up outside capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


# (workgroups per KV head, 16-byte loads in flight per thread and tensor) of the floor sweep;
# on MI355X the fastest 67-134 MB reads used >= 512 workgroups and 4-8 loads
STREAM_SWEEP = ((52, 16), (64, 16), (128, 4), (128, 8), (256, 4), (256, 8), (512, 4), (512, 8))
MIN_WARMUP_REPLAYS = 30  # the reference's time_graph warms each graph up 30 times
MIN_WARMUP_SECONDS = 0.1  # and at least this long per graph: clocks ramp over tens of ms
# MFMA-bound graphs (the prefill legs) take longer to reach steady clocks: after 0.1 s of replays
# the first timing of a prefill graph read 5-10% slow in same-process A/Bs on MI355X
MIN_WARMUP_SECONDS_MFMA = 1.0
# prefill calls per graph: a model's prefill runs its attention layers back to back in one graph,
# as the decode legs time 16 layer-calls per graph; one call per graph adds the graph launch to
# every call (reported as *_1call)
PREFILL_CALLS = 8


class Timing:
    """Per-replay graph timings in ms: ``mean`` over the bracketed run of exactly ``steps``
    replays, and the median / min / max of the individual replays (HIP events between replays on
    the stream the graphs run on)."""

    def __init__(self, mean: float, per: list):
        per = sorted(per)
        self.mean, self.median, self.min, self.max = mean, statistics.median(per), per[0], per[-1]

    def us(self, div: int = 1) -> dict:
        return {k: round(getattr(self, k) * 1e3 / div, 3) for k in ("median", "mean", "min", "max")}


def time_graphs(torch, graphs, steps: int, warmup: int,
                min_seconds: float = MIN_WARMUP_SECONDS) -> Timing:
    """The reference's graph timing (bench/engine/micro_kernels.py:16-32): at least 30 warm-up
    replays (and at least ``min_seconds`` of them), then ``steps`` timed replays (graphs
    round-robin), each bracketed by events on the current stream, the one the graphs' kernels
    run on."""
    t0, i = time.perf_counter(), 0
    while i < max(warmup, MIN_WARMUP_REPLAYS) or time.perf_counter() - t0 < min_seconds:
        for _ in range(10):
            graphs[i % len(graphs)].replay()
            i += 1
        torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    ev[0].record()
    for i in range(steps):
        graphs[i % len(graphs)].replay()
        ev[i + 1].record()
    torch.cuda.synchronize()
    per = [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]
    return Timing(ev[0].elapsed_time(ev[steps]) / steps, per)


def warm_device(torch, seconds: float = 1.0) -> float:
    """At least ``seconds`` of streaming reads before the first timed graph, so clocks and HBM
    have left idle (the reference warms up before timing: micro_kernels.py:16-32)."""
    import qengine_amd.capi as capi
    buf = torch.ones(256 * 2 ** 20 // 4, dtype=torch.int32, device="cuda")
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(50):
            capi.hbm_read_probe(buf, buf.numel() * 4, sink)
        torch.cuda.synchronize()
    del buf
    return time.perf_counter() - t0


def bench_length(torch, C, qa, L: int, steps: int, warmup: int, ns: int | None):
    """Layer-calls at KV length L (16 per graph on distinct caches, >= 512 MB in rotation): the
    whole op, its partials kernel alone, its combine alone (on partials already written), and
    the two ceilings measured the same way: the streaming probe on the partials grid (the K/V
    bytes, no arithmetic) and an empty launch."""
    import qengine_amd.capi as capi
    ns = ns or qa.default_splits(L, HKV)
    nsets = max(1, math.ceil(ROTATE_BYTES / (LAYERS * L * 4096)))
    gen = torch.Generator(device="cuda").manual_seed(L)
    sets = [LayerSet(torch, C, L, ns, gen) for _ in range(nsets)]
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")

    def probe_all(s):
        for k, v in zip(s.kc, s.vc):
            capi.kv_stream_probe(k, v, s.pos, HKV, L, ns, sink)

    def sweep_all(s, gph, depth):
        for k, v in zip(s.kc, s.vc):
            capi.kv_stream_sweep(k, v, s.pos, HKV, L, gph, depth, sink)
    full = [capture(torch, s.decode_all) for s in sets]
    part = [capture(torch, s.partials_all) for s in sets]
    probe = [capture(torch, lambda s=s: probe_all(s)) for s in sets]
    comb = [capture(torch, s.combine_all) for s in sets]
    t_full = time_graphs(torch, full, steps, warmup)
    t_part = time_graphs(torch, part, steps, warmup)
    t_probe = time_graphs(torch, probe, steps, warmup)
    t_comb = time_graphs(torch, comb, steps, warmup)
    us_layer = t_full.median * 1e3 / LAYERS
    us_part = t_part.median * 1e3 / LAYERS
    us_probe = t_probe.median * 1e3 / LAYERS
    # the one-launch floor whatever the grid: the same bytes swept over grid size (workgroups per
    # KV head) and loads in flight per thread; the fastest configuration is the floor
    stream = {}
    for gph, depth in STREAM_SWEEP:
        gs = [capture(torch, lambda s=s: sweep_all(s, gph, depth)) for s in sets]
        stream[f"{gph}x{depth}"] = round(
            time_graphs(torch, gs, steps, warmup).median * 1e3 / LAYERS, 3)
        del gs
    best = min(stream, key=stream.get)
    res = {
        "L": L, "NS": ns, "split_size": qa.split_size(L, ns), "kv_rotation_MB":
            round(nsets * LAYERS * L * 4096 / 2 ** 20, 1),
        "ms_per_step": t_full.mean, "ms_per_step_median": t_full.median,
        "us_per_layer": us_layer, "us_per_layer_stats": t_full.us(LAYERS),
        "GBps": alg_bytes_layer(L) / (us_layer * 1e3),
        "partials_us": us_part, "partials_us_stats": t_part.us(LAYERS),
        "partials_GBps": alg_bytes_partials(L) / (us_part * 1e3),
        "partials_us_mean": t_part.mean * 1e3 / LAYERS,
        "kv_stream_probe_us": us_probe,
        "stream_sweep_us": stream,
        "best_stream_us": stream[best], "best_stream_cfg": best,
        "combine_us": t_comb.median * 1e3 / LAYERS,
    }
    res["frac"] = res["GBps"] / HBM_PEAK_GBS
    res["partials_frac"] = res["partials_GBps"] / HBM_PEAK_GBS
    del sets, full, part, probe, comb
    torch.cuda.empty_cache()
    return res


def ceiling(sweep, node_us: float) -> dict:
    """What any design can reach on this box, per KV length, in µs per graph node: the fastest
    streaming read of the K/V bytes over a sweep of grids and load depths is the floor of one
    launch that reads them (best_stream_us); the same read on the partials kernel's own grid is
    kv_stream_probe_us; adding one empty graph node gives the floor of a two-launch layer-call
    (partials + combine); the combine alone is what this build's second node costs; the BASELINE
    target is 75% of 8 TB/s on the algorithmic bytes."""
    out = {"graph_node_us": round(node_us, 3), "per_L": {}}
    for r in sweep:
        L = r["L"]
        out["per_L"][str(L)] = {
            "best_stream_us": r["best_stream_us"], "best_stream_cfg": r["best_stream_cfg"],
            "kv_stream_probe_us": round(r["kv_stream_probe_us"], 3),
            "one_launch_floor_us": r["best_stream_us"],
            "two_launch_floor_us": round(r["best_stream_us"] + node_us, 3),
            "partials_us": round(r["partials_us"], 3),
            "partials_minus_best_stream_us": round(r["partials_us"] - r["best_stream_us"], 3),
            "measured_us": round(r["us_per_layer"], 3),
            "measured_minus_two_launch_floor_us": round(
                r["us_per_layer"] - r["best_stream_us"] - node_us, 3),
            "combine_alone_us": round(r["combine_us"], 3),
            "target_75pct_us": round(alg_bytes_layer(L) / (0.75 * HBM_PEAK_GBS * 1e3), 3)}
    return out


def launch_floor_us(torch, steps: int, warmup: int) -> float:
    """µs per node of a graph of 16 empty launches: what every kernel in a graph pays."""
    import qengine_amd.capi as capi

    def run():
        for _ in range(LAYERS):
            capi.launch_probe()
    return time_graphs(torch, [capture(torch, run)], steps, warmup).median * 1e3 / LAYERS


def time_fn_graph(torch, fn, steps: int, warmup: int,
                  min_seconds: float = MIN_WARMUP_SECONDS) -> float:
    """ms per replay (median) of a graph capturing fn()."""
    return time_graphs(torch, [capture(torch, fn)], steps, warmup, min_seconds).median


def rotated(bytes_per_set: int) -> int:
    """Sets of LAYERS caches (one graph each, replayed round-robin) so that >= 512 MB of distinct
    KV bytes rotate: the 256 MB Infinity Cache cannot serve a repeated read."""
    return max(1, math.ceil(ROTATE_BYTES / bytes_per_set))


def time_sets(torch, fns, steps: int, warmup: int) -> float:
    """ms per replay (median) over one graph per set, replayed round-robin."""
    return time_graphs(torch, [capture(torch, f) for f in fns], steps, warmup).median


def bench_configs(torch, C, qa, steps: int, warmup: int) -> dict:
    """The other BASELINE configs, each timed as graph replays on the GPU (values per call). Every
    HBM-bound leg rotates >= 512 MB of distinct KV (kv_rotation_MB)."""
    dev, BF = "cuda", torch.bfloat16
    gen = torch.Generator(device=dev).manual_seed(1)
    res = {}

    def rnd(*shape, scale=1.0):
        return (torch.randn(*shape, device=dev, generator=gen) * scale).to(BF)

    inv = (1.0 / (1e7 ** (torch.arange(0, 64, 2, dtype=torch.float32) / 64))).to(dev)
    qnw, knw = rnd(D, scale=0.3), rnd(D, scale=0.3)

    # cfg 1: prep + decode, one row at KV 1024, 16 layers per step
    L, nl = 1024, 16
    nsets = rotated(nl * L * 4096)
    sets = [([rnd(HKV, L, D) for _ in range(nl)], [rnd(HKV, L, D) for _ in range(nl)])
            for _ in range(nsets)]
    rot_mb = round(nsets * nl * L * 4096 / 2 ** 20, 1)
    proj = rnd(1, HQ * 2 * D + 2 * HKV * D + 8, scale=3.0)
    qg, k, v = proj[:, :HQ * 2 * D], proj[:, HQ * 2 * D:HQ * 2 * D + HKV * D], proj[:, HQ * 2 * D + HKV * D:HQ * 2 * D + 2 * HKV * D]
    q = torch.empty(1, HQ * D, dtype=BF, device=dev)
    out = torch.empty(1, HQ * D, dtype=BF, device=dev)
    ns = qa.default_splits(L, HKV)
    po, pml = qa.alloc_partials(1, HQ, ns, dev)
    pos = torch.tensor([L - 1], dtype=torch.int32, device=dev)

    def cfg1(kcs, vcs):
        for kk, vv in zip(kcs, vcs):
            C.attn_prep(qg, k, v, qnw, knw, inv, pos, q, kk, vv, 1e-6)
            C.attn_decode(q, kk, vv, pos, qg, po, pml, out)
    us = time_sets(torch, [lambda s=s: cfg1(*s) for s in sets], steps, warmup) * 1e3 / nl
    res["cfg1_prep_decode_1k"] = {"us_per_layer": round(us, 3),
                                  "GBps": round((alg_bytes_layer(L) + 45056) / (us * 1e3), 1),
                                  "kv_rotation_MB": rot_mb}

    def cfg1_fused(kcs, vcs):
        for kk, vv in zip(kcs, vcs):
            C.attn_prep_decode(qg, k, v, qnw, knw, inv, pos, q, kk, vv, 1e-6, po, pml, out)
    us = time_sets(torch, [lambda s=s: cfg1_fused(*s) for s in sets], steps, warmup) * 1e3 / nl
    res["cfg1_prep_decode_1k_fused"] = {"us_per_layer": round(us, 3),
                                        "GBps": round((alg_bytes_layer(L) + 45056) / (us * 1e3), 1),
                                        "kv_rotation_MB": rot_mb}
    del sets

    # prep + decode per layer at KV 16384 (16 layers on distinct caches), separate and fused ops
    L, nl = 16384, 16
    kcs = [rnd(HKV, L, D) for _ in range(nl)]
    vcs = [rnd(HKV, L, D) for _ in range(nl)]
    ns16 = qa.default_splits(L, HKV)
    po16, pml16 = qa.alloc_partials(1, HQ, ns16, dev)
    pos16 = torch.tensor([L - 1], dtype=torch.int32, device=dev)

    def sep16():
        for kk, vv in zip(kcs, vcs):
            C.attn_prep(qg, k, v, qnw, knw, inv, pos16, q, kk, vv, 1e-6)
            C.attn_decode(q, kk, vv, pos16, qg, po16, pml16, out)

    def fused16():
        for kk, vv in zip(kcs, vcs):
            C.attn_prep_decode(qg, k, v, qnw, knw, inv, pos16, q, kk, vv, 1e-6, po16, pml16, out)
    for name, fn in (("prep_decode_16k", sep16), ("prep_decode_16k_fused", fused16)):
        us = time_fn_graph(torch, fn, steps, warmup) * 1e3 / nl
        res[name] = {"us_per_layer": round(us, 3),
                     "GBps": round((alg_bytes_layer(L) + 45056) / (us * 1e3), 1),
                     "kv_rotation_MB": round(nl * L * 4096 / 2 ** 20, 1)}
    del kcs, vcs

    # cfg 3: MTP verify, 5 rows at pos 4096 over 4096 cached + 5 new positions
    L, n, nl = 4096 + 5, 5, 16
    nsets = rotated(nl * L * 4096)
    sets = [([rnd(HKV, L, D) for _ in range(nl)], [rnd(HKV, L, D) for _ in range(nl)])
            for _ in range(nsets)]
    q5, qg5 = rnd(n, HQ * D), rnd(n, HQ * 2 * D)
    out5 = torch.empty(n, HQ * D, dtype=BF, device=dev)
    ns = qa.default_splits(L, HKV)
    po5, pml5 = qa.alloc_partials(n, HQ, ns, dev)
    pos5 = torch.tensor([4096], dtype=torch.int32, device=dev)

    def cfg3(kcs, vcs):
        for kk, vv in zip(kcs, vcs):
            C.attn_decode(q5, kk, vv, pos5, qg5, po5, pml5, out5)
    us = time_sets(torch, [lambda s=s: cfg3(*s) for s in sets], steps, warmup) * 1e3 / nl
    res["cfg3_mtp_verify_5rows_4k"] = {"us_per_layer": round(us, 3),
                                       "GBps": round(alg_bytes_layer(L, n) / (us * 1e3), 1),
                                       "kv_rotation_MB": round(nsets * nl * L * 4096 / 2 ** 20, 1)}
    del sets

    # MTP verify at 8 rows (7 drafts) at pos 4096 and 16384, on bf16 and on fp8 caches: 48 columns
    # at GQA 6, the multi-column kernel (its fp8 mode for the second)
    def codes(L):
        return fp8_codes(torch, (HKV, L, D), gen)
    for P in (4096, 16384):
        L, n, nl = P + 8, 8, 16
        q8, qg8 = rnd(n, HQ * D), rnd(n, HQ * 2 * D)
        out8 = torch.empty(n, HQ * D, dtype=BF, device=dev)
        pos8 = torch.tensor([P], dtype=torch.int32, device=dev)
        for fp8 in (False, True):
            ns = qa.default_splits(L, HKV, kv8=fp8)
            po8, pml8 = qa.alloc_partials(n, HQ, ns, dev)
            per_pos = 2048 if fp8 else 4096
            nsets = rotated(nl * L * per_pos)
            sets = [([codes(L) if fp8 else rnd(HKV, L, D) for _ in range(nl)],
                     [codes(L) if fp8 else rnd(HKV, L, D) for _ in range(nl)])
                    for _ in range(nsets)]

            def verify8(kcs, vcs, fp8=fp8, po8=po8, pml8=pml8):
                for kk, vv in zip(kcs, vcs):
                    if fp8:
                        C.attn_decode_fp8(q8, kk, vv, pos8, qg8, po8, pml8, out8, 1 / 16, 1 / 16)
                    else:
                        C.attn_decode(q8, kk, vv, pos8, qg8, po8, pml8, out8)
            us = time_sets(torch, [lambda s=s: verify8(*s) for s in sets], steps, warmup) * 1e3 / nl
            nbytes = (2048 * L + 36864 * n) if fp8 else alg_bytes_layer(L, n)
            res[f"{'fp8kv_' if fp8 else ''}verify_8rows_{P // 1024}k"] = {
                "us_per_layer": round(us, 3), "GBps": round(nbytes / (us * 1e3), 1),
                "kv_rotation_MB": round(nsets * nl * L * per_pos / 2 ** 20, 1)}
            del sets

    # cfg 4: KV 131072 (537 MB per layer: two layers rotate past the Infinity Cache), plus the
    # variant with 1% of key rows scaled by 8
    L, nl = 131072, 2
    kcs = [rnd(HKV, L, D) for _ in range(nl)]
    vcs = [rnd(HKV, L, D) for _ in range(nl)]
    q1, qg1 = rnd(1, HQ * D), rnd(1, HQ * 2 * D)
    ns = qa.default_splits(L, HKV)
    po1, pml1 = qa.alloc_partials(1, HQ, ns, dev)
    pos1 = torch.tensor([L - 1], dtype=torch.int32, device=dev)
    for name in ("cfg4_long_128k", "cfg4_long_128k_keys_x8"):
        if name.endswith("x8"):
            idx = torch.randperm(L, device=dev, generator=gen)[: L // 100]
            for kk in kcs:
                kk[:, idx] = (kk[:, idx].float() * 8).to(BF)

        def cfg4():
            for kk, vv in zip(kcs, vcs):
                C.attn_decode(q1, kk, vv, pos1, qg1, po1, pml1, out)
        us = time_fn_graph(torch, cfg4, steps, warmup) * 1e3 / nl
        res[name] = {"us_per_layer": round(us, 3), "GBps": round(alg_bytes_layer(L) / (us * 1e3), 1),
                     "hbm_frac": round(alg_bytes_layer(L) / (us * 1e3) / HBM_PEAK_GBS, 4),
                     "kv_rotation_MB": round(nl * L * 4096 / 2 ** 20, 1)}
    del kcs, vcs

    # one row attending 4096 positions of 131072-position caches (a cache sized for long context,
    # early in a generation), 16 layers: the slices follow the attended length, so this runs like
    # the 4096-position sweep entry, not like a 131072-position cache cut into fixed slices
    Lc, La, nl = 131072, 4096, 16
    nsets = rotated(nl * La * 4096)  # the attended prefixes rotate

    def cache_pair():
        kk = torch.empty(HKV, Lc, D, dtype=BF, device=dev)
        vv = torch.empty(HKV, Lc, D, dtype=BF, device=dev)
        kk[:, :La] = rnd(HKV, La, D)
        vv[:, :La] = rnd(HKV, La, D)
        return kk, vv
    sets = [list(zip(*[cache_pair() for _ in range(nl)])) for _ in range(nsets)]
    ns = qa.default_splits(Lc, HKV)
    poc, pmlc = qa.alloc_partials(1, HQ, ns, dev)
    posc = torch.tensor([La - 1], dtype=torch.int32, device=dev)

    def short_in_long(kcs, vcs):
        for kk, vv in zip(kcs, vcs):
            C.attn_decode(q1, kk, vv, posc, qg1, poc, pmlc, out)
    us = time_sets(torch, [lambda s=s: short_in_long(*s) for s in sets], steps, warmup) * 1e3 / nl
    res["decode_4k_in_128k_cache"] = {"us_per_layer": round(us, 3),
                                      "GBps": round(alg_bytes_layer(La) / (us * 1e3), 1),
                                      "kv_rotation_MB": round(nsets * nl * La * 4096 / 2 ** 20, 1)}
    del sets

    for L in (4096, 16384, 32768, 131072):
        res[f"fp8kv_decode_{L // 1024}k"] = bench_length_fp8(torch, C, qa, L, steps, warmup)
    res.update(bench_prefill(torch, C, steps, warmup))
    res.update(bench_gemv(torch, C, qa, steps, warmup))
    res.update(bench_step_ops(torch, C, steps, warmup))
    res.update(bench_gdn(torch, C, steps, warmup))
    return res


def bench_gemv(torch, C, qa, steps: int, warmup: int) -> dict:
    """The projections on either side of the attention path (F1's neighbours): in_proj
    [14336 x 5120] and o_proj [5120 x 6144] GEMV at 1 and 5 rows, each call on a different copy
    of the weights (>= 600 MB in rotation, past the 256 MB Infinity Cache); plus the streaming
    read probe over 2 GiB, the achievable HBM read rate on the same box."""
    import qengine_amd.capi as capi
    dev, BF = "cuda", torch.bfloat16
    gen = torch.Generator(device=dev).manual_seed(2)
    res = {}
    for name, N, K in (("gemv_in_proj_14336x5120", 14336, 5120),
                       ("gemv_o_proj_5120x6144", 5120, 6144)):
        wbytes = N * K * 2
        copies = max(4, -(-600 * 2 ** 20 // wbytes))
        Ws = [(torch.randn(N, K, device=dev, generator=gen) * K ** -0.5).to(BF)
              for _ in range(copies)]
        for nr in (1, 5):
            x = torch.randn(nr, K, device=dev, generator=gen).to(BF)
            out = torch.empty(nr, N, dtype=BF, device=dev)

            def run():
                for W in Ws:
                    C.gemv_bf16(W, x, out)
            us = time_fn_graph(torch, run, steps, warmup) * 1e3 / copies
            gbps = wbytes / (us * 1e3)
            res[f"{name}_rows{nr}"] = {"us": round(us, 3), "GBps": round(gbps, 1),
                                       "hbm_frac": round(gbps / HBM_PEAK_GBS, 4),
                                       "kparts": capi.gemv_kparts(N, K),
                                       "tile_rows": capi.gemv_tile_rows(N, K)}
        del Ws
    nbytes = 2 * 2 ** 30
    buf = torch.ones(nbytes // 4, dtype=torch.int32, device=dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    us = time_fn_graph(torch, lambda: capi.hbm_read_probe(buf, nbytes, sink), steps, warmup) * 1e3
    res["hbm_read_probe_2GiB"] = {"us": round(us, 2), "GBps": round(nbytes / (us * 1e3), 1),
                                  "hbm_frac": round(nbytes / (us * 1e3) / HBM_PEAK_GBS, 4)}
    del buf
    return res


def bench_step_ops(torch, C, steps: int, warmup: int) -> dict:
    """The rest of a decode step at the reference model's shapes (hidden 5120, intermediate
    17408, vocab 248320): embed, rmsnorm1p with the fused residual, swiglu, argmax (two launches),
    accept + commit. Each is 16 calls per graph on rotating buffers; values are per call. These
    kernels are launch- and latency-bound (2-20 KB per row, 0.5 MB per logits row)."""
    dev, BF, I32 = "cuda", torch.bfloat16, torch.int32
    gen = torch.Generator(device=dev).manual_seed(4)
    H, I, V, nl = 5120, 17408, 248320, 16
    res = {}

    def per_call(fn):
        return round(time_fn_graph(torch, fn, steps, warmup) * 1e3 / nl, 3)

    tab = torch.randn(V, H, device=dev, generator=gen).to(BF)
    tok = torch.randint(0, V, (8,), device=dev, generator=gen, dtype=I32)
    outs = [torch.empty(8, H, dtype=BF, device=dev) for _ in range(nl)]
    for n in (1, 5):
        res[f"embed_rows{n}"] = {"us": per_call(lambda: [C.embed(tab, tok, o[:n]) for o in outs])}
    del tab
    xs = [torch.randn(8, H, device=dev, generator=gen).to(BF) for _ in range(nl)]
    ds = [torch.randn(8, H, device=dev, generator=gen).to(BF) for _ in range(nl)]
    w = torch.randn(H, device=dev, generator=gen).to(BF)
    for n in (1, 5):
        res[f"rmsnorm1p_residual_rows{n}"] = {
            "us": per_call(lambda: [C.rmsnorm1p(x[:n], d[:n], w, o[:n], 1e-6)
                                    for x, d, o in zip(xs, ds, outs)])}
    gus = [torch.randn(8, 2 * I, device=dev, generator=gen).to(BF) for _ in range(nl)]
    acts = [torch.empty(8, I, dtype=BF, device=dev) for _ in range(nl)]
    for n in (1, 5):
        us = per_call(lambda: [C.swiglu(g[:n], a[:n]) for g, a in zip(gus, acts)])
        res[f"swiglu_rows{n}"] = {"us": us, "GBps": round(n * I * 6 / (us * 1e3), 1)}
    del gus, acts
    lgs = [torch.randn(8, V, device=dev, generator=gen).to(BF) for _ in range(nl)]
    wv, wi = torch.empty(8 * 256, device=dev), torch.empty(8 * 256, dtype=I32, device=dev)
    am = torch.empty(8, dtype=I32, device=dev)
    for n in (1, 5):
        us = per_call(lambda: [C.argmax(lg[:n], wv[:n * 256], wi[:n * 256], am) for lg in lgs])
        res[f"argmax_vocab_rows{n}"] = {"us": us, "GBps": round(n * V * 2 / (us * 1e3), 1)}
    del lgs
    ctl = torch.zeros(32, dtype=I32, device=dev)
    in_tok = torch.zeros(9, dtype=I32, device=dev)
    nt, dr = torch.zeros(8, dtype=I32, device=dev), torch.zeros(8, dtype=I32, device=dev)
    log = torch.zeros(1 << 20, dtype=I32, device=dev)
    res["accept_commit_rows5"] = {"us": per_call(lambda: [(C.accept(in_tok, am, 5, ctl, nt, log),
                                                           C.commit(ctl, in_tok, am, dr, 4))
                                                          for _ in range(nl)])}
    return res


GDN_HK, GDN_HV, GDN_LAYERS = 16, 48, 48


def gdn_alg_bytes(n: int, pend: int, hk: int = GDN_HK, hv: int = GDN_HV) -> int:
    """Algorithmic HBM bytes of one gdn_step_n call: the fp32 state read and written back (the
    write only when rows are replayed), the replayed and the newly staged rows (k, v, decay,
    beta in fp32), conv weights, the 3-position ring history and the n ring slots written, and
    the bf16 rows qkv / z / b / a in and out."""
    Cd, Vd = 2 * hk * 128 + hv * 128, hv * 128
    state = hv * 128 * 128 * 4 * (2 if pend > 0 else 1)
    staged = (pend + n) * hv * (128 + 128 + 2) * 4
    conv = Cd * 4 * 2 + 3 * Cd * 2 + n * Cd * 2
    rows = n * (Cd + Vd + 2 * hv) * 2 + n * Vd * 2
    return state + staged + conv + rows + hv * 2 * 2 + 128 * 2


def bench_gdn(torch, C, steps: int, warmup: int, rows=(1, 2, 4, 6, 8)) -> dict:
    """Gated DeltaNet step (gdn_step_n) at the reference model's shapes (Hk 16, Hv 48: 48 value
    heads with a 128 x 128 fp32 state, 3 MB per layer), the way the reference times it
    (bench/engine/micro_kernels.py:35-56): 48 layer-calls per graph on separate states, with
    pending = n staged rows replayed by every call. Two graphs alternate over 2 x 48 states
    (about 360 MB) so the 256 MB Infinity Cache cannot hold them; values are per call."""
    dev, BF, I32 = "cuda", torch.bfloat16, torch.int32
    hk, hv, nl = GDN_HK, GDN_HV, GDN_LAYERS
    Cd, Vd = 2 * hk * 128 + hv * 128, hv * 128
    w = Cd + Vd + 2 * hv
    gen = torch.Generator(device=dev).manual_seed(5)
    pr = (torch.randn(8, (w + 7) // 8 * 8, device=dev, generator=gen) * 0.5).to(BF)
    qkv, z, b, a = pr[:, :Cd], pr[:, Cd:Cd + Vd], pr[:, Cd + Vd:Cd + Vd + hv], pr[:, Cd + Vd + hv:w]
    conv_w = (torch.randn(Cd, 1, 4, device=dev, generator=gen) * 0.3).to(BF)
    A_log = torch.zeros(hv, dtype=BF, device=dev)
    dt = torch.zeros(hv, dtype=BF, device=dev)
    nw = torch.ones(128, dtype=BF, device=dev)
    out = torch.empty(8, Vd, dtype=BF, device=dev)

    def layer():
        return dict(ring=torch.zeros(16, Cd, dtype=BF, device=dev),
                    S=torch.randn(hv, 128, 128, device=dev, generator=gen) * 0.01,
                    st=[torch.zeros(8, hv, 128, device=dev), torch.zeros(8, hv, 128, device=dev),
                        torch.zeros(8, hv, 2, device=dev)])

    def call(Ld, n, ctl):
        C.gdn_step_n(qkv[:n], z[:n], b[:n], a[:n], Ld["ring"], conv_w, A_log, dt, nw, Ld["S"],
                     *Ld["st"], ctl, out[:n], hk, 1e-6)

    res = {}
    for n in rows:
        sets = [[layer() for _ in range(nl)] for _ in range(2)]
        prime = torch.tensor([100, 0, 0, 0, 0, 0, 0, 0], dtype=I32, device=dev)
        ctl = torch.tensor([100, n, 0, 0, 0, 0, 0, 0], dtype=I32, device=dev)
        for s in sets:  # stage n real rows in every layer, then time calls that replay them
            for Ld in s:
                call(Ld, n, prime)
        graphs = [capture(torch, lambda s=s: [call(Ld, n, ctl) for Ld in s]) for s in sets]
        us = time_graphs(torch, graphs, steps, warmup).median * 1e3 / nl
        nb = gdn_alg_bytes(n, n)
        res[f"gdn_step_rows{n}"] = {"us": round(us, 3), "alg_bytes": nb,
                                    "GBps": round(nb / (us * 1e3), 1),
                                    "hbm_frac": round(nb / (us * 1e3) / HBM_PEAK_GBS, 4)}
        del sets, graphs
        torch.cuda.empty_cache()
    return res


def bench_prefill(torch, C, steps: int, warmup: int) -> dict:
    """a 2048-row causal chunk appended to a 2048-position cache (attn_prep_chunk
    + attn_prefill), timed as replays of graphs holding PREFILL_CALLS calls (values per call), and
    of graphs holding one call (``*_1call``). FLOPs = 4 * D * Hq * sum of attended lengths."""
    dev, BF = "cuda", torch.bfloat16
    gen = torch.Generator(device=dev).manual_seed(5)
    res = {}

    def rnd(*shape, scale=1.0):
        return (torch.randn(*shape, device=dev, generator=gen) * scale).to(BF)

    inv = (1.0 / (1e7 ** (torch.arange(0, 64, 2, dtype=torch.float32) / 64))).to(dev)
    qnw, knw = rnd(D, scale=0.3), rnd(D, scale=0.3)
    T, pos0 = 2048, 2048
    L = pos0 + T
    kc, vc = rnd(HKV, L, D), rnd(HKV, L, D)
    projT = rnd(T, HQ * 2 * D + 2 * HKV * D, scale=3.0)
    qgT, kT, vT = projT[:, :HQ * 2 * D], projT[:, HQ * 2 * D:HQ * 2 * D + HKV * D], projT[:, HQ * 2 * D + HKV * D:]
    qT = torch.empty(T, HQ * D, dtype=BF, device=dev)
    outT = torch.empty(T, HQ * D, dtype=BF, device=dev)
    posT = torch.tensor([pos0], dtype=torch.int32, device=dev)
    C.attn_prep_chunk(qgT, kT, vT, qnw, knw, inv, posT, qT, kc, vc, 1e-6)
    flops = 4 * D * HQ * sum(pos0 + 1 + t for t in range(T))
    mw = MIN_WARMUP_SECONDS_MFMA
    nc = PREFILL_CALLS

    def per_call(fn):  # ms per call: graphs of nc calls, and graphs of one
        many = time_fn_graph(torch, lambda: [fn() for _ in range(nc)], steps, warmup, mw) / nc
        return many, time_fn_graph(torch, fn, steps, warmup, mw)

    ms_attn, ms_attn1 = per_call(lambda: C.attn_prefill(qT, kc, vc, posT, qgT, outT))

    def full():
        C.attn_prep_chunk(qgT, kT, vT, qnw, knw, inv, posT, qT, kc, vc, 1e-6)
        C.attn_prefill(qT, kc, vc, posT, qgT, outT)
    ms_full, ms_full1 = per_call(full)
    tflops = flops / (ms_attn * 1e-3) / 1e12
    res["cfg5_prefill_2048_on_2048"] = {
        "us_attention": round(ms_attn * 1e3, 2), "us_prep_plus_attention": round(ms_full * 1e3, 2),
        "calls_per_graph": nc, "us_attention_1call": round(ms_attn1 * 1e3, 2),
        "us_prep_plus_attention_1call": round(ms_full1 * 1e3, 2),
        "GFLOP": round(flops / 1e9, 2), "TFLOPs": round(tflops, 1),
        "mfma_frac_of_2500_TFLOPs_bf16_dense": round(tflops / 2500.0, 4)}

    # the same chunk over an fp8 cache (codes of the bf16 cache at scale 1/16): attn_prep_fp8
    # writes the chunk's codes, attn_prefill_fp8 converts each tile once in LDS
    ks = vs = 1.0 / 16
    kc8 = torch.empty(HKV, L, D, dtype=torch.float8_e4m3fn, device=dev)
    vc8 = torch.empty_like(kc8)
    kc8.copy_((kc.float() * 16).clamp(-448, 448).to(torch.float8_e4m3fn))
    vc8.copy_((vc.float() * 16).clamp(-448, 448).to(torch.float8_e4m3fn))
    C.attn_prep_fp8(qgT, kT, vT, qnw, knw, inv, posT, qT, kc8, vc8, 1e-6, ks, vs)
    ms8, ms8_1 = per_call(lambda: C.attn_prefill_fp8(qT, kc8, vc8, posT, qgT, outT, ks, vs))

    def full8():
        C.attn_prep_fp8(qgT, kT, vT, qnw, knw, inv, posT, qT, kc8, vc8, 1e-6, ks, vs)
        C.attn_prefill_fp8(qT, kc8, vc8, posT, qgT, outT, ks, vs)
    ms8_full, ms8_full1 = per_call(full8)
    tf8 = flops / (ms8 * 1e-3) / 1e12
    res["cfg5_prefill_fp8kv"] = {
        "us_attention": round(ms8 * 1e3, 2), "us_prep_plus_attention": round(ms8_full * 1e3, 2),
        "calls_per_graph": nc, "us_attention_1call": round(ms8_1 * 1e3, 2),
        "us_prep_plus_attention_1call": round(ms8_full1 * 1e3, 2),
        "TFLOPs": round(tf8, 1), "mfma_frac_of_2500_TFLOPs_bf16_dense": round(tf8 / 2500.0, 4)}
    return res


def _median_us(fn, reps: int, warm: int) -> float:
    ts = []
    for i in range(warm + reps):
        t0 = time.perf_counter()
        fn()
        if i >= warm:
            ts.append(time.perf_counter() - t0)
    return statistics.median(ts) * 1e6


def cpu_baseline(torch, lengths=(1024, 4096, 16384, 32768, 131072), reps: int = 5,
                 warm: int = 2) -> dict:
    """The reference's PyTorch attention path (reference.py:252-280, restated op for op in
    oracle/) timed on this host's CPU cores, per layer-call: one decode row at each KV length
    (attention_core, which repeats K/V per GQA group in fp32 as the reference does), config 1 as
    prep + decode at 1024, config 3 (5 causal rows at pos 4096, sequential attention_core calls as
    reference.py:275-280 runs them), and config 5 timed on 64 evenly spaced rows of the 2048-row
    chunk and extrapolated to 2048 rows (labelled). Medians of ``reps`` after ``warm``."""
    import oracle as O
    torch.set_num_threads(os.cpu_count() or 1)
    res = {}
    g = torch.Generator().manual_seed(7)
    bf = torch.bfloat16

    def rnd(*shape, scale=1.0):
        return (torch.randn(*shape, generator=g) * scale).to(bf)
    q, gate = rnd(HQ, D), rnd(HQ * D)
    for L in lengths:
        kc, vc = rnd(HKV, L, D), rnd(HKV, L, D)
        r = reps if L < 131072 else 3
        res[f"decode_{L // 1024}k"] = round(_median_us(lambda: O.attention_core(q, gate, kc, vc, L), r, warm if L < 131072 else 1), 1)
        if L == 1024:
            proj = rnd(1, HQ * 2 * D + 2 * HKV * D, scale=3.0)
            qg1, k1, v1 = proj[:, :HQ * 2 * D], proj[:, HQ * 2 * D:HQ * 2 * D + HKV * D], proj[:, HQ * 2 * D + HKV * D:]
            qnw, knw = rnd(D, scale=0.3), rnd(D, scale=0.3)
            inv = O.rope_inv_freq(1e7, 64)

            def cfg1():
                qq = O.attn_prep(qg1, k1, v1, qnw, knw, inv, L - 1, kc, vc, 1e-6, HQ)
                O.attention_core(qq[0].reshape(HQ, D), gate, kc, vc, L)
            res["cfg1_prep_decode_1k"] = round(_median_us(cfg1, reps, warm), 1)
        del kc, vc
    L3, n3 = 4096 + 5, 5
    kc, vc = rnd(HKV, L3, D), rnd(HKV, L3, D)
    q5, qg5 = rnd(n3, HQ * D), rnd(n3, HQ * 2 * D)
    res["cfg3_mtp_verify_5rows_4k"] = round(_median_us(
        lambda: O.attn_decode(q5, kc, vc, 4096, qg5, HQ, grouped=False), reps, warm), 1)
    T, pos0 = 2048, 2048
    kc, vc = rnd(HKV, pos0 + T, D), rnd(HKV, pos0 + T, D)
    rows = [round(i * (T - 1) / 63) for i in range(64)]

    def cfg5_sample():
        for t in rows:
            O.attention_core(q, gate, kc, vc, pos0 + t + 1)
    us64 = _median_us(cfg5_sample, 3, 1)
    res["cfg5_prefill_2048_on_2048_extrapolated"] = round(us64 * T / len(rows), 1)
    res["cfg5_sample"] = "64 evenly spaced rows of the 2048-row chunk, x 2048/64"
    return res


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def traffic_from_profiles(L: int):
    """HBM bytes per partials launch measured with rocprofv3 counters (profiles/traffic.json,
    written from FETCH_SIZE + WRITE_SIZE runs scaled by a copy-kernel calibration), if present."""
    p = ROOT / "profiles" / "traffic.json"
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text()).get("partials_bytes_per_launch", {}).get(str(L))
    except (ValueError, OSError):
        return None


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=MIN_WARMUP_REPLAYS,
                    help="untimed replays before each timed graph (at least 30 are run)")
    ap.add_argument("--lengths", default="4096,16384,32768")
    ap.add_argument("--ns", type=int, default=0, help="split count (0 = default policy)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only BASELINE config 5 (chunked prefill); prints its timing as JSON")
    ap.add_argument("--fp8-only", action="store_true",
                    help="only the fp8 KV decode sweep (4k-128k), as JSON")
    ap.add_argument("--step-ops-only", action="store_true",
                    help="only embed / rmsnorm1p / swiglu / argmax / accept+commit, as JSON")
    ap.add_argument("--gdn-only", action="store_true",
                    help="only the Gated DeltaNet step at the model's shapes, as JSON")
    ap.add_argument("--gdn-rows", default="1,2,4,6,8",
                    help="row counts of the --gdn-only leg (one profile per row count)")
    ap.add_argument("--gemv-only", action="store_true",
                    help="only the in_proj / o_proj GEMV and the HBM read probe, as JSON")
    ap.add_argument("--sweep-only", action="store_true",
                    help="only the decode sweep over exactly --lengths (one JSON object per "
                         "length); the per-length runs that rocprofv3 profiles")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the other BASELINE configs (1, 3, 4, 5)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run 5 plain device copies of MIB MiB (reads MIB, writes MIB): the "
                         "reference kernel that scales rocprofv3 FETCH_SIZE/WRITE_SIZE to bytes")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build's decode path runs on a single MI355X and "
              "has no multi-GPU mode (run with --gpus 1).", file=sys.stderr)
        sys.exit(2)

    if args.copy_calibration:
        import torch
        n = args.copy_calibration * 2 ** 20 // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_MiB": args.copy_calibration, "launches": 5}))
        return

    build_if_missing()
    import torch
    import qengine_amd as qa
    C = qa._C
    torch.backends.cuda.matmul.allow_tf32 = False
    warm_s = warm_device(torch)
    if args.prefill_only:
        print(json.dumps(bench_prefill(torch, C, args.steps, args.warmup)))
        return
    if args.gemv_only:
        print(json.dumps(bench_gemv(torch, C, qa, args.steps, args.warmup)))
        return
    if args.fp8_only:
        print(json.dumps({f"fp8kv_decode_{L // 1024}k": bench_length_fp8(torch, C, qa, L, args.steps,
                                                                          args.warmup)
                          for L in (4096, 16384, 32768, 131072)}))
        return
    if args.step_ops_only:
        print(json.dumps(bench_step_ops(torch, C, args.steps, args.warmup)))
        return
    if args.gdn_only:
        rows = tuple(int(x) for x in args.gdn_rows.split(",") if x)
        print(json.dumps(bench_gdn(torch, C, args.steps, args.warmup, rows)))
        return
    lengths = [int(x) for x in args.lengths.split(",") if x]
    if args.sweep_only:
        for L in lengths:
            r = bench_length(torch, C, qa, L, args.steps, args.warmup, args.ns or None)
            print(json.dumps({k: (round(v, 4) if isinstance(v, float) else v)
                              for k, v in r.items()}), flush=True)
        return
    if HEADLINE_L not in lengths:
        lengths.append(HEADLINE_L)
    node_us = launch_floor_us(torch, args.steps, args.warmup)
    print(f"# warm-up {warm_s:.2f} s; empty graph node {node_us:.2f} us", file=sys.stderr,
          flush=True)
    sweep = []
    for L in lengths:
        r = bench_length(torch, C, qa, L, args.steps, args.warmup, args.ns or None)
        print(f"# L={L}: {r['us_per_layer']:.2f} us/layer-call, {r['GBps']:.0f} GB/s "
              f"({100 * r['frac']:.1f}%), partials {r['partials_us']:.2f} us "
              f"({100 * r['partials_frac']:.1f}%); stream probe {r['kv_stream_probe_us']:.2f} us"
              f", best stream {r['best_stream_us']:.2f} us ({r['best_stream_cfg']})",
              file=sys.stderr, flush=True)
        sweep.append(r)
    head = next(r for r in sweep if r["L"] == HEADLINE_L)
    configs = None
    if not args.no_configs:
        configs = bench_configs(torch, C, qa, args.steps, args.warmup)
        for k, v in configs.items():
            print(f"# {k}: {v}", file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu:
        per = cpu_baseline(torch)
        cpu = {"value": per[f"decode_{HEADLINE_L // 1024}k"], "unit": "us/layer-call",
               "cores": torch.get_num_threads(), "kind": "port",
               "sample": f"oracle.attention_core (reference.py:263-272 restated in torch, CPU), "
                         f"1 layer-call at KV {HEADLINE_L}, median of 5 after 2 warm-ups; "
                         f"per_config holds every length and configs 1, 3, 5 (5 extrapolated "
                         f"from 64 rows)",
               "per_config_us": per, "cpu_model": cpu_model(), "os_cpu_count": os.cpu_count()}
        print(f"# cpu baseline: {per}", file=sys.stderr, flush=True)

    line = {
        "metric": METRIC,
        "value": round(head["us_per_layer"], 3),
        "unit": "us/layer-call",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "split-KV decode sweep (BASELINE configs[1]), 16 layer-calls "
                               "per step in one hipGraph", "L": HEADLINE_L, "layers_per_step": LAYERS,
                   "hq": HQ, "hkv": HKV, "head_dim": D, "rows": 1, "NS": head["NS"],
                   "split_size": head["split_size"], "kv_rotation_MB": head["kv_rotation_MB"]},
        "achieved_GBps": round(head["GBps"], 1),
        "hbm_frac": round(head["frac"], 4),
        "roofline": {"bound": "hbm", "kernel": "attn_partials_kernel",
                     "achieved": round(alg_bytes_partials(HEADLINE_L) / (head["partials_us_mean"] * 1e3), 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(alg_bytes_partials(HEADLINE_L) / (head["partials_us_mean"] * 1e3) / HBM_PEAK_GBS, 4),
                     "traffic": traffic_from_profiles(HEADLINE_L),
                     "alg_bytes_per_launch": alg_bytes_partials(HEADLINE_L),
                     "avg_launch_us": round(head["partials_us_mean"], 3)},
        "ceiling": ceiling(sweep, node_us),
        "cpu_baseline": cpu,
        "configs": configs,
        "sweep": [{k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()}
                  for r in sweep],
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
