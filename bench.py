"""Benchmark of the MI355X MUL_MAT offload path (one GPU).

Headline workload (value): the decode GEMV set — every TinyLlama-1.1B
projection (q/o 2048x2048, k/v 256x2048, gate/up 5632x2048 in Q4_K, down
2048x5632 in Q6_K) of all 22 layers, at M=1 and then M=4, each activation
quantised to Q8_K and multiplied through the Q4_K/Q6_K x Q8_K GEMV. One step
is one such pass (22 distinct layers, 0.61 GB of weights, so the 256 MB
last-level cache cannot hold it); the step is captured once in a HIP graph and
replayed. value = algorithmic HBM bytes per step / step time.

Extra fields: the dominant kernel's roofline (the 4-row Q4_K GEMV on the
matrix cores) and the single-row kernel's beside it; the repack and A8
quantisation rooflines; the W8A8 prefill GEMM (int8 TOPS on the 5632x2048 Q4_K
weight at 128 tokens and on larger shapes, rotating >1 GiB of weights); the
prefill MUL_MAT tokens/s of TinyLlama-1.1B (128, 512 tokens), Llama-3.2-1B
(128, 512, 2048) and Llama-3-8B (4096), every layer and the output head on
repacked Q4_K/Q6_K weights; large and batched decode GEMVs; and the CPU oracle
timed on the host cores (all usable threads up to 16, and one) as a baseline.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--no-cpu]
       python bench.py --profile {gemv-q4k,gemv-q4k-m4,gemm,gemm-512,gemm-128,gemm-128-split,repack-q4k,repack-q6k,a8-4096,a8-512,copy}
           (workload only, for rocprofv3 counter runs)
       python bench.py --vs-hipblaslt   (W8A8 GEMM against torch._int_mm over 155 prefill shapes, one JSON line each)
       python bench.py --gemv-shapes    (single decode GEMV launches per shape and row count, one JSON line each)
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "W8A8 MUL_MAT int8 TOPS + prefill tok/s; Q4_K decode GEMV HBM GB/s"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--quick", action="store_true", help="skip the extra W8A8 shapes and the CPU baseline")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--profile", choices=["gemv-q4k", "gemv-q4k-m4", "gemm", "gemm-512", "gemm-128", "gemm-128-split", "copy",
                                          "repack-q4k", "repack-q6k", "a8-4096", "a8-512"],
                    help="run one workload eagerly a few times and exit (for rocprofv3 --pmc passes)")
    ap.add_argument("--vs-hipblaslt", action="store_true",
                    help="time the W8A8 GEMM against torch._int_mm over a grid of prefill shapes and exit")
    ap.add_argument("--gemv-shapes", action="store_true",
                    help="time single decode GEMV launches per projection shape and row count, one JSON line each, "
                         "and exit")
    return ap.parse_args()


TRAFFIC_FILE = ROOT / "profiles" / "traffic.json"


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the counter runs recorded in
    profiles/traffic.json (FETCH_SIZE + WRITE_SIZE, each scaled by what the
    counter reads for a plain copy of known size), or None."""
    try:
        rec = json.loads(TRAFFIC_FILE.read_text())[kernel]
        return int(rec["traffic_bytes_per_launch"])
    except (OSError, KeyError, ValueError):
        return None


# ----------------------------------------------------------------------------- decode GEMV set
class DecodeSet:
    """Device-resident TinyLlama projection weights and the per-step launch list."""

    def __init__(self, torch, hip, synth, layers: int):
        self.torch, self.hip = torch, hip
        dev = "cuda"
        self.layers = []
        for li in range(layers):
            lw = {}
            for pi, (name, k, n, kind) in enumerate(synth.TINYLLAMA_LAYER):
                blocks = synth.kquant(kind, n, k, index=10_000 + li * 16 + pi)
                lw[name] = (torch.from_numpy(blocks).to(dev), k, n, kind)
            self.layers.append(lw)
        # the decode cache's tile-interleaved copies, written once before any
        # timing (the C ABI builds them on a weight's first call of 2+ rows)
        self.tiled = [{name: hip.gemv_tile_weights(kind, w, k, n) for name, (w, k, n, kind) in lw.items()}
                      for lw in self.layers]
        # activations: one input per distinct projection input, per M
        self.inputs = {}
        self.outs = {}
        for m in (1, 4):
            for tag, k in (("attn", 2048), ("o", 2048), ("ffn", 2048), ("down", 5632)):
                x = torch.from_numpy(synth.activations(m, k, index=20_000 + m * 8 + k)).to(dev)
                self.inputs[(m, tag)] = x
            for li in range(layers):
                for name, k, n, kind in synth.TINYLLAMA_LAYER:
                    self.outs[(m, li, name)] = torch.empty((m, n), dtype=torch.float32, device=dev)
        self.groups = (("attn", ("q", "k", "v")), ("o", ("o",)), ("ffn", ("gate", "up")), ("down", ("down",)))

    def _launches(self, only_kind, only_m=None):
        for m in (1, 4):
            if only_m is not None and m != only_m:
                continue
            for li, lw in enumerate(self.layers):
                for tag, names in self.groups:
                    kind = lw[names[0]][3]
                    if only_kind is not None and kind != only_kind:
                        continue
                    yield m, li, tag, names, kind

    def step(self, only_kind: int | None = None, only_m: int | None = None):
        """One pass: per layer and M, one fused launch per shared input
        (q/k/v, o, gate/up, down), each quantising its f32 input to Q8_K; the
        raw rows or the tiled copies as the library's rule picks (tiled from
        2 rows), as the C ABI's decode entries do."""
        hip = self.hip
        for m, li, tag, names, kind in self._launches(only_kind, only_m):
            lw, lt = self.layers[li], self.tiled[li]
            k = lw[names[0]][1]
            hip.gemv_decode(kind, [lw[nm][0] for nm in names], [lt[nm] for nm in names], k,
                            [lw[nm][2] for nm in names], self.inputs[(m, tag)],
                            outs=[self.outs[(m, li, nm)] for nm in names])

    def bytes_per_step(self, only_kind: int | None = None, only_m: int | None = None) -> tuple[int, int]:
        """(algorithmic HBM bytes, launches) per step: each launch reads its
        weights (the raw GGUF bytes; every TinyLlama projection has a multiple
        of 16 rows, so its tiled copy holds exactly those bytes) and the f32
        activation rows once and writes the f32 outputs."""
        total = 0
        launches = 0
        for m, li, tag, names, kind in self._launches(only_kind, only_m):
            lw = self.layers[li]
            k = lw[names[0]][1]
            total += m * k * 4
            for nm in names:
                w, k, n, kind = lw[nm]
                total += w.numel() + m * n * 4
            launches += 1
        return total, launches


_SIDE_STREAM = None


SETTLE_S = 0.03  # seconds of warm-up replays before a timed region


def time_graph(torch, fn, steps: int, warmup: int) -> tuple[float, object]:
    """Capture fn() in a HIP graph, replay warmup + steps times; returns
    (ms per replay over the timed steps, graph). Every capture runs on one
    side stream, so the library's per-stream K-split workspaces are made once."""
    global _SIDE_STREAM
    if _SIDE_STREAM is None:
        _SIDE_STREAM = torch.cuda.Stream()
    s = _SIDE_STREAM
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # eager warm-up on the side stream (loads code objects, makes its split workspaces)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    # captured on the warm-up's stream, whose K-split workspaces the graph reuses
    with torch.cuda.graph(g, stream=s):
        fn()
    # warm-up: at least `warmup` replays and at least SETTLE_S of replaying (a
    # short shape timed right after its set-up, with three warm-up replays,
    # ran up to 15 % slower than the same graph timed again: 1024 x 2048 x
    # 2048 11.2 against 9.5 us)
    t0 = time.perf_counter()
    done = 0
    while done < warmup or (time.perf_counter() - t0 < SETTLE_S and done < 1000):
        for _ in range(max(1, warmup)):
            g.replay()
        done += max(1, warmup)
        torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps, g


# ----------------------------------------------------------------------------- W8A8 GEMM
def w8a8_route(torch, hip, synth, m: int, n: int, k: int, reps: int, rotate_bytes: int) -> dict:
    """The W8A8 prompt route of one Q4_K MUL_MAT as the reference serves it once
    its W8 is cached (execute_cached_w8a8_mtile_pool_padded, lib.rs:1776-1791
    quantise, :1868-1884 GEMM + rescale): per-token A8 quantisation of the f32
    activations, then the int8 GEMM with the fused rescale, as one graph over
    distinct W8 copies totalling >= rotate_bytes; and the one-time repack of the
    Q4_K blocks to W8 beside it (cold, rotating distinct copies)."""
    dev = "cuda"
    kp = hip.k_pad_of(k)
    blocks = torch.from_numpy(synth.kquant(4, n, k, index=31_000 + n)).to(dev)
    copies = max(1, min(128, rotate_bytes // (n * kp) + 1))
    w8s = [hip.repack_w8(4, blocks, k, n) for _ in range(copies)]
    a = torch.from_numpy(synth.activations(m, k, index=30_000 + m)).to(dev)
    a8 = torch.empty((m, kp), dtype=torch.int8, device=dev)
    asc = torch.empty(m, dtype=torch.float32, device=dev)
    out = torch.empty((m, n), dtype=torch.float32, device=dev)

    def route():
        for w8, wsc in w8s:
            hip.quantize_a8(a, kp, a8, asc)
            hip.gemm_w8a8(a8, asc, w8, wsc, out=out)

    def quant():
        for _ in w8s:
            hip.quantize_a8(a, kp, a8, asc)

    iters = max(1, reps // copies)
    route_ms, _ = time_graph(torch, route, iters, 2)
    quant_ms, _ = time_graph(torch, quant, iters, 2)
    route_us, quant_us = route_ms * 1e3 / copies, quant_ms * 1e3 / copies
    # the repack, once per weight: cold blocks rotating through > 1 GB
    rcopies = max(2, min(64, int(1.2e9 // (blocks.numel() + n * kp)) + 1))
    srcs = [blocks] + [blocks.clone() for _ in range(rcopies - 1)]
    dst = [(torch.empty((n, kp), dtype=torch.int8, device=dev), torch.empty(n, dtype=torch.float32, device=dev))
           for _ in range(rcopies)]

    def repack():
        for b, (w8, sc) in zip(srcs, dst):
            hip.repack_w8(4, b, k, n, w8=w8, scales=sc)

    rp_ms, _ = time_graph(torch, repack, 5, 2)
    ops = 2.0 * m * n * k
    byts = n * kp + 4 * n + 4 * m * k + 4 * m * n  # W8, scales, f32 activations, f32 out (A8 stays in L2)
    return {"route_us": round(route_us, 3), "a8_quant_us": round(quant_us, 3),
            "route_tops": round(ops / (route_us * 1e-6) / 1e12, 2),
            "route_hbm_roofline_us": round(byts / (HBM_PEAK_GBS * 1e3), 3),
            "repack_us": round(rp_ms * 1e3 / rcopies, 3), "repack_copies": rcopies, "weight_copies": copies}


def w8a8_gemm(torch, hip, synth, m: int, n: int, k: int, reps: int, rotate_bytes: int) -> dict:
    """Time the int8 MFMA GEMM on distinct weight copies totalling >= rotate_bytes."""
    dev = "cuda"
    kp = hip.k_pad_of(k)
    copies = max(1, min(128, rotate_bytes // (n * kp) + 1))
    g = torch.Generator(device=dev)
    g.manual_seed(m * 7 + n + k)
    ws = [torch.randint(-127, 128, (n, kp), dtype=torch.int8, device=dev, generator=g) for _ in range(copies)]
    wsc = torch.rand(n, device=dev, generator=g) / 127 + 1e-3
    a = torch.from_numpy(synth.activations(m, k, index=30_000 + m)).to(dev)
    a8, asc = hip.quantize_a8(a, kp)
    out = torch.empty((m, n), dtype=torch.float32, device=dev)

    def run():
        for w in ws:
            hip.gemm_w8a8(a8, asc, w, wsc, out=out)

    # at least three timed replays after three untimed ones: the first replay
    # of a large shape runs ~6 % slow (4096 x 14336 x 4096: 275 us, then
    # 259-261 us on every later replay)
    iters = max(3, reps // copies)
    ms, _ = time_graph(torch, run, iters, 3)
    per = ms / copies
    ops = 2.0 * m * n * k
    byts = n * kp + m * kp + 4 * (m + n) + 4 * m * n
    tops = ops / (per * 1e-3) / 1e12
    bound_tops = min(INT8_PEAK_TOPS, HBM_PEAK_GBS * ops / byts / 1e3)
    return {"m": m, "n": n, "k": k, "k_splits": hip.gemm_workspace(m, n, kp)[1],
            "column_split": hip.gemm_column_split(m, n, kp), "us": round(per * 1e3, 3),
            "tops": round(tops, 2),
            "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
            "roofline_tops": round(bound_tops, 1), "frac_roofline": round(tops / bound_tops, 4),
            "bound": "mfma" if bound_tops >= INT8_PEAK_TOPS else "hbm", "weight_copies": copies}


# layers, hidden, FFN, K/V rows (KV heads x head dim), vocab
MODELS = {
    "tinyllama_1.1b": (22, 2048, 5632, 256, 32000),
    "llama3.2_1b": (16, 2048, 8192, 512, 128256),
    "llama3_8b": (32, 4096, 14336, 1024, 128256),
}


class PrefillModel:
    """Every prefill MUL_MAT of one model on device-resident W8, in the order and
    grouping the routing runs them: per layer q/k/v as one GEMM over their
    concatenated W8 (one A8 quantisation of the shared input), o, gate+up as
    one GEMM, down; then the output head. Weights are seeded Q4_K (Q6_K for
    ffn_down and the head) repacked on the GPU into distinct buffers per layer,
    so a step streams every layer's weights from HBM."""

    def __init__(self, torch, hip, synth, model: str, m_max: int):
        self.torch, self.hip = torch, hip
        layers, hidden, ffn, kv, vocab = MODELS[model]
        dev = "cuda"
        groups = (("qkv", hidden, ((4, hidden), (4, kv), (4, kv))), ("o", hidden, ((4, hidden),)),
                  ("gateup", hidden, ((4, ffn), (4, ffn))), ("down", ffn, ((6, hidden),)))
        # one set of seeded blocks per projection shape, repacked into every layer's buffers
        blocks = {}
        for gname, k, members in groups:
            for j, (kind, n) in enumerate(members):
                blocks[(gname, j)] = torch.from_numpy(synth.kquant(kind, n, k, index=60_000 + 8 * len(blocks))).to(dev)
        head_rows = 8192  # seeded rows, tiled to the vocabulary
        hb = synth.kquant(6, head_rows, hidden, index=61_000).reshape(head_rows, -1)
        reps = (vocab + head_rows - 1) // head_rows
        head_blocks = torch.from_numpy(np.ascontiguousarray(np.tile(hb, (reps, 1))[:vocab])).to(dev)
        self.layers = []
        self.weight_bytes = 0
        for _ in range(layers):
            lw = []
            for gname, k, members in groups:
                kp = hip.k_pad_of(k)
                n_total = sum(n for _, n in members)
                w8 = torch.empty((n_total, kp), dtype=torch.int8, device=dev)
                sc = torch.empty(n_total, dtype=torch.float32, device=dev)
                r0 = 0
                for j, (kind, n) in enumerate(members):
                    hip.repack_w8(kind, blocks[(gname, j)], k, n, w8=w8[r0:r0 + n], scales=sc[r0:r0 + n])
                    r0 += n
                lw.append((k, w8, sc))
                self.weight_bytes += w8.numel() + 4 * n_total
            self.layers.append(lw)
        self.head = (hidden, *hip.repack_w8(6, head_blocks, hidden, vocab))
        self.weight_bytes += self.head[1].numel() + 4 * vocab
        del blocks, head_blocks
        self.ops_per_token = 2.0 * sum(w8.shape[0] * k for lw in self.layers for k, w8, _ in lw)
        self.ops_per_token += 2.0 * vocab * hidden
        self.model, self.m_max = model, m_max
        self.x = {k: torch.from_numpy(synth.activations(m_max, k, index=62_000 + k)).to(dev) for k in {hidden, ffn}}
        self.a8 = {k: (torch.empty((m_max, hip.k_pad_of(k)), dtype=torch.int8, device=dev),
                       torch.empty(m_max, dtype=torch.float32, device=dev)) for k in {hidden, ffn}}
        n_max = max(max(w8.shape[0] for _, w8, _ in self.layers[0]), vocab)
        self.out = torch.empty(m_max * n_max, dtype=torch.float32, device=dev)
        torch.cuda.synchronize()

    def step(self, m: int, quant_only: bool = False):
        hip = self.hip
        for k, w8, sc in [g for lw in self.layers for g in lw] + [self.head]:
            a8, asc = self.a8[k]
            hip.quantize_a8(self.x[k][:m], hip.k_pad_of(k), a8[:m], asc[:m])
            if not quant_only:
                hip.gemm_w8a8(a8[:m], asc[:m], w8, sc, out=self.out[:m * w8.shape[0]].view(m, w8.shape[0]))

    def time(self, m: int, steps: int) -> dict:
        ms, _ = time_graph(self.torch, lambda: self.step(m), steps, 2)
        # the A8 quantisation launches of the same step alone: their share of it
        qms, _ = time_graph(self.torch, lambda: self.step(m, quant_only=True), steps, 2)
        tops = self.ops_per_token * m / (ms * 1e-3) / 1e12
        return {"m": m, "ms": round(ms, 4), "tok_s": round(m / (ms * 1e-3), 1), "int8_tops": round(tops, 1),
                "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4), "a8_quant_ms": round(qms, 4),
                "a8_quant_share": round(qms / ms, 4)}


def prefill_sequences(torch, hip, synth, steps: int) -> dict:
    """Prefill MUL_MAT tokens/s of the three model shapes at their prompt sizes."""
    res = {}
    for model, ms in (("tinyllama_1.1b", (128, 512)), ("llama3.2_1b", (128, 512, 2048)), ("llama3_8b", (4096,))):
        pm = PrefillModel(torch, hip, synth, model, max(ms))
        layers, hidden, ffn, kv, vocab = MODELS[model]
        res[model] = {"layers": layers, "hidden": hidden, "ffn": ffn, "kv": kv, "vocab": vocab,
                      "w8_bytes": pm.weight_bytes, "launches_per_step": 2 * (4 * layers + 1),
                      "runs": [pm.time(m, steps if m < 4096 else max(2, steps // 4)) for m in ms]}
        del pm
        torch.cuda.empty_cache()
    return res


def repack_roofline(torch, hip, synth) -> dict:
    """Kernel (a) on the Llama-3-8B gate weight (Q4_K 14336 x 4096) and the
    Llama-3.2-1B head (Q6_K 128256 x 2048), rotating distinct copies through
    more than 1 GB: algorithmic bytes (blocks read, W8 and scales written) per
    launch over the launch time."""
    dev = "cuda"
    res = {}
    for name, kind, n, k in (("q4k_14336x4096", 4, 14336, 4096), ("q6k_128256x2048", 6, 128256, 2048)):
        src = torch.from_numpy(synth.kquant(kind, n, k, index=63_000 + kind)).to(dev)
        kp = hip.k_pad_of(k)
        byts = src.numel() + n * kp + 4 * n
        copies = max(2, min(16, int(1.2e9 // byts) + 1))
        srcs = [src] + [src.clone() for _ in range(copies - 1)]
        outs = [(torch.empty((n, kp), dtype=torch.int8, device=dev), torch.empty(n, dtype=torch.float32, device=dev))
                for _ in range(copies)]

        def run():
            for b, (w8, sc) in zip(srcs, outs):
                hip.repack_w8(kind, b, k, n, w8=w8, scales=sc)

        ms, _ = time_graph(torch, run, 5, 2)
        us = ms * 1e3 / copies
        gbs = byts / (us * 1e-6) / 1e9
        res[name] = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(f"repack_{name}"),
                     "avg_launch_us": round(us, 3), "bytes_per_launch": byts}
        del srcs, outs
        torch.cuda.empty_cache()
    return res


def a8_roofline(torch, hip, synth) -> dict:
    """Kernel (b) on 4096 tokens x 4096 and 512 tokens x 5632 f32 activations,
    rotating distinct copies through more than 1 GB: f32 read, A8 and scales
    written, per launch over the launch time."""
    dev = "cuda"
    res = {}
    for m, k in ((4096, 4096), (512, 5632)):
        kp = hip.k_pad_of(k)
        byts = m * k * 4 + m * kp + 4 * m
        copies = max(2, min(32, int(1.2e9 // byts) + 1))
        xs = [torch.from_numpy(synth.activations(m, k, index=64_000 + i)).to(dev) for i in range(copies)]
        outs = [(torch.empty((m, kp), dtype=torch.int8, device=dev), torch.empty(m, dtype=torch.float32, device=dev))
                for _ in range(copies)]

        def run():
            for x, (a8, sc) in zip(xs, outs):
                hip.quantize_a8(x, kp, a8, sc)

        ms, _ = time_graph(torch, run, 5, 2)
        us = ms * 1e3 / copies
        gbs = byts / (us * 1e-6) / 1e9
        res[f"m{m}_k{k}"] = {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(f"a8_m{m}_k{k}"),
                             "avg_launch_us": round(us, 3), "bytes_per_launch": byts}
        del xs, outs
        torch.cuda.empty_cache()
    return res


def decode_large(torch, hip, synth) -> dict:
    """Llama-3-8B decode projections at M=1 (gate+up 2 x [14336 x 4096] Q4_K in
    one launch, down [4096 x 14336] Q6_K), rotating distinct weight copies:
    the GEMV on matrices large enough for the launch cost not to dominate."""
    dev = "cuda"
    res = {}
    for name, kind, ns, k in (("gate_up_q4k", 4, (14336, 14336), 4096), ("down_q6k", 6, (4096,), 14336)):
        wbytes = sum(n * k // 256 * synth.BLOCK_BYTES[kind] for n in ns)
        copies = max(2, min(24, int(1.2e9 // wbytes)))
        tiled = hip.gemv_tiled_preferred(kind, 1, k)
        W = []
        for c in range(copies):
            ws = []
            for j, n in enumerate(ns):
                raw = torch.from_numpy(synth.kquant(kind, n, k, index=50_000 + 8 * c + j)).to(dev)
                ws.append(hip.gemv_tile_weights(kind, raw, k, n) if tiled else raw)
            W.append(ws)
        x = torch.from_numpy(synth.activations(1, k, index=51_000 + k)).to(dev)
        outs = [torch.empty((1, n), dtype=torch.float32, device=dev) for n in ns]

        def run():
            for ws in W:
                hip.gemv_decode(kind, ws, ws, k, list(ns), x, outs=outs)

        ms, _ = time_graph(torch, run, 5, 2)
        us = ms * 1e3 / copies
        byts = wbytes + k * 4 + sum(ns) * 4
        gbs = byts / (us * 1e-6) / 1e9
        res[name] = {"kind": kind, "n": list(ns), "k": k, "layout": "tiled" if tiled else "raw", "us": round(us, 3),
                     "gb_s": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "weight_copies": copies}
        del W
        torch.cuda.empty_cache()
    return res


def decode_crossover(torch, hip, synth) -> dict:
    """Llama-3-8B gate+up (2 x [14336 x 4096] Q4_K) at batched decode sizes:
    the GEMV route (f32 activations quantised to Q8_K in-kernel, the Q4_K
    weights' tiled copy) against the W8A8 route (per-token A8 quant + int8 GEMM
    on weights repacked once to W8), to locate the batch where the GEMM takes
    over. Weight copies rotate through > 256 MB for both routes."""
    dev = "cuda"
    n, k = 14336, 4096
    res = {}
    wq = [[torch.from_numpy(synth.kquant(4, n, k, index=52_000 + 2 * c + j)).to(dev) for j in range(2)]
          for c in range(4)]
    wt = [[hip.gemv_tile_weights(4, blk, k, n) for blk in pair] for pair in wq]
    w8 = []
    for pair in wq[:3]:
        parts = [hip.repack_w8(4, blk, k, n) for blk in pair]
        w8.append((torch.cat([p[0] for p in parts]), torch.cat([p[1] for p in parts])))
    for m in (1, 4, 8, 16, 32, 64):
        x = torch.from_numpy(synth.activations(m, k, index=53_000 + m)).to(dev)
        outs = [torch.empty((m, n), dtype=torch.float32, device=dev) for _ in range(2)]
        a8 = torch.empty((m, k), dtype=torch.int8, device=dev)
        asc = torch.empty(m, dtype=torch.float32, device=dev)
        out = torch.empty((m, 2 * n), dtype=torch.float32, device=dev)

        def gemv():
            for pair, tpair in zip(wq, wt):
                hip.gemv_decode(4, pair, tpair, k, [n, n], x, outs=outs)

        def gemm():
            for w, wsc in w8:
                hip.quantize_a8(x, k, a8, asc)
                hip.gemm_w8a8(a8, asc, w, wsc, out=out)

        gv_ms, _ = time_graph(torch, gemv, 5, 2)
        gm_ms, _ = time_graph(torch, gemm, 5, 2)
        gv, gm = gv_ms * 1e3 / len(wq), gm_ms * 1e3 / len(w8)
        res[f"m{m}"] = {"gemv_us": round(gv, 2), "w8a8_us": round(gm, 2), "faster": "gemv" if gv < gm else "w8a8"}
    return res


def vs_hipblaslt(torch, hip, synth) -> None:
    """One line per shape: this GEMM (rescale fused, f32 out) against
    hipBLASLt's int8 GEMM through torch._int_mm (i32 out, no rescale), both
    on weight copies rotating through >= 512 MiB, M x N x K over prefill
    sizes of the TinyLlama, Llama-3.2-1B and Llama-3-8B projections, and
    their down projections' long K."""
    rotate = 512 << 20
    shapes = [(m, n, k) for m in (64, 128, 256, 384, 512, 768, 1024, 1536, 2048, 4096)
              for n in (2048, 2560, 4096, 5632, 11264, 14336, 28672) for k in (2048, 4096)]
    # the down projections' long K (TinyLlama 5632, Llama-3.2-1B 8192, Llama-3-8B 14336)
    shapes += [(m, n, k) for m in (64, 128, 256, 512, 2048) for n, k in ((2048, 5632), (2048, 8192), (4096, 14336))]
    for m, n, k in shapes:
        ours = w8a8_gemm(torch, hip, synth, m, n, k, reps=20, rotate_bytes=rotate)["us"]
        copies = max(1, min(64, rotate // (n * k) + 1))
        ws = [torch.randint(-127, 128, (n, k), dtype=torch.int8, device="cuda") for _ in range(copies)]
        a = torch.randint(-127, 128, (max(m, 17), k), dtype=torch.int8, device="cuda")  # _int_mm needs m > 16

        def run():
            for w in ws:
                torch._int_mm(a, w.t())

        ms, _ = time_graph(torch, run, max(1, 20 // copies), 2)
        theirs = ms * 1e3 / copies
        print(json.dumps({"m": m, "n": n, "k": k, "k_splits": hip.gemm_workspace(m, n, k)[1], "us": ours,
                          "int_mm_us": round(theirs, 3), "speedup": round(theirs / ours, 3)}), flush=True)
        del ws


def gemv_shapes(torch, hip, synth) -> None:
    """One line per decode shape, row count and weight layout (raw GGUF rows,
    the tiled copy): single fused launches (Q8_K quantisation in-kernel) of the
    TinyLlama projections and the Llama-3-8B FFN, replayed in a graph on weight
    copies rotating through >= 1 GiB; `picked` marks the layout the library's
    rule takes."""
    shapes = [("o", 4, 2048, [2048]), ("qkv", 4, 2048, [2048, 256, 256]), ("gate+up", 4, 2048, [5632, 5632]),
              ("down", 6, 5632, [2048]), ("llama3_8b gate+up", 4, 4096, [14336, 14336]),
              ("llama3_8b down", 6, 14336, [4096])]
    for name, kind, k, ns in shapes:
        per = sum(n * (k // synth.QK) * hip.BLOCK_BYTES[kind] for n in ns)
        copies = max(2, (1 << 30) // per + 1)
        base = [[torch.from_numpy(synth.kquant(kind, n, k, index=500 + c * 8 + i)).to("cuda")
                 for i, n in enumerate(ns)] for c in range(min(copies, 2))]
        tbase = [[hip.gemv_tile_weights(kind, w, k, n) for w, n in zip(ws, ns)] for ws in base]
        for layout, src in (("raw", base), ("tiled", tbase)):
            sets = [src[c] if c < len(src) else [t.clone() for t in src[c % len(src)]] for c in range(copies)]
            for m in ((1, 2, 4, 8) if name.startswith("llama3_8b") else (1, 2, 4, 8)):
                x = torch.from_numpy(synth.activations(m, k, index=900 + m)).to("cuda")
                outs = [torch.empty((m, n), device="cuda") for n in ns]
                call = hip.gemv_q_f32 if layout == "raw" else hip.gemv_q_f32_tiled

                def run():
                    for ws in sets:
                        call(kind, ws, k, ns, x, outs=outs)

                ms, _ = time_graph(torch, run, max(1, 100 // copies), 2)
                us = ms * 1e3 / copies
                byts = per + m * k * 4 + m * sum(ns) * 4
                print(json.dumps({"shape": name, "kind": kind, "m": m, "k": k, "n": ns, "layout": layout,
                                  "picked": hip.gemv_tiled_preferred(kind, m, k) == (layout == "tiled"),
                                  "us": round(us, 3), "gb_s": round(byts / us / 1e3, 1),
                                  "weight_mb": round(per / 1e6, 2)}), flush=True)
            del sets
        del base, tbase
        torch.cuda.empty_cache()


def profile_workload(torch, hip, synth, which: str) -> None:
    """Run one workload eagerly (3 times) for rocprofv3 counter passes."""
    if which in ("gemv-q4k", "gemv-q4k-m4"):
        ds = DecodeSet(torch, hip, synth, synth.TINYLLAMA_LAYERS)
        for _ in range(3):
            ds.step(only_kind=4, only_m=1 if which == "gemv-q4k" else 4)
    elif which.startswith("gemm"):
        # Llama-3-8B FFN at M=4096; TinyLlama gate+up at M=512; 128 x 5632 x 2048; TinyLlama
        # down at M=128 (K split in two)
        m, n, k = {"gemm": (4096, 14336, 4096), "gemm-512": (512, 11264, 2048), "gemm-128": (128, 5632, 2048),
                   "gemm-128-split": (128, 2048, 5632)}[which]
        w = torch.randint(-127, 128, (n, k), dtype=torch.int8, device="cuda")
        wsc = torch.rand(n, device="cuda") / 127 + 1e-3
        a8, asc = hip.quantize_a8(torch.from_numpy(synth.activations(m, k, index=5)).to("cuda"), k)
        out = torch.empty((m, n), dtype=torch.float32, device="cuda")
        for _ in range(3):
            hip.gemm_w8a8(a8, asc, w, wsc, out=out)
    elif which.startswith("repack"):
        # the roofline entries' shapes: Llama-3-8B gate (Q4_K) and the Llama-3.2-1B head (Q6_K)
        kind, n, k = (4, 14336, 4096) if which == "repack-q4k" else (6, 128256, 2048)
        src = torch.from_numpy(synth.kquant(kind, n, k, index=63_000 + kind)).to("cuda")
        for _ in range(3):
            hip.repack_w8(kind, src, k, n)
    elif which.startswith("a8"):
        m, k = (4096, 4096) if which == "a8-4096" else (512, 5632)
        x = torch.from_numpy(synth.activations(m, k, index=64_000)).to("cuda")
        for _ in range(3):
            hip.quantize_a8(x, hip.k_pad_of(k))
    else:  # a plain copy of known size: 256 MiB read, 256 MiB written
        src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
    torch.cuda.synchronize()
    print(f"profiled {which}", flush=True)


# ----------------------------------------------------------------------------- CPU baseline
def cpu_threads() -> int:
    """Threads for the CPU legs: the CPUs this process may run on, at most 16
    (one GPU's share of the host)."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def cpu_topology() -> str:
    """Host CPU model, sockets x cores x threads, and the CPUs this process may use."""
    model, sockets, cores, siblings = "unknown CPU", set(), None, None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            key, _, val = line.partition(":")
            key, val = key.strip(), val.strip()
            if key == "model name":
                model = val
            elif key == "physical id":
                sockets.add(val)
            elif key == "cpu cores" and cores is None:
                cores = int(val)
            elif key == "siblings" and siblings is None:
                siblings = int(val)
    except (OSError, ValueError):
        pass
    try:
        allowed = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        allowed = os.cpu_count() or 1
    shape = ""
    if sockets and cores and siblings:
        shape = f"{len(sockets)} socket(s) x {cores} cores x {siblings // cores} threads, "
    return f"{model}: {shape}{os.cpu_count()} logical CPUs, {allowed} usable by this process"


def _use_native_oracle(orc) -> str:
    """Time a -march=native build of the oracle (same floating-point flags);
    fall back to the shipped build when no compiler is found."""
    import shutil
    import tempfile

    if shutil.which("gcc") is None:
        return "shipped -march=x86-64-v3 build"
    orc.use_native_build(tempfile.mkdtemp(prefix="oracle_native_"))
    return "-O3 -march=native build"


def cpu_baseline(synth, budget_s: float = 10.0, budget_1t_s: float = 5.0) -> dict:
    """The C oracle's decode GEMV (ggml generic arithmetic) on the host cores,
    over layer 0 of the same set at M=1 and M=4, repeated for ~budget_s on
    cpu_threads() threads and ~budget_1t_s on one thread."""
    from oracle import oracle as orc

    build = _use_native_oracle(orc)
    threads = cpu_threads()
    layer = [(synth.kquant(kind, n, k, index=10_000 + pi), k, n, kind)
             for pi, (name, k, n, kind) in enumerate(synth.TINYLLAMA_LAYER)]
    q8 = {(m, k): orc.quantize_q8_k(synth.activations(m, k, index=20_000 + m * 8 + k))
          for m in (1, 4) for k in (2048, 5632)}

    def run(nthreads, budget):
        total_bytes, reps = 0, 0
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < budget:
            for m in (1, 4):
                for w, k, n, kind in layer:
                    orc.gemv_q8_k(kind, w, k, n, q8[(m, k)], threads=nthreads)
                    total_bytes += w.nbytes + q8[(m, k)].nbytes + m * n * 4
            reps += 1
        dt = time.perf_counter() - t0
        return total_bytes / dt / 1e9, reps, dt

    gbs, reps, dt = run(threads, budget_s)
    gbs1, reps1, dt1 = run(1, budget_1t_s)
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "value_1thread": round(gbs1, 3),
            "topology": cpu_topology(),
            "sample": f"oracle decode GEMV (ggml generic dot, OpenMP, {build}) over TinyLlama layer 0's 7 "
                      f"projections at M=1 and M=4: {reps} passes in {dt:.1f} s on {threads} threads, "
                      f"{reps1} passes in {dt1:.1f} s on 1 thread"}


def cpu_baseline_w8a8(synth, budget_s: float = 8.0, budget_1t_s: float = 5.0) -> dict:
    """The C oracle's W8A8 prefill route on the 5632 x 2048 Q4_K weight at 128
    tokens, in the reference's steady state: the W8 repacked once (as its cache
    serves it after the first miss, lib.rs:1731-1989), then per call A8 quant
    + exact i32 GEMM + rescale (value); beside it the same call with the repack
    included (the cold first call, value_with_repack)."""
    from oracle import oracle as orc

    threads = cpu_threads()
    n, k, m = 5632, 2048, 128
    blocks = synth.kquant(4, n, k, index=1)
    a = synth.activations(m, k, index=2)
    w8, wsc = orc.repack_w8(4, blocks, k, n, threads=threads)
    ops = 2.0 * m * n * k

    def timed(fn, budget):
        reps = 0
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < budget:
            fn()
            reps += 1
        dt = time.perf_counter() - t0
        return ops * reps / dt / 1e12, reps, dt

    def cached(nthreads):
        a8, asc = orc.quantize_a8(a)
        return orc.rescale(orc.gemm_i32(a8, w8, threads=nthreads), asc, wsc)

    tops, reps, dt = timed(lambda: cached(threads), budget_s)
    tops1, reps1, dt1 = timed(lambda: cached(1), budget_1t_s)
    cold, creps, cdt = timed(lambda: orc.matmul_q_w8a8(4, blocks, a, n, threads=threads), budget_s / 2)
    return {"value": round(tops, 4), "unit": "int8 TOPS (W8 cached: A8 quant + i32 GEMM + rescale)",
            "cores": threads, "kind": "port", "value_1thread": round(tops1, 4),
            "value_with_repack": round(cold, 4), "topology": cpu_topology(),
            "sample": f"oracle W8A8 route, Q4_K 5632x2048 weight x 128 tokens, W8 repacked once: {reps} calls in "
                      f"{dt:.1f} s on {threads} threads, {reps1} calls in {dt1:.1f} s on 1 thread; repack included: "
                      f"{creps} calls in {cdt:.1f} s on {threads} threads"}


# ----------------------------------------------------------------------------- main
def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}): the split of weight rows or K "
              "over several GPUs is not built, so no multi-GPU figure exists.", file=sys.stderr)
        sys.exit(2)
    import torch

    from rocknpu_amd import hip, synth

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.set_device(0)
    if args.profile:
        profile_workload(torch, hip, synth, args.profile)
        return
    if args.vs_hipblaslt:
        vs_hipblaslt(torch, hip, synth)
        return
    if args.gemv_shapes:
        gemv_shapes(torch, hip, synth)
        return

    ds = DecodeSet(torch, hip, synth, synth.TINYLLAMA_LAYERS)
    torch.cuda.synchronize()
    step_bytes, n_gemv = ds.bytes_per_step()
    ms, graph = time_graph(torch, ds.step, args.steps, args.warmup)
    value = step_bytes / (ms * 1e-3) / 1e9

    # graph replays must reproduce the eager result bit for bit
    ref = {key: t.clone() for key, t in ds.outs.items()}
    for t in ds.outs.values():
        t.zero_()
    graph.replay()
    torch.cuda.synchronize()
    assert all(torch.equal(ref[key], ds.outs[key]) for key in ref), "graph replay differs"

    # dominant kernel: the Q4_K x Q8_K GEMV at M=4 on the matrix cores (the
    # largest share of a step), its launches timed alone in the same sequence;
    # the single-row launches of the same weights are timed beside it
    def kernel_rate(only_m, kind=4):
        b, launches = ds.bytes_per_step(only_kind=kind, only_m=only_m)
        t_ms, _ = time_graph(torch, lambda: ds.step(only_kind=kind, only_m=only_m), args.steps, args.warmup)
        us = t_ms * 1e3 / launches
        return b // launches, us, b / launches / (us * 1e-6) / 1e9

    q4_bpl, q4_us, achieved = kernel_rate(1)
    m4_bpl, m4_us, m4_achieved = kernel_rate(4)
    # the Q6_K down projections of the same step (the other kind), for where the time goes
    q6 = {}
    for m in (1, 4):
        bpl, us, gbs = kernel_rate(m, kind=6)
        q6[f"m{m}"] = {"achieved": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4), "avg_launch_us": round(us, 3),
                       "bytes_per_launch": bpl, "launches_per_step": synth.TINYLLAMA_LAYERS}

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k/q6_k x q8_k (int8 dot4, f32 accumulate)",
        "data": "synthetic (seeded Q4_K/Q6_K weights, N(0,1) activations)",
        "config": {"workload": "decode GEMV set: TinyLlama-1.1B projections x 22 layers, M=1 and M=4, "
                               "Q8_K activation quant fused into the Q4_K/Q6_K x Q8_K GEMV, one launch per "
                               "shared input (qkv, o, gate+up, down), the decode cache's tiled copies (the Q6_K "
                               "down at M=1: raw rows), HIP graph",
                   "layers": synth.TINYLLAMA_LAYERS, "m": [1, 4], "launches_per_step": n_gemv,
                   "bytes_per_step": step_bytes},
        "roofline": {"bound": "hbm", "kernel": "Q4_K x Q8_K decode GEMV at M=4 on the matrix cores over the "
                                               "tiled copies, fused Q8_K quant (gemv_tiled_kernel<4,4,true,8,true,1,1,1> "
                                               "for q/k/v and o, gemv_tiled_kernel<4,4,true,8,true,3,2,1> for "
                                               "gate+up), the 66 Q4_K launches of a step",
                     "achieved": round(m4_achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(m4_achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic("gemv_q4k_m4"),
                     "avg_launch_us": round(m4_us, 3), "bytes_per_launch": m4_bpl},
        "roofline_m1": {"bound": "hbm", "kernel": "Q4_K x Q8_K decode GEMV with fused Q8_K quant at M=1 "
                                                  "on the tiled copies (gemv_tiled_kernel<4,4,true,8,...>), the 66 "
                                                  "Q4_K launches of a step",
                        "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic("gemv_q4k"),
                        "avg_launch_us": round(q4_us, 3), "bytes_per_launch": q4_bpl},
        "decode_q6k_down": {"kernel": "Q6_K x Q8_K decode GEMV with fused Q8_K quant (M=1: gemv_q6_stream_kernel "
                                      "on raw rows; M=4: gemv_tiled_kernel<6,4,true,8,false,2,2,2,true,2> on the "
                                      "tiled copies, each tile's 22 blocks as two ranges of 11 on two workgroups), "
                                      "the 22 down launches of a step at each M", "peak": HBM_PEAK_GBS,
                            "unit": "GB/s",
                            **q6},
    }
    if not args.quick:
        rot = 1 << 30
        result["w8a8"] = {
            "q4k_5632x2048_m128": {**w8a8_gemm(torch, hip, synth, 128, 5632, 2048, 200, rot),
                                   **w8a8_route(torch, hip, synth, 128, 5632, 2048, 200, rot)},
            "tinyllama_gateup_m512": w8a8_gemm(torch, hip, synth, 512, 11264, 2048, 100, rot),
            "llama3_8b_ffn_m4096": w8a8_gemm(torch, hip, synth, 4096, 14336, 4096, 8, rot),
        }
        result["roofline_repack"] = repack_roofline(torch, hip, synth)
        result["roofline_a8_quant"] = a8_roofline(torch, hip, synth)
        result["prefill_mul_mat_tok_s"] = prefill_sequences(torch, hip, synth, 5)
        result["decode_gemv_large_m1"] = decode_large(torch, hip, synth)
        result["decode_crossover_llama3_8b_gate_up"] = decode_crossover(torch, hip, synth)
    if not (args.quick or args.no_cpu):
        result["cpu_baseline"] = cpu_baseline(synth)
        result["cpu_baseline_w8a8"] = cpu_baseline_w8a8(synth)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
