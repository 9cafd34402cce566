#!/usr/bin/env python3
"""Benchmark: Qwen3-A3B-shaped selected-expert MoE layer stack on one MI355X.

Headline workload: 48 MoE layers, hidden 2048, 128 experts, top-8,
moe_intermediate 768, SwiGLU experts with Q4_0 weights ~N(0, 0.02) (18-byte
blocks), router W_r ~N(0, 0.02) with logits biased by ln Zipf(s=1.1) over a
per-layer rank permutation, hidden ~N(0, 1), batch 1 decode. Each layer computes
    h <- h + sum_j w_j * down_j(silu(gate_j h) * up_j h)
over the router's softmax -> top-8 -> renormalised selection. Every expert of every
layer is resident in HBM (16.3 GB). One step is one token through all 48 layers,
three kernels per layer (router + top-8, fused gate/up + SiLU, down + combine)
replayed from a hipGraph; `value` is step time / 48 in us per token per layer.

Also measured in the same run (each in its own object of the JSON line):
- kernels: each layer kernel alone (router, gate/up, down), replayed from a graph
  of launches that rotate over more weight bytes than the 256 MB MALL holds; one
  roofline entry each, and `roofline` names the one with the most time;
- batch: 16 and 32 tokens per step through the same 48 layers: the layer entry
  point (grouped-token MFMA products from 12 tokens) against the router plus the
  per-assignment kernels;
- gemv: Q4_0 [1024 x 4096] batch 1, and Q4_0 / Q5_0 / IQ3_0 at [4096 x 4096] and
  [14336 x 4096], batch 1 and 8, each over a >= 4 GB rotated working set;
- stack4: the 4-layer x 8-expert top-2 Q4_0 stack (hidden 2048, intermediate 1024),
  batch 1, over >= 4 GB of rotated replicas (its 113 MB would sit in the MALL);
- deepseek: one H 7168 / 256 routed + 1 shared / top-8 / I 2048 FP4 layer at
  batch 1 and 32;
- official: the same routed experts through the FP8-activation ("official
  arithmetic") layer with an FP8 shared expert, batch 1 and 32;
- router: the router alone at the DeepSeek and Qwen3-A3B shapes for 1 to 32 tokens;
- misses: the headline stack with the experts in pinned host memory behind the
  expert cache at 25% of the expert bytes (objeta_hip_moe_stack_cached), batch 1
  and a 16-token batch, without and with next-layer prefetch: end-to-end us per
  token including the PCIe copies of the misses, against the PCIe floor of the
  bytes loaded;
- cpu_baseline: the oracle's C restatement of the reference CPU path
  (cpu_router + selected_moe_cpu) on the box's host cores, one pinned core and all
  cores, median of 5 runs over a bounded sample of the same layers.

--report-dir DIR also writes QGemvStatsReport / MoeStatsReport JSON lines with the
reference's field names (bench_qgemv.rs:6-37, bench_selected_moe.rs:19-101).

Synthetic data generated on the device (no checkpoints).
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import platform
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from objeta_amd.workloads import zipf_bias  # noqa: E402

HBM_PEAK_GBPS = 8000.0
ROTATE_BYTES = 4 << 30  # working set of the rotated GEMV measurements (>> 256 MB MALL)
SECTIONS = ("headline", "kernels", "batch", "gemv", "stack4", "deepseek", "official", "router", "misses", "cpu")
# not in the default run: kernels of known traffic for scaling rocprofv3's FETCH_SIZE / WRITE_SIZE
EXTRA_SECTIONS = ("calibrate",)
TRAFFIC_PROFILE = "profiles/moe_layer_q4_qwen3a3b_hbm_traffic.md"


def stats(values) -> dict:
    """avg/min/max/p50/p95 with the reference's percentile rule (bench_qgemv.rs:59-100)."""
    from objeta_amd.reports import stats as report_stats
    return report_stats(values)


def rnd(d: dict, n: int = 3) -> dict:
    return {k: round(x, n) for k, x in d.items()}


def cpu_model() -> str:
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return platform.processor() or "unknown"


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE + WRITE_SIZE
    summary (counter runs cannot share a process with this measurement)."""
    try:
        for line in open(os.path.join(ROOT, TRAFFIC_PROFILE)):
            if line.startswith(f"traffic_bytes_per_launch {kernel}:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


class Env:
    """Backend, library, stream and event helpers."""

    def __init__(self):
        from objeta_amd import HipBackend, MoeExecutor, check
        from objeta_amd._lib import load
        self.check = check
        self.be = HipBackend(0, 2)
        self.lib = load()
        self.ctx = self.be.ctx
        self.stream = self.be.stream(0)
        self.moe = MoeExecutor(self.be)

    def event(self):
        e = C.c_void_p()
        self.check(self.lib.objeta_hip_event_create(self.ctx, C.byref(e)))
        return e

    def drop_events(self, evs):
        for e in evs:
            self.check(self.lib.objeta_hip_event_destroy(self.ctx, e))

    def record(self, e):
        self.check(self.lib.objeta_hip_event_record(self.ctx, e, self.stream))

    def elapsed_us(self, a, b) -> float:
        ms = C.c_float()
        self.check(self.lib.objeta_hip_event_elapsed_ms(self.ctx, a, b, C.byref(ms)))
        return ms.value * 1000.0

    def capture(self, enqueue):
        self.check(self.lib.objeta_hip_graph_begin_capture(self.ctx, self.stream))
        enqueue()
        g = C.c_void_p()
        self.check(self.lib.objeta_hip_graph_end_capture(self.ctx, self.stream, C.byref(g)))
        return g

    def launch(self, g):
        self.check(self.lib.objeta_hip_graph_launch(self.ctx, g, self.stream))

    def destroy(self, graphs):
        for g in graphs:
            self.check(self.lib.objeta_hip_graph_destroy(self.ctx, g))

    def per_step(self, launch, steps: int):
        """Times `steps` calls of launch(i) with an event between consecutive steps:
        (total us, list of per-step us)."""
        evs = [self.event() for _ in range(steps + 1)]
        self.record(evs[0])
        for i in range(steps):
            launch(i)
            self.record(evs[i + 1])
        self.be.synchronize(self.stream)
        per = [self.elapsed_us(evs[i], evs[i + 1]) for i in range(steps)]
        total = self.elapsed_us(evs[0], evs[-1])
        self.drop_events(evs)
        if self.moe.device_error() != 0:
            raise RuntimeError("device error word set during a timed run")
        return total, per

    def fill_q(self, fmt: int, ptr: int, rows: int, cols: int, seed: int, sigma: float = 0.02):
        self.check(self.lib.objeta_hip_fill_gauss_quantized_device(self.ctx, fmt, None, C.c_void_p(ptr), rows, cols,
                                                                   seed, C.c_float(sigma)))

    def fill_gauss(self, ptr: int, n: int, seed: int, sigma: float):
        self.check(self.lib.objeta_hip_fill_gauss_device(self.ctx, None, C.c_void_p(ptr), n, seed, 0,
                                                         C.c_float(sigma)))


class QwenStack:
    """Device-resident Q4_0 MoE layer stack (weights, router, expert tables). Each
    layer's arena holds all experts' gate and up matrices as one [E * 2 * I][H] Q4_0
    matrix (expert e: rows [2eI, 2eI + I) gate, the next I rows up) followed by all
    down matrices as one [E * H][I] matrix, each generated by one fill."""

    def __init__(self, env: Env, layers, hidden, n_experts, k, inter, seed):
        from objeta_amd import ExpertTable
        self.env = env
        be = env.be
        self.layers, self.H, self.E, self.K, self.I = layers, hidden, n_experts, k, inter
        self.fmt = 0
        self.gu_bytes = inter * (hidden // 32) * 18
        self.dn_bytes = hidden * (inter // 32) * 18
        self.expert_bytes = 2 * self.gu_bytes + self.dn_bytes
        self.seed = seed
        self.gu_region = n_experts * 2 * self.gu_bytes
        self.arenas, self.tables, self.router_w, self.router_b, self.bias_host = [], [], [], [], []
        for l in range(layers):
            arena = be.alloc(n_experts * self.expert_bytes)
            env.fill_q(0, arena.ptr, n_experts * 2 * inter, hidden, self.gu_key(l))
            env.fill_q(0, arena.ptr + self.gu_region, n_experts * hidden, inter, self.dn_key(l))
            entries = []
            for e in range(n_experts):
                g, u, d = (self.offsets(e)[j] + arena.ptr for j in range(3))
                entries.append((g, u, d))
            self.arenas.append(arena)
            self.tables.append(ExpertTable(be, entries))
            w = be.alloc(4 * n_experts * hidden)
            env.fill_gauss(w.ptr, n_experts * hidden, seed + 10_000_000 + l, 0.02)
            self.router_w.append(w)
            b = zipf_bias(n_experts, 1.1, seed + l)
            self.bias_host.append(b)
            self.router_b.append(be.to_device(b))
        be.synchronize()

    def gu_key(self, l: int) -> int:
        return self.seed + 2 * l

    def dn_key(self, l: int) -> int:
        return self.seed + 2 * l + 1

    def offsets(self, e: int):
        """Byte offsets of expert e's gate, up and down matrices in its layer's arena."""
        g = e * 2 * self.gu_bytes
        return g, g + self.gu_bytes, self.gu_region + e * self.dn_bytes

    def f32_first(self, e: int):
        """(key, first element) of the N(0, 0.02) draws behind expert e's gate, up and
        down matrices of layer l, for regenerating them unquantized."""
        return ((0, e * 2 * self.I * self.H), (0, e * 2 * self.I * self.H + self.I * self.H), (1, e * self.H * self.I))

    def expert_host_bytes(self, layer: int, e: int):
        g, u, d = self.offsets(e)
        a = self.arenas[layer]
        return (a.download(np.uint8, self.gu_bytes, offset=g), a.download(np.uint8, self.gu_bytes, offset=u),
                a.download(np.uint8, self.dn_bytes, offset=d))


# --------------------------------------------------------------------- headline
def run_headline(env: Env, st: QwenStack, args, xs, P):
    L, H, K, I = st.layers, st.H, st.K, st.I
    h = env.be.alloc(4 * H)
    ids = env.be.alloc(4 * L * K)
    wts = env.be.alloc(4 * L * K)

    def enqueue_token(p: int):
        x0 = xs.addr(4 * p * H)
        for l in range(L):
            src = x0 if l == 0 else h.addr()
            env.moe.layer_device(st.fmt, st.tables[l], st.router_w[l], st.router_b[l], K, 1, src, src, h.addr(),
                                 ids.addr(4 * l * K), wts.addr(4 * l * K), H, I, H, stream=env.stream)

    enqueue_token(0)
    env.be.synchronize(env.stream)
    graphs = [env.capture(lambda p=p: enqueue_token(p)) for p in range(P)]
    for i in range(args.warmup):
        env.launch(graphs[i % P])
    env.be.synchronize(env.stream)
    total, per = env.per_step(lambda i: env.launch(graphs[i % P]), args.steps)
    token_us = total / args.steps
    env.destroy(graphs)
    # every token of the pool layer by layer, keeping each layer's input, ids and
    # weights: the inputs of the kernel timing below, so that each kernel alone does
    # the work it does inside the graph (the same logits, so the router meets the
    # same close calls and fallbacks)
    h_in = env.be.alloc(4 * P * L * H)
    ids_all, wts_all = env.be.alloc(4 * P * L * K), env.be.alloc(4 * P * L * K)
    for p in range(P):
        base = p * L
        env.check(env.lib.objeta_hip_copy_d2d(env.ctx, env.stream, h_in.addr(4 * base * H), xs.addr(4 * p * H),
                                              4 * H))
        for l in range(L):
            i = base + l
            dst = h_in.addr(4 * (i + 1) * H) if l + 1 < L else h.addr()
            env.moe.layer_device(st.fmt, st.tables[l], st.router_w[l], st.router_b[l], K, 1, h_in.addr(4 * i * H),
                                 h_in.addr(4 * i * H), dst, ids_all.addr(4 * i * K), wts_all.addr(4 * i * K), H, I,
                                 H, stream=env.stream)
    env.be.synchronize(env.stream)
    return token_us, stats(per), (h_in, ids_all, wts_all, P)


# ------------------------------------------------------------- kernels alone
KERNEL_NAMES = {"router": "router_split_kernel<2>", "gate_up": "moe_gate_up_kernel", "down": "moe_down_kernel"}


def run_kernels(env: Env, st: QwenStack, layer_io, reps: int):
    """Each layer kernel alone: per token of the pool a graph of 48 launches, launch l
    doing layer l's work for that token on the layer's recorded input (the work of a
    headline step, so the same share of router fallbacks); the P graphs are replayed
    `reps` times each, and a step's time / 48 is one sample of the us per launch
    (avg, p50, p95 over the samples). The router reads its
    weights from 1 GiB of replicas (copies of the 48 layers' W_r), gate/up and down the
    layers' selected experts (16 GB in all), so that the weights come from HBM, not
    the 256 MB MALL."""
    L, H, E, K, I = st.layers, st.H, st.E, st.K, st.I
    be = env.be
    h_in, d_ids, d_w, P = layer_io
    n = P * L
    act = be.alloc(4 * n * K * I)
    out = be.alloc(4 * H)
    rid, rw = be.alloc(4 * K), be.alloc(4 * K)
    rb = 4 * E * H
    n_rep = max(L, ((1 << 30) // rb) // L * L)
    replicas = be.alloc(n_rep * rb)
    for r in range(n_rep):
        env.check(env.lib.objeta_hip_copy_d2d(env.ctx, env.stream, replicas.addr(r * rb), st.router_w[r % L].addr(),
                                              rb))
    be.synchronize(env.stream)
    res = {}

    def router(i):
        l = i % L
        env.check(env.lib.objeta_hip_router_topk_device(env.ctx, env.stream, replicas.addr((i % n_rep) * rb),
                                                        st.router_b[l].addr(), h_in.addr(4 * i * H), 1, E, H, K, 1,
                                                        rid.addr(), rw.addr()))

    def gate_up(i):
        l = i % L
        env.moe.gate_up_device(st.fmt, st.tables[l], d_ids.addr(4 * i * K), 1, K, h_in.addr(4 * i * H),
                               act.addr(4 * i * K * I), H, I, stream=env.stream)

    def down(i):
        l = i % L
        env.moe.down_device(st.fmt, st.tables[l], d_ids.addr(4 * i * K), d_w.addr(4 * i * K), 1, K,
                            act.addr(4 * i * K * I), h_in.addr(4 * i * H), out.addr(), I, H, stream=env.stream)

    for name, fn in (("router", router), ("gate_up", gate_up), ("down", down)):
        fn(0)
        be.synchronize(env.stream)
        # one graph per token of the pool: that token's 48 launches, one per layer
        graphs = [env.capture(lambda p=p, fn=fn: [fn(p * L + l) for l in range(L)]) for p in range(P)]
        for g in graphs:
            env.launch(g)
        be.synchronize(env.stream)
        _, per = env.per_step(lambda i: env.launch(graphs[i % P]), reps * P)
        res[name] = stats([t / L for t in per])
        env.destroy(graphs)
    replicas.free()
    # algorithmic bytes per launch (one layer, one token)
    bytes_per = {
        "router": 4 * E * H + 4 * H + 4 * E + 8 * K,          # W_r, x, bias, ids + weights
        "gate_up": K * 2 * st.gu_bytes + 4 * H + 4 * K * I,   # 8 experts' gate and up, x, activations
        "down": K * st.dn_bytes + 4 * K * I + 8 * H,          # 8 experts' down, activations, residual + out
    }
    entries = {}
    for k, s in res.items():
        achieved = bytes_per[k] / (s["avg"] * 1e-6) / 1e9
        traffic = measured_traffic(KERNEL_NAMES[k])
        entries[k] = {"kernel": KERNEL_NAMES[k], "bound": "hbm", "achieved": round(achieved, 1),
                      "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                      "traffic": traffic,
                      "traffic_source": (f"copied from {TRAFFIC_PROFILE}: rocprofv3 --pmc FETCH_SIZE, then "
                                         "WRITE_SIZE, per dispatch of this kernel in the headline graph replays "
                                         "(`python bench.py --sections headline --steps 20`), scaled by the "
                                         "calibration kernels in that file") if traffic else None,
                      "algorithmic_bytes_per_launch": bytes_per[k], "avg_launch_us": round(s["avg"], 3),
                      "p50_us": round(s["p50"], 3), "p95_us": round(s["p95"], 3)}
    return entries


# ------------------------------------------------------------------- batches
def run_batch(env: Env, st: QwenStack, args, seed):
    """Batches of args.batch and 2 * args.batch tokens through every layer: the layer
    entry point (router, then the grouped-token products from 12 tokens on) against
    the router followed by the per-assignment kernels, and the router followed by the
    grouped-token products at every batch size."""
    L, H, E, K, I = st.layers, st.H, st.E, st.K, st.I
    be = env.be
    out = {"path": "objeta_hip_moe_layer_device (router + grouped-token MFMA products from 12 tokens) vs "
                   "router + objeta_hip_moe_selected_device (per-assignment kernels) vs router + "
                   "objeta_hip_moe_grouped_device (grouped-token products); one graph per pass of "
                   f"{L} layers"}
    for B in (args.batch, 2 * args.batch):
        xb = be.alloc(4 * B * H)
        env.fill_gauss(xb.ptr, B * H, seed + 99 + B, 1.0)
        hb = be.alloc(4 * B * H)
        idsb = be.alloc(4 * L * B * K)
        wtsb = be.alloc(4 * L * B * K)

        def enqueue(mode: str, B=B, xb=xb, hb=hb, idsb=idsb, wtsb=wtsb):
            for l in range(L):
                src = xb.addr() if l == 0 else hb.addr()
                li, lw = idsb.addr(4 * l * B * K), wtsb.addr(4 * l * B * K)
                if mode == "entry":
                    env.moe.layer_device(st.fmt, st.tables[l], st.router_w[l], st.router_b[l], K, B, src, src,
                                         hb.addr(), li, lw, H, I, H, stream=env.stream)
                    continue
                env.check(env.lib.objeta_hip_router_topk_device(env.ctx, env.stream, st.router_w[l].addr(),
                                                                st.router_b[l].addr(), src, B, E, H, K, 1, li, lw))
                if mode == "grouped":
                    env.moe.grouped_device(st.fmt, st.tables[l], li, lw, B, K, src, src, hb.addr(), H, I, H,
                                           stream=env.stream)
                else:
                    env.moe.selected_device(st.fmt, st.tables[l], li, lw, B, K, src, src, hb.addr(), H, I, H,
                                            stream=env.stream)

        res = {}
        for mode in ("entry", "per_assignment", "grouped"):
            enqueue(mode)
            be.synchronize(env.stream)
            g = env.capture(lambda m=mode: enqueue(m))
            for _ in range(3):
                env.launch(g)
            be.synchronize(env.stream)
            _, per = env.per_step(lambda i: env.launch(g), max(5, args.steps // 20))
            res[mode] = stats(per)
            env.destroy([g])
        ids_all = idsb.download(np.uint32, L * B * K).reshape(L, B * K)
        uniq = [len(set(int(v) for v in ids_all[l])) for l in range(L)]
        ub = sum(uniq) * st.expert_bytes
        out[f"batch{B}"] = {
            "tokens": B, "us_per_step": rnd(res["entry"], 1),
            "us_per_token_layer": round(res["entry"]["avg"] / (L * B), 3),
            "per_assignment_us_per_step": rnd(res["per_assignment"], 1),
            "grouped_us_per_step": rnd(res["grouped"], 1),
            "speedup_vs_per_assignment": round(res["per_assignment"]["avg"] / res["entry"]["avg"], 3),
            "grouped_speedup_vs_per_assignment": round(res["per_assignment"]["avg"] / res["grouped"]["avg"], 3),
            "unique_experts_per_layer": round(sum(uniq) / L, 1), "unique_expert_bytes_per_step": ub,
            "expert_hbm_gbps": round(ub / (res["entry"]["avg"] * 1e-6) / 1e9, 1),
            "per_assignment_expert_hbm_gbps": round(ub / (res["per_assignment"]["avg"] * 1e-6) / 1e9, 1),
            "grouped_expert_hbm_gbps": round(ub / (res["grouped"]["avg"] * 1e-6) / 1e9, 1)}
        for b in (xb, hb, idsb, wtsb):
            b.free()
    return out


# ------------------------------------------------------------------ GEMV sweep
GEMV_CASES = [(0, 1024, 4096, 1)] + [(f, r, 4096, b) for f in (0, 1, 2) for r in (4096, 14336) for b in (1, 8)]
FMT_NAME = {0: "Q4_0", 1: "Q5_0", 2: "IQ3_0", 3: "DeepSeekFp4E2M1"}
KERNEL_NAME = {0: "q4_gemv", 1: "q5_gemv", 2: "iq3_gemv", 3: "fp4_e2m1_gemv"}
BB = {0: 18, 1: 22, 2: 14}


def run_gemv(env: Env, reps: int, checks: list | None = None, calls: int = 512, rotate: int = ROTATE_BYTES):
    """Each case's matrix replicated over >= 4 GB (one fill of R * rows rows); graphs of
    launches cycle through the replicas, so the weights come from HBM. `checks`
    receives (format, rows, cols, seed, replica-0 bytes, x, y of token 0) per case for
    the numerics of the reports."""
    be = env.be
    out = []
    big = be.alloc(rotate + (64 << 20))
    xs = be.alloc(4 * 8 * 14336)
    env.fill_gauss(xs.ptr, 8 * 14336, 31337, 1.0)
    ys = be.alloc(4 * 8 * 14336)
    filled = None
    for fmt, rows, cols, B in GEMV_CASES:
        mb = rows * (cols // 32) * BB[fmt]
        R = max(1, rotate // mb)
        if filled != (fmt, rows):
            env.fill_q(fmt, big.ptr, R * rows, cols, 777 + fmt)
            be.synchronize()
            filled = (fmt, rows)
        n = min(R, calls)  # calls per graph

        def launch(i, fmt=fmt, rows=rows, cols=cols, B=B, mb=mb, R=R):
            env.check(env.lib.objeta_hip_qgemv_device(env.ctx, fmt, env.stream, big.addr((i % R) * mb), xs.addr(),
                                                      ys.addr(), rows, cols, B))
        launch(0)
        be.synchronize(env.stream)
        if checks is not None:
            checks.append((fmt, rows, cols, 777 + fmt, big.download(np.uint8, mb), xs.download(np.float32, cols),
                           ys.download(np.float32, rows)))
        ng = (R + n - 1) // n
        graphs = [env.capture(lambda g0=g0: [launch(g0 * n + i) for i in range(n)]) for g0 in range(ng)]
        env.launch(graphs[0])
        be.synchronize(env.stream)
        _, per = env.per_step(lambda i: env.launch(graphs[i % ng]), max(reps, ng))
        s = stats([p / n for p in per])
        alg = mb + 4 * B * cols + 4 * B * rows
        ref_bytes = mb + 4 * cols  # the reference's bytes_read (quant.rs:282)
        out.append({"format": FMT_NAME[fmt], "rows": rows, "cols": cols, "batch": B,
                    "working_set_bytes": R * mb, "us": rnd(s), "samples_us": [p / n for p in per],
                    "algorithmic_bytes": alg,
                    "gbps": round(alg / (s["avg"] * 1e-6) / 1e9, 1),
                    "frac_of_peak": round(alg / (s["avg"] * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
                    "reference_effective_gbps": round(ref_bytes / (s["avg"] * 1e-6) / 1e9, 1)})
        env.destroy(graphs)
    big.free()
    return out


# ------------------------------------------------------- DeepSeek-V3-class FP4
def run_deepseek(env: Env, args, seed):
    from objeta_amd import ExpertTable
    be = env.be
    H, I, E, K = 7168, 2048, 256, 8
    w_b, s_b = I * H // 2, I * H // 32
    dw_b, ds_b = H * I // 2, H * I // 32
    eb = 2 * (w_b + s_b) + dw_b + ds_b
    arena = be.alloc((E + 1) * eb)
    entries = []
    for e in range(E + 1):
        base = arena.ptr + e * eb
        gw, gs = base, base + w_b
        uw, us = gs + s_b, gs + s_b + w_b
        dw, ds = us + s_b, us + s_b + dw_b
        for j, (wp, sp, r, c) in enumerate(((gw, gs, I, H), (uw, us, I, H), (dw, ds, H, I))):
            env.check(env.lib.objeta_hip_fill_fp4_split_device(env.ctx, None, C.c_void_p(wp), C.c_void_p(sp), r, c,
                                                               seed + 3 * e + j))
        entries.append((gw, uw, dw, gs, us, ds))
    table = ExpertTable(be, entries[:E])
    shared = ExpertTable(be, entries[E:])
    w_r = be.alloc(4 * E * H)
    env.fill_gauss(w_r.ptr, E * H, seed + 5, 0.02)
    res = {"hidden": H, "intermediate": I, "experts": E, "shared_experts": 1, "top_k": K, "format": "DeepSeekFp4E2M1",
           "expert_bytes": eb, "path": "objeta_hip_moe_layer_shared_device replayed from a hipGraph: batch 1 on the "
                                       "per-assignment kernels (router, gate/up + SiLU, down + combine, shared "
                                       "expert last with weight 1), batch 4 and 32 on the grouped-token products "
                                       "(from 2 tokens at this expert size) with the shared expert as one more "
                                       "group"}
    for T in (1, 4, 32):
        P = 8
        xs = be.alloc(4 * P * T * H)
        env.fill_gauss(xs.ptr, P * T * H, seed + 10 + T, 1.0)
        out = be.alloc(4 * T * H)
        ids = be.alloc(4 * T * K)
        wts = be.alloc(4 * T * K)

        def enq(p, T=T, xs=xs, out=out, ids=ids, wts=wts):
            env.moe.layer_device(3, table, w_r, None, K, T, xs.addr(4 * p * T * H), xs.addr(4 * p * T * H), out.addr(),
                                 ids.addr(), wts.addr(), H, I, H, stream=env.stream, shared=shared)
        enq(0)
        be.synchronize(env.stream)
        graphs = [env.capture(lambda p=p: enq(p)) for p in range(P)]
        for i in range(5):
            env.launch(graphs[i % P])
        be.synchronize(env.stream)
        _, per = env.per_step(lambda i: env.launch(graphs[i % P]), max(20, args.steps // 4))
        s = stats(per)
        sel = ids.download(np.uint32, T * K)
        distinct = len(set(int(v) for v in sel)) + 1  # + the shared expert
        ebytes = distinct * eb
        res[f"batch{T}"] = {"us_per_layer": rnd(s), "us_per_token": round(s["avg"] / T, 3),
                            "expert_bytes_read": ebytes, "distinct_experts_incl_shared": distinct,
                            "expert_hbm_gbps": round(ebytes / (s["avg"] * 1e-6) / 1e9, 1),
                            "expert_hbm_frac_of_peak": round(ebytes / (s["avg"] * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)}
        env.destroy(graphs)
    arena.free()
    return res


# ------------------------------------------- four-layer eight-expert stack
def run_stack4(env: Env, args, seed):
    """The 4-layer x 8-expert top-2 Q4_0 stack (hidden 2048, intermediate 1024, W_r
    [8 x 2048] ~N(0, 0.02), softmax -> top-2 -> renormalised, batch 1). The whole model
    is 113 MB and would sit in the 256 MB MALL, so it is replicated over >= 4 GB (the
    generated layers copied into every replica) and step i runs one token through the
    four layers of replica i mod R: the expert bytes come from HBM. One hipGraph per
    replica (12 launches: router, gate/up, down per layer)."""
    from objeta_amd import ExpertTable
    be = env.be
    L, H, E, K, I = 4, 2048, 8, 2, 1024
    gu = I * (H // 32) * 18
    dn = H * (I // 32) * 18
    eb = 2 * gu + dn
    model = L * (E * eb + 4 * E * H)
    R = max(1, -(-ROTATE_BYTES // model))
    arena = be.alloc(R * model)
    layer_b = E * eb + 4 * E * H
    for l in range(L):
        base = arena.ptr + l * layer_b
        for e in range(E):
            env.fill_q(0, base + e * eb, 2 * I, H, seed + 100 * l + 3 * e)
            env.fill_q(0, base + e * eb + 2 * gu, H, I, seed + 100 * l + 3 * e + 2)
        env.fill_gauss(base + E * eb, E * H, seed + 100 * l + 99, 0.02)
    for r in range(1, R):
        env.check(env.lib.objeta_hip_copy_d2d(env.ctx, env.stream, arena.addr(r * model), arena.addr(), model))
    be.synchronize(env.stream)
    tables = []
    for r in range(R):
        row = []
        for l in range(L):
            base = arena.ptr + r * model + l * layer_b
            row.append((ExpertTable(be, [(base + e * eb, base + e * eb + gu, base + e * eb + 2 * gu)
                                         for e in range(E)]), base + E * eb))
        tables.append(row)
    P = 16
    xs = be.alloc(4 * P * H)
    env.fill_gauss(xs.ptr, P * H, seed + 7, 1.0)
    h = be.alloc(4 * H)
    ids, wts = be.alloc(4 * L * K), be.alloc(4 * L * K)

    def enq(r):
        x0 = xs.addr(4 * (r % P) * H)
        for l in range(L):
            src = x0 if l == 0 else h.addr()
            tab, wr = tables[r][l]
            env.moe.layer_device(0, tab, C.c_void_p(wr), None, K, 1, src, src, h.addr(), ids.addr(4 * l * K),
                                 wts.addr(4 * l * K), H, I, H, stream=env.stream)
    enq(0)
    be.synchronize(env.stream)
    graphs = [env.capture(lambda r=r: enq(r)) for r in range(R)]
    for i in range(min(R, 10)):
        env.launch(graphs[i])
    be.synchronize(env.stream)
    steps = max(2 * R, args.steps)
    total, per = env.per_step(lambda i: env.launch(graphs[i % R]), steps)
    env.destroy(graphs)
    s = stats(per)
    tok_us = total / steps
    layer_bytes = K * eb
    arena.free()
    return {"layers": L, "hidden": H, "experts": E, "top_k": K, "intermediate": I, "format": "Q4_0",
            "expert_bytes": eb, "expert_bytes_per_layer": layer_bytes, "replicas": R,
            "rotated_bytes": R * model,
            "path": "objeta_hip_moe_layer_device per layer (router, gate/up + SiLU, down + combine), one hipGraph "
                    "per replica",
            "us_per_token": round(tok_us, 3), "us_per_token_stats": rnd(s), "us_per_layer": round(tok_us / L, 3),
            "expert_hbm_gbps": round(L * layer_bytes / (tok_us * 1e-6) / 1e9, 1),
            "expert_hbm_frac_of_peak": round(L * layer_bytes / (tok_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)}


# ------------------------------------------------------------- router alone
def run_router(env: Env, args, seed):
    """objeta_hip_router_topk_device alone at the DeepSeek (256 experts, hidden 7168)
    and Qwen3-A3B (128 experts, hidden 2048) shapes, top-8, for 1 to 32 tokens: one
    token runs router_split_kernel (logits and the selecting workgroup in one launch),
    a batch the two-launch form (router_logits_batch_kernel, router_select_batch_kernel).
    A hipGraph holds 32 consecutive calls over a pool of 32 tokens (T tokens per call,
    the groups in turn) and the figure is the graph's time over 32, so it includes the
    gap between dependent launches as a layer does. A call whose exact-sum bounds
    cannot separate a decision recomputes the undecided logits in the reference's
    sequential order; with a batch the slowest token sets the call's time."""
    be = env.be
    res = {"path": "32 calls of objeta_hip_router_topk_device per hipGraph (renormalised top-8)"}
    for name, E, H in (("deepseek", 256, 7168), ("qwen3a3b", 128, 2048)):
        K, P, N = 8, 32, 32
        w = be.alloc(4 * E * H)
        env.fill_gauss(w.ptr, E * H, seed + E, 0.02)
        xs = be.alloc(4 * P * H)
        env.fill_gauss(xs.ptr, P * H, seed + 7 + E, 1.0)
        ids = be.alloc(4 * P * K)
        wts = be.alloc(4 * P * K)
        r = {"experts": E, "hidden": H, "top_k": K, "weight_bytes": 4 * E * H}
        for T in (1, 2, 4, 8, 16, 32):
            groups = P // T

            def enq(T=T, groups=groups):
                for i in range(N):
                    g = i % groups
                    env.check(env.lib.objeta_hip_router_topk_device(env.ctx, env.stream, w.addr(), None,
                                                                    xs.addr(4 * g * T * H), T, E, H, K, 1,
                                                                    ids.addr(4 * g * T * K), wts.addr(4 * g * T * K)))
            enq()
            be.synchronize(env.stream)
            g = env.capture(enq)
            for _ in range(3):
                env.launch(g)
            be.synchronize(env.stream)
            _, per = env.per_step(lambda i: env.launch(g), max(10, args.steps // 4))
            sc = stats([v / N for v in per])
            r[f"tokens{T}"] = {"us_per_call": rnd(sc), "us_per_token": round(sc["avg"] / T, 3)}
            env.destroy([g])
        res[name] = r
        for b in (w, xs, ids, wts):
            b.free()
    return res


# ------------------------------------------- DeepSeek official arithmetic (FP8)
def run_official(env: Env, args, seed):
    """The FP8-activation ("official arithmetic") layer at the DeepSeek shape: router,
    then objeta_hip_moe_official_fp4_device (act_quant of x, FP4 routed gate/up with the
    official SwiGLU, the FP8 shared expert, act_quant of the intermediates, FP4 routed
    down, shared down), replayed from a hipGraph at batch 1 and 32."""
    from objeta_amd import ExpertTable
    from objeta_amd.workloads import fp8_random_expert
    be = env.be
    H, I, E, K = 7168, 2048, 256, 8
    w_b, s_b = I * H // 2, I * H // 32
    dw_b, ds_b = H * I // 2, H * I // 32
    eb = 2 * (w_b + s_b) + dw_b + ds_b
    arena = be.alloc(E * eb)
    entries = []
    for e in range(E):
        base = arena.ptr + e * eb
        gw, gs = base, base + w_b
        uw, us = gs + s_b, gs + s_b + w_b
        dw, ds = us + s_b, us + s_b + dw_b
        for j, (wp, sp, r, c) in enumerate(((gw, gs, I, H), (uw, us, I, H), (dw, ds, H, I))):
            env.check(env.lib.objeta_hip_fill_fp4_split_device(env.ctx, None, C.c_void_p(wp), C.c_void_p(sp), r, c,
                                                               seed + 3 * e + j))
        entries.append((gw, uw, dw, gs, us, ds))
    table = ExpertTable(be, entries)
    sh = [be.to_device(a) for a in fp8_random_expert(H, I, H, seed + 7)]
    shared = ExpertTable(be, [(sh[0].addr(), sh[2].addr(), sh[4].addr(), sh[1].addr(), sh[3].addr(), sh[5].addr())])
    shared_bytes = sum(int(a.nbytes) for a in sh)
    w_r = be.alloc(4 * E * H)
    env.fill_gauss(w_r.ptr, E * H, seed + 5, 0.02)
    res = {"hidden": H, "intermediate": I, "experts": E, "top_k": K, "routed_format": "DeepSeekFp4E2M1",
           "shared_format": "F8_E4M3, E8M0 128x128 tiles", "routed_expert_bytes": eb, "shared_expert_bytes": shared_bytes,
           "path": "router, then objeta_hip_moe_official_fp4_device (FP8 activations), replayed from a hipGraph"}
    for T in (1, 32):
        P = 8
        xs = be.alloc(4 * P * T * H)
        env.fill_gauss(xs.ptr, P * T * H, seed + 10 + T, 1.0)
        out = be.alloc(4 * T * H)
        ids = be.alloc(4 * T * K)
        wts = be.alloc(4 * T * K)

        def enq(p, T=T, xs=xs, out=out, ids=ids, wts=wts):
            x = xs.addr(4 * p * T * H)
            env.check(env.lib.objeta_hip_router_topk_device(env.ctx, env.stream, w_r.addr(), None, x, T, E, H, K, 1,
                                                            ids.addr(), wts.addr()))
            env.moe.official_fp4_device(table, ids, wts, T, K, x, out, H, I, H, 10.0, stream=env.stream,
                                        shared_fp8=shared)
        enq(0)
        be.synchronize(env.stream)
        graphs = [env.capture(lambda p=p: enq(p)) for p in range(P)]
        for i in range(5):
            env.launch(graphs[i % P])
        be.synchronize(env.stream)
        _, per = env.per_step(lambda i: env.launch(graphs[i % P]), max(20, args.steps // 4))
        s = stats(per)
        sel = ids.download(np.uint32, T * K)
        distinct = len(set(int(v) for v in sel))
        ebytes = distinct * eb + shared_bytes
        res[f"batch{T}"] = {"us_per_layer": rnd(s), "us_per_token": round(s["avg"] / T, 3),
                            "expert_bytes_read": ebytes, "distinct_routed_experts": distinct,
                            "expert_hbm_gbps": round(ebytes / (s["avg"] * 1e-6) / 1e9, 1),
                            "expert_hbm_frac_of_peak": round(ebytes / (s["avg"] * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)}
        env.destroy(graphs)
        for b in (xs, out, ids, wts):
            b.free()
    arena.free()
    return res


# ------------------------------------------------------------- cache misses
def run_misses(env: Env, st: QwenStack, args, xs, P, report):
    """The stack with every expert in pinned host memory behind the expert cache at 25%
    of the expert bytes, through objeta_hip_moe_stack_cached: per layer the router on
    the device, its ids to the host once, the union of the step's selected experts
    resolved by the cache (misses copied on the copy stream), the layer's kernels after
    its own copies; the hidden state stays on the device. Batch 1 and a 16-token batch,
    each from an empty cache, without and with next-layer prefetch (layer l+1's router
    evaluated on layer l's input; its predicted experts' absent tensors copied behind
    layer l's misses). Two warm-up steps fill the cache; then `miss_tokens` steps are
    timed end to end on the host clock. The PCIe floor of a step is its loaded bytes at
    the rate of a 256 MiB pinned-host copy measured in the same run. With a report
    directory, a few tokens also go through execute_selected_moe_cuda per layer (the
    reference's executor, host x in and host out) for the MoeStatsReport."""
    from objeta_amd import ExpertCache, HostExpertSet, PinnedHostBuffer
    be = env.be
    L, H, E, K, I = st.layers, st.H, st.E, st.K, st.I
    eb = st.expert_bytes
    pin = PinnedHostBuffer(be, L * E * eb)
    host = pin.array(np.uint8)
    t0 = time.time()
    for l in range(L):
        env.check(env.lib.objeta_hip_copy_d2h(env.ctx, None, C.c_void_p(pin.ptr + l * E * eb), st.arenas[l].addr(),
                                              E * eb))
    be.synchronize()
    stage_s = time.time() - t0

    def tensors(l, e):
        base = l * E * eb
        g, u, d = st.offsets(e)
        return (host[base + g:base + g + st.gu_bytes], host[base + u:base + u + st.gu_bytes],
                host[base + d:base + d + st.dn_bytes])
    experts = [[tensors(l, e) for e in range(E)] for l in range(L)]
    sets = [HostExpertSet(experts[l]) for l in range(L)]
    layers = [(sets[l], st.router_w[l], st.router_b[l], l) for l in range(L)]
    # PCIe probe: one 256 MiB pinned -> device copy
    probe = be.alloc(256 << 20)
    ev0, ev1 = env.event(), env.event()
    env.record(ev0)
    env.check(env.lib.objeta_hip_copy_h2d(env.ctx, env.stream, probe.addr(), C.c_void_p(pin.ptr), 256 << 20))
    env.record(ev1)
    be.synchronize(env.stream)
    probe_gbps = (256 << 20) / (env.elapsed_us(ev0, ev1) * 1e-6) / 1e9
    env.drop_events([ev0, ev1])
    probe.free()
    capacity = (L * E * eb) // 4
    n_steps = args.miss_tokens

    def run(T: int, prefetch: bool):
        cache = ExpertCache(capacity, be)
        d_h = be.alloc(4 * T * H)
        wall, tels = [], []
        for step in range(n_steps + 2):
            for t in range(T):
                env.check(env.lib.objeta_hip_copy_d2d(env.ctx, env.stream, d_h.addr(4 * t * H),
                                                      xs.addr(4 * ((step * T + t) % P) * H), 4 * H))
            c0 = time.perf_counter()
            _, _, tel = env.moe.stack_cached(0, layers, K, T, d_h, H, I, cache=cache, prefetch_next=prefetch,
                                             stream=env.stream)
            if step >= 2:
                wall.append((time.perf_counter() - c0) * 1e6)
                tels.append(tel)
        cst = cache.stats()
        cache.close()
        d_h.free()
        s = stats(wall)
        loaded = sum(t["actual_expert_bytes_loaded"] for t in tels) / len(tels)
        logical = sum(t["logical_expert_bytes_requested"] for t in tels) / len(tels)
        pf_bytes = sum(t["prefetch_bytes_issued"] for t in tels) / len(tels)
        copy_ms = sum(t["copy_ms"] for t in tels) / len(tels)
        floor_us = (loaded + pf_bytes) / (probe_gbps * 1e9) * 1e6
        res = {"tokens_per_step": T, "us_per_step_end_to_end": rnd(s, 1), "us_per_token": round(s["avg"] / T, 1),
               "us_per_token_layer": round(s["avg"] / T / L, 2),
               "hit_rate_bytes": round(1.0 - loaded / logical, 4) if logical else None,
               "expert_bytes_loaded_per_step": int(loaded), "prefetch_bytes_per_step": int(pf_bytes),
               "distinct_experts_per_layer": round(sum(t["distinct_experts"] for t in tels) / len(tels) / L, 1),
               "pcie_floor_us_per_step": round(floor_us, 1),
               "end_to_end_over_pcie_floor": round(s["avg"] / floor_us, 3) if floor_us > 0 else None,
               "copy_stream_gbps": round((loaded / (copy_ms * 1e-3) / 1e9), 1) if copy_ms > 0 else None,
               "host_wait_ms_per_step": round(sum(t["host_wait_ms"] for t in tels) / len(tels), 3),
               "device_ms_per_step": round(sum(t["total_ms"] for t in tels) / len(tels), 3),
               "cache": {k: cst[k] for k in ("hit_count", "miss_count", "eviction_count", "resident_bytes",
                                              "cache_insert_accept_count")}}
        if prefetch:
            pred = sum(t["prefetch_experts_predicted"] for t in tels)
            res["prediction_accuracy"] = round(sum(t["prefetch_experts_correct"] for t in tels) / pred, 4) if pred else None
        return res

    res = {"layers": L, "cache_capacity_bytes": capacity, "expert_bytes_total": L * E * eb, "steps": n_steps,
           "pcie_probe_gbps": round(probe_gbps, 1), "host_staging_s": round(stage_s, 1),
           "path": "objeta_hip_moe_stack_cached: router on the device, ids to the host once per layer, the union of "
                   "the step's experts resolved through the 25% cache (misses copied on the copy stream from pinned "
                   "host memory), the layer's kernels after its own copies; hidden state on the device"}
    for T in (1, args.batch):
        res[f"batch{T}"] = run(T, False)
        res[f"batch{T}_prefetch"] = run(T, True)
    if report is not None:
        # the reference's executor, one call per layer, for the MoeStatsReport
        cache = ExpertCache(capacity, be)
        d_h = be.alloc(4 * H)
        d_ids, d_w = be.alloc(4 * K), be.alloc(4 * K)
        tel_runs, last = [], None
        for t in range(3):
            h = xs.download(np.float32, H, offset=4 * (t % P) * H)
            for l in range(L):
                d_h.upload(h)
                env.check(env.lib.objeta_hip_router_topk_device(env.ctx, None, st.router_w[l].addr(),
                                                                st.router_b[l].addr(), d_h.addr(), 1, E, H, K, 1,
                                                                d_ids.addr(), d_w.addr()))
                ids = d_ids.download(np.uint32, K)
                ws = d_w.download(np.float32, K)
                sel = [(int(i), float(w)) for i, w in zip(ids, ws)]
                out, tel = env.moe.execute_selected_moe_cuda(None, None, sets[l], sel, h, H, I, H, l, cache)
                last = (l, sel, h.copy(), out.copy())
                h = (h + out).astype(np.float32)
                if t >= 1:
                    tel_runs.append(tel)
        cache.close()
        report["moe_tel"] = tel_runs
        report["moe_shape"] = (H, I, H, K)
        report["moe_last"] = last
    del experts, host, sets, layers
    pin.free()
    return res


# ------------------------------------------------------------- CPU baseline
def run_cpu(env: Env, st: QwenStack, xs, args):
    """The oracle's C restatement of cpu_router + selected_moe_cpu on the host cores:
    one core (pinned with sched_setaffinity) and all cores (row-parallel OpenMP),
    median of `runs` runs over the same sample of layers; also the parity of the
    GPU layer against it (ids bit-exact, outputs relative error)."""
    from oracle import oracle as orc
    be = env.be
    L, H, E, K, I = st.layers, st.H, st.E, st.K, st.I
    layers = list(range(0, L, max(1, L // args.cpu_layers)))[:args.cpu_layers]
    hin, hout = be.alloc(4 * H), be.alloc(4 * H)
    lids, lwts = be.alloc(4 * K), be.alloc(4 * K)
    cases = []
    mism, max_rel = 0, 0.0
    hg = xs.download(np.float32, H)
    for l in layers:
        hin.upload(hg)
        env.moe.layer_device(st.fmt, st.tables[l], st.router_w[l], st.router_b[l], K, 1, hin.addr(), hin.addr(),
                             hout.addr(), lids.addr(), lwts.addr(), H, I, H)
        be.synchronize()
        gpu_out = hout.download(np.float32, H)
        gpu_ids = lids.download(np.uint32, K)
        w_r = st.router_w[l].download(np.float32, E * H)
        rid, rw, _, _ = orc.router(w_r, hg, E, H, K, bias=st.bias_host[l], renormalize=True)
        mism += int(not np.array_equal(rid, gpu_ids))
        ex = {int(e): st.expert_host_bytes(l, int(e)) for e in rid}
        order = sorted(ex)
        remap = {e: i for i, e in enumerate(order)}
        sel = [(remap[int(e)], float(w)) for e, w in zip(rid, rw)]
        exl = [ex[e] for e in order]
        ref = (hg + orc.selected_moe(0, exl, sel, hg, H, I, H)).astype(np.float32)
        max_rel = max(max_rel, float(np.max(np.abs(gpu_out - ref))) / float(np.max(np.abs(ref))))
        cases.append((w_r, st.bias_host[l], hg.copy(), exl, order))
        hg = gpu_out

    def one_pass():
        t0 = time.perf_counter()
        for w_r, b, x, exl, order in cases:
            rid, rw, _, _ = orc.router(w_r, x, E, H, K, bias=b, renormalize=True)
            orc.selected_moe(0, exl, [(order.index(int(e)), float(w)) for e, w in zip(rid, rw)], x, H, I, H)
        return (time.perf_counter() - t0) * 1e6 / len(cases)

    ncpu = os.cpu_count() or 1
    allowed = sorted(os.sched_getaffinity(0))
    out = {}
    for label, threads in (("one_core", 1), ("all_cores", len(allowed))):
        orc.set_threads(threads)
        if threads == 1:
            os.sched_setaffinity(0, {allowed[0]})
        try:
            one_pass()
            runs = [one_pass() for _ in range(args.cpu_runs)]
        finally:
            os.sched_setaffinity(0, set(allowed))
            orc.set_threads(1)
        out[label] = {"us_per_token_layer": round(float(np.median(runs)), 1), "runs_us": [round(r, 1) for r in runs],
                      "threads": threads}
    sample = (f"{len(cases)} layer calls (layers {layers[0]}..{layers[-1]} of one token, each from the GPU's input "
              f"of that layer): cpu_router + selected_moe_cpu, oracle C restatement built -O2 -ffp-contract=off; "
              f"median of {args.cpu_runs} runs after one warm-up run")
    return {"value": out["one_core"]["us_per_token_layer"], "unit": "us/token/layer", "cores": 1, "kind": "port",
            "sample": sample, "pinned_core": allowed[0],
            "all_cores": {"value": out["all_cores"]["us_per_token_layer"], "unit": "us/token/layer",
                          "cores": out["all_cores"]["threads"], "kind": "port (row-parallel OpenMP)"},
            "runs": out, "nproc": ncpu, "affinity_cpus": len(allowed), "cpu_model": cpu_model(),
            "parity_vs_gpu": {"layers_checked": len(cases), "router_id_mismatched_layers": mism,
                              "layer_output_max_rel_err": max_rel}}


# ------------------------------------------------------------------- reports
def report_numerics(env: Env, st: QwenStack, args, gemv_checks, report):
    """The numerics of the reports, as the reference's benches compute them
    (bench_qgemv.rs:145-156, bench_selected_moe.rs:396-406): the device result against
    the oracle's quantized CPU path (cuda_vs_cpu_quant) and against the fp32 path on
    the unquantized weights (quant_vs_fp32), both through compare_outputs."""
    from oracle import oracle as orc
    from objeta_amd import reports
    be = env.be
    gemv_num = []
    for fmt, rows, cols, seed, q, x, y in gemv_checks:
        ref = orc.gemv(fmt, q, x, rows, cols)
        m = be.alloc(4 * rows * cols)
        env.fill_gauss(m.ptr, rows * cols, seed, 0.02)
        dense = orc.dense_gemv(m.download(np.float32, rows * cols), x, rows, cols)
        m.free()
        gemv_num.append(reports.numerics_suite(orc.compare(ref, y), orc.compare(dense, y)))
    moe_num = None
    if report and report.get("moe_last"):
        l, sel, h, out = report["moe_last"]
        H, E, I = st.H, st.E, st.I
        ids = [e for e, _ in sel]
        order = sorted(set(ids))
        remap = {e: i for i, e in enumerate(order)}
        sel2 = [(remap[e], w) for e, w in sel]
        q = [st.expert_host_bytes(l, e) for e in order]
        ref = orc.selected_moe(0, q, sel2, h, H, I, H)
        f32 = []
        for e in order:
            mats = []
            for (which, first), n in zip(st.f32_first(e), (I * H, I * H, H * I)):
                m = be.alloc(4 * n)
                key = st.gu_key(l) if which == 0 else st.dn_key(l)
                env.check(env.lib.objeta_hip_fill_gauss_device(env.ctx, None, m.addr(), n, key, first,
                                                               C.c_float(0.02)))
                mats.append(m.download(np.float32, n))
                m.free()
            f32.append(tuple(mats))
        ref32 = orc.selected_moe(-1, f32, sel2, h, H, I, H)
        moe_num = reports.numerics_suite(orc.compare(ref, out), orc.compare(ref32, out))
    return gemv_num, moe_num


def write_reports(path: str, gemv, report, gemv_num, moe_num):
    """QGemvStatsReport lines (bench_qgemv.rs:6-37) for the GEMV sweep and a
    MoeStatsReport (bench_selected_moe.rs:19-101) for the cache-miss executor runs."""
    from objeta_amd import reports
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "qgemv_stats_reports.jsonl"), "w") as f:
        for i, g in enumerate(gemv or []):
            fmt = {"Q4_0": 0, "Q5_0": 1, "IQ3_0": 2}[g["format"]]
            f.write(json.dumps(reports.qgemv_stats_report(
                backend="hip", kernel=KERNEL_NAME[fmt], fmt=g["format"], rows=g["rows"], cols=g["cols"],
                kernel_ms=[v / 1000.0 for v in g["samples_us"]],
                bytes_read=g["rows"] * (g["cols"] // 32) * BB[fmt] + 4 * g["cols"],
                numerics=gemv_num[i] if gemv_num and i < len(gemv_num) else None)) + "\n")
    if report and report.get("moe_tel"):
        H, I, O, K = report["moe_shape"]
        with open(os.path.join(path, "moe_stats_report.json"), "w") as f:
            f.write(json.dumps(reports.moe_stats_report(source="synthetic", backend="hip", fmt="Q4_0", hidden=H,
                                                        intermediate=I, out=O, telemetries=report["moe_tel"],
                                                        numerics=moe_num)) + "\n")


def pmc_calibration(env: Env) -> int:
    """Kernels of known traffic for scaling rocprofv3's FETCH_SIZE / WRITE_SIZE: a zero
    fill of 64 MiB (writes only) and a Q4_0 GEMV over a 16384 x 4096 matrix (37,748,736
    weight bytes read once, plus 16 KiB of x), five of each."""
    ctx, lib = env.ctx, env.lib
    fill = env.be.alloc(64 << 20)
    rows, cols = 16384, 4096
    wq = env.be.alloc(rows * (cols // 32) * 18)
    env.fill_q(0, wq.ptr, rows, cols, 5)
    x, y = env.be.alloc(4 * cols), env.be.alloc(4 * rows)
    env.fill_gauss(x.ptr, cols, 6, 1.0)
    env.be.synchronize()
    for _ in range(5):
        env.check(lib.objeta_hip_zero_device(ctx, None, fill.addr(), 64 << 20))
        env.check(lib.objeta_hip_qgemv_device(ctx, 0, None, wq.addr(), x.addr(), y.addr(), rows, cols, 1))
    env.be.synchronize()
    print(json.dumps({"calibration": {"fill_bytes": 64 << 20, "gemv_weight_bytes": rows * (cols // 32) * 18,
                                      "gemv_x_bytes": 4 * cols, "gemv_y_bytes": 4 * rows}}), flush=True)
    env.be.close()
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--tokens-pool", type=int, default=16, help="distinct input tokens cycled over steps")
    ap.add_argument("--seed", type=int, default=20251201)
    ap.add_argument("--batch", type=int, default=16, help="tokens of the batched side measurement")
    ap.add_argument("--kernel-reps", type=int, default=10, help="replays of each kernel's rotation graph")
    ap.add_argument("--gemv-calls", type=int, default=512,
                    help="GEMV calls per graph in the gemv section (small values keep profiler runs short)")
    ap.add_argument("--gemv-rotate-mb", type=int, default=ROTATE_BYTES >> 20,
                    help="bytes of matrix replicas the gemv section cycles through, in MiB (>= 512 keeps "
                         "the weights out of the 256 MB MALL)")
    ap.add_argument("--miss-tokens", type=int, default=16, help="steps timed through the 25%% cache (each of 1 and --batch tokens)")
    ap.add_argument("--cpu-layers", type=int, default=8, help="layer calls in the CPU-baseline sample")
    ap.add_argument("--cpu-runs", type=int, default=5)
    ap.add_argument("--sections", default=",".join(SECTIONS), help="comma list of " + ", ".join(SECTIONS))
    ap.add_argument("--report-dir", default=None, help="write reference-schema JSON reports here")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "one GPU is measured; --gpus > 1 is not supported (a layer would "
                                   "shard each selected expert's rows over the GPUs and all-reduce "
                                   "the partial outputs)"}))
        return 2
    sections = set(s.strip() for s in args.sections.split(",") if s.strip())
    bad = sections - set(SECTIONS) - set(EXTRA_SECTIONS)
    if bad:
        print(json.dumps({"error": f"unknown sections {sorted(bad)}"}))
        return 2

    env = Env()
    if "calibrate" in sections:
        return pmc_calibration(env)
    H, E, K, I, L = 2048, 128, 8, 768, args.layers
    t0 = time.time()
    st = QwenStack(env, L, H, E, K, I, args.seed)
    print(f"# generated {L} layers x {E} experts ({L * E * st.expert_bytes / 1e9:.2f} GB) in {time.time() - t0:.1f}s",
          file=sys.stderr, flush=True)
    P = args.tokens_pool
    xs = env.be.alloc(4 * P * H)
    env.fill_gauss(xs.ptr, P * H, args.seed + 77, 1.0)
    env.be.synchronize()

    def stage(name):
        print(f"# {name} ({time.time() - t0:.1f}s)", file=sys.stderr, flush=True)

    token_us, step_stats, layer_io = None, None, None
    if "headline" in sections or "kernels" in sections:
        stage("headline")
        token_us, step_stats, layer_io = run_headline(env, st, args, xs, P)
    kernels = None
    if "kernels" in sections:
        stage("kernels")
        kernels = run_kernels(env, st, layer_io, args.kernel_reps)
    batch = None
    if "batch" in sections and args.batch > 0:
        stage("batch")
        batch = run_batch(env, st, args, args.seed)
    gemv, gemv_checks = None, []
    if "gemv" in sections:
        stage("gemv")
        gemv = run_gemv(env, max(8, args.kernel_reps // 4), gemv_checks if args.report_dir else None,
                        calls=max(1, args.gemv_calls), rotate=max(64, args.gemv_rotate_mb) << 20)
    stack4 = None
    if "stack4" in sections:
        stage("stack4")
        stack4 = run_stack4(env, args, args.seed + 3000)
    deepseek = None
    if "deepseek" in sections:
        stage("deepseek")
        deepseek = run_deepseek(env, args, args.seed + 5000)
    official = None
    if "official" in sections:
        stage("official")
        official = run_official(env, args, args.seed + 6000)
    router = None
    if "router" in sections:
        stage("router")
        router = run_router(env, args, args.seed + 7000)
    report = {} if args.report_dir else None
    misses = None
    if "misses" in sections:
        stage("misses")
        misses = run_misses(env, st, args, xs, P, report)
    cpu = None
    if "cpu" in sections:
        stage("cpu")
        cpu = run_cpu(env, st, xs, args)
    if args.report_dir:
        stage("reports")
        gemv_num, moe_num = report_numerics(env, st, args, gemv_checks, report)
        write_reports(args.report_dir, gemv, report, gemv_num, moe_num)
    stage("done")
    for g in gemv or []:
        g.pop("samples_us", None)

    expert_bytes_token = L * K * st.expert_bytes
    roof = None
    if kernels:
        dom = max(kernels, key=lambda k: kernels[k]["avg_launch_us"])
        roof = dict(kernels[dom])
        roof["dominant_of"] = "router, gate_up, down (largest average launch time)"
    dev = env.be.device_info
    rec = {
        "metric": "MoE layer us/token + achieved HBM GB/s (% of peak), Q4_0 Qwen3-A3B shape",
        "value": round(token_us / L, 3) if token_us else None,
        "unit": "us/token/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(token_us / 1000.0, 4) if token_us else None,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 weights, fp32 compute",
        "data": "synthetic (device-generated N(0,0.02) Q4_0 weights, Zipf(1.1)-biased router, N(0,1) tokens)",
        "config": {"workload": "qwen3_a3b_moe_stack", "layers": L, "hidden": H, "experts": E, "top_k": K,
                   "moe_intermediate": I, "batch": 1, "format": "Q4_0", "residency": "all experts in HBM",
                   "tokens_pool": P},
        "path": "three kernels per layer (router, gate/up + SiLU, down + combine) replayed from a hipGraph",
        "us_per_token": round(token_us, 2) if token_us else None,
        "us_per_step_stats": rnd(step_stats, 2) if step_stats else None,
        "us_per_token_layer_p50": round(step_stats["p50"] / L, 3) if step_stats else None,
        "us_per_token_layer_p95": round(step_stats["p95"] / L, 3) if step_stats else None,
        "expert_bytes_per_token": expert_bytes_token,
        "expert_hbm_gbps": round(expert_bytes_token / (token_us * 1e-6) / 1e9, 1) if token_us else None,
        "expert_hbm_frac_of_peak": (round(expert_bytes_token / (token_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4)
                                    if token_us else None),
        "roofline": roof,
        "kernels": kernels,
        "batch": batch,
        "gemv": gemv,
        "stack4": stack4,
        "deepseek": deepseek,
        "official": official,
        "router": router,
        "misses": misses,
        "cpu_baseline": cpu,
        "device": {"name": dev["name"], "arch": dev["arch"], "compute_units": dev["compute_units"]},
    }
    print(json.dumps(rec), flush=True)
    env.be.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
