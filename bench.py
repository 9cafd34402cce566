#!/usr/bin/env python3
"""Benchmark: Qwen3-A3B-shaped selected-expert MoE layer stack on one MI355X.

Workload (the headline configuration): 48 MoE layers, hidden 2048, 128 experts,
top-8, moe_intermediate 768, SwiGLU experts with Q4_0 weights ~N(0, 0.02) (18-byte
blocks), router W_r ~N(0, 0.02) with logits biased by ln Zipf(s=1.1) over a
per-layer rank permutation, hidden ~N(0, 1), batch 1 decode. Each layer computes
    h <- h + sum_j w_j * down_j(silu(gate_j h) * up_j h)
over the router's softmax -> top-8 -> renormalised selection. Every expert of every
layer is resident in HBM (16.3 GB); one step is one token through all 48 layers,
three kernels per layer (router + top-8, fused gate/up + SiLU, down + combine)
replayed from a hipGraph.

Reported: MoE layer us/token (step time / 48), the step's us/token, achieved HBM
GB/s on expert-weight bytes (8 experts x 2,654,208 B per layer) and its fraction of
MI355X's 8 TB/s, a roofline record for a layer kernel timed with HIP events on
its stream, and the CPU
baseline: the oracle's single-thread restatement of the reference CPU path
(cpu_router + selected_moe_cpu) on a few tokens.

Synthetic data generated on the device with the counter-based generator shared
with the oracle (no checkpoints).
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

HBM_PEAK_GBPS = 8000.0

from objeta_amd.workloads import zipf_bias  # noqa: E402


def cpu_model() -> str:
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return platform.processor() or "unknown"


class Stack:
    """Device-resident Q4_0 MoE layer stack (weights, router, expert tables)."""

    def __init__(self, be, layers, hidden, n_experts, k, inter, seed):
        from objeta_amd import ExpertTable, QuantFormat, check
        self.be, self.L = be, be.L
        self.layers, self.H, self.E, self.K, self.I = layers, hidden, n_experts, k, inter
        self.fmt = int(QuantFormat.Q4_0)
        ctx = be.ctx
        self.gu_bytes = inter * (hidden // 32) * 18
        self.dn_bytes = hidden * (inter // 32) * 18
        self.expert_bytes = 2 * self.gu_bytes + self.dn_bytes
        self.arenas, self.tables, self.router_w, self.router_b = [], [], [], []
        for l in range(layers):
            arena = be.alloc(n_experts * self.expert_bytes)
            entries = []
            for e in range(n_experts):
                base = arena.ptr + e * self.expert_bytes
                g, u, d = base, base + self.gu_bytes, base + 2 * self.gu_bytes
                key = seed + ((l * n_experts + e) * 3)
                check(self.L.objeta_hip_fill_gauss_quantized_device(ctx, self.fmt, None, C.c_void_p(g), inter, hidden,
                                                                    key, C.c_float(0.02)))
                check(self.L.objeta_hip_fill_gauss_quantized_device(ctx, self.fmt, None, C.c_void_p(u), inter, hidden,
                                                                    key + 1, C.c_float(0.02)))
                check(self.L.objeta_hip_fill_gauss_quantized_device(ctx, self.fmt, None, C.c_void_p(d), hidden, inter,
                                                                    key + 2, C.c_float(0.02)))
                entries.append((g, u, d))
            self.arenas.append(arena)
            self.tables.append(ExpertTable(be, entries))
            w = be.alloc(4 * n_experts * hidden)
            check(self.L.objeta_hip_fill_gauss_device(ctx, None, w.addr(), n_experts * hidden, seed + 10_000_000 + l, 0,
                                                      C.c_float(0.02)))
            self.router_w.append(w)
            self.router_b.append(be.to_device(zipf_bias(n_experts, 1.1, seed + l)))
        be.synchronize()

    def expert_host_bytes(self, layer: int, e: int):
        """(gate, up, down) bytes of one expert, copied back from HBM."""
        buf = self.arenas[layer].download(np.uint8, self.expert_bytes, offset=e * self.expert_bytes)
        g = buf[:self.gu_bytes]
        u = buf[self.gu_bytes:2 * self.gu_bytes]
        d = buf[2 * self.gu_bytes:]
        return g, u, d


TRAFFIC_PROFILE = "profiles/moe_layer_q4_qwen3a3b_hbm_traffic.md"


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary of this workload (counters cannot be read from inside the run)."""
    path = os.path.join(ROOT, TRAFFIC_PROFILE)
    try:
        for line in open(path):
            if line.startswith(f"traffic_bytes_per_launch {kernel}:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def pmc_calibration(be, lib) -> int:
    """Kernels of known traffic for scaling rocprofv3's FETCH_SIZE / WRITE_SIZE: a fill of
    64 MiB (writes only) and a Q4_0 GEMV over a 16384 x 4096 matrix (37,748,736 B read
    once, plus 16 KiB of x)."""
    from objeta_amd import check
    ctx = be.ctx
    fill = be.alloc(64 << 20)
    rows, cols = 16384, 4096
    wq = be.alloc(rows * (cols // 32) * 18)
    check(lib.objeta_hip_fill_gauss_quantized_device(ctx, 0, None, wq.addr(), rows, cols, 5, C.c_float(0.02)))
    x = be.alloc(4 * cols)
    y = be.alloc(4 * rows)
    check(lib.objeta_hip_fill_gauss_device(ctx, None, x.addr(), cols, 6, 0, C.c_float(1.0)))
    be.synchronize()
    for _ in range(5):
        check(lib.objeta_hip_zero_device(ctx, None, fill.addr(), 64 << 20))
        check(lib.objeta_hip_qgemv_device(ctx, 0, None, wq.addr(), x.addr(), y.addr(), rows, cols, 1))
    be.synchronize()
    print(json.dumps({"calibration": {"fill_bytes": 64 << 20, "gemv_weight_bytes": rows * (cols // 32) * 18,
                                      "gemv_x_bytes": 4 * cols, "gemv_y_bytes": 4 * rows}}), flush=True)
    be.close()
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--tokens-pool", type=int, default=16, help="distinct input tokens cycled over steps")
    ap.add_argument("--cpu-tokens", type=int, default=4, help="tokens in the CPU-baseline sample (0 = skip)")
    ap.add_argument("--seed", type=int, default=20251201)
    ap.add_argument("--pmc-calibrate", action="store_true",
                    help="only run the counter calibration kernels (a 64 MiB fill, a 37.7 MB streaming read)")
    ap.add_argument("--batch", type=int, default=16,
                    help="tokens of the batched side measurement (layer entry point and grouped-token path); 0 skips it")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "one GPU is measured; --gpus > 1 is not supported (a layer would "
                                   "shard each selected expert's rows over the GPUs and all-reduce "
                                   "the partial outputs)"}))
        return 2

    from objeta_amd import HipBackend, MoeExecutor, check
    from objeta_amd._lib import load

    H, E, K, I, L = 2048, 128, 8, 768, args.layers
    be = HipBackend(0, 2)
    lib = load()
    ctx = be.ctx
    if args.pmc_calibrate:
        return pmc_calibration(be, lib)
    t0 = time.time()
    stack = Stack(be, L, H, E, K, I, args.seed)
    print(f"# generated {L} layers x {E} experts ({L * E * stack.expert_bytes / 1e9:.2f} GB) in "
          f"{time.time() - t0:.1f}s", file=sys.stderr, flush=True)

    P = args.tokens_pool
    xs = be.alloc(4 * P * H)
    check(lib.objeta_hip_fill_gauss_device(ctx, None, xs.addr(), P * H, args.seed + 77, 0, C.c_float(1.0)))
    h = be.alloc(4 * H)
    ids = be.alloc(4 * L * K)
    wts = be.alloc(4 * L * K)
    moe = MoeExecutor(be)
    stream = be.stream(0)

    def enqueue_token(p: int):
        x0 = xs.addr(4 * p * H)
        for l in range(L):
            src = x0 if l == 0 else h.addr()
            moe.layer_device(stack.fmt, stack.tables[l], stack.router_w[l], stack.router_b[l], K, 1, src, src,
                             h.addr(), ids.addr(4 * l * K), wts.addr(4 * l * K), H, I, H, stream=stream)

    ev0, ev1 = C.c_void_p(), C.c_void_p()
    check(lib.objeta_hip_event_create(ctx, C.byref(ev0)))
    check(lib.objeta_hip_event_create(ctx, C.byref(ev1)))
    ms = C.c_float()

    expert_bytes_token = L * K * stack.expert_bytes
    router_bytes_token = L * (4 * E * H)

    def timed(launch, steps):
        check(lib.objeta_hip_event_record(ctx, ev0, stream))
        for i in range(steps):
            launch(i)
        check(lib.objeta_hip_event_record(ctx, ev1, stream))
        check(lib.objeta_hip_event_elapsed_ms(ctx, ev0, ev1, C.byref(ms)))
        be.synchronize(stream)
        if moe.device_error() != 0:
            raise RuntimeError("device error word set during a timed run")
        return ms.value * 1000.0 / steps

    # ---- three kernels per layer (router, gate/up + SiLU, down + combine), replayed from a hipGraph ----
    graph_us = None
    gu_us = None
    if True:
        enqueue_token(0)
        be.synchronize(stream)
        graphs = []
        for p in range(P):
            check(lib.objeta_hip_graph_begin_capture(ctx, stream))
            enqueue_token(p)
            g = C.c_void_p()
            check(lib.objeta_hip_graph_end_capture(ctx, stream, C.byref(g)))
            graphs.append(g)
        for i in range(args.warmup):
            check(lib.objeta_hip_graph_launch(ctx, graphs[i % P], stream))
        be.synchronize(stream)
        graph_us = timed(lambda i: check(lib.objeta_hip_graph_launch(ctx, graphs[i % P], stream)), args.steps)
        # the graph's largest kernel on its own: gate/up + SiLU of one layer's 8 selected experts
        act = be.alloc(4 * K * I)
        lids = ids.addr(4 * 0 * K)

        def gate_up(i):
            moe.gate_up_device(stack.fmt, stack.tables[i % L], lids, 1, K, xs.addr(4 * (i % P) * H), act.addr(),
                               H, I, stream=stream)
        for i in range(args.warmup):
            gate_up(i)
        be.synchronize(stream)
        gu_us = timed(gate_up, args.steps)

    token_us = graph_us
    layer_us = token_us / L
    gbps = expert_bytes_token / (token_us * 1e-6) / 1e9
    if True:
        # 8 experts' gate and up matrices + x in + activations out
        kernel_bytes = K * 2 * stack.gu_bytes + 4 * H + 4 * K * I
        traffic = measured_traffic("moe_gate_up_kernel")
        roof = {"kernel": "moe_gate_up_kernel (fused gate/up + SiLU, 8 selected experts, one layer)", "bound": "hbm",
                "achieved": round(kernel_bytes / (gu_us * 1e-6) / 1e9, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(kernel_bytes / (gu_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4), "traffic": traffic,
                "traffic_source": TRAFFIC_PROFILE if traffic else None,
                "avg_launch_us": round(gu_us, 3), "algorithmic_bytes_per_launch": kernel_bytes}

    # ---- side measurement: a batch of tokens through the same 48 layers ----
    batch = None
    if args.batch > 0:
        B = args.batch
        xb = be.alloc(4 * B * H)
        check(lib.objeta_hip_fill_gauss_device(ctx, None, xb.addr(), B * H, args.seed + 99, 0, C.c_float(1.0)))
        hb = be.alloc(4 * B * H)
        idsb = be.alloc(4 * L * B * K)
        wtsb = be.alloc(4 * L * B * K)

        def enqueue_batch(grouped: bool):
            for l in range(L):
                src = xb.addr() if l == 0 else hb.addr()
                li, lw = idsb.addr(4 * l * B * K), wtsb.addr(4 * l * B * K)
                if grouped:  # router, then the grouped-token product (each selected expert read once)
                    check(lib.objeta_hip_router_topk_device(ctx, stream, stack.router_w[l].addr(),
                                                            stack.router_b[l].addr(), src, B, E, H, K, 1, li, lw))
                    moe.grouped_device(stack.fmt, stack.tables[l], li, lw, B, K, src, src, hb.addr(), H, I, H,
                                       stream=stream)
                else:  # the layer entry point: router, then one expert pass per (token, slot)
                    moe.layer_device(stack.fmt, stack.tables[l], stack.router_w[l], stack.router_b[l], K, B, src,
                                     src, hb.addr(), li, lw, H, I, H, stream=stream)

        res = {}
        for grouped in (True, False):
            enqueue_batch(grouped)
            be.synchronize(stream)
            check(lib.objeta_hip_graph_begin_capture(ctx, stream))
            enqueue_batch(grouped)
            gb = C.c_void_p()
            check(lib.objeta_hip_graph_end_capture(ctx, stream, C.byref(gb)))
            for i in range(3):
                check(lib.objeta_hip_graph_launch(ctx, gb, stream))
            be.synchronize(stream)
            res[grouped] = timed(lambda i: check(lib.objeta_hip_graph_launch(ctx, gb, stream)),
                                 max(5, args.steps // 20))
        ids_all = idsb.download(np.uint32, L * B * K).reshape(L, B * K)
        uniq = [len(set(int(v) for v in ids_all[l])) for l in range(L)]
        unique_bytes = sum(uniq) * stack.expert_bytes
        batch = {"tokens": B, "path": "layer entry point: router + per-assignment gate/up and down kernels",
                 "us_per_step": round(res[False], 1),
                 "us_per_token_layer": round(res[False] / (L * B), 3),
                 "grouped_path_us_per_step": round(res[True], 1),
                 "unique_experts_per_layer": round(sum(uniq) / L, 1),
                 "unique_expert_bytes_per_step": unique_bytes,
                 "expert_hbm_gbps": round(unique_bytes / (res[False] * 1e-6) / 1e9, 1)}

    # ---- CPU baseline: oracle restatement, one thread, same layers ----
    cpu = None
    if args.cpu_tokens > 0:
        from oracle import oracle as orc
        cpu_time = 0.0
        n_layer_calls = 0
        mism = 0
        max_rel = 0.0
        hin = be.alloc(4 * H)
        hout = be.alloc(4 * H)
        lids, lwts = be.alloc(4 * K), be.alloc(4 * K)
        for p in range(args.cpu_tokens):
            # layer by layer, both sides start from the GPU's own input of that layer
            hg = xs.download(np.float32, H, offset=4 * p * H)
            for l in range(L):
                hin.upload(hg)
                moe.layer_device(stack.fmt, stack.tables[l], stack.router_w[l], stack.router_b[l], K, 1, hin.addr(),
                                 hin.addr(), hout.addr(), lids.addr(), lwts.addr(), H, I, H)
                be.synchronize()
                gpu_out = hout.download(np.float32, H)
                gpu_ids = lids.download(np.uint32, K)
                w_r = stack.router_w[l].download(np.float32, E * H)
                bias = stack.router_b[l].download(np.float32, E)
                t1 = time.perf_counter()
                rid, rw, _, _ = orc.router(w_r, hg, E, H, K, bias=bias, renormalize=True)
                cpu_time += time.perf_counter() - t1
                mism += int(not np.array_equal(rid, gpu_ids))
                experts = {int(e): stack.expert_host_bytes(l, int(e)) for e in rid}
                order = sorted(experts)
                remap = {e: i for i, e in enumerate(order)}
                sel = [(remap[int(e)], float(w)) for e, w in zip(rid, rw)]
                t1 = time.perf_counter()
                out = orc.selected_moe(0, [experts[e] for e in order], sel, hg, H, I, H)
                ref = (hg + out).astype(np.float32)
                cpu_time += time.perf_counter() - t1
                n_layer_calls += 1
                max_rel = max(max_rel, float(np.max(np.abs(gpu_out - ref))) / float(np.max(np.abs(ref))))
                hg = gpu_out
        cpu_layer_us = cpu_time * 1e6 / n_layer_calls
        cpu = {"value": round(cpu_layer_us, 1), "unit": "us/token/layer", "cores": 1, "kind": "port",
               "sample": f"{args.cpu_tokens} token(s) x {L} layers: cpu_router + selected_moe_cpu (oracle C "
                         f"restatement, -O2 -ffp-contract=off, 1 thread) on the same weights",
               "cpu_model": cpu_model(), "stack_us_per_token": round(cpu_layer_us * L, 1),
               "parity_vs_gpu": {"layers_checked": n_layer_calls, "router_id_mismatched_layers": mism,
                                 "layer_output_max_rel_err": max_rel}}

    dev = be.device_info
    rec = {
        "metric": "MoE layer us/token + achieved HBM GB/s (% of peak), Q4_0 Qwen3-A3B shape",
        "value": round(layer_us, 3),
        "unit": "us/token/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(token_us / 1000.0, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 weights, fp32 compute",
        "data": "synthetic (device-generated N(0,0.02) Q4_0 weights, Zipf(1.1)-biased router, N(0,1) tokens)",
        "config": {"workload": "qwen3_a3b_moe_stack", "layers": L, "hidden": H, "experts": E, "top_k": K,
                   "moe_intermediate": I, "batch": 1, "format": "Q4_0", "residency": "all experts in HBM",
                   "tokens_pool": P},
        "path": "three kernels per layer from a hipGraph",
        "us_per_token": round(token_us, 2),
        "expert_bytes_per_token": expert_bytes_token,
        "expert_hbm_gbps": round(gbps, 1),
        "expert_hbm_frac_of_peak": round(gbps / HBM_PEAK_GBPS, 4),
        "roofline": roof,
        "gate_up_kernel_us": round(gu_us, 3) if gu_us is not None else None,
        "batch": batch,
        "cpu_baseline": cpu,
        "device": {"name": dev["name"], "arch": dev["arch"], "compute_units": dev["compute_units"]},
    }
    print(json.dumps(rec), flush=True)
    be.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
