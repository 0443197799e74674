#!/usr/bin/env python3
"""Benchmark of the MoE expert-FFN decode section on one MI355X.

Workload: the 30-layer Gemma-4-26B-A4B-shaped
expert section (H 2816, I 704, 128 experts, top-8, q4_0 banks of seeded
Irwin-Hall(4) weights of sd 0.02, f32 routers of the same), decoding tokens at batch 1
with the residual chain x <- x + MoE_l(rmsnorm(x)) between layers (attention
stubbed as identity; the unweighted pre-norm is the reference model's, and
without it (--input-norm 0) the chain's GELU*up, quadratic in the scale of x,
overflows to inf within the 30 layers of the Zipf stack and 3 of the
large-expert stack). One step = one token through all 30 layers; inputs (banks,
routers, the tokens' hidden states) are resident in HBM before timing.

Prints one JSON line: value = mean us/token (lower is better), plus achieved
HBM GB/s over the algorithmic expert bytes (802,897,920 B/token), the
roofline of the dominant kernel, and a CPU baseline (the oracle's restatement
of ft-core's AVX2 path, timed on this host's cores on a bounded sample).

--config picks one of BASELINE.json's other configurations instead (cfg3 Zipf
routing, cfg4 batched decode at 16/64 tokens, cfg5 the large-expert shape at
batch 1 and 32). One step is then one batch of B tokens through all layers;
value stays us/token (step time / B) and GB/s counts each step's unique
experts once per layer (the bytes a grouped product has to stream).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "freetoken-rs_amd"))

HBM_PEAK_GBPS = 8000.0
# HBM bytes per launch of the kernel each config's `roofline` names (per step where that is the
# whole HIP graph of a step), measured with rocprofv3 --pmc FETCH_SIZE and, in a second run,
# WRITE_SIZE on `bench.py --config NAME --steps 4 --warmup 2 --no-cpu --copy-calib 256` (default
# options otherwise): FETCH_SIZE x 1.9982 + WRITE_SIZE x 1.0, the two factors being what a plain
# 256 MiB torch copy in the same run reads and writes over what the counters report for it.
# Summaries and commands: profiles/hbm_traffic.md. Reported only for runs with those options.
MEASURED_TRAFFIC = {
    "gemma30": 883615384,    # k_moe_stack_fused, one launch (algorithmic 846,151,680 B)
    "zipf": 888320417,       # k_moe_stack_fused, one launch
    "batch16": 7918487317,   # whole step, 30 grouped layers
    "batch64": 12209286449,  # whole step, 30 grouped layers (MFMA)
    "large32": 25578821695,  # whole step, 32 grouped layers
    "large1": 132269060,     # k_gemv_gu_long, one launch (algorithmic 132,120,576 B)
}
METRIC = "MoE expert-FFN µs/token at batch 1 + achieved HBM GB/s (% of MI355X peak)"
# name -> (shape, tokens per step, Zipf exponent of the router bias, BASELINE.json config)
CONFIGS = {
    "gemma30": ("GEMMA", 1, None, 2),
    "zipf": ("GEMMA", 1, 1.1, 3),
    "batch16": ("GEMMA", 16, None, 4),
    "batch64": ("GEMMA", 64, None, 4),
    "large1": ("LARGE", 1, None, 5),
    "large32": ("LARGE", 32, None, 5),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--config", choices=list(CONFIGS) + ["dense", "hbm"], default="gemma30",
                    help="gemma30 = the headline (cfg2); zipf = cfg3; batch16/batch64 = cfg4; large1/large32 = "
                         "cfg5; dense = the dense q4r GEMVs around the expert section (qkv, o_proj, shared MLP, "
                         "lm_head); hbm = the achievable HBM read rate")
    ap.add_argument("--path", choices=["auto", "fused", "grouped", "multikernel"], default="auto",
                    help="auto: fused whole-stack kernel at batch 1 of the Gemma shape, grouped layers (dot4 and "
                         "int8 MFMA kernels) for batched decode, launch-by-launch layers for the large-expert "
                         "shape at batch 1")
    ap.add_argument("--mfma-min", type=int, default=0,
                    help="grouped path: experts with at least this many tokens take the int8 MFMA kernels "
                         "(0: automatic, every expert on MFMA from 4 pairs per expert on)")
    ap.add_argument("--gemv-lanes", type=int, choices=[0, 8, 16, 32, 64], default=0,
                    help="dense config: lanes per row of the q4r GEMV launches (0: automatic)")
    ap.add_argument("--layers", type=int, default=0, help="0 = the config's layer count")
    ap.add_argument("--prefetch", type=int, choices=[0, 1], default=1,
                    help="fused path: stream the early-routed experts of the next layer ahead (1) or not (0)")
    ap.add_argument("--refine", type=int, choices=[0, 1], default=1,
                    help="fused path: prefetch the refined prediction (R_{l+1} x_l + sum_p w_p M_p a_p, from the "
                         "table ft_hip_fused_build_predictor builds at setup) (1) or the early routing's alone (0)")
    ap.add_argument("--trace", default="", metavar="NPY",
                    help="fused path: after timing, run one more token recording every workgroup's phase stamps "
                         "(wall clock, 100 MHz) into this .npy file, shape [workgroups][layers+1][32]")
    ap.add_argument("--input-norm", type=int, choices=[0, 1], default=1,
                    help="1: each layer runs on rmsnorm(x) (the reference model's pre-norm; keeps the 30/32-layer "
                         "residual chains finite); 0: on x as is")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--copy-calib", type=int, default=0, metavar="MIB",
                    help="before warmup, run 3 int32->f32 copies of MIB MiB each (a plain copy kernel of known "
                         "size, read MIB and written MIB per launch) to scale rocprofv3 FETCH_SIZE/WRITE_SIZE")
    return ap.parse_args()


def chunk_size(steps, warmup):
    for c in (16, 8, 4, 2, 1):
        if steps % c == 0 and warmup % c == 0:
            return c
    return 1


class GraphRunner:
    """Layer-by-layer paths: C steps of B tokens through all layers per
    captured HIP graph. step(src, dst, ids, wts, stream) enqueues all layers
    for the B tokens of src ([B, H]) into dst, with ids/wts [L, B*k]; or,
    without it, layer(l, src, dst, ids, wts, stream) enqueues one layer. The
    routing of every step of a chunk lands in ids/wts [C, L, B*k] (read after
    timing only)."""

    def __init__(self, model, B, chunk, layer, step=None):
        import torch
        self.m, self.B, self.C, self.layer, self.step = model, B, chunk, layer, step
        H, k = model.shape.hidden, model.shape.top_k
        dev = model.device
        self.xin = torch.zeros((chunk, B, H), dtype=torch.float32, device=dev)
        self.out = torch.zeros((chunk, B, H), dtype=torch.float32, device=dev)
        self.state = [torch.zeros((B, H), dtype=torch.float32, device=dev) for _ in range(2)]
        self.ids = torch.zeros((chunk, model.L, B * k), dtype=torch.int32, device=dev)
        self.wts = torch.zeros((chunk, model.L, B * k), dtype=torch.float32, device=dev)
        self.stream = torch.cuda.Stream()
        self.graph = torch.cuda.CUDAGraph()
        self._enqueue(self.stream)  # one eager pass before capture
        torch.cuda.synchronize()
        with torch.cuda.graph(self.graph, stream=self.stream):
            self._enqueue(self.stream)
        torch.cuda.synchronize()

    def _enqueue(self, stream):
        L = self.m.L
        for c in range(self.C):
            src = self.xin[c]
            if self.step is not None:
                self.step(src, self.out[c], self.ids[c], self.wts[c], stream)
                continue
            for l in range(L):
                dst = self.out[c] if l == L - 1 else self.state[l & 1]
                self.layer(l, src, dst, self.ids[c, l], self.wts[c, l], stream)
                src = dst

    def run_chunk(self, hidden_rows):
        """hidden_rows: [C, B, H]; the outputs land in self.out."""
        self.xin.copy_(hidden_rows)
        self.graph.replay()


def time_dominant_kernel(g, model, reps=3):
    """Average duration of the layer's gate|up launch (k_gemv_gu_long for q4r
    rows of 64 or 128 blocks, else k_gemv_gu_act: the gate|up GEMV with
    GELU*up and q8, moving 2/3 of the bytes) with
    HIP events on the stream it runs on, rotating over all layers so that no
    layer's bank is cache-resident."""
    import torch
    s = model.shape
    H, I, E, k = s.hidden, s.inter, s.n_experts, s.top_k
    stream = torch.cuda.Stream()
    ids = torch.arange(0, E, E // k, dtype=torch.int32, device=model.device)[:k].contiguous()
    q8x = torch.zeros(H // 32 * 40, dtype=torch.uint8, device=model.device)
    q8a = torch.zeros(k * (I // 32) * 40, dtype=torch.uint8, device=model.device)
    x = model.hidden(0)
    with torch.cuda.stream(stream):
        g.quantize_q8(x, 0, q8x, H, 1, stream=stream)
        eb = model.expert_bytes

        def launch(l):
            bank = model.banks[l * E * eb:(l + 1) * E * eb]
            g.gemv_gate_up_act(bank, eb, ids, k, k, q8x, H, I, q8a, layout=model.layout, stream=stream)

        for l in range(model.L):
            launch(l)
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n = 0
        ev0.record(stream)
        for _ in range(reps):
            for l in range(model.L):
                launch(l)
                n += 1
        ev1.record(stream)
    torch.cuda.synchronize()
    us = ev0.elapsed_time(ev1) * 1000.0 / n
    nbytes = k * 2 * I * (H // 32) * 18
    return us, nbytes


def bench_dense(args, g):
    """--config dense: the dense q4r GEMVs around Gemma's expert section
    (moe_synth.DENSE) through ft_hip_gemv_q4_grouped_slots with one entry,
    as the reference's gemv_q4r_idx with a dense index. Each GEMV rotates over
    enough seeded weight copies (>= 1.5 GB) that no launch finds its matrix in
    the 256 MB last-level cache; `args.steps` launches per GEMV are captured
    in one HIP graph and timed with HIP events on the graph's stream. value =
    30 x (qkv + o_proj + shared gate|up + shared down) + lm_head, the dense
    GEMV time of one decoded token. The shared MLP is also timed as the chain
    a step runs (its input q8 and GELU*up included): the reference's four
    launches and this library's three with the gate|up launch applying
    GELU*up and the q8, and two (ft_hip_gemv_q4r_f32in: the gate|up GEMV with
    the q8 of x in its launch and GELU*up as its f32 second output, the down
    GEMV with the q8 of that in its launch) (config.shared_mlp_chain_us; the
    token with the fastest chain: config.us_per_token_with_shared_chain)."""
    import numpy as np
    import torch
    import ft_hip
    import moe_synth
    dev = "cuda:0"
    order = ["qkv", "o_proj", "shared_gate_up", "shared_down", "lm_head"]
    per = {}
    stream = torch.cuda.Stream()
    for name in order:
        rows, k = moe_synth.DENSE[name]
        rb = ft_hip.row_bytes(k, ft_hip.LAYOUT_Q4R)
        mbytes = rows * rb
        copies = max(2, -(-1_500_000_000 // mbytes))
        W = moe_synth.dense_weights(g, name, copies=copies, device=dev)
        x = torch.from_numpy(np.random.default_rng(rows + k).standard_normal(k).astype(np.float32)).to(dev)
        q8 = torch.zeros(k // 32 * 40, dtype=torch.uint8, device=dev)
        y = torch.zeros(rows, dtype=torch.float32, device=dev)
        slots = torch.zeros(1, dtype=torch.int32, device=dev)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            g.quantize_q8(x, 0, q8, k, 1, stream=stream)

            def launches(n):
                for i in range(n):
                    c = i % copies
                    g.gemv_grouped_slots(W[c * mbytes:(c + 1) * mbytes], 0, 0, slots, None, 1, q8, 0, y, rows,
                                         rows, k, stream=stream)

            launches(args.warmup)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                launches(args.steps)
            graph.replay()
            ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            ev0.record(stream)
            graph.replay()
            ev1.record(stream)
        torch.cuda.synchronize()
        us = ev0.elapsed_time(ev1) * 1000.0 / args.steps
        gbps = mbytes / (us * 1e-6) / 1e9
        per[name] = {"rows": rows, "k": k, "bytes": mbytes, "us": round(us, 3), "GBps": round(gbps, 1),
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "copies": copies}
        log(f"[dense] {name:15s} {rows:6d} x {k}: {mbytes / 1e6:7.2f} MB, {us:8.2f} us/launch, {gbps:6.0f} GB/s "
            f"({gbps / HBM_PEAK_GBPS:.1%} of peak), {copies} rotating copies")
        del W, graph
        torch.cuda.empty_cache()
    # the shared MLP as the chain a decode step runs, from the f32 (normed) input: the reference's
    # four launches (quantize_q8, gate|up GEMV, gelu_mul_q8, down GEMV; ft-model/src/lib.rs:
    # 1368-1395), this library's three (quantize_q8, gemv_gate_up_act, down GEMV) and two
    # (gemv_q4r_f32in for gate|up from x with GELU*up out, then for down from that), each over
    # rotating weight copies, `args.steps` chains per graph
    (gu_rows, H), (_, I) = moe_synth.DENSE["shared_gate_up"], moe_synth.DENSE["shared_down"]
    gb, db = gu_rows * ft_hip.row_bytes(H, ft_hip.LAYOUT_Q4R), H * ft_hip.row_bytes(I, ft_hip.LAYOUT_Q4R)
    gc, dc = max(2, -(-1_500_000_000 // gb)), max(2, -(-1_500_000_000 // db))
    Wg = moe_synth.dense_weights(g, "shared_gate_up", copies=gc, device=dev)
    Wd = moe_synth.dense_weights(g, "shared_down", copies=dc, device=dev)
    xs = torch.from_numpy(np.random.default_rng(7).standard_normal(H).astype(np.float32)).to(dev)
    q8x = torch.zeros(H // 32 * 40, dtype=torch.uint8, device=dev)
    ygu = torch.zeros(gu_rows, dtype=torch.float32, device=dev)
    q8a = torch.zeros(I // 32 * 40, dtype=torch.uint8, device=dev)
    ys = torch.zeros(H, dtype=torch.float32, device=dev)
    actf = torch.zeros(I, dtype=torch.float32, device=dev)
    slots = torch.zeros(1, dtype=torch.int32, device=dev)
    chains = {}
    for cname in ("reference_4_launches", "fused_3_launches", "f32in_2_launches"):
        def chain(n, cname=cname):
            for i in range(n):
                wg, wd = Wg[(i % gc) * gb:(i % gc + 1) * gb], Wd[(i % dc) * db:(i % dc + 1) * db]
                if cname == "f32in_2_launches":
                    g.gemv_q4r_f32in(wg, xs, ygu, actf, gu_rows, H, stream=stream)
                    g.gemv_q4r_f32in(wd, actf, ys, None, H, I, stream=stream)
                    continue
                g.quantize_q8(xs, 0, q8x, H, 1, stream=stream)
                if cname == "reference_4_launches":
                    g.gemv_grouped_slots(wg, 0, 0, slots, None, 1, q8x, 0, ygu, gu_rows, gu_rows, H, stream=stream)
                    g.gelu_mul_q8(ygu, q8a, I, 1, stream=stream)
                else:
                    g.gemv_gate_up_act(wg, gb, slots, 1, 1, q8x, H, I, q8a, stream=stream)
                g.gemv_grouped_slots(wd, 0, 0, slots, None, 1, q8a, 0, ys, H, H, I, stream=stream)

        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            chain(args.warmup)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                chain(args.steps)
            graph.replay()
            ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            ev0.record(stream)
            graph.replay()
            ev1.record(stream)
        torch.cuda.synchronize()
        chains[cname] = round(ev0.elapsed_time(ev1) * 1000.0 / args.steps, 3)
        log(f"[dense] shared MLP chain, {cname}: {chains[cname]:.2f} us")
        del graph
    del Wg, Wd
    torch.cuda.empty_cache()
    # the floor of one launch in the graph: the same entry point on a 1 x 32 matrix
    Wf = torch.empty(ft_hip.row_bytes(32, ft_hip.LAYOUT_Q4R), dtype=torch.uint8, device=dev)
    g.gen_q4_rows(moe_synth.tensor_key(moe_synth.DENSE_CFG, 0, 0, 0), 0, 1, 32, moe_synth.gen_scale(0.02), Wf,
                  ft_hip.LAYOUT_Q4R)
    q8f = torch.zeros(40, dtype=torch.uint8, device=dev)
    yf = torch.zeros(1, dtype=torch.float32, device=dev)
    slots = torch.zeros(1, dtype=torch.int32, device=dev)
    with torch.cuda.stream(stream):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for _ in range(args.steps):
                g.gemv_grouped_slots(Wf, 0, 0, slots, None, 1, q8f, 0, yf, 1, 1, 32, stream=stream)
        graph.replay()
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record(stream)
        graph.replay()
        ev1.record(stream)
    torch.cuda.synchronize()
    floor_us = ev0.elapsed_time(ev1) * 1000.0 / args.steps
    log(f"[dense] launch floor (1 x 32 matrix): {floor_us:.2f} us/launch")
    L = moe_synth.GEMMA.n_layers
    layer = ["qkv", "o_proj", "shared_gate_up", "shared_down"]
    tok_us = L * sum(per[n]["us"] for n in layer) + per["lm_head"]["us"]
    # the same token with the shared MLP as the fastest of the chains (its input q8 and GELU*up
    # included, which the GEMV-only figure above leaves out)
    tok_chain_us = L * (per["qkv"]["us"] + per["o_proj"]["us"] + min(chains.values())) + per["lm_head"]["us"]
    tok_bytes = L * sum(per[n]["bytes"] for n in layer) + per["lm_head"]["bytes"]
    dom = max(order, key=lambda n: per[n]["us"] * (L if n in layer else 1))
    d = per[dom]
    res = {
        "metric": "dense q4r GEMV µs/token (30 x qkv, o_proj, shared MLP + lm_head) + achieved HBM GB/s",
        "value": round(tok_us, 2), "unit": "us/token", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(tok_us / 1000.0, 5), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "q4r x q8 (int8 dot, f32 accumulate)",
        "data": "synthetic (seeded Irwin-Hall(4) values of sd 0.02 as q4r weights, sd 1 input)",
        "config": {"workload": "dense q4r GEMVs of the Gemma-4-26B-A4B-shaped decode step, batch 1",
                   "name": "dense", "gemvs": per, "layers": L, "gemv_lanes": args.gemv_lanes or "auto",
                   "launch_floor_us": round(floor_us, 3), "shared_mlp_chain_us": chains,
                   "us_per_token_with_shared_chain": round(tok_chain_us, 2)},
        "achieved_GBps": round(tok_bytes / (tok_us * 1e-6) / 1e9, 1),
        "hbm_frac": round(tok_bytes / (tok_us * 1e-6) / 1e9 / HBM_PEAK_GBPS, 4),
        "roofline": {"bound": "hbm", "achieved": d["GBps"], "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": d["frac"], "traffic": None, "kernel": f"q4r GEMV launch ({dom})",
                     "bytes_per_launch": d["bytes"], "us_per_launch": d["us"]},
        "cpu_baseline": None,
    }
    print(json.dumps(res), flush=True)


def bench_hbm(args, g):
    """--config hbm: the achievable HBM read rate. ft_hip_stream_read over
    one 8 GiB buffer (32x the 256 MB last-level cache), `args.steps` reads
    per grid size, timed with HIP events on the launch stream; value = the
    best grid's GB/s."""
    import torch
    dev = "cuda:0"
    nbytes = 8 << 30
    buf = torch.ones(nbytes // 4, dtype=torch.int32, device=dev)
    out = torch.zeros(65536, dtype=torch.int32, device=dev)
    stream = torch.cuda.Stream()
    rates = {}
    with torch.cuda.stream(stream):
        for nwg in (1024, 2048, 4096, 8192, 16384, 32768, 65536):
            for _ in range(max(1, args.warmup // 8)):
                g.stream_read(buf, out, nwg, stream=stream)
            ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            ev0.record(stream)
            for _ in range(args.steps):
                g.stream_read(buf, out, nwg, stream=stream)
            ev1.record(stream)
            torch.cuda.synchronize()
            us = ev0.elapsed_time(ev1) * 1000.0 / args.steps
            rates[nwg] = {"us": round(us, 1), "GBps": round(nbytes / (us * 1e-6) / 1e9, 1)}
            log(f"[hbm] {nwg:5d} workgroups: {us:9.1f} us per 8 GiB read, {rates[nwg]['GBps']:.0f} GB/s")
    best = max(rates, key=lambda n: rates[n]["GBps"])
    gbps = rates[best]["GBps"]
    res = {
        "metric": "achievable HBM read GB/s (one read of an 8 GiB buffer)", "value": gbps, "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(rates[best]["us"] / 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u8",
        "data": "synthetic (constant buffer)",
        "config": {"workload": "read-only stream over 8 GiB of device memory", "name": "hbm", "bytes": nbytes,
                   "workgroups": best, "by_workgroups": rates},
        "roofline": {"bound": "hbm", "achieved": gbps, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None, "kernel": "k_stream_read",
                     "bytes_per_launch": nbytes, "us_per_launch": rates[best]["us"]},
        "cpu_baseline": None,
    }
    print(json.dumps(res), flush=True)


def cpu_baseline(model, hidden, seconds, threads, input_norm, max_tokens=None):
    """The oracle's restatement of ft-core's AVX2 CPU path (row-parallel over
    `threads` host threads, as rayon's par_iter_mut) over the same section,
    on a time-bounded sample of the same tokens, each token free-running
    through all layers. Returns (us/token, tokens, per-token layer states
    [L+1][H], per-token routing ids [L][k])."""
    import numpy as np
    import ctypes
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    s = model.shape
    H, I, E, k = s.hidden, s.inter, s.n_experts, s.top_k
    t0 = time.time()
    banks = model.banks.cpu().numpy()
    routers = model.routers.cpu().numpy()
    log(f"[cpu] banks copied to host in {time.time() - t0:.1f}s")
    bias = None if model.bias is None else model.bias.cpu().numpy()
    eb, gb = model.expert_bytes, model.gu_bytes
    base = banks.ctypes.data
    gu_ptrs = [(ctypes.c_void_p * E)(*[base + (l * E + e) * eb for e in range(E)]) for l in range(model.L)]
    dn_ptrs = [(ctypes.c_void_p * E)(*[base + (l * E + e) * eb + gb for e in range(E)]) for l in range(model.L)]
    L = orc.lib()
    P = ctypes.c_void_p
    limit = len(hidden) if max_tokens is None else min(len(hidden), max_tokens)
    states, ids_all = [], []
    t_start = time.perf_counter()
    while True:
        xs = np.zeros((model.L + 1, H), np.float32)
        ids = np.zeros((model.L, k), np.int32)
        xs[0] = hidden[len(states)]
        for l in range(model.L):
            b = None if bias is None else bias[l].ctypes.data_as(P)
            rc = L.orc_moe_layer(xs[l].ctypes.data_as(P), H, I, E, k, routers[l].ctypes.data_as(P), b, None,
                                 ctypes.cast(gu_ptrs[l], P), ctypes.cast(dn_ptrs[l], P), model.layout, threads,
                                 int(input_norm), xs[l + 1].ctypes.data_as(P), None, ids[l].ctypes.data_as(P),
                                 None, None, None, None, None, None)
            assert rc == 0
        states.append(xs)
        ids_all.append(ids)
        if time.perf_counter() - t_start >= seconds or len(states) >= limit:
            break
    dt = time.perf_counter() - t_start
    return dt * 1e6 / len(states), len(states), states, ids_all


def teacher_forced(model, gpu_states, gpu_ids, threads, input_norm, n_tok):
    """Each layer of the oracle run on the GPU's own input state of that
    layer (untimed): per (token, layer) whether the oracle's top-k ids equal
    the GPU's, and max|x_gpu_{l+1} - x_orc_{l+1}| over the norm of the
    oracle's update ||x_orc_{l+1} - x_gpu_l||."""
    import numpy as np
    import ctypes
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    s = model.shape
    H, I, E, k = s.hidden, s.inter, s.n_experts, s.top_k
    banks = model.banks.cpu().numpy()
    routers = model.routers.cpu().numpy()
    bias = None if model.bias is None else model.bias.cpu().numpy()
    eb, gb = model.expert_bytes, model.gu_bytes
    base = banks.ctypes.data
    P = ctypes.c_void_p
    L = orc.lib()
    same, errs = [], []
    x_out = np.zeros(H, np.float32)
    ids = np.zeros(k, np.int32)
    for l in range(model.L):
        gu = (ctypes.c_void_p * E)(*[base + (l * E + e) * eb for e in range(E)])
        dn = (ctypes.c_void_p * E)(*[base + (l * E + e) * eb + gb for e in range(E)])
        b = None if bias is None else bias[l].ctypes.data_as(P)
        for t in range(n_tok):
            xin = np.ascontiguousarray(gpu_states[t][l])
            rc = L.orc_moe_layer(xin.ctypes.data_as(P), H, I, E, k, routers[l].ctypes.data_as(P), b, None,
                                 ctypes.cast(gu, P), ctypes.cast(dn, P), model.layout, threads, int(input_norm),
                                 x_out.ctypes.data_as(P), None, ids.ctypes.data_as(P), None, None, None, None,
                                 None, None)
            assert rc == 0
            same.append(np.array_equal(ids, gpu_ids[t][l]))
            upd = np.linalg.norm(x_out.astype(np.float64) - xin)
            errs.append(np.max(np.abs(gpu_states[t][l + 1].astype(np.float64) - x_out)) / max(upd, 1e-30))
    return {"tokens": n_tok, "layers": model.L, "topk_agreement": round(float(np.mean(same)), 5),
            "max_err": float(f"{max(errs):.3e}"), "median_err": float(f"{np.median(errs):.3e}")}


def host_cpu():
    """(model name with its family/model/stepping and vector extensions, logical CPUs) of this host.
    Virtualised hosts often report a bare "AMD EPYC" as the model name; the CPUID family and model
    and the AVX2 / AVX-512 flags (the reference's CPU path is AVX2) identify the part further."""
    fields = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if not line.strip():
                    break  # the first processor's block
                k, _, v = line.partition(":")
                fields[k.strip()] = v.strip()
    except OSError:
        pass
    name = fields.get("model name", "unknown")
    flags = fields.get("flags", "").split()
    extra = [f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields]
    if flags:
        extra.append("AVX2 " + ("yes" if "avx2" in flags else "no"))
        extra.append("AVX-512 " + ("yes" if "avx512f" in flags else "no"))
    if extra:
        name += " (" + ", ".join(extra) + ")"
    return name, os.cpu_count() or 1


def q8_quants(x):
    """ft-core's Q8Vec::quantize quants of x (q4_0.rs:62-78; f32 as there)."""
    import numpy as np
    b = x.astype(np.float32).reshape(-1, 32)
    d = (np.fmax.reduce(np.abs(b), axis=1) / np.float32(127.0)).astype(np.float32)  # NaN-skipping, as f32::max
    with np.errstate(divide="ignore", invalid="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
        r = (b * inv[:, None]).astype(np.float32)
    q = np.sign(r) * np.floor(np.abs(r) + np.float32(0.5))
    return np.nan_to_num(np.clip(q, -127, 127), nan=0.0).astype(np.int8)


def chain_check(gpu_states, gpu_ids, cpu_states, cpu_ids):
    """GPU vs oracle over free-running chains of the same tokens: per
    (token, layer) top-k agreement, the first layer whose ids differ, and the
    error of every layer's state up to it, max|x_gpu - x_cpu| over the norm
    of the oracle's own update of that layer; also the first layer whose
    input q8 quants differ (a rounding flip of q8, after which the chains
    take different integer dots) and the error before it."""
    import numpy as np
    n, L = len(cpu_states), cpu_ids[0].shape[0]
    q8_first = np.array([next((l for l in range(L) if not np.array_equal(q8_quants(gpu_states[t][l]),
                                                                         q8_quants(cpu_states[t][l]))), L)
                         for t in range(n)])
    agree = np.array([[np.array_equal(gpu_ids[t][l], cpu_ids[t][l]) for l in range(L)] for t in range(n)])
    first = np.array([int(np.argmin(a)) if not a.all() else L for a in agree])
    errs = np.zeros((n, L))
    for t in range(n):
        xc, xg = cpu_states[t], gpu_states[t]
        for l in range(L):
            upd = np.linalg.norm(xc[l + 1].astype(np.float64) - xc[l])
            errs[t, l] = np.max(np.abs(xg[l + 1].astype(np.float64) - xc[l + 1])) / max(upd, 1e-30)
    before = [errs[t, :first[t]].max() for t in range(n) if first[t] > 0]
    before_q8 = [errs[t, :q8_first[t] - 1].max() for t in range(n) if q8_first[t] > 1]
    same = first == L
    return {"tokens": n, "layers": L, "topk_agreement": round(float(agree.mean()), 5),
            "first_q8_diff_layer_min": int(q8_first.min()),
            "first_q8_diff_layer_median": float(np.median(q8_first)),
            "max_err_before_first_q8_diff": float(f"{max(before_q8):.3e}") if before_q8 else None,
            "tokens_without_flip": int(same.sum()),
            "first_flip_layer_min": int(first.min()), "first_flip_layer_median": float(np.median(first)),
            "max_err_before_first_flip": float(f"{max(before):.3e}") if before else None,
            "max_err_final_no_flip": float(f"{errs[same, -1].max():.3e}") if same.any() else None,
            "nonfinite_gpu": int(sum((~np.isfinite(x)).sum() for x in gpu_states[:n]))}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no multi-GPU path. "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch
    import ft_hip
    import moe_synth

    if args.config == "hbm":
        bench_hbm(args, ft_hip.Q4Gemv(0))
        return
    if args.config == "dense":
        g = ft_hip.Q4Gemv(0)
        g.set_gemv_lanes(args.gemv_lanes)
        bench_dense(args, g)
        return
    shape_name, B, zipf_s, cfg_id = CONFIGS[args.config]
    shape = getattr(moe_synth, shape_name)
    path = args.path
    if path == "auto":
        path = "grouped" if B > 1 else ("fused" if shape is moe_synth.GEMMA else "multikernel")
    if path == "fused" and B != 1:
        sys.exit("the fused whole-stack kernel decodes one token per launch: use --path grouped or multikernel")
    if path == "fused" and shape is not moe_synth.GEMMA:
        sys.exit("--path fused is built for the Gemma shape only: use --path grouped or multikernel")

    g = ft_hip.Q4Gemv(0)
    g.set_input_norm(args.input_norm)
    g.set_grouped_mfma_min(args.mfma_min)
    t0 = time.time()

    def progress(l):
        if l % 10 == 9:
            torch.cuda.synchronize()
            log(f"[setup] layer {l + 1} generated ({time.time() - t0:.1f}s)")

    model = moe_synth.SyntheticMoE(g, shape, n_layers=args.layers or None, zipf_s=zipf_s, progress=progress)
    torch.cuda.synchronize()
    log(f"[setup] {args.config}: {model.L} layers x {shape.n_experts} experts generated on the GPU in "
        f"{time.time() - t0:.1f}s ({model.banks.numel() / 1e9:.2f} GB of banks), {B} token(s) per step, path {path}")
    H, I, E, k = shape.hidden, shape.inter, shape.n_experts, shape.top_k
    n_steps = args.warmup + args.steps
    hidden = torch.stack([model.hidden(t) for t in range(n_steps * B)]).view(n_steps, B, H)
    outs = torch.zeros((n_steps, B, H), dtype=torch.float32, device=model.device)
    runner = None
    if path == "fused":
        t1 = time.time()
        g.fused_set_prefetch(args.prefetch)
        stack = moe_synth.FusedStack(model, predictor=bool(args.refine))
        torch.cuda.synchronize()
        log(f"[setup] banks repacked for the fused kernel in {time.time() - t1:.1f}s")

        def run(t0_, n, marks=None):
            for t in range(t0_, t0_ + n):
                stack.run(hidden[t, 0], outs[t, 0])
                if marks is not None:
                    marks.append(torch.cuda.Event(enable_timing=True))
                    marks[-1].record()
    else:
        step = None
        if path == "grouped":
            packed = moe_synth.FusedStack(model, workspace=False)
            gstack = moe_synth.GroupedStack(packed, B)
            bstack = moe_synth.BatchedStack(packed, B)

            def layer(l, src, dst, ids, wts, stream):
                gstack.layer(l, src, dst, ids, wts, stream=stream)

            def step(src, dst, ids, wts, stream):  # all layers in one call (ft_hip_moe_stack_grouped)
                bstack.run(src, dst, B, ids, wts, stream=stream)
        else:
            ws = model.workspace(B)
            sws = model.stack_workspace(B)

            def layer(l, src, dst, ids, wts, stream):
                model.layer(l, src, dst, ids, wts, ws, n_seqs=B, stream=stream)

            def step(src, dst, ids, wts, stream):  # all layers in one call (ft_hip_moe_stack)
                model.stack(src, dst, ids, wts, sws, n_seqs=B, stream=stream)
        C = chunk_size(args.steps, args.warmup)
        runner = GraphRunner(model, B, C, layer, step)
        log(f"[setup] {C} step(s) per captured HIP graph")

        def run(t0_, n, marks=None):
            for c in range(t0_, t0_ + n, C):
                runner.run_chunk(hidden[c:c + C])
                outs[c:c + C].copy_(runner.out)
                if marks is not None:
                    marks.append(torch.cuda.Event(enable_timing=True))
                    marks[-1].record()

    if args.copy_calib > 0:
        n = args.copy_calib << 18
        src = torch.ones(n, dtype=torch.int32, device=model.device)
        dst = torch.empty(n, dtype=torch.float32, device=model.device)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[calib] 3 copies of {n * 4} B read + {n * 4} B written each")
        del src, dst

    run(0, args.warmup)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_wall = time.perf_counter()
    ev0.record()
    run(args.warmup, args.steps)
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    ms = ev0.elapsed_time(ev1)
    us_step = ms * 1000.0 / args.steps
    us_tok = us_step / B
    # the distribution, from a second pass over the same steps with an event after each token
    # (fused) or captured chunk of steps (kept out of the timed pass above)
    marks = []
    ev2 = torch.cuda.Event(enable_timing=True)
    ev2.record()
    run(args.warmup, args.steps, marks)
    torch.cuda.synchronize()
    per = args.steps / max(1, len(marks))  # steps per mark
    spans = [a.elapsed_time(b) * 1000.0 / (per * B) for a, b in zip([ev2] + marks[:-1], marks)]
    us_tok_p50, us_tok_p90 = float(np.percentile(spans, 50)), float(np.percentile(spans, 90))
    e_bytes = moe_synth.algorithmic_expert_bytes(shape)
    router_bytes = E * H * 4 * model.L
    if B == 1:
        uniq = float(k)
    else:  # unique experts per layer, averaged over the timed steps (replayed untimed: same inputs, same ids)
        counts = []
        for c in range(args.warmup, args.warmup + args.steps, runner.C):
            runner.run_chunk(hidden[c:c + runner.C])
            ids = runner.ids.cpu().numpy()
            counts += [len(np.unique(ids[i, l])) for i in range(runner.C) for l in range(model.L)]
        uniq = float(np.mean(counts))
    step_bytes = int(round(uniq * e_bytes * model.L))
    gbps = step_bytes / (us_step * 1e-6) / 1e9
    log(f"[gpu] {us_tok:.1f} us/token, {us_step:.1f} us/step (wall {wall * 1e6 / args.steps:.1f}), "
        f"{uniq:.2f} unique experts/layer, {gbps:.0f} GB/s expert bytes, "
        f"{(step_bytes + router_bytes) / (us_step * 1e-6) / 1e9:.0f} GB/s incl. router")

    if path == "fused":
        stack.check()
        if args.trace:
            nw = stack.n_workgroups()
            tr = torch.zeros(nw * (model.L + 1) * 32, dtype=torch.int64, device=model.device)
            stack.run(hidden[0, 0], torch.empty_like(hidden[0, 0]), trace=tr)
            stack.check()
            np.save(args.trace, tr.cpu().numpy().reshape(nw, model.L + 1, 32))
            log(f"[trace] {nw} workgroups x {model.L + 1} rows of phase stamps -> {args.trace}")
        # the fused kernel is the only kernel of a step: one launch per token
        k_us, k_bytes = us_tok, step_bytes + router_bytes
        k_name = f"k_moe_stack_fused (whole {model.L}-layer section, one launch per token)"
    elif B == 1:
        k_us, k_bytes = time_dominant_kernel(g, model)
        gu = "k_gemv_gu_long" if model.layout == ft_hip.LAYOUT_Q4R and shape.hidden in (2048, 4096) else "k_gemv_gu_act"
        k_name = f"{gu} (gate|up GEMV + GELU*up q8, {k} experts)"
    else:  # the step's graph as a whole: its expert bytes over the step time
        k_us, k_bytes = us_step, step_bytes
        k_name = f"whole step ({model.L} {path} layers of {B} tokens in one HIP graph; not a single kernel)"
    k_gbps = k_bytes / (k_us * 1e-6) / 1e9
    log(f"[kernel] {k_name}: {k_us:.2f} us/launch, {k_bytes} B -> {k_gbps:.0f} GB/s")

    def gpu_states(n_tok):
        """Per-layer states [L+1][H] and routing ids [L][k] of the first n_tok
        tokens, run again through the timed path (fused: the dbg_x record;
        layer paths: each layer into its own buffer), and whether every final
        state equals the timed run's output bit for bit."""
        Lm = model.L
        st, idl = [], []
        if path == "fused":
            xs = torch.zeros((Lm + 1) * H, dtype=torch.float32, device=model.device)
            ids = torch.zeros(Lm * k, dtype=torch.int32, device=model.device)
            wts = torch.zeros(Lm * k, dtype=torch.float32, device=model.device)
            tmp = torch.zeros(H, dtype=torch.float32, device=model.device)
            for t in range(n_tok):
                stack.run(hidden[t, 0], tmp, ids=ids, wts=wts, dbg_x=xs)
                stack.check()
                st.append(xs.cpu().numpy().reshape(Lm + 1, H))
                idl.append(ids.cpu().numpy().reshape(Lm, k))
        else:
            bufs = torch.zeros((Lm + 1, B, H), dtype=torch.float32, device=model.device)
            ids = torch.zeros((Lm, B * k), dtype=torch.int32, device=model.device)
            wts = torch.zeros((Lm, B * k), dtype=torch.float32, device=model.device)
            cur = torch.cuda.current_stream()
            for c in range((n_tok + B - 1) // B):
                bufs[0].copy_(hidden[c])
                for l in range(Lm):
                    layer(l, bufs[l], bufs[l + 1], ids[l], wts[l], cur)
                xs_h, ids_h = bufs.cpu().numpy(), ids.cpu().numpy()
                for b in range(B):
                    st.append(xs_h[:, b].copy())
                    idl.append(ids_h[:, b * k:(b + 1) * k].copy())
        st, idl = st[:n_tok], idl[:n_tok]
        final = outs.view(n_steps * B, H)[:n_tok].cpu().numpy()
        same = all(np.array_equal(final[t].view(np.uint32), st[t][-1].view(np.uint32)) for t in range(n_tok))
        return st, idl, same

    cpu = None
    chain = None
    if not args.no_cpu:
        # the GPU box's CPU share for one GPU (OMP_NUM_THREADS there), else every logical CPU
        threads = int(os.environ.get("OMP_NUM_THREADS") or 0) or (os.cpu_count() or 1)
        cpu_name, n_logical = host_cpu()
        hid = hidden.view(n_steps * B, H).cpu().numpy()
        cpu_us, cpu_n, cpu_states, cpu_ids = cpu_baseline(model, hid, args.cpu_seconds, threads, args.input_norm)
        gst, gids, replay_same = gpu_states(cpu_n)
        chain = chain_check(gst, gids, cpu_states, cpu_ids)
        chain["gpu_rerun_bit_identical"] = bool(replay_same)
        chain["teacher_forced"] = teacher_forced(model, gst, gids, threads, args.input_norm, min(cpu_n, 16))
        log(f"[cpu] {cpu_us:.0f} us/token over {cpu_n} tokens on {threads} threads ({cpu_name}, "
            f"{n_logical} logical CPUs)")
        log(f"[chain] {json.dumps(chain)}")
        one_us, one_n, _, _ = cpu_baseline(model, hid, args.cpu_seconds / 2, 1, args.input_norm)
        log(f"[cpu] 1 thread: {one_us:.0f} us/token over {one_n} tokens")
        cpu = {"value": round(cpu_us, 1), "unit": "us/token", "cores": threads, "kind": "port",
               "sample": f"{cpu_n} tokens x {model.L} layers of the same workload, one token at a time "
                         f"(libm GELU and exp), {threads} threads = this host's CPU share for one GPU",
               "value_1_thread": round(one_us, 1), "sample_1_thread": f"{one_n} tokens",
               "host_cpu": cpu_name, "host_logical_cpus": n_logical}

    workload = {1: "", 2: "", 3: ", Zipf(1.1) router bias", 4: "", 5: ""}[cfg_id]
    profiled_opts = (args.path == "auto" and args.prefetch == 1 and args.refine == 1 and args.input_norm == 1
                     and args.mfma_min == 0
                     and args.layers == 0 and not args.trace)
    traffic = MEASURED_TRAFFIC.get(args.config) if profiled_opts else None
    res = {
        "metric": METRIC,
        "value": round(us_tok, 2),
        "unit": "us/token",
        "us_per_token_p50": round(us_tok_p50, 2),
        "us_per_token_p90": round(us_tok_p90, 2),
        "p50_over": f"{len(marks)} spans of {per:g} step(s) each, HIP events between them, in a second pass",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 x q8 (int8 dot, f32 accumulate)",
        "data": "synthetic (seeded Irwin-Hall(4) values: sd 0.02 q4_0 banks and f32 routers, sd 1 hidden)",
        "config": {"workload": f"{shape.name} MoE expert FFN, {model.L} layers, batch {B}, residual chain"
                               f"{' on rmsnorm(x)' if args.input_norm else ''}{workload}",
                   "baseline_config": cfg_id, "name": args.config,
                   "hidden": H, "inter": I, "experts": E, "top_k": k, "layers": model.L, "batch": B,
                   "path": path, "prefetch": bool(args.prefetch) if path == "fused" else None,
                   "prediction": ("refined" if args.refine else "early routing") if path == "fused" and args.prefetch
                   else None,
                   "input_norm": bool(args.input_norm),
                   "zipf_tau": moe_synth.ZIPF_TAU[(shape.name, zipf_s)] if zipf_s else None,
                   "mfma_min_tokens": args.mfma_min if path == "grouped" else None,
                   "unique_experts_per_layer": round(uniq, 2)},
        "achieved_GBps": round(gbps, 1),
        "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
        "roofline": {"bound": "hbm", "achieved": round(k_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(k_gbps / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "traffic_unit": "B per launch" if traffic else None,
                     "kernel": k_name, "bytes_per_launch": k_bytes,
                     "us_per_launch": round(k_us, 3)},
        "cpu_baseline": cpu,
        "chain_check": chain,
    }
    # Parity gate: the oracle run on the timed path's own layer inputs must pick
    # the same experts in every (token, layer) and land within 1e-3 of the norm
    # of its update, and a rerun of the timed path must give the same bits.
    # Free-running chains are reported, not gated: once a layer's input q8
    # rounds differently on the two sides (GPU and AVX2 f32 sums differing in
    # the last bit at a rounding tie), the chains take different integer dots
    # and drift apart without either being wrong.
    if chain is not None:
        tf = chain["teacher_forced"]
        bad = []
        if tf["topk_agreement"] < 1.0:
            bad.append(f"teacher-forced top-k agreement {tf['topk_agreement']} < 1")
        if not tf["max_err"] <= 1e-3:
            bad.append(f"teacher-forced max error {tf['max_err']} > 1e-3")
        if not chain["gpu_rerun_bit_identical"]:
            bad.append("a rerun of the timed path gave other bits")
        if bad:
            print("bench.py: parity gate failed: " + "; ".join(bad), file=sys.stderr, flush=True)
            sys.exit(3)
        res["parity_gate"] = "passed"
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
