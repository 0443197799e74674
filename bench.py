#!/usr/bin/env python3
"""Benchmark of the MoE expert-FFN decode section on one MI355X.

Workload: the 30-layer Gemma-4-26B-A4B-shaped
expert section (H 2816, I 704, 128 experts, top-8, q4_0 banks of seeded
N(0, 0.02) weights, f32 routers of N(0, 0.02)), decoding tokens at batch 1
with the residual chain x <- x + MoE_l(x) between layers (attention stubbed
as identity). One step = one token through all 30 layers; inputs (banks,
routers, the tokens' hidden states) are resident in HBM before timing.

Prints one JSON line: value = mean us/token (lower is better), plus achieved
HBM GB/s over the algorithmic expert bytes (802,897,920 B/token), the
roofline of the dominant kernel, and a CPU baseline (the oracle's restatement
of ft-core's AVX2 path, timed on this host's cores on a bounded sample).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "freetoken-rs_amd"))

HBM_PEAK_GBPS = 8000.0
METRIC = "MoE expert-FFN µs/token at batch 1 + achieved HBM GB/s (% of MI355X peak)"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--path", choices=["fused", "multikernel"], default="fused")
    ap.add_argument("--layers", type=int, default=30)
    ap.add_argument("--prefetch", type=int, choices=[0, 1], default=1,
                    help="fused path: stream the early-routed experts of the next layer ahead (1) or not (0)")
    ap.add_argument("--trace", default="", metavar="NPY",
                    help="fused path: after timing, run one more token recording every workgroup's phase stamps "
                         "(wall clock, 100 MHz) into this .npy file, shape [workgroups][layers+1][32]")
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


class MultiKernelRunner:
    """Launch-by-launch path: 7 kernels per layer, C tokens per captured HIP graph."""

    def __init__(self, model, chunk):
        import torch
        self.m, self.C = model, chunk
        H, k = model.shape.hidden, model.shape.top_k
        dev = model.device
        self.xin = torch.zeros((chunk, H), dtype=torch.float32, device=dev)
        self.out = torch.zeros((chunk, H), dtype=torch.float32, device=dev)
        self.state = torch.zeros(H, dtype=torch.float32, device=dev)
        self.ids = torch.zeros((model.L, chunk, k), dtype=torch.int32, device=dev)
        self.wts = torch.zeros((model.L, chunk, k), dtype=torch.float32, device=dev)
        self.ws = model.workspace(1)
        self.stream = torch.cuda.Stream()
        self.graph = torch.cuda.CUDAGraph()
        self._enqueue(self.stream)  # one eager pass before capture
        torch.cuda.synchronize()
        with torch.cuda.graph(self.graph, stream=self.stream):
            self._enqueue(self.stream)
        torch.cuda.synchronize()

    def _enqueue(self, stream):
        m = self.m
        for t in range(self.C):
            for l in range(m.L):
                src = self.xin[t] if l == 0 else self.state
                dst = self.out[t] if l == m.L - 1 else self.state
                m.layer(l, src, dst, self.ids[l, t], self.wts[l, t], self.ws, 1, stream)

    def run_chunk(self, hidden_rows):
        self.xin.copy_(hidden_rows)
        self.graph.replay()


def time_dominant_kernel(g, model, reps=3):
    """Average duration of the gate|up grouped GEMV (the kernel moving 2/3 of
    the bytes) with HIP events on the stream it runs on, rotating over all
    layers so that no layer's bank is cache-resident."""
    import torch
    s = model.shape
    H, I, E, k = s.hidden, s.inter, s.n_experts, s.top_k
    stream = torch.cuda.Stream()
    ids = torch.arange(0, E, E // k, dtype=torch.int32, device=model.device)[:k].contiguous()
    q8x = torch.zeros(H // 32 * 40, dtype=torch.uint8, device=model.device)
    ygu = torch.zeros(k * 2 * I, dtype=torch.float32, device=model.device)
    x = model.hidden(0)
    with torch.cuda.stream(stream):
        g.quantize_q8(x, 0, q8x, H, 1, stream=stream)
        eb = model.expert_bytes

        def launch(l):
            bank = model.banks[l * E * eb:(l + 1) * E * eb]
            g.gemv_grouped_slots(bank, eb, 0, ids, None, k, q8x, 0, ygu, 2 * I, 2 * I, H, model.layout,
                                 stream=stream)

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


def cpu_baseline(model, hidden, seconds, threads):
    """The oracle's restatement of ft-core's AVX2 CPU path (row-parallel over
    `threads` host threads, as rayon's par_iter_mut) over the same section,
    on a time-bounded sample of the same tokens."""
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
    eb, gb = model.expert_bytes, model.gu_bytes
    base = banks.ctypes.data
    gu_ptrs = [(ctypes.c_void_p * E)(*[base + (l * E + e) * eb for e in range(E)]) for l in range(model.L)]
    dn_ptrs = [(ctypes.c_void_p * E)(*[base + (l * E + e) * eb + gb for e in range(E)]) for l in range(model.L)]
    L = orc.lib()
    P = ctypes.c_void_p
    x_out = np.zeros(H, np.float32)
    n_tok = 0
    outs = []
    t_start = time.perf_counter()
    while True:
        x = hidden[n_tok].copy()
        for l in range(model.L):
            rc = L.orc_moe_layer(x.ctypes.data_as(P), H, I, E, k, routers[l].ctypes.data_as(P), None, None,
                                 ctypes.cast(gu_ptrs[l], P), ctypes.cast(dn_ptrs[l], P), model.layout, threads,
                                 orc.GELU_LIBM, x_out.ctypes.data_as(P), None, None, None, None, None, None,
                                 None, None)
            assert rc == 0
            x, x_out = x_out, x
        outs.append(x.copy())
        n_tok += 1
        if time.perf_counter() - t_start >= seconds or n_tok >= len(hidden):
            break
    dt = time.perf_counter() - t_start
    return dt * 1e6 / n_tok, n_tok, outs


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

    g = ft_hip.Q4Gemv(0)
    t0 = time.time()
    def progress(l):
        if l % 10 == 9:
            torch.cuda.synchronize()
            log(f"[setup] layer {l + 1} generated ({time.time() - t0:.1f}s)")

    model = moe_synth.SyntheticMoE(g, moe_synth.GEMMA, n_layers=args.layers, progress=progress)
    torch.cuda.synchronize()
    log(f"[setup] {model.L} layers x {model.shape.n_experts} experts generated on the GPU in {time.time() - t0:.1f}s "
        f"({model.banks.numel() / 1e9:.2f} GB of banks)")
    n_tok = args.warmup + args.steps
    H = model.shape.hidden
    hidden = torch.stack([model.hidden(t) for t in range(n_tok)])
    outs = torch.zeros((n_tok, H), dtype=torch.float32, device=model.device)
    if args.path == "fused":
        t1 = time.time()
        g.fused_set_prefetch(args.prefetch)
        stack = moe_synth.FusedStack(model)
        torch.cuda.synchronize()
        log(f"[setup] banks repacked for the fused kernel in {time.time() - t1:.1f}s")

        def run(t0_, n):
            for t in range(t0_, t0_ + n):
                stack.run(hidden[t], outs[t])
    else:
        C = chunk_size(args.steps, args.warmup)
        runner = MultiKernelRunner(model, C)

        def run(t0_, n):
            for c in range(t0_, t0_ + n, C):
                runner.run_chunk(hidden[c:c + C])
                outs[c:c + C].copy_(runner.out)

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
    us_tok = ms * 1000.0 / args.steps
    exp_bytes = moe_synth.algorithmic_expert_bytes(model.shape) * model.shape.top_k * model.L
    router_bytes = model.shape.n_experts * H * 4 * model.L
    gbps = exp_bytes / (us_tok * 1e-6) / 1e9
    log(f"[gpu] {us_tok:.1f} us/token (wall {wall * 1e6 / args.steps:.1f}), {gbps:.0f} GB/s expert bytes, "
        f"{(exp_bytes + router_bytes) / (us_tok * 1e-6) / 1e9:.0f} GB/s incl. router")

    if args.path == "fused":
        stack.check()
        if args.trace:
            nw = stack.n_workgroups()
            tr = torch.zeros(nw * (model.L + 1) * 32, dtype=torch.int64, device=model.device)
            stack.run(hidden[0], torch.empty_like(hidden[0]), trace=tr)
            stack.check()
            np.save(args.trace, tr.cpu().numpy().reshape(nw, model.L + 1, 32))
            log(f"[trace] {nw} workgroups x {model.L + 1} rows of phase stamps -> {args.trace}")
        # the fused kernel is the only kernel of a step: one launch per token
        k_us, k_bytes = us_tok, exp_bytes + router_bytes
        k_name = "k_moe_stack_fused (whole 30-layer section, one launch per token)"
    else:
        k_us, k_bytes = time_dominant_kernel(g, model)
        k_name = "k_gemv_q4_grouped (gate|up, 8 experts)"
    k_gbps = k_bytes / (k_us * 1e-6) / 1e9
    log(f"[kernel] {k_name}: {k_us:.2f} us/launch, {k_bytes} B -> {k_gbps:.0f} GB/s")

    cpu = None
    if not args.no_cpu:
        threads = min(16, os.cpu_count() or 1)
        hid = hidden.cpu().numpy()
        cpu_us, cpu_n, cpu_outs = cpu_baseline(model, hid, args.cpu_seconds, threads)
        gpu_outs = outs.cpu().numpy()
        errs = [float(np.max(np.abs(gpu_outs[i] - cpu_outs[i])) / np.linalg.norm(cpu_outs[i] - hid[i]))
                for i in range(cpu_n)]
        log(f"[cpu] {cpu_us:.0f} us/token over {cpu_n} tokens on {threads} threads; "
            f"GPU vs CPU max|dx|/||dx_ref|| = {max(errs):.2e}")
        cpu = {"value": round(cpu_us, 1), "unit": "us/token", "cores": threads, "kind": "port",
               "sample": f"{cpu_n} tokens x {model.L} layers of the same workload (libm GELU mode)"}

    res = {
        "metric": METRIC,
        "value": round(us_tok, 2),
        "unit": "us/token",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 x q8 (int8 dot, f32 accumulate)",
        "data": "synthetic (seeded N(0,0.02) q4_0 banks, N(0,1) hidden)",
        "config": {"workload": f"gemma-shaped MoE expert FFN, {model.L} layers, batch 1, residual chain",
                   "hidden": H, "inter": model.shape.inter, "experts": model.shape.n_experts,
                   "top_k": model.shape.top_k, "layers": model.L, "path": args.path,
                   "prefetch": bool(args.prefetch) if args.path == "fused" else None},
        "achieved_GBps": round(gbps, 1),
        "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
        "roofline": {"bound": "hbm", "achieved": round(k_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(k_gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                     "kernel": k_name, "bytes_per_launch": k_bytes,
                     "us_per_launch": round(k_us, 3)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
