"""Seeded synthetic MoE expert stacks resident in HBM, and the layer chain.

This is the host side of the benchmark configurations: it owns the device
buffers (expert banks, routers, hidden states) and drives the library
through ft_hip.Q4Gemv, like ft-bench's decode microbenchmark does through
ft_cuda::Q4Gemv (ft-bench/src/bin/decode.rs:93-331). Unlike that bench, whose
weights are one template block (:111-116), every expert of every layer here
is distinct seeded data quantized to q4_0, generated on the GPU. Values are
Irwin-Hall(4) sums of hashed 16-bit fields scaled to sd sigma (bounded at
+-3.46 sigma; integer arithmetic, so the device and the host oracle produce
the same bits), not Gaussian.

Bank layout (the reference's q4r bank layout, ft-model/src/lib.rs:570-609):
expert (l, e) occupies bytes [(l*E + e) * expert_bytes, +expert_bytes) of one
device allocation: gate rows (I x H), then up rows (I x H), then down rows
(H x I), each row in the chosen layout. All banks stay resident: with 288 GB
of HBM there is no slot cache and no host split.
"""
import math
from dataclasses import dataclass

import numpy as np
import torch

import ft_hip

SEED = 0xF7EE2026
T_HIDDEN, T_GU, T_DN, T_ROUTER = 1, 2, 3, 4
MASK64 = (1 << 64) - 1


@dataclass(frozen=True)
class Shape:
    name: str
    hidden: int
    inter: int
    n_experts: int
    top_k: int
    n_layers: int
    cfg_id: int


# G (configs 1-4) and X (config 5).
GEMMA = Shape("gemma4-26b-a4b-moe", 2816, 704, 128, 8, 30, 1)
LARGE = Shape("large-expert-h4096-i14336", 4096, 14336, 8, 2, 32, 5)

# The dense q4r GEMVs around Gemma's expert section, (rows, k): qkv
# (ft-model/src/lib.rs:1255-1265), o_proj (:1335-1345), the shared MLP's
# gate|up and down (:1371-1396) and lm_head (:1675-1682). The reference reads
# the widths from its GGUF; these take the row widths of its own q4r test
# (ft-cuda/tests/q4r.rs: k in {2816, 2112, 704, 4096}): 16 query heads x 256
# (4096 rows, o_proj k 4096), k and v of 2048 rows each, a shared-MLP width of
# 2112, and Gemma's 262,144-token vocabulary.
DENSE = {"qkv": (8192, 2816), "o_proj": (2816, 4096), "shared_gate_up": (4224, 2816),
         "shared_down": (2816, 2112), "lm_head": (262144, 2816)}
DENSE_CFG = 200  # generator config id of the dense weights


def dense_weights(gemv, name, copies=1, device="cuda", sigma=0.02):
    """`copies` seeded q4r matrices of DENSE[name] in one allocation (copy c
    at c * rows * row_bytes), generated on the device."""
    rows, k = DENSE[name]
    rb = ft_hip.row_bytes(k, ft_hip.LAYOUT_Q4R)
    w = torch.empty(copies * rows * rb, dtype=torch.uint8, device=device)
    idx = sorted(DENSE).index(name)
    for c in range(copies):
        gemv.gen_q4_rows(tensor_key(DENSE_CFG, c, idx, T_GU), 0, rows, k, gen_scale(sigma),
                         w[c * rows * rb:(c + 1) * rows * rb], ft_hip.LAYOUT_Q4R)
    return w


def _mix64(z):
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    return z ^ (z >> 31)


def tensor_key(cfg, layer, expert, tensor, seed=SEED):
    """Key of one seeded tensor (the same chain as the device generator's callers)."""
    h = _mix64((seed + 0x9E3779B97F4A7C15) & MASK64)
    h = _mix64(h ^ ((cfg << 32) | tensor))
    h = _mix64(h ^ ((layer << 32) | expert))
    return h


def gen_scale(sigma):
    """sigma*sqrt(3)/65536 rounded to f32: the Irwin-Hall(4) sum then has sd sigma."""
    return float(np.float32(sigma * math.sqrt(3.0) / 65536.0))


def expert_geometry(shape, layout):
    rb_h = ft_hip.row_bytes(shape.hidden, layout)
    rb_i = ft_hip.row_bytes(shape.inter, layout)
    gu_bytes = 2 * shape.inter * rb_h
    dn_bytes = shape.hidden * rb_i
    return gu_bytes, dn_bytes, gu_bytes + dn_bytes


def algorithmic_expert_bytes(shape):
    """q4_0 bytes of one expert (18 B per 32 weights): 3*H*I*18/32."""
    return 3 * shape.hidden * shape.inter * 18 // 32


class SyntheticMoE:
    """All layers of one config, resident on the GPU."""

    def __init__(self, gemv, shape, n_layers=None, layout=ft_hip.LAYOUT_Q4R, zipf_s=None, device="cuda",
                 w_sigma=0.02, r_sigma=0.02, progress=None):
        self.g = gemv
        self.shape = shape
        self.L = n_layers or shape.n_layers
        self.layout = layout
        self.device = device
        H, I, E = shape.hidden, shape.inter, shape.n_experts
        self.gu_bytes, self.dn_bytes, self.expert_bytes = expert_geometry(shape, layout)
        self.banks = torch.empty(self.L * E * self.expert_bytes, dtype=torch.uint8, device=device)
        self.routers = torch.empty((self.L, E, H), dtype=torch.float32, device=device)
        ws, ss = gen_scale(w_sigma), gen_scale(r_sigma)
        for l in range(self.L):
            for e in range(E):
                off = (l * E + e) * self.expert_bytes
                gemv.gen_q4_rows(tensor_key(shape.cfg_id, l, e, T_GU), 0, 2 * I, H, ws,
                                 self.banks[off:off + self.gu_bytes], layout)
                gemv.gen_q4_rows(tensor_key(shape.cfg_id, l, e, T_DN), 0, H, I, ws,
                                 self.banks[off + self.gu_bytes:off + self.expert_bytes], layout)
            gemv.gen_values(tensor_key(shape.cfg_id, l, 0, T_ROUTER), 0, E * H, ss, self.routers[l])
            if progress:
                progress(l)
        self.bias = None
        if zipf_s is not None:
            self.bias = torch.from_numpy(zipf_router_bias(shape, self.L, zipf_s)).to(device)

    def hidden(self, token, out=None):
        """Seeded hidden state (Irwin-Hall(4), sd 1) of one decode token."""
        H = self.shape.hidden
        if out is None:
            out = torch.empty(H, dtype=torch.float32, device=self.device)
        self.g.gen_values(tensor_key(self.shape.cfg_id, 0, token, T_HIDDEN), 0, H, gen_scale(1.0), out)
        return out

    def bank_of(self, layer, expert):
        off = (layer * self.shape.n_experts + expert) * self.expert_bytes
        return self.banks[off:off + self.expert_bytes]

    def layer_bias(self, layer):
        return None if self.bias is None else self.bias[layer]

    def workspace(self, n_seqs):
        s = self.shape
        nbytes = ft_hip.Q4Gemv.moe_layer_workspace_bytes(n_seqs, s.hidden, s.inter, s.n_experts, s.top_k)
        return torch.empty(nbytes, dtype=torch.uint8, device=self.device)

    def layer(self, l, x, x_out, ids, wts, ws, n_seqs=1, stream=None):
        """One layer through the launch-by-launch kernels: x_out = x + MoE_l(x)."""
        s = self.shape
        E = s.n_experts
        bank = self.banks[l * E * self.expert_bytes:(l + 1) * E * self.expert_bytes]
        self.g.moe_layer(x, x_out, n_seqs, s.hidden, s.inter, E, s.top_k, self.routers[l], self.layer_bias(l),
                         None, bank, self.expert_bytes, self.layout, ids, wts, ws, stream)

    def stack_workspace(self, n_seqs):
        s = self.shape
        nbytes = ft_hip.Q4Gemv.moe_stack_workspace_bytes(n_seqs, s.hidden, s.inter, s.n_experts, s.top_k)
        return torch.empty(nbytes, dtype=torch.uint8, device=self.device)

    def stack(self, x, x_out, ids, wts, ws, n_seqs=1, stream=None):
        """All L layers through ft_hip_moe_stack (the launch-by-launch kernels, each
        layer's router head folded into the previous down launch); ids/wts [L][n_seqs*k]."""
        s = self.shape
        self.g.moe_stack(x, x_out, n_seqs, s.hidden, s.inter, s.n_experts, s.top_k, self.L, self.routers,
                         self.bias, None, self.banks, self.expert_bytes, self.layout, ids, wts, ws, stream)


def gen_values_np(key, n, scale):
    """Host restatement of the device generator (ft_hip_gen_values): value i
    is the Irwin-Hall(4) sum of the four 16-bit fields of
    splitmix64(key + (i+1) * 0x9E3779B97F4A7C15), centred, times scale (an f32
    product, as on the device)."""
    i = np.arange(1, n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(key) + i * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    m = np.uint64(0xFFFF)
    f = ((z & m) + ((z >> np.uint64(16)) & m) + ((z >> np.uint64(32)) & m) + (z >> np.uint64(48))).astype(np.int64)
    return (f - 131070).astype(np.float32) * np.float32(scale)


def zipf_mass(n_experts, top_k, s):
    """Share of Zipf(s) mass over n_experts ranks carried by the top_k ranks."""
    p = np.arange(1, n_experts + 1, dtype=np.float64) ** -s
    return float(p[:top_k].sum() / p.sum())


def zipf_ranks(shape, n_layers, seed=SEED):
    """Popularity rank (1 = most popular) of every expert per layer: a seeded
    permutation per layer."""
    E = shape.n_experts
    out = np.empty((n_layers, E), np.int64)
    for l in range(n_layers):
        rng = np.random.default_rng([seed, shape.cfg_id, l, 7])
        perm = rng.permutation(E)
        out[l, perm] = np.arange(1, E + 1)
    return out


def zipf_top_share(shape, n_layers, s, tau, n_tokens=256, r_sigma=0.02):
    """Share of the routed (token, expert) pairs that land on each layer's
    top_k most popular experts, routing the seeded hidden states of n_tokens
    tokens (RMS-normalised, as the router sees them) through each layer's
    seeded router plus the Zipf bias with this tau (float64 on the host)."""
    H, E, k = shape.hidden, shape.n_experts, shape.top_k
    xs = np.stack([gen_values_np(tensor_key(shape.cfg_id, 0, t, T_HIDDEN), H, gen_scale(1.0))
                   for t in range(n_tokens)]).astype(np.float64)
    xs /= np.sqrt((xs * xs).mean(axis=1, keepdims=True) + 1e-6)
    ranks = zipf_ranks(shape, n_layers)
    hits = 0
    for l in range(n_layers):
        W = gen_values_np(tensor_key(shape.cfg_id, l, 0, T_ROUTER), E * H, gen_scale(r_sigma)).reshape(E, H)
        logits = xs @ W.astype(np.float64).T - tau * s * np.log(ranks[l])[None, :]
        top = np.argsort(-logits, axis=1, kind="stable")[:, :k]
        hits += int((ranks[l][top] <= k).sum())
    return hits / (n_layers * n_tokens * k)


def calibrate_zipf_tau(shape, s=1.1, n_layers=8, n_tokens=256, lo=0.0, hi=4.0, iters=20):
    """tau for which zipf_top_share equals zipf_mass(E, k, s): the routed
    pairs' share on the top_k popularity ranks follows Zipf(s) (bisection;
    the share grows with tau)."""
    target = zipf_mass(shape.n_experts, shape.top_k, s)
    for _ in range(iters):
        mid = 0.5 * (lo + hi)
        if zipf_top_share(shape, n_layers, s, mid, n_tokens) < target:
            lo = mid
        else:
            hi = mid
    return 0.5 * (lo + hi)


# calibrate_zipf_tau(GEMMA, 1.1) = 0.8949 (8 layers x 256 tokens): the Zipf configuration's bias scale
ZIPF_TAU = {(GEMMA.name, 1.1): 0.895}


def zipf_router_bias(shape, n_layers, s=1.1, tau=None, seed=SEED):
    """Per-layer router bias for the skewed-routing config: expert at
    popularity rank r (zipf_ranks) gets tau * ln(r^-s), so the router favours
    experts in Zipf(s) order. tau defaults to the calibrated ZIPF_TAU, for
    which the share of routed pairs on the top_k ranks equals Zipf(s)'s mass
    there (57 % for 8 of 128 experts at s = 1.1)."""
    E = shape.n_experts
    if tau is None:
        tau = ZIPF_TAU[(shape.name, s)]
    ranks = zipf_ranks(shape, n_layers, seed)
    return (tau * (-s) * np.log(ranks)).astype(np.float32)


class FusedStack:
    """A SyntheticMoE's banks and routers repacked for the fused whole-stack
    kernel (ft_hip_moe_stack_fused): one launch runs all layers of one token.
    The packed banks also serve the grouped batched path (GroupedStack)."""

    def __init__(self, model, workspace=True, predictor=True):
        """workspace=False: the packed banks and routers only (for the grouped
        path on shapes the fused kernel does not take). predictor: build the
        refined-prediction table (ft_hip_fused_build_predictor) and use it in
        run(); False: the early routing's prediction alone."""
        g, s = model.g, model.shape
        H, I, E, K = s.hidden, s.inter, s.n_experts, s.top_k
        self.m, self.g = model, g
        self.expert_bytes = g.fused_expert_bytes(H, I)
        self.banks = torch.empty(model.L * E * self.expert_bytes, dtype=torch.uint8, device=model.device)
        g.pack_experts_fused(model.banks, model.layout, model.expert_bytes, self.banks, model.L * E, H, I)
        self.routers = torch.empty_like(model.routers)
        g.pack_router_fused(model.routers, self.routers, model.L, E, H)
        self.ws = None
        if workspace:
            self.ws = torch.empty(g.fused_workspace_bytes(H, I, E, K), dtype=torch.uint8, device=model.device)
            g.fused_workspace_init(self.ws)
        self.pred = None
        if workspace and predictor and model.L > 1:
            self.pred = torch.empty(g.fused_predictor_bytes(H, I, E, model.L), dtype=torch.uint8, device=model.device)
            g.fused_build_predictor(self.banks, self.routers, H, I, E, model.L, self.pred)

    def n_workgroups(self):
        s = self.m.shape
        return self.g.fused_workgroups(s.hidden, s.inter, s.n_experts, s.top_k)

    def run(self, x_in, x_out, ids=None, wts=None, dbg_gu=None, dbg_act=None, dbg_x=None, trace=None,
            stream=None):
        s = self.m.shape
        self.g.fused_set_predictor(self.pred, self.m.L)  # the context's setting is shared by every stack
        self.g.moe_stack_fused(x_in, x_out, s.hidden, s.inter, s.n_experts, s.top_k, self.m.L, self.banks,
                               self.routers, self.m.bias, None, ids, wts, self.ws, dbg_gu, dbg_act, dbg_x, trace,
                               stream)

    def reset(self):
        """Re-initialise the workspace (required after a launch that timed out)."""
        self.g.fused_workspace_init(self.ws)

    def check(self):
        """Raise if a launch gave up a bounded wait (synchronises first)."""
        torch.cuda.synchronize()
        self.g.fused_status(self.ws)


class GroupedStack:
    """Batched decode through ft_hip_moe_layer_grouped: n_seqs tokens per step,
    layer by layer, pairs grouped by expert; the banks are a FusedStack's."""

    def __init__(self, fused, n_seqs):
        self.f, self.m, self.B = fused, fused.m, n_seqs
        g, s = self.m.g, self.m.shape
        self.g = g
        nbytes = g.moe_layer_grouped_workspace_bytes(n_seqs, s.hidden, s.inter, s.n_experts, s.top_k)
        self.ws = torch.empty(nbytes, dtype=torch.uint8, device=self.m.device)
        self.buf = [torch.zeros((n_seqs, s.hidden), dtype=torch.float32, device=self.m.device) for _ in range(2)]
        self.ids = torch.zeros((self.m.L, n_seqs * s.top_k), dtype=torch.int32, device=self.m.device)
        self.wts = torch.zeros((self.m.L, n_seqs * s.top_k), dtype=torch.float32, device=self.m.device)

    def bank(self, l):
        E, eb = self.m.shape.n_experts, self.f.expert_bytes
        return self.f.banks[l * E * eb:(l + 1) * E * eb]

    def layer(self, l, x, x_out, ids=None, wts=None, dbg_gu=None, dbg_act=None, stream=None):
        s = self.m.shape
        self.g.moe_layer_grouped(x, x_out, self.B, s.hidden, s.inter, s.n_experts, s.top_k, self.m.routers[l],
                                 self.m.layer_bias(l), None, self.bank(l), self.ids[l] if ids is None else ids,
                                 self.wts[l] if wts is None else wts, self.ws, dbg_gu, dbg_act, stream)

    def run(self, x_in, x_out, stream=None):
        """All layers for the batch: x_out = x_L (x_in, x_out: [n_seqs, H])."""
        src = x_in
        for l in range(self.m.L):
            dst = x_out if l == self.m.L - 1 else self.buf[l & 1]
            self.layer(l, src, dst, stream=stream)
            src = dst


class BatchedStack:
    """Batched decode through ft_hip_moe_stack_grouped: all layers of a step
    of n_seqs <= max_seqs tokens in one call, on one workspace for every
    batch size up to max_seqs; the banks are a FusedStack's."""

    def __init__(self, fused, max_seqs):
        self.f, self.m, self.max_seqs = fused, fused.m, max_seqs
        g, s = self.m.g, self.m.shape
        self.g = g
        nbytes = g.moe_stack_grouped_workspace_bytes(max_seqs, s.hidden, s.inter, s.n_experts, s.top_k, self.m.L)
        self.ws = torch.empty(nbytes, dtype=torch.uint8, device=self.m.device)

    def run(self, x_in, x_out, n_seqs, ids=None, wts=None, stream=None):
        """x_out[:n_seqs] = the stack applied to x_in[:n_seqs]; ids/wts: [L][n_seqs*k] or None."""
        s = self.m.shape
        self.g.moe_stack_grouped(x_in, x_out, n_seqs, self.max_seqs, s.hidden, s.inter, s.n_experts, s.top_k,
                                 self.m.L, self.f.banks, self.m.routers, self.m.bias, None, ids, wts, self.ws,
                                 stream)
