"""GPU parity tests of the grouped batched layer (ft_hip_moe_layer_grouped).

Batched decode of BASELINE configs 4 (B = 16, 64 tokens, uniform routing) and
3 (Zipf-skewed routing), on seeded Gemma-shaped layers. Per token the routing
is checked bit-exact against the oracle's R-order logits and top-k; per
(token, expert) pair the act q8 blocks bit-exact against the oracle's
GELU*up q8 of the kernel's own gate|up sums (teacher forcing); gate|up sums
and layer outputs within max|d| <= 1e-3 * ||ref||_2.
The ungrouped launch-by-launch layer (one GEMV per pair, as the reference's
batched path, ft-model/src/lib.rs:1507-1606) must pick the same experts with
the same weights. With the input RMS norm on, its scale enters the logits
and the gate|up sums; the same checks hold. The default (mfma_min 0) puts every
expert on the int8 MFMA tile kernels from 4 pairs per expert on (B = 64, 128)
and on the dot4 kernels below (B = 16); cases also split the experts at 16 tokens
(both families in one layer) and force every expert onto one family (mfma_min
1 or 10**6); the large-expert shape (inter 14336) always takes the MFMA
kernels.
"""
import numpy as np
import pytest
import torch

import moe_synth

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.fixture(scope="module")
def gstack(gemv):
    m = moe_synth.SyntheticMoE(gemv, moe_synth.GEMMA, n_layers=2, zipf_s=1.1)
    return moe_synth.FusedStack(m)


def _hidden(m, B, first=0):
    x = torch.empty((B, m.shape.hidden), dtype=torch.float32, device=DEV)
    for t in range(B):
        m.hidden(first + t, x[t])
    return x


def _banks(m, layer, ids):
    gu, dn = {}, {}
    for e in set(int(v) for v in ids):
        b = m.bank_of(layer, e).cpu().numpy()
        gu[e], dn[e] = b[:m.gu_bytes], b[m.gu_bytes:]
    return gu, dn


@pytest.mark.parametrize("B,zipf,norm,mfma_min", [(16, False, False, 0), (64, False, False, 0), (128, False, False, 0),
                                                   (64, True, False, 16),
                                                  (16, True, True, 16), (16, False, False, 1), (64, True, True, 1),
                                                  (64, True, False, 10**6)])
def test_grouped_layer_matches_oracle(gemv, orc, gstack, B, zipf, norm, mfma_min):
    m = gstack.m
    s = m.shape
    H, I, E, K = s.hidden, s.inter, s.n_experts, s.top_k
    gs = moe_synth.GroupedStack(gstack, B)
    saved = m.bias
    if not zipf:
        m.bias = None
    try:
        x = _hidden(m, B, first=100 * B + zipf)
        xo = torch.zeros_like(x)
        ids = torch.zeros(B * K, dtype=torch.int32, device=DEV)
        wts = torch.zeros(B * K, dtype=torch.float32, device=DEV)
        dgu = torch.zeros((B * K, 2 * I), dtype=torch.float32, device=DEV)
        dact = torch.zeros((B * K, I // 32, 40), dtype=torch.uint8, device=DEV)
        layer = 1
        gemv.set_input_norm(norm)
        gemv.set_grouped_mfma_min(mfma_min)
        gs.layer(layer, x, xo, ids, wts, dgu, dact)
        X, XO, IDS, WTS = host(x), host(xo), host(ids).reshape(B, K), host(wts).reshape(B, K)
        GU, ACT = host(dgu).reshape(B, K, 2 * I), host(dact).reshape(B, K, I // 32, 40)
        W_r = host(m.routers[layer])
        bias = None if m.bias is None else host(m.bias[layer])
        # routing: bit-exact per token
        for t in range(B):
            lg = orc.router_logits(W_r, X[t])
            if norm:
                lg = (lg * orc.rms_inv(X[t])).astype(np.float32)
            if bias is not None:
                lg = (lg + bias).astype(np.float32)
            ie, we = orc.topk_softmax(lg, K)
            assert np.array_equal(IDS[t], ie), f"token {t}"
            assert np.array_equal(WTS[t].view(np.uint32), we.view(np.uint32)), f"token {t}"
        if zipf:  # the skew must put many tokens on some expert (chunked groups)
            assert np.bincount(IDS.ravel(), minlength=E).max() > 8
        # per pair: act q8 bit-exact from the kernel's own gate|up sums; sums within tolerance
        d8, q8 = orc.q8_quantize(X[0])
        for t in range(0, B, max(1, B // 8)):
            gub, dnb = _banks(m, layer, IDS[t])
            d8, q8 = orc.q8_quantize(X[t])
            for k in range(K):
                e = int(IDS[t, k])
                _, ad, aq = orc.gelu_mul_q8(GU[t, k], I)
                blk = ACT[t, k]
                assert np.array_equal(blk[:, 0:4].copy().view(np.float32)[:, 0].view(np.uint32), ad.view(np.uint32))
                assert np.array_equal(blk[:, 8:40].copy().view(np.int8).ravel(), aq)
                ref = orc.gemv_q8(gub[e].reshape(2 * I, -1), 2 * I, d8, q8, H, layout=m.layout)
                if norm:
                    ref = (ref * orc.rms_inv(X[t])).astype(np.float32)
                assert np.max(np.abs(GU[t, k] - ref)) <= 1e-3 * np.linalg.norm(ref)
            r = orc.moe_layer(X[t], W_r, gub, dnb, H, I, K, bias=bias, layout=m.layout,
                              input_norm=norm)
            assert np.array_equal(r["ids"], IDS[t])
            dref = r["x_out"] - X[t]
            assert np.max(np.abs((XO[t] - X[t]) - dref)) <= 1e-3 * np.linalg.norm(dref), f"token {t}"
        # the ungrouped launch-by-launch layer on the same batch
        ws = m.workspace(B)
        xo2 = torch.zeros_like(x)
        ids2 = torch.zeros_like(ids)
        wts2 = torch.zeros_like(wts)
        m.layer(layer, x, xo2, ids2, wts2, ws, n_seqs=B)
        assert np.array_equal(host(ids2).reshape(B, K), IDS)
        assert np.array_equal(host(wts2).reshape(B, K).view(np.uint32), WTS.view(np.uint32))
        XO2 = host(xo2)
        for t in range(B):
            d2 = XO2[t] - X[t]
            assert np.max(np.abs((XO[t] - X[t]) - d2)) <= 1e-3 * np.linalg.norm(d2)
    finally:
        m.bias = saved
        gemv.set_input_norm(0)
        gemv.set_grouped_mfma_min(0)


def test_grouped_repeatable_and_empty(gemv, gstack):
    """Fixed orders: two runs give identical bits; a zero-token batch is a no-op."""
    m = gstack.m
    B = 32
    gs = moe_synth.GroupedStack(gstack, B)
    x = _hidden(m, B, first=7)
    a, b = torch.zeros_like(x), torch.zeros_like(x)
    gs.run(x, a)
    gs.run(x, b)
    assert np.array_equal(host(a).view(np.uint32), host(b).view(np.uint32))
    s = m.shape
    gemv.moe_layer_grouped(x, a, 0, s.hidden, s.inter, s.n_experts, s.top_k, m.routers[0], None, None,
                           gs.bank(0), gs.ids[0], gs.wts[0], gs.ws)


@pytest.mark.parametrize("norm,B", [(False, 12), (True, 12), (True, 32)])
def test_grouped_large_expert_mfma(gemv, orc, norm, B):
    """Config 5's shape (H 4096, 8 experts of I 14336, top-2), 12 tokens and
    config 5's own batch of 32 in one grouped layer (MFMA kernels, K-split
    down rows): per token routing bit-exact, act q8 bit-exact from the
    kernel's own gate|up sums, gate|up sums and outputs within the
    north-star tolerance."""
    m = moe_synth.SyntheticMoE(gemv, moe_synth.LARGE, n_layers=1)
    st = moe_synth.FusedStack(m, workspace=False)
    s = m.shape
    H, I, E, K = s.hidden, s.inter, s.n_experts, s.top_k
    gs = moe_synth.GroupedStack(st, B)
    x = _hidden(m, B, first=40)
    xo = torch.zeros_like(x)
    ids = torch.zeros(B * K, dtype=torch.int32, device=DEV)
    wts = torch.zeros(B * K, dtype=torch.float32, device=DEV)
    dgu = torch.zeros((B * K, 2 * I), dtype=torch.float32, device=DEV)
    dact = torch.zeros((B * K, I // 32, 40), dtype=torch.uint8, device=DEV)
    gemv.set_input_norm(norm)
    try:
        gs.layer(0, x, xo, ids, wts, dgu, dact)
    finally:
        gemv.set_input_norm(0)
    X, XO, IDS, WTS = host(x), host(xo), host(ids).reshape(B, K), host(wts).reshape(B, K)
    GU, ACT = host(dgu).reshape(B, K, 2 * I), host(dact).reshape(B, K, I // 32, 40)
    W_r = host(m.routers[0])
    gub, dnb = _banks(m, 0, IDS.ravel())
    for t in range(B):
        r = orc.moe_layer(X[t], W_r, gub, dnb, H, I, K, layout=m.layout, threads=8, input_norm=norm)
        assert np.array_equal(IDS[t], r["ids"]), t
        assert np.array_equal(WTS[t].view(np.uint32), r["wts"].view(np.uint32)), t
        for k in range(K):
            assert np.max(np.abs(GU[t, k] - r["y_gu"][k])) <= 1e-3 * np.linalg.norm(r["y_gu"][k]), (t, k)
            _, ad, aq = orc.gelu_mul_q8(GU[t, k], I)
            blk = ACT[t, k]
            assert np.array_equal(blk[:, 0:4].copy().view(np.float32)[:, 0].view(np.uint32), ad.view(np.uint32))
            assert np.array_equal(blk[:, 8:40].copy().view(np.int8).ravel(), aq)
        dref = r["x_out"] - X[t]
        assert np.max(np.abs((XO[t] - X[t]) - dref)) <= 1e-3 * np.linalg.norm(dref), t


@pytest.mark.parametrize("norm", [False, True])
def test_batched_stack_variable_batch(gemv, norm):
    """ft_hip_moe_stack_grouped over a 3-layer Zipf stack on ONE workspace
    sized for 64 tokens, with the batch changing between steps (16, 5, 64,
    1, 0, 33 tokens, as forward_batch sees under continuous batching): every
    step's outputs and per-layer routing equal the layer-by-layer calls on
    the same tokens (each with a workspace of its own size), bit for bit;
    rows past n_seqs are untouched; an in-place call gives the same bits."""
    m = moe_synth.SyntheticMoE(gemv, moe_synth.GEMMA, n_layers=3, zipf_s=1.1)
    st = moe_synth.FusedStack(m, workspace=False)
    bs = moe_synth.BatchedStack(st, 64)
    H, k, L = m.shape.hidden, m.shape.top_k, m.L
    gemv.set_input_norm(int(norm))
    try:
        first = 0
        for B in (16, 5, 64, 1, 0, 33):
            x = _hidden(m, max(B, 1), first)
            first += B
            out = torch.full((64, H), 7.0, dtype=torch.float32, device=DEV)
            ids = torch.zeros((L, max(B, 1) * k), dtype=torch.int32, device=DEV)
            wts = torch.zeros((L, max(B, 1) * k), dtype=torch.float32, device=DEV)
            bs.run(x, out, B, ids, wts)
            o = host(out)
            assert np.all(o[B:] == 7.0)
            if B == 0:
                continue
            ref = moe_synth.GroupedStack(st, B)
            ro = torch.zeros((B, H), dtype=torch.float32, device=DEV)
            ref.run(x, ro)
            assert np.array_equal(o[:B].view(np.uint32), host(ro).view(np.uint32)), B
            assert np.array_equal(host(ids), host(ref.ids)), B
            assert np.array_equal(host(wts).view(np.uint32), host(ref.wts).view(np.uint32)), B
            xi = x.clone()
            bs.run(xi, xi, B)  # in place, no routing record
            assert np.array_equal(host(xi).view(np.uint32), o[:B].view(np.uint32)), B
    finally:
        gemv.set_input_norm(0)


def test_batched_stack_rejects(gemv, gstack):
    m = gstack.m
    bs = moe_synth.BatchedStack(gstack, 8)
    x = _hidden(m, 9)
    with pytest.raises(Exception):
        bs.run(x, x, 9)  # more tokens than the workspace was sized for
    s = m.shape
    small = torch.empty(bs.ws.numel() - 256, dtype=torch.uint8, device=DEV)
    with pytest.raises(Exception):
        gemv.moe_stack_grouped(x, x, 4, 8, s.hidden, s.inter, s.n_experts, s.top_k, m.L, gstack.banks, m.routers,
                               m.bias, None, None, None, small)
