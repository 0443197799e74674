"""Stage-level bit-exact parity of the launch-by-launch layer path.

ft_hip_moe_layer / ft_hip_moe_stack run their layers as k_route_prep (or,
in a folded stack, the head inside the gate|up launch), k_gemv_gu_act or
k_gemv_gu_long (gate|up, GELU*up, q8) and k_gemv_down_combine or
k_gemv_down_head (down with the combine). ft_hip_set_layer_record makes
those kernels store what they compute, and every stage is checked against
the oracle on the kernel's own input to that stage (teacher forcing):

  q8(x_l)         == Q8Vec::quantize(x_l)            (ft-core/src/q4_0.rs:62-78)
  top-k ids, wts  == the oracle's routing of x_l      (ft-model/src/lib.rs:1487-1504)
  gate|up dots    == integer block dots vs q8(x_l)    (q4_0.rs:105-118)
  act q8          == GELU*up -> q8 of the kernel's OWN gate|up sums
                                                     (lib.rs:435-437, :1625-1632)
  down dots       == integer block dots vs that act   (q4_0.rs:105-118)
  gate|up sums, x_{l+1}: within 1e-3 of the L2 norm of the oracle's value
  (f32 sums run in another lane order than the AVX2 lanes).

The last test does the same for the production fused kernel at full depth:
the 30-layer Gemma stack, oracle on layers 0, 15 and 29 of the states the
kernel itself produced (its debug build records them and is checked to give
the production build's bits).
"""
import numpy as np
import pytest
import torch

import ft_hip
import moe_synth
from cases import q4r_to_q4_0

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def q8_blocks(orc, x):
    """The 40-byte wire blocks {d, qsum, qs} of the oracle's q8 of x."""
    d, qs = orc.q8_quantize(x)
    nb = len(d)
    b = np.zeros((nb, 40), np.uint8)
    b[:, 0:4] = d.view(np.uint8).reshape(nb, 4)
    b[:, 4:8] = qs.reshape(nb, 32).astype(np.int32).sum(axis=1).astype(np.int32).view(np.uint8).reshape(nb, 4)
    b[:, 8:40] = qs.view(np.uint8).reshape(nb, 32)
    return b


def act_blocks(orc, gu, inter):
    """GELU*up -> q8 wire blocks of one pair's gate|up sums (teacher forcing)."""
    _, d, qs = orc.gelu_mul_q8(gu, inter)
    return q8_blocks_from(d, qs)


def q8_blocks_from(d, qs):
    nb = len(d)
    b = np.zeros((nb, 40), np.uint8)
    b[:, 0:4] = d.astype(np.float32).view(np.uint8).reshape(nb, 4)
    b[:, 4:8] = qs.reshape(nb, 32).astype(np.int32).sum(axis=1).astype(np.int32).view(np.uint8).reshape(nb, 4)
    b[:, 8:40] = qs.view(np.uint8).reshape(nb, 32)
    return b


class LayerRecord:
    """Record buffers for L layers of B seqs (top_k pairs each), set on the
    context for the duration of a with-block."""

    def __init__(self, gemv, L, B, shape):
        H, I, k = shape.hidden, shape.inter, shape.top_k
        P = B * k
        self.g = gemv
        z = lambda *s, dt=torch.int32: torch.full(s, -(2 ** 31) if dt == torch.int32 else 0, dtype=dt, device=DEV)
        self.x = torch.full((L, B, H), float("nan"), dtype=torch.float32, device=DEV)
        self.q8x = torch.zeros((L, B, H // 32, 40), dtype=torch.uint8, device=DEV)
        self.gu = torch.full((L, P, 2 * I), float("nan"), dtype=torch.float32, device=DEV)
        self.act = torch.zeros((L, P, I // 32, 40), dtype=torch.uint8, device=DEV)
        self.gu_dots = z(L, P, 2 * I, H // 32)
        self.dn_dots = z(L, P, H, I // 32)

    def __enter__(self):
        self.g.set_layer_record(self.x, self.q8x, self.gu, self.act, self.gu_dots, self.dn_dots)
        return self

    def __exit__(self, *a):
        self.g.set_layer_record()

    def host(self):
        return {k: host(getattr(self, k)) for k in ("x", "q8x", "gu", "act", "gu_dots", "dn_dots")}


def expert_rows(m, layer, e):
    """q4_0 rows (gate|up, down) of one expert, as the oracle's block dots take them."""
    b = m.bank_of(layer, e).cpu().numpy()
    s = m.shape
    gu, dn = b[:m.gu_bytes], b[m.gu_bytes:]
    if m.layout == ft_hip.LAYOUT_Q4R:
        return q4r_to_q4_0(gu, 2 * s.inter, s.hidden), q4r_to_q4_0(dn, s.hidden, s.inter)
    return gu.reshape(2 * s.inter, -1), dn.reshape(s.hidden, -1)


def check_layer(orc, m, l, R, ids, wts, x_next, norm, tag):
    """Teacher-forced checks of layer l of a record R (host dict) for every seq."""
    s = m.shape
    H, I, k = s.hidden, s.inter, s.top_k
    B = R["x"].shape[1]
    Wr = host(m.routers[l])
    bias = None if m.bias is None else host(m.bias[l])
    rows, gu_b, dn_b = {}, {}, {}
    for e in sorted(set(ids.ravel().tolist())):
        b = m.bank_of(l, e).cpu().numpy()
        gu_b[e], dn_b[e] = b[:m.gu_bytes], b[m.gu_bytes:]
        rows[e] = expert_rows(m, l, e)
    for t in range(B):
        X = R["x"][l, t]
        where = f"{tag} layer {l} seq {t}"
        assert np.array_equal(R["q8x"][l, t], q8_blocks(orc, X)), f"q8(x) {where}"
        ref = orc.moe_layer(X, Wr, gu_b, dn_b, H, I, k, bias=bias, layout=m.layout, threads=8, input_norm=norm)
        assert np.array_equal(ids[t], ref["ids"]) and np.array_equal(wts[t], ref["wts"]), f"routing {where}"
        _, qs8 = orc.q8_quantize(X)
        for kk in range(k):
            p, e = t * k + kk, int(ids[t, kk])
            gu = R["gu"][l, p]
            # the kernel's sums against the oracle's (both times the norm's scale: GELU's input)
            y_ref = ref["y_gu"][kk]
            assert np.max(np.abs(gu - y_ref)) <= 1e-3 * np.linalg.norm(y_ref), f"gate|up sums {where} pair {kk}"
            assert np.array_equal(R["act"][l, p], act_blocks(orc, gu, I)), f"act q8 {where} pair {kk}"
            assert np.array_equal(R["gu_dots"][l, p], orc.block_dots(rows[e][0], qs8, H)), f"gate|up dots {where}"
            aq = R["act"][l, p][:, 8:40].copy().view(np.int8).ravel()
            assert np.array_equal(R["dn_dots"][l, p], orc.block_dots(rows[e][1], aq, I)), f"down dots {where}"
        d_ref = ref["x_out"] - X
        err = np.max(np.abs((x_next[t] - X) - d_ref)) / np.linalg.norm(d_ref)
        assert err <= 1e-3, f"x_out {where}: {err}"


def _layer_case(gemv, shape, B, norm, seed):
    m = moe_synth.SyntheticMoE(gemv, shape, n_layers=1)
    s = m.shape
    x = torch.stack([m.hidden(seed + t) for t in range(B)])
    xo = torch.zeros_like(x)
    ids = torch.zeros(B * s.top_k, dtype=torch.int32, device=DEV)
    wts = torch.zeros(B * s.top_k, dtype=torch.float32, device=DEV)
    gemv.set_input_norm(norm)
    try:
        with LayerRecord(gemv, 1, B, s) as rec:
            m.layer(0, x, xo, ids, wts, m.workspace(B), n_seqs=B)
            R = rec.host()
    finally:
        gemv.set_input_norm(0)
    return m, R, host(ids).reshape(B, -1), host(wts).reshape(B, -1), host(xo)


@pytest.mark.parametrize("shape,B,norm", [("gemma", 1, False), ("gemma", 1, True), ("gemma", 3, False),
                                          ("large", 1, True), ("large", 3, False)])
def test_moe_layer_stages_bit_exact(gemv, orc, shape, B, norm):
    """ft_hip_moe_layer: Gemma (k_route_prep, k_gemv_gu_act, k_gemv_down_combine
    with 8 lanes per row) and the large-expert shape (k_gemv_gu_long, 16 lanes
    per down row), every stage of every pair."""
    sh = moe_synth.GEMMA if shape == "gemma" else moe_synth.LARGE
    m, R, ids, wts, xo = _layer_case(gemv, sh, B, norm, 40)
    assert np.array_equal(R["x"][0], np.stack([host(m.hidden(40 + t)) for t in range(B)]))
    check_layer(orc, m, 0, R, ids, wts, xo, norm, f"moe_layer {shape} B={B}")


@pytest.mark.parametrize("shape,B,L,norm", [("gemma", 1, 2, True), ("large", 1, 2, False), ("large", 3, 2, True)])
def test_moe_stack_stages_bit_exact(gemv, orc, shape, B, L, norm):
    """ft_hip_moe_stack: the Gemma stack (plain layers) and the large-expert
    stack, whose later layers take q8(x), logits and norm scale from the head
    inside the gate|up launch (k_gemv_gu_long<HEAD>) and whose down launch is
    k_gemv_down_head; every layer's stages against the oracle on that layer's
    own input (teacher forcing), and each layer's output is the next one's
    recorded input bit for bit."""
    sh = moe_synth.GEMMA if shape == "gemma" else moe_synth.LARGE
    m = moe_synth.SyntheticMoE(gemv, sh, n_layers=L)
    s = m.shape
    k = s.top_k
    x = torch.stack([m.hidden(50 + t) for t in range(B)])
    out = torch.zeros_like(x)
    ids = torch.zeros((L, B * k), dtype=torch.int32, device=DEV)
    wts = torch.zeros((L, B * k), dtype=torch.float32, device=DEV)
    gemv.set_input_norm(norm)
    try:
        with LayerRecord(gemv, L, B, s) as rec:
            m.stack(x, out, ids, wts, m.stack_workspace(B), n_seqs=B)
            R = rec.host()
    finally:
        gemv.set_input_norm(0)
    ids_h, wts_h, out_h = host(ids).reshape(L, B, k), host(wts).reshape(L, B, k), host(out)
    assert np.array_equal(R["x"][0], host(x))
    for l in range(L):
        x_next = R["x"][l + 1] if l + 1 < L else out_h
        check_layer(orc, m, l, R, ids_h[l], wts_h[l], x_next, norm, f"moe_stack {shape} B={B}")


@pytest.mark.parametrize("shape", ["small", "large"])
def test_gemv_gate_up_act_stages_bit_exact(gemv, orc, shape):
    """ft_hip_gemv_gate_up_act (the shared MLP's gate|up with GELU*up and q8 in
    one launch): its block dots equal the oracle's, and its act q8 equals
    GELU*up -> q8 of its own recorded sums (times the per-row scale)."""
    sh = moe_synth.Shape("small", 384, 160, 24, 3, 1, 9) if shape == "small" else moe_synth.LARGE
    m = moe_synth.SyntheticMoE(gemv, sh, n_layers=1)
    H, I = sh.hidden, sh.inter
    n, xdiv = 3, 2
    x = torch.stack([m.hidden(t) for t in range(2)])
    q8x = torch.zeros(2 * (H // 32) * 40, dtype=torch.uint8, device=DEV)
    gemv.quantize_q8(x, H, q8x, H, 2)
    slots = torch.tensor([3 % sh.n_experts, 5 % sh.n_experts, 0], dtype=torch.int32, device=DEV)
    sc = torch.tensor([0.75, 1.3125], dtype=torch.float32, device=DEV)
    bank = m.banks[:sh.n_experts * m.expert_bytes]
    out = torch.zeros(n * (I // 32) * 40, dtype=torch.uint8, device=DEV)
    gu = torch.full((n, 2 * I), float("nan"), dtype=torch.float32, device=DEV)
    dots = torch.full((n, 2 * I, H // 32), -(2 ** 31), dtype=torch.int32, device=DEV)
    gemv.set_layer_record(gu=gu, gu_dots=dots)
    try:
        gemv.gemv_gate_up_act(bank, m.expert_bytes, slots, n, xdiv, q8x, H, I, out, layout=m.layout, in_scale=sc)
        G, D, A = host(gu), host(dots), host(out).reshape(n, I // 32, 40)
    finally:
        gemv.set_layer_record()
    X, S = host(x), host(sc)
    for p in range(n):
        e, row = int(host(slots)[p]), p // xdiv
        _, qs8 = orc.q8_quantize(X[row])
        rows = expert_rows(m, 0, e)[0]
        assert np.array_equal(D[p], orc.block_dots(rows, qs8, H)), f"gate|up dots pair {p}"
        assert np.array_equal(A[p], act_blocks(orc, G[p], I)), f"act q8 pair {p}"
        ref = orc.gemv(rows, X[row], 2 * I) * S[row]
        assert np.max(np.abs(G[p] - ref)) <= 1e-3 * np.linalg.norm(ref), f"sums pair {p}"


def test_record_off_is_production(gemv):
    """With the record off again the layer gives the same bits as with it on
    (the record instantiations compute the same arithmetic)."""
    m, R, ids, wts, xo = _layer_case(gemv, moe_synth.GEMMA, 2, True, 80)
    s = m.shape
    x = torch.stack([m.hidden(80 + t) for t in range(2)])
    xo2 = torch.zeros_like(x)
    ids2 = torch.zeros(2 * s.top_k, dtype=torch.int32, device=DEV)
    wts2 = torch.zeros(2 * s.top_k, dtype=torch.float32, device=DEV)
    gemv.set_input_norm(1)
    try:
        m.layer(0, x, xo2, ids2, wts2, m.workspace(2), n_seqs=2)
    finally:
        gemv.set_input_norm(0)
    assert np.array_equal(host(xo2).view(np.uint32), xo.view(np.uint32))
    assert np.array_equal(host(ids2).reshape(2, -1), ids) and np.array_equal(host(wts2).reshape(2, -1), wts)


@pytest.mark.parametrize("zipf", [False, True])
def test_fused_30_layers_teacher_forced(gemv, orc, zipf):
    """The production fused kernel on the full 30-layer Gemma stack (the
    headline configuration, input norm on): its output equals its debug
    build's bit for bit, and on layers 0, 15 and 29 of the states the kernel
    produced, the oracle gives the same top-k ids and weights, GELU*up -> q8
    of the kernel's own gate|up sums gives its act quants, and x_{l+1} agrees
    within 1e-3 of the norm of the oracle's update."""
    m = moe_synth.SyntheticMoE(gemv, moe_synth.GEMMA, zipf_s=1.1 if zipf else None)
    st = moe_synth.FusedStack(m)
    s = m.shape
    H, I, K, L = s.hidden, s.inter, s.top_k, m.L
    x = m.hidden(7)
    gemv.set_input_norm(1)
    try:
        out_p = torch.zeros_like(x)
        ids_p = torch.zeros(L * K, dtype=torch.int32, device=DEV)
        wts_p = torch.zeros(L * K, dtype=torch.float32, device=DEV)
        st.run(x, out_p, ids_p, wts_p)
        st.check()
        out_d = torch.zeros_like(x)
        ids_d = torch.zeros_like(ids_p)
        wts_d = torch.zeros_like(wts_p)
        dgu = torch.zeros(L * K * 2 * I, dtype=torch.float32, device=DEV)
        dact = torch.zeros(L * K * (I // 32) * 40, dtype=torch.uint8, device=DEV)
        dx = torch.zeros((L + 1) * H, dtype=torch.float32, device=DEV)
        st.run(x, out_d, ids_d, wts_d, dgu, dact, dx)
        st.check()
    finally:
        gemv.set_input_norm(0)
    assert np.array_equal(host(out_d).view(np.uint32), host(out_p).view(np.uint32))
    assert torch.equal(ids_d, ids_p) and torch.equal(wts_d, wts_p)
    IDS, WTS = host(ids_p).reshape(L, K), host(wts_p).reshape(L, K)
    GU, ACT, XS = host(dgu).reshape(L, K, 2 * I), host(dact).reshape(L, K, I // 32, 40), host(dx).reshape(L + 1, H)
    assert np.array_equal(XS[L].view(np.uint32), host(out_p).view(np.uint32))
    for l in (0, 15, 29):
        Wr = host(m.routers[l])
        bias = None if m.bias is None else host(m.bias[l])
        gu_b, dn_b = {}, {}
        for e in IDS[l]:
            b = m.bank_of(l, int(e)).cpu().numpy()
            gu_b[int(e)], dn_b[int(e)] = b[:m.gu_bytes], b[m.gu_bytes:]
        ref = orc.moe_layer(XS[l], Wr, gu_b, dn_b, H, I, K, bias=bias, layout=m.layout, threads=8, input_norm=True)
        assert np.array_equal(IDS[l], ref["ids"]) and np.array_equal(WTS[l], ref["wts"]), f"routing layer {l}"
        for p in range(K):
            assert np.array_equal(ACT[l, p], act_blocks(orc, GU[l, p], I)), f"act q8 layer {l} slot {p}"
        d_ref = ref["x_out"] - XS[l]
        err = np.max(np.abs((XS[l + 1] - XS[l]) - d_ref)) / np.linalg.norm(d_ref)
        assert err <= 1e-3, f"x layer {l}: {err}"
