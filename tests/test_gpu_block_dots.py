"""Per-block int32 dots of the inner loops the bench times, bit-exact.

north_star requires the per-block int32 dots sum_i (q4_i - 8) * q8_i
(ft-core/src/q4_0.rs:105-118, the integer part of dot_q4_q8_avx2 :123-160)
to be bit-exact. ft_hip_set_block_dot_record makes the grouped layer's
kernels (v_dot4 gate|up and down, int8 MFMA gate|up and down) and the fused
whole-stack kernel store every block dot their production loops compute;
each is compared with the oracle's integer block dots of the same weight rows
against the same q8 activations: q8(x) for gate|up (the quants of x itself,
with or without the input norm), the kernel's own act q8 blocks for down
(themselves pinned bit-exact by the teacher-forced tests).
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


def q4_0_rows(m, layer, e):
    b = m.bank_of(layer, e).cpu().numpy()
    s = m.shape
    gu, dn = b[:m.gu_bytes], b[m.gu_bytes:]
    if m.layout == ft_hip.LAYOUT_Q4R:
        return q4r_to_q4_0(gu, 2 * s.inter, s.hidden), q4r_to_q4_0(dn, s.hidden, s.inter)
    return gu.reshape(2 * s.inter, -1), dn.reshape(s.hidden, -1)


class Record:
    """Block-dot record buffers set on the context for the duration of a with-block."""

    def __init__(self, gemv, n_slots, H, I):
        self.g = gemv
        self.gu = torch.full((n_slots, 2 * I, H // 32), -(2 ** 31), dtype=torch.int32, device=DEV)
        self.dn = torch.full((n_slots, H, I // 32), -(2 ** 31), dtype=torch.int32, device=DEV)

    def __enter__(self):
        self.g.set_block_dot_record(self.gu, self.dn)
        return self

    def __exit__(self, *a):
        self.g.set_block_dot_record(None, None)


def check_pair(orc, rec_gu, rec_dn, gu_rows, dn_rows, x, act_blk, where):
    _, qs8 = orc.q8_quantize(x)
    assert np.array_equal(rec_gu, orc.block_dots(gu_rows, qs8, x.size)), f"gate|up {where}"
    aq = act_blk[:, 8:40].copy().view(np.int8).ravel()
    assert np.array_equal(rec_dn, orc.block_dots(dn_rows, aq, aq.size)), f"down {where}"


@pytest.mark.parametrize("shape,B,mfma_min,norm", [("gemma", 16, 0, False),       # dot4, 1 pair per expert
                                                   ("gemma", 64, 10 ** 6, True),  # dot4, ~4 pairs per expert
                                                   ("gemma", 16, 1, False),       # int8 MFMA tiles
                                                   ("large", 3, 0, False)])       # MFMA, K-split long down rows
def test_grouped_block_dots_bit_exact(gemv, orc, shape, B, mfma_min, norm):
    sh = moe_synth.GEMMA if shape == "gemma" else moe_synth.LARGE
    m = moe_synth.SyntheticMoE(gemv, sh, n_layers=1)
    st = moe_synth.FusedStack(m, workspace=False)
    s = m.shape
    H, I, K = s.hidden, s.inter, s.top_k
    gs = moe_synth.GroupedStack(st, B)
    x = torch.empty((B, H), dtype=torch.float32, device=DEV)
    for t in range(B):
        m.hidden(60 + t, x[t])
    xo = torch.zeros_like(x)
    ids = torch.zeros(B * K, dtype=torch.int32, device=DEV)
    wts = torch.zeros(B * K, dtype=torch.float32, device=DEV)
    dgu = torch.zeros((B * K, 2 * I), dtype=torch.float32, device=DEV)
    dact = torch.zeros((B * K, I // 32, 40), dtype=torch.uint8, device=DEV)
    gemv.set_grouped_mfma_min(mfma_min)
    gemv.set_input_norm(norm)
    try:
        with Record(gemv, B * K, H, I) as rec:
            gs.layer(0, x, xo, ids, wts, dgu, dact)
            RG, RD = host(rec.gu), host(rec.dn)
    finally:
        gemv.set_grouped_mfma_min(0)
        gemv.set_input_norm(0)
    X, IDS, ACT = host(x), host(ids), host(dact)
    rows = {}
    for p in range(B * K):
        e = int(IDS[p])
        if e not in rows:
            rows[e] = q4_0_rows(m, 0, e)
        check_pair(orc, RG[p], RD[p], rows[e][0], rows[e][1], X[p // K], ACT[p], f"pair {p} expert {e}")


@pytest.mark.parametrize("zipf,norm", [(False, False), (True, True)])
def test_fused_block_dots_bit_exact(gemv, orc, zipf, norm):
    """Every (layer, slot, row, block) dot of the fused kernel's debug build
    (its owner's waves or, for a mispredicted tile, the helper waves), which
    the plain build's results equal bit for bit."""
    m = moe_synth.SyntheticMoE(gemv, moe_synth.GEMMA, n_layers=3, zipf_s=1.1 if zipf else None)
    st = moe_synth.FusedStack(m)
    s = m.shape
    H, I, K, L = s.hidden, s.inter, s.top_k, m.L
    x = m.hidden(70)
    out = torch.zeros_like(x)
    ids = torch.zeros(L * K, dtype=torch.int32, device=DEV)
    dbg_act = torch.zeros(L * K * (I // 32) * 40, dtype=torch.uint8, device=DEV)
    dbg_x = torch.zeros((L + 1) * H, dtype=torch.float32, device=DEV)
    gemv.set_input_norm(norm)
    try:
        with Record(gemv, L * K, H, I) as rec:
            st.run(x, out, ids, None, None, dbg_act, dbg_x)
            st.check()
            RG = host(rec.gu).reshape(L, K, 2 * I, H // 32)
            RD = host(rec.dn).reshape(L, K, H, I // 32)
    finally:
        gemv.set_input_norm(0)
    IDS = host(ids).reshape(L, K)
    ACT = host(dbg_act).reshape(L, K, I // 32, 40)
    XS = host(dbg_x).reshape(L + 1, H)
    for l in range(L):
        for p in range(K):
            e = int(IDS[l, p])
            gu_rows, dn_rows = q4_0_rows(m, l, e)
            check_pair(orc, RG[l, p], RD[l, p], gu_rows, dn_rows, XS[l], ACT[l, p], f"layer {l} slot {p} expert {e}")
