"""GPU parity tests of the launch-by-launch kernels against the CPU oracle.

Bit-exact: q8 quants (d, qs, integer sum), per-block int32 dots, GELU*up q8
given the same gate|up inputs (libm tanhf, as ft-core), router logits (R-order),
top-k ids and weights, the weighted combine, the seeded generators and the
q4r repack. f32 GEMV outputs: max|dy| <= 1e-3 * ||y_ref||_2 (the north-star
tolerance) and, tighter, |dy| <= 1e-5 * sum|w*x| per row.
Models: ft-cuda/tests/{parity,grouped,v3,q4r}.rs.
"""
import numpy as np
import pytest
import torch

import ft_hip
import moe_synth
from cases import nonfinite_q8_blocks

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def q8_split(buf, n, nb):
    b = np.ascontiguousarray(buf).view(np.uint8).reshape(n, nb, 40)
    d = b[:, :, 0:4].copy().view(np.float32)[:, :, 0]
    qsum = b[:, :, 4:8].copy().view(np.int32)[:, :, 0]
    qs = b[:, :, 8:40].copy().view(np.int8).reshape(n, nb * 32)
    return d, qsum, qs


def gpu_quantize(gemv, x, k, n, x_stride):
    q8 = torch.zeros(n * (k // 32) * 40, dtype=torch.uint8, device=DEV)
    gemv.quantize_q8(dev(x), x_stride, q8, k, n)
    return q8_split(host(q8), n, k // 32), q8


def q8_from_oracle(orc, x):
    d, qs = orc.q8_quantize(x)
    nb = len(d)
    b = np.zeros((nb, 40), np.uint8)
    b[:, 0:4] = d.view(np.uint8).reshape(nb, 4)
    b[:, 4:8] = qs.reshape(nb, 32).astype(np.int32).sum(axis=1).astype(np.int32).view(np.uint8).reshape(nb, 4)
    b[:, 8:40] = qs.view(np.uint8).reshape(nb, 32)
    return b.ravel()


def test_context(gemv):
    assert gemv.device == 0


@pytest.mark.parametrize("k,n,stride", [(32, 1, 0), (2816, 3, 2816), (704, 8, 736), (4096, 2, 0), (14336, 1, 0)])
def test_quantize_q8_bit_exact(gemv, orc, k, n, stride):
    rng = np.random.default_rng(k + n)
    rows = stride if stride else k
    x = (rng.standard_normal(max(n, 1) * rows) * rng.choice([1e-3, 1.0, 30.0])).astype(np.float32)
    x[:32] = 0.0                                               # zero block
    if k >= 64:
        x[32:64] = np.array([127.0, 2.5, -2.5, 0.5, -0.5, 126.5] + [1.5] * 26, np.float32)  # exact ties
    (d, qsum, qs), _ = gpu_quantize(gemv, x, k, n, stride)
    for r in range(n):
        xr = x[r * stride:r * stride + k] if stride else x[:k]
        de, qe = orc.q8_quantize(xr)
        assert np.array_equal(d[r].view(np.uint32), de.view(np.uint32))
        assert np.array_equal(qs[r], qe)
        assert np.array_equal(qsum[r], qe.reshape(-1, 32).astype(np.int32).sum(axis=1))


def test_quantize_q8_nonfinite_blocks(gemv):
    """inf, NaN and subnormal-scale blocks: the quants Rust's `as i8` gives
    (NaN products -> 0), closed form in cases.nonfinite_q8_blocks."""
    x, de, qe = nonfinite_q8_blocks()
    (d, qsum, qs), _ = gpu_quantize(gemv, x, x.size, 1, 0)
    assert np.array_equal(d[0].view(np.uint32), de.view(np.uint32)), (d[0], de)
    assert np.array_equal(qs[0], qe)
    assert np.array_equal(qsum[0], qe.reshape(-1, 32).astype(np.int32).sum(axis=1))


def test_quantize_q8_division_sweep(gemv, orc):
    """d = amax/127 and 1/d must be IEEE-exact: sweep amax over 2^18 random f32
    values spanning 1e-30..1e30, one block each."""
    rng = np.random.default_rng(99)
    nblk = 1 << 18
    amax = (10.0 ** rng.uniform(-30, 30, nblk)).astype(np.float32)
    u = rng.uniform(-1, 1, (nblk, 32)).astype(np.float32)
    x = (u * amax[:, None]).astype(np.float32)
    x[:, 0] = amax
    x = x.ravel()
    (d, qsum, qs), _ = gpu_quantize(gemv, x, x.size, 1, 0)
    de, qe = orc.q8_quantize(x)
    assert np.array_equal(d[0].view(np.uint32), de.view(np.uint32))
    assert np.array_equal(qs[0], qe)


def make_bank(orc, n_exp, n_rows, k, seed, layout):
    """n_exp experts of n_rows q4 rows each (xorshift-like seeded normal data), in layout."""
    rng = np.random.default_rng(seed)
    w = orc.quantize_row((rng.standard_normal((n_exp * n_rows, k)) * 0.02).astype(np.float32))
    if layout == ft_hip.LAYOUT_Q4R:
        w = orc.repack_q4r(w, k)
    return w.reshape(n_exp, -1)


@pytest.mark.parametrize("layout", [ft_hip.LAYOUT_Q4_0, ft_hip.LAYOUT_Q4R])
@pytest.mark.parametrize("k,n_rows", [(2816, 64), (2112, 64), (704, 64), (4096, 32), (32, 7), (704, 2816),
                                      (2816, 1408), (14336, 8)])
def test_block_dots_and_gemv(gemv, orc, layout, k, n_rows):
    """ft-cuda/tests/q4r.rs shapes, plus the Gemma gate|up / down shapes; shuffled
    slots as ft-cuda/tests/grouped.rs ([3,0,4,1,2]) and an x_idx indirection."""
    n_exp = 5
    bank = make_bank(orc, n_exp, n_rows, k, k * 7 + n_rows, layout)
    eb = bank.shape[1]
    rng = np.random.default_rng(k)
    xs = rng.standard_normal((2, k)).astype(np.float32)
    q8 = np.concatenate([q8_from_oracle(orc, xs[0]), q8_from_oracle(orc, xs[1])])
    slots = np.array([3, 0, 4, 1, 2], np.int32)
    x_idx = np.array([1, 0, 0, 1, 1], np.int32)
    nb = k // 32
    bank_d, q8_d, slots_d, xidx_d = dev(bank.ravel()), dev(q8), dev(slots), dev(x_idx)
    dots = torch.zeros(5 * n_rows * nb, dtype=torch.int32, device=DEV)
    gemv.block_dots(bank_d, eb, 0, slots_d, xidx_d, 5, q8_d, nb, dots, n_rows, k, layout)
    y = torch.zeros(5 * n_rows, dtype=torch.float32, device=DEV)
    gemv.gemv_grouped_slots(bank_d, eb, 0, slots_d, xidx_d, 5, q8_d, nb, y, n_rows, n_rows, k, layout)
    dots, y = host(dots).reshape(5, n_rows, nb), host(y).reshape(5, n_rows)
    rb0 = orc.row_bytes(k)
    for e in range(5):
        raw = bank[slots[e]].reshape(n_rows, -1)
        if layout == ft_hip.LAYOUT_Q4R:  # the oracle's integer dots read q4_0 rows: undo the repack
            so = orc.q4r_scales_bytes(k)
            q40 = np.zeros((n_rows, nb, 18), np.uint8)
            q40[:, :, :2] = raw[:, :2 * nb].reshape(n_rows, nb, 2)
            q40[:, :, 2:] = raw[:, so:].reshape(n_rows, nb, 16)
            raw = q40.reshape(n_rows, rb0)
        d8, qs8 = orc.q8_quantize(xs[x_idx[e]])
        assert np.array_equal(dots[e], orc.block_dots(raw, qs8, k)), f"entry {e}"
        ref = orc.gemv_q8(raw, n_rows, d8, qs8, k)
        assert np.max(np.abs(y[e] - ref)) <= 1e-3 * np.linalg.norm(ref)
        # per-row bound against the magnitude of the terms
        from test_oracle import unpack_q4
        nib, d4 = unpack_q4(raw, k)
        mag = np.abs((nib.astype(np.float64) - 8) * np.repeat(d4, 32, axis=1)) @ np.abs(
            qs8.astype(np.float64) * np.repeat(d8, 32))
        assert np.all(np.abs(y[e].astype(np.float64) - ref) <= 1e-5 * mag + 1e-30)


def test_gemv_ptr_form_and_shared_activation(gemv, orc):
    k, n_rows, n_exp = 2816, 96, 3
    bank = make_bank(orc, n_exp, n_rows, k, 0xFACE, ft_hip.LAYOUT_Q4R)
    bank_d = dev(bank.ravel())
    eb = bank.shape[1]
    x = np.random.default_rng(1).standard_normal(k).astype(np.float32)
    q8_d = dev(q8_from_oracle(orc, x))
    bases = torch.tensor([bank_d.data_ptr() + e * eb for e in (2, 0, 1)], dtype=torch.int64, device=DEV)
    y1 = torch.zeros(3 * n_rows, dtype=torch.float32, device=DEV)
    gemv.gemv_q4r_ptr(bases, 0, None, 3, q8_d, 0, y1, n_rows, n_rows, k)
    y2 = torch.zeros(3 * n_rows, dtype=torch.float32, device=DEV)
    gemv.gemv_q4r_idx(bank_d, eb, 0, dev(np.array([2, 0, 1], np.int32)), None, 3, q8_d, 0, y2, n_rows, n_rows, k)
    assert torch.equal(y1, y2)
    d8, qs8 = orc.q8_quantize(x)
    raw = make_bank(orc, n_exp, n_rows, k, 0xFACE, ft_hip.LAYOUT_Q4_0)
    ref = np.concatenate([orc.gemv_q8(raw[e], n_rows, d8, qs8, k) for e in (2, 0, 1)])
    y = host(y1)
    assert np.max(np.abs(y - ref)) <= 1e-3 * np.linalg.norm(ref)


def test_gelu_mul_q8_bit_exact(gemv, orc):
    """Teacher-forced GELU*up -> q8 on identical gate|up inputs: bit-exact with the
    oracle, whose tanh is the host libm's tanhf (ft-model/src/lib.rs:436 calls
    glibc's tanhf through f32::tanh). Includes the branch points of glibc's
    tanhf/expm1f (|z| = 1, 22, 2^-55, ln2/2, 3ln2/2) on the GELU argument."""
    I, n = 704, 64
    rng = np.random.default_rng(5)
    gu = (rng.standard_normal((n, 2 * I)) * rng.choice([0.05, 1.0, 4.0], (n, 1))).astype(np.float32)
    gu[0, :40] = [0.0, -0.0, 10.0, -10.0, 9.5, -9.5, 1e-30, -1e-30] + [1e-4] * 32
    # gate values g whose GELU argument 0.7978845608*(g + 0.044715 g^3) lands near tanhf's branches
    gu[1, :I] = np.concatenate([np.linspace(-30, 30, 352), np.geomspace(1e-12, 2.0, 176),
                                -np.geomspace(1e-12, 2.0, 176)]).astype(np.float32)
    q8 = torch.zeros(n * (I // 32) * 40, dtype=torch.uint8, device=DEV)
    gemv.gelu_mul_q8(dev(gu), q8, I, n)
    d, qsum, qs = q8_split(host(q8), n, I // 32)
    for e in range(n):
        _, de, qe = orc.gelu_mul_q8(gu[e], I)
        assert np.array_equal(d[e].view(np.uint32), de.view(np.uint32)), e
        assert np.array_equal(qs[e], qe), e
        assert np.array_equal(qsum[e], qe.reshape(-1, 32).astype(np.int32).sum(axis=1))


def test_router_logits_bit_exact(gemv, orc):
    E, H, S = 128, 2816, 3
    rng = np.random.default_rng(6)
    W = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    x = rng.standard_normal((S, H)).astype(np.float32)
    bias = rng.standard_normal(E).astype(np.float32)
    for b in (None, bias):
        y = torch.zeros(S * E, dtype=torch.float32, device=DEV)
        gemv.gemv_f32_rows_dev(dev(W), dev(x), y, H, E, S, bias=None if b is None else dev(b))
        y = host(y).reshape(S, E)
        for s in range(S):
            assert np.array_equal(y[s].view(np.uint32), orc.router_logits(W, x[s], b).view(np.uint32))


@pytest.mark.parametrize("E,k", [(128, 8), (8, 2), (1024, 32), (3, 3)])
def test_topk_router_bit_exact(gemv, orc, E, k):
    S = 6
    rng = np.random.default_rng(E + k)
    lg = rng.standard_normal((S, E)).astype(np.float32)
    lg[1, :] = 0.5                                  # all tied
    lg[2, rng.integers(0, E, E // 2)] = lg[2, 0]    # many ties
    lg[3, rng.integers(0, E, max(1, E // 3))] = np.nan  # NaN ranks after every number
    lg[4, : (E + 1) // 2] = -0.0                    # signed zeros tie
    lg[4, (E + 1) // 2:] = 0.0
    scale = (rng.random(E) + 0.5).astype(np.float32)
    for es in (None, scale):
        ids = torch.zeros(S * k, dtype=torch.int32, device=DEV)
        wts = torch.zeros(S * k, dtype=torch.float32, device=DEV)
        gemv.topk_router_dev(dev(lg), None if es is None else dev(es), ids, wts, E, k, S)
        ids, wts = host(ids).reshape(S, k), host(wts).reshape(S, k)
        for s in range(S):
            ie, we = orc.topk_softmax(lg[s], k, es)
            assert np.array_equal(ids[s], ie)
            nan = np.isnan(we)                      # a chosen NaN makes every weight NaN
            assert np.array_equal(np.isnan(wts[s]), nan)
            assert np.array_equal(wts[s][~nan].view(np.uint32), we[~nan].view(np.uint32))


def test_reduce_pairs_weighted_bit_exact(gemv, orc):
    H, S, k = 2816, 4, 8
    rng = np.random.default_rng(7)
    y = rng.standard_normal((S * k, H)).astype(np.float32)
    w = rng.random(S * k).astype(np.float32)
    seq_of = np.repeat(np.arange(S, dtype=np.int32), k)
    rng.shuffle(seq_of)
    out0 = rng.standard_normal((S, H)).astype(np.float32)
    out = dev(out0)
    gemv.reduce_pairs_weighted(dev(y), dev(w), dev(seq_of), out, H, S * k, S)
    out = host(out)
    for s in range(S):
        ps = np.nonzero(seq_of == s)[0]
        exp = orc.combine(y[ps], w[ps], out0[s])
        assert np.array_equal(out[s].view(np.uint32), exp.view(np.uint32))


def test_generators_bit_exact(gemv, orc):
    key = moe_synth.tensor_key(1, 3, 17, moe_synth.T_GU)
    assert key == orc.tensor_key(1, 3, 17, orc.T_GU)
    scale = moe_synth.gen_scale(0.02)
    assert np.float32(scale) == np.float32(orc.gen_scale(0.02))
    v = torch.zeros(100000, dtype=torch.float32, device=DEV)
    gemv.gen_values(key, 12345, 100000, scale, v)
    assert np.array_equal(host(v), orc.gen_values(key, 12345, 100000, 0.02))
    for k, rows, row0 in [(2816, 40, 0), (704, 33, 1000)]:
        exp = orc.gen_q4_rows(key, row0, rows, k, 0.02)
        for layout in (ft_hip.LAYOUT_Q4_0, ft_hip.LAYOUT_Q4R):
            out = torch.zeros(rows * ft_hip.row_bytes(k, layout), dtype=torch.uint8, device=DEV)
            gemv.gen_q4_rows(key, row0, rows, k, scale, out, layout)
            e = exp if layout == ft_hip.LAYOUT_Q4_0 else orc.repack_q4r(exp, k)
            assert np.array_equal(host(out).reshape(e.shape), e)


def test_repack_rows(gemv, orc):
    k, rows = 704, 50
    w = make_bank(orc, 1, rows, k, 3, ft_hip.LAYOUT_Q4_0).reshape(rows, -1)
    src = dev(w.ravel())
    dst = torch.full((rows * ft_hip.row_bytes(k, ft_hip.LAYOUT_Q4R),), 0xEE, dtype=torch.uint8, device=DEV)
    gemv.repack_rows(src, ft_hip.LAYOUT_Q4_0, dst, ft_hip.LAYOUT_Q4R, rows, k)
    assert np.array_equal(host(dst).reshape(rows, -1), orc.repack_q4r(w, k))
    back = torch.zeros_like(src)
    gemv.repack_rows(dst, ft_hip.LAYOUT_Q4R, back, ft_hip.LAYOUT_Q4_0, rows, k)
    assert torch.equal(back, src)


def _oracle_banks(model, layer, ids):
    """Host copies of the routed experts' banks, split into gate|up and down."""
    gu, dn = {}, {}
    for e in ids:
        b = model.bank_of(layer, int(e)).cpu().numpy()
        gu[int(e)] = b[:model.gu_bytes]
        dn[int(e)] = b[model.gu_bytes:]
    return gu, dn


@pytest.fixture(scope="module")
def gemma_layers(gemv):
    """Two seeded Gemma-shaped layers (config 1 is layer 0)."""
    return moe_synth.SyntheticMoE(gemv, moe_synth.GEMMA, n_layers=2)


def test_moe_layer_config1_stages(gemv, orc, gemma_layers):
    """Config 1: one Gemma layer, one token. Stage by stage against the oracle,
    each stage teacher-forced on the GPU's own input to that stage."""
    m = gemma_layers
    s = m.shape
    H, I, E, k = s.hidden, s.inter, s.n_experts, s.top_k
    x = m.hidden(0)
    xh = host(x)
    assert np.array_equal(xh, orc.gen_values(orc.tensor_key(1, 0, 0, orc.T_HIDDEN), 0, H, 1.0))
    Wr = host(m.routers[0])
    # router -> top-k
    lg = torch.zeros(E, dtype=torch.float32, device=DEV)
    gemv.gemv_f32_rows_dev(m.routers[0], x, lg, H, E, 1)
    lg_h = host(lg)
    assert np.array_equal(lg_h.view(np.uint32), orc.router_logits(Wr, xh).view(np.uint32))
    ids = torch.zeros(k, dtype=torch.int32, device=DEV)
    wts = torch.zeros(k, dtype=torch.float32, device=DEV)
    gemv.topk_router_dev(lg, None, ids, wts, E, k, 1)
    ie, we = orc.topk_softmax(lg_h, k)
    assert np.array_equal(host(ids), ie) and np.array_equal(host(wts), we)
    # q8(x) -> grouped gate|up
    q8x = torch.zeros(H // 32 * 40, dtype=torch.uint8, device=DEV)
    gemv.quantize_q8(x, 0, q8x, H, 1)
    assert np.array_equal(host(q8x), q8_from_oracle(orc, xh))
    ygu = torch.zeros(k * 2 * I, dtype=torch.float32, device=DEV)
    gemv.gemv_q4r_idx(m.banks[:E * m.expert_bytes], m.expert_bytes, 0, ids, None, k, q8x, 0, ygu, 2 * I, 2 * I, H)
    ygu_h = host(ygu).reshape(k, 2 * I)
    gu_b, dn_b = _oracle_banks(m, 0, ie)
    ref = orc.moe_layer(xh, Wr, gu_b, dn_b, H, I, k, layout=1)
    for p in range(k):
        assert np.max(np.abs(ygu_h[p] - ref["y_gu"][p])) <= 1e-3 * np.linalg.norm(ref["y_gu"][p])
    # GELU*up -> q8, teacher-forced on the GPU's own gate|up
    q8a = torch.zeros(k * I // 32 * 40, dtype=torch.uint8, device=DEV)
    gemv.gelu_mul_q8(ygu, q8a, I, k)
    q8a_h = host(q8a).reshape(k, -1)
    for p in range(k):
        _, de, qe = orc.gelu_mul_q8(ygu_h[p], I)
        b = np.zeros((I // 32, 40), np.uint8)
        b[:, :4] = de.view(np.uint8).reshape(-1, 4)
        b[:, 4:8] = qe.reshape(-1, 32).astype(np.int32).sum(1).astype(np.int32).view(np.uint8).reshape(-1, 4)
        b[:, 8:] = qe.view(np.uint8).reshape(-1, 32)
        assert np.array_equal(q8a_h[p], b.ravel()), p
    # whole layer through moe_layer: ids and weights exact, output within tolerance
    x_out = torch.zeros_like(x)
    ids2 = torch.zeros_like(ids)
    wts2 = torch.zeros_like(wts)
    m.layer(0, x, x_out, ids2, wts2, m.workspace(1))
    assert torch.equal(ids2, ids) and torch.equal(wts2, wts)
    xo = host(x_out)
    d_ref = ref["x_out"] - xh
    assert np.max(np.abs((xo - xh) - d_ref)) <= 1e-3 * np.linalg.norm(d_ref)


def test_moe_layer_batched_two_layers(gemv, orc, gemma_layers):
    """4 tokens through 2 layers; per layer the ids are checked against the oracle
    on the GPU's own layer input (teacher forcing), outputs within tolerance."""
    m = gemma_layers
    s = m.shape
    H, I, E, k, B = s.hidden, s.inter, s.n_experts, s.top_k, 4
    x = torch.stack([m.hidden(t) for t in range(B)])
    ws = m.workspace(B)
    ids = torch.zeros(B * k, dtype=torch.int32, device=DEV)
    wts = torch.zeros(B * k, dtype=torch.float32, device=DEV)
    for l in range(2):
        xin = host(x)
        xo = torch.zeros_like(x)
        m.layer(l, x, xo, ids, wts, ws, n_seqs=B)
        ids_h, wts_h, xo_h = host(ids).reshape(B, k), host(wts).reshape(B, k), host(xo)
        Wr = host(m.routers[l])
        for t in range(B):
            gu_b, dn_b = _oracle_banks(m, l, ids_h[t])
            ref = orc.moe_layer(xin[t], Wr, gu_b, dn_b, H, I, k, layout=1)
            assert np.array_equal(ids_h[t], ref["ids"]) and np.array_equal(wts_h[t], ref["wts"])
            d_ref = ref["x_out"] - xin[t]
            assert np.max(np.abs((xo_h[t] - xin[t]) - d_ref)) <= 1e-3 * np.linalg.norm(d_ref)
        x = xo


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("scaled", [False, True])
def test_gemv_gate_up_act_matches_two_launches(gemv, layout, scaled):
    """ft_hip_gemv_gate_up_act against the grouped gate|up GEMV followed by
    gelu_mul_q8 (on the sums times the scale, in f32), for 5 pairs over 2 q8
    rows (x_div 3) of a small bank in both layouts. The two sum each row in a
    different lane order, so the activations agree to the north-star
    tolerance (max-abs 1e-3 of the L2 norm) and nearly every quant is equal."""
    shape = moe_synth.Shape("small", 384, 160, 24, 3, 1, 9)
    m = moe_synth.SyntheticMoE(gemv, shape, n_layers=1, layout=layout)
    H, I, n = shape.hidden, shape.inter, 5
    x = torch.stack([m.hidden(t) for t in range(2)])
    q8x = torch.zeros(2 * (H // 32) * 40, dtype=torch.uint8, device=DEV)
    gemv.quantize_q8(x, H, q8x, H, 2)
    slots = torch.tensor([3, 17, 3, 0, 23], dtype=torch.int32, device=DEV)
    sc = torch.tensor([0.75, 1.3125], dtype=torch.float32, device=DEV)
    bank = m.banks[:shape.n_experts * m.expert_bytes]
    out = torch.zeros(n * (I // 32) * 40, dtype=torch.uint8, device=DEV)
    gemv.gemv_gate_up_act(bank, m.expert_bytes, slots, n, 3, q8x, H, I, out, layout=layout,
                          in_scale=sc if scaled else None)
    xi = torch.tensor([p // 3 for p in range(n)], dtype=torch.int32, device=DEV)
    ygu = torch.zeros(n * 2 * I, dtype=torch.float32, device=DEV)
    gemv.gemv_grouped_slots(bank, m.expert_bytes, 0, slots, xi, n, q8x, H // 32, ygu, 2 * I, 2 * I, H, layout)
    if scaled:
        ygu = (ygu.view(n, 2 * I) * sc[xi.long()].view(n, 1)).contiguous()
    ref = torch.zeros_like(out)
    gemv.gelu_mul_q8(ygu, ref, I, n)
    d, _, qs = q8_split(host(out), n, I // 32)
    d_r, _, qs_r = q8_split(host(ref), n, I // 32)
    a_out = (d[:, :, None] * qs.reshape(n, I // 32, 32)).ravel()
    a_ref = (d_r[:, :, None] * qs_r.reshape(n, I // 32, 32)).ravel()
    assert np.max(np.abs(a_out - a_ref)) <= 1e-3 * np.linalg.norm(a_ref)
    assert np.mean(qs == qs_r) >= 0.99


@pytest.mark.parametrize("layout,top_k,n_experts,hidden,inter",
                         [(0, 2, 24, 384, 160), (1, 4, 24, 384, 160), (0, 3, 24, 384, 160), (1, 6, 24, 384, 160),
                          (1, 4, 300, 384, 160), (0, 2, 8, 128, 8192), (1, 8, 16, 256, 8192)])
def test_moe_layer_small_shapes(gemv, orc, layout, top_k, n_experts, hidden, inter):
    """Small layers in both weight layouts, 3 tokens: top-k 2, 4 and 8 take the
    down launch that combines the k pairs of a token in one workgroup (16 lanes
    per row for rows of 256+ blocks and k dividing 16, else 8), 3 and 6 (not
    dividing 32) the separate down and combine launches; up to 256 experts
    are routed inside the gate|up launch, 300 by the separate top-k launch.
    Ids and weights exact against the oracle, outputs within tolerance."""
    shape = moe_synth.Shape("small", hidden, inter, n_experts, top_k, 1, 9)
    m = moe_synth.SyntheticMoE(gemv, shape, n_layers=1, layout=layout)
    H, I, k, B = shape.hidden, shape.inter, top_k, 3
    x = torch.stack([m.hidden(t) for t in range(B)])
    ws = m.workspace(B)
    ids = torch.zeros(B * k, dtype=torch.int32, device=DEV)
    wts = torch.zeros(B * k, dtype=torch.float32, device=DEV)
    xo = torch.zeros_like(x)
    m.layer(0, x, xo, ids, wts, ws, n_seqs=B)
    xin, ids_h, wts_h, xo_h = host(x), host(ids).reshape(B, k), host(wts).reshape(B, k), host(xo)
    Wr = host(m.routers[0])
    gu_b, dn_b = _oracle_banks(m, 0, sorted(set(ids_h.ravel().tolist())))
    for t in range(B):
        ref = orc.moe_layer(xin[t], Wr, gu_b, dn_b, H, I, k, layout=layout)
        assert np.array_equal(ids_h[t], ref["ids"]) and np.array_equal(wts_h[t], ref["wts"]), t
        d_ref = ref["x_out"] - xin[t]
        assert np.max(np.abs((xo_h[t] - xin[t]) - d_ref)) <= 1e-3 * np.linalg.norm(d_ref), t


@pytest.mark.parametrize("norm", [False, True])
def test_moe_layer_large_expert(gemv, orc, norm):
    """Config 5's shape (H 4096, 8 experts of I 14336, top-2): one layer, 3 tokens
    (the batched launch), per token ids/weights exact against the oracle and the
    output within tolerance (with and without the input RMS norm); gate|up of
    the long rows within tolerance per pair."""
    m = moe_synth.SyntheticMoE(gemv, moe_synth.LARGE, n_layers=1)
    s = m.shape
    H, I, E, k, B = s.hidden, s.inter, s.n_experts, s.top_k, 3
    x = torch.stack([m.hidden(t) for t in range(B)])
    ws = m.workspace(B)
    ids = torch.zeros(B * k, dtype=torch.int32, device=DEV)
    wts = torch.zeros(B * k, dtype=torch.float32, device=DEV)
    xo = torch.zeros_like(x)
    gemv.set_input_norm(norm)
    try:
        m.layer(0, x, xo, ids, wts, ws, n_seqs=B)
    finally:
        gemv.set_input_norm(0)
    xin, ids_h, wts_h, xo_h = host(x), host(ids).reshape(B, k), host(wts).reshape(B, k), host(xo)
    Wr = host(m.routers[0])
    gu_b, dn_b = _oracle_banks(m, 0, sorted(set(ids_h.ravel().tolist())))
    refs = [orc.moe_layer(xin[t], Wr, gu_b, dn_b, H, I, k, layout=1, threads=8, input_norm=norm) for t in range(B)]
    for t, ref in enumerate(refs):
        assert np.array_equal(ids_h[t], ref["ids"]) and np.array_equal(wts_h[t], ref["wts"]), t
        d_ref = ref["x_out"] - xin[t]
        assert np.max(np.abs((xo_h[t] - xin[t]) - d_ref)) <= 1e-3 * np.linalg.norm(d_ref), t
    # the first pair's gate|up sums on their own
    q8x = torch.zeros(H // 32 * 40, dtype=torch.uint8, device=DEV)
    gemv.quantize_q8(x[0], 0, q8x, H, 1)
    ygu = torch.zeros(2 * I, dtype=torch.float32, device=DEV)
    gemv.gemv_q4r_idx(m.banks, m.expert_bytes, 0, ids[:1], None, 1, q8x, 0, ygu, 2 * I, 2 * I, H)
    ygu_h = host(ygu) * (orc.rms_inv(xin[0]) if norm else np.float32(1))
    assert np.max(np.abs(ygu_h - refs[0]["y_gu"][0])) <= 1e-3 * np.linalg.norm(refs[0]["y_gu"][0])
