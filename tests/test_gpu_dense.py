"""The dense q4r GEMVs around Gemma's expert section (qkv, o_proj, the shared
MLP, lm_head; ft-model/src/lib.rs:1255-1265, :1335-1345, :1371-1396,
:1675-1682) on the same kernel family, at the shapes of moe_synth.DENSE.

The reference runs each as gemv_q4r_idx with a dense index (one "expert",
ft-model/src/lib.rs:1259-1262); here ft_hip_gemv_q4_grouped_slots with
slots = [0]. Per-(row, block) int32 dots bit-exact against the oracle's
integer dots (ft-core/src/q4_0.rs:105-118); outputs within 1e-3 * ||y||_2
and 1e-5 * sum|w*x| per row. The shared MLP runs gate|up -> GELU*up q8 ->
down: the q8 activation bit-exact against the oracle's GELU*up q8 of the
GPU's own gate|up sums, in two launches (gemv + gelu_mul_q8, as the reference)
and in one (ft_hip_gemv_gate_up_act). The f32-input GEMV
(ft_hip_gemv_q4r_f32in: the q8 of its f32 row computed in the launch, and on
a gate|up matrix GELU*up as a second output) equals quantize_q8 + the GEMV bit
for bit, and the shared MLP in its two launches equals the reference's four.
lm_head is checked on a slice of its 262,144 rows (the launch covers all of
them).
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


def q8_dev(gemv, x):
    k = x.numel()
    q8 = torch.zeros(k // 32 * 40, dtype=torch.uint8, device=DEV)
    gemv.quantize_q8(x, 0, q8, k, 1)
    return q8


def check_gemv(gemv, orc, W, rows, k, x, check_rows, lanes=0):
    """y = W q8(x) through the grouped entry point with one entry, `lanes`
    lanes per row (0: automatic); the block dots the GEMV launch itself
    computes (block-dot record) and those of the dump entry point are both
    checked bit-exact. Returns y."""
    q8 = q8_dev(gemv, x)
    slots = torch.zeros(1, dtype=torch.int32, device=DEV)
    y = torch.zeros(rows, dtype=torch.float32, device=DEV)
    nb = k // 32
    rec = torch.full((rows * nb,), -(1 << 30), dtype=torch.int32, device=DEV)
    unused = torch.zeros(1, dtype=torch.int32, device=DEV)
    gemv.set_gemv_lanes(lanes)
    gemv.set_block_dot_record(rec, unused)
    try:
        gemv.gemv_grouped_slots(W, 0, 0, slots, None, 1, q8, 0, y, rows, rows, k)
    finally:
        gemv.set_block_dot_record(None, None)
    y_rec = host(y)
    y.zero_()
    gemv.gemv_grouped_slots(W, 0, 0, slots, None, 1, q8, 0, y, rows, rows, k)
    gemv.set_gemv_lanes(0)
    dots = torch.zeros(check_rows * nb, dtype=torch.int32, device=DEV)
    gemv.block_dots(W, 0, 0, slots, None, 1, q8, 0, dots, check_rows, k)
    y, dots = host(y), host(dots).reshape(check_rows, nb)
    assert np.array_equal(y.view(np.uint32), y_rec.view(np.uint32))  # recording changes no bit of y
    raw = q4r_to_q4_0(host(W[:check_rows * ft_hip.row_bytes(k, ft_hip.LAYOUT_Q4R)]), check_rows, k)
    d8, qs8 = orc.q8_quantize(host(x))
    ref_dots = orc.block_dots(raw, qs8, k)
    assert np.array_equal(dots, ref_dots)
    assert np.array_equal(host(rec).reshape(rows, nb)[:check_rows], ref_dots)
    ref = orc.gemv_q8(raw, check_rows, d8, qs8, k, threads=8)
    assert np.max(np.abs(y[:check_rows] - ref)) <= 1e-3 * np.linalg.norm(ref)
    from test_oracle import unpack_q4
    nib, d4 = unpack_q4(raw, k)
    mag = np.abs((nib.astype(np.float64) - 8) * np.repeat(d4, 32, axis=1)) @ np.abs(
        qs8.astype(np.float64) * np.repeat(d8, 32))
    assert np.all(np.abs(y[:check_rows].astype(np.float64) - ref) <= 1e-5 * mag + 1e-30)
    return y


@pytest.mark.parametrize("lanes", [0, 8, 16, 32, 64])
@pytest.mark.parametrize("name", ["qkv", "o_proj", "shared_gate_up", "shared_down", "lm_head"])
def test_dense_gemv(gemv, orc, name, lanes):
    rows, k = moe_synth.DENSE[name]
    W = moe_synth.dense_weights(gemv, name)
    x = torch.from_numpy(np.random.default_rng(rows + k).standard_normal(k).astype(np.float32)).to(DEV)
    y = check_gemv(gemv, orc, W, rows, k, x, rows if rows <= 8192 else 2048, lanes)
    assert np.all(np.isfinite(y))  # every row of the launch was written


@pytest.mark.parametrize("lanes", [16, 32, 64])
@pytest.mark.parametrize("rows,k", [(1, 32), (7, 64), (33, 2048), (100, 32 * 17), (257, 4096)])
def test_short_gemv_ragged(gemv, orc, rows, k, lanes):
    """The short-launch kernel at ragged row counts (last workgroup partly
    empty) and row lengths (lanes with fewer blocks than others, nb < lanes)."""
    W = torch.empty(rows * ft_hip.row_bytes(k, ft_hip.LAYOUT_Q4R), dtype=torch.uint8, device=DEV)
    gemv.gen_q4_rows(moe_synth.tensor_key(moe_synth.DENSE_CFG, 99, rows, k), 0, rows, k,
                     moe_synth.gen_scale(0.02), W, ft_hip.LAYOUT_Q4R)
    x = torch.from_numpy(np.random.default_rng(rows * k).standard_normal(k).astype(np.float32)).to(DEV)
    check_gemv(gemv, orc, W, rows, k, x, rows, lanes)


def test_gemv_lanes_rejects(gemv):
    with pytest.raises(ft_hip.FtHipError):
        gemv.set_gemv_lanes(12)


def test_shared_mlp_chain(gemv, orc):
    """gate|up (4224 x 2816) -> GELU*up q8 (2112) -> down (2816 x 2112)."""
    (gu_rows, H), (_, I) = moe_synth.DENSE["shared_gate_up"], moe_synth.DENSE["shared_down"]
    assert gu_rows == 2 * I
    Wgu = moe_synth.dense_weights(gemv, "shared_gate_up")
    Wdn = moe_synth.dense_weights(gemv, "shared_down")
    x = torch.from_numpy(np.random.default_rng(11).standard_normal(H).astype(np.float32)).to(DEV)
    ygu = check_gemv(gemv, orc, Wgu, gu_rows, H, x, gu_rows)
    # GELU*up q8 of the GPU's own gate|up sums: bit-exact (two launches, as the reference)
    q8a = torch.zeros(I // 32 * 40, dtype=torch.uint8, device=DEV)
    gemv.gelu_mul_q8(torch.from_numpy(ygu).to(DEV), q8a, I, 1)
    blk = host(q8a).reshape(I // 32, 40)
    _, ad, aq = orc.gelu_mul_q8(ygu, I)
    assert np.array_equal(blk[:, :4].copy().view(np.float32)[:, 0].view(np.uint32), ad.view(np.uint32))
    assert np.array_equal(blk[:, 8:].copy().view(np.int8).ravel(), aq)
    # one launch: gate|up GEMV with GELU*up and q8 (ft_hip_gemv_gate_up_act). Its f32 gate|up sums
    # run in another lane order than the GEMV above, so its q8 may differ from the two-launch one by
    # the rounding of those sums only: per block d within 1e-5 relative and quants within 1. Teacher-
    # forced on its own sums (the layer record) it is bit-exact: GELU*up q8 of those sums equals the
    # launch's act q8, and its gate|up block dots equal the oracle's
    q8b = torch.zeros_like(q8a)
    slots = torch.zeros(1, dtype=torch.int32, device=DEV)
    gsum = torch.full((1, gu_rows), float("nan"), dtype=torch.float32, device=DEV)
    gdots = torch.full((1, gu_rows, H // 32), -(2 ** 31), dtype=torch.int32, device=DEV)
    gemv.set_layer_record(gu=gsum, gu_dots=gdots)
    try:
        gemv.gemv_gate_up_act(Wgu, Wgu.numel(), slots, 1, 1, q8_dev(gemv, x), H, I, q8b)
        G, GD = host(gsum)[0], host(gdots)[0]
    finally:
        gemv.set_layer_record()
    b1 = host(q8b).reshape(I // 32, 40)
    d1 = b1[:, :4].copy().view(np.float32)[:, 0]
    assert np.all(np.abs(d1 - ad) <= 1e-5 * np.abs(ad))
    assert np.max(np.abs(b1[:, 8:].copy().view(np.int8).astype(int).ravel() - aq.astype(int))) <= 1
    _, fd, fq = orc.gelu_mul_q8(G, I)
    assert np.array_equal(d1.view(np.uint32), fd.view(np.uint32))
    assert np.array_equal(b1[:, 8:].copy().view(np.int8).ravel(), fq)
    _, xq8 = orc.q8_quantize(host(x))
    assert np.array_equal(GD, orc.block_dots(q4r_to_q4_0(host(Wgu), gu_rows, H), xq8, H))
    # down from the act q8, through the grouped GEMV: dots bit-exact, f32 within tolerance
    nb = I // 32
    y = torch.zeros(H, dtype=torch.float32, device=DEV)
    gemv.gemv_grouped_slots(Wdn, 0, 0, slots, None, 1, q8a, 0, y, H, H, I)
    dots = torch.zeros(H * nb, dtype=torch.int32, device=DEV)
    gemv.block_dots(Wdn, 0, 0, slots, None, 1, q8a, 0, dots, H, I)
    raw = q4r_to_q4_0(host(Wdn), H, I)
    assert np.array_equal(host(dots).reshape(H, nb), orc.block_dots(raw, aq, I))
    ref = orc.gemv_q8(raw, H, ad, aq, I, threads=8)
    assert np.max(np.abs(host(y) - ref)) <= 1e-3 * np.linalg.norm(ref)


def _q4r(gemv, rows, k, seed):
    W = torch.empty(rows * ft_hip.row_bytes(k, ft_hip.LAYOUT_Q4R), dtype=torch.uint8, device=DEV)
    gemv.gen_q4_rows(moe_synth.tensor_key(moe_synth.DENSE_CFG, seed, rows, k), 0, rows, k,
                     moe_synth.gen_scale(0.02), W, ft_hip.LAYOUT_Q4R)
    return W


@pytest.mark.parametrize("lanes", [0, 16, 32, 64])
@pytest.mark.parametrize("act", [False, True])
@pytest.mark.parametrize("rows,k", [(4224, 2816), (2816, 2112), (8, 64), (34, 2048), (258, 4096)])
def test_gemv_q4r_f32in(gemv, orc, rows, k, act, lanes):
    """ft_hip_gemv_q4r_f32in: the q8 of the f32 row x computed in the launch. y
    equals the reference's two calls (quantize_q8, then the GEMV at the same lane
    count) bit for bit; the launch's own block dots (block-dot record) equal the
    oracle's integer dots against the oracle's q8 of x; with act (the matrix as
    gate|up rows), act equals the oracle's GELU*up of the launch's own sums, and
    gelu_mul_q8 of those sums quantizes exactly what q8(act) gives."""
    W = _q4r(gemv, rows, k, 50 + rows)
    xin = np.random.default_rng(rows * 7 + k).standard_normal(k).astype(np.float32)
    x = torch.from_numpy(xin).to(DEV)
    q8 = q8_dev(gemv, x)
    slots = torch.zeros(1, dtype=torch.int32, device=DEV)
    y2 = torch.zeros(rows, dtype=torch.float32, device=DEV)
    y1 = torch.full((rows,), float("nan"), dtype=torch.float32, device=DEV)
    a1 = torch.full((rows // 2,), float("nan"), dtype=torch.float32, device=DEV) if act else None
    nb = k // 32
    rec = torch.full((rows * nb,), -(1 << 30), dtype=torch.int32, device=DEV)
    unused = torch.zeros(1, dtype=torch.int32, device=DEV)
    try:
        # the same lanes per row: with act (automatic) 32 where the row fits
        gemv.set_gemv_lanes(lanes or (32 if act and nb <= 256 else 0))
        gemv.gemv_grouped_slots(W, 0, 0, slots, None, 1, q8, 0, y2, rows, rows, k)
        gemv.set_gemv_lanes(lanes)
        gemv.set_block_dot_record(rec, unused)
        try:
            gemv.gemv_q4r_f32in(W, x, y1, a1, rows, k)
        finally:
            gemv.set_block_dot_record(None, None)
        y3 = torch.full_like(y1, float("nan"))
        a3 = torch.full_like(a1, float("nan")) if act else None
        gemv.gemv_q4r_f32in(W, x, y3, a3, rows, k)  # without the record: the same bits
    finally:
        gemv.set_gemv_lanes(0)
    Y = host(y2)
    assert np.array_equal(host(y1).view(np.uint32), Y.view(np.uint32))
    assert np.array_equal(host(y3).view(np.uint32), Y.view(np.uint32))
    _, qs8 = orc.q8_quantize(xin)
    raw = q4r_to_q4_0(host(W), rows, k)
    assert np.array_equal(host(rec).reshape(rows, nb), orc.block_dots(raw, qs8, k))
    if act:
        A = host(a1)
        assert np.array_equal(host(a3).view(np.uint32), A.view(np.uint32))
        if rows // 2 % 32 == 0:  # whole q8 blocks: the oracle's GELU*up (and its q8) of the launch's sums
            ref_a, ad, aq = orc.gelu_mul_q8(Y, rows // 2)
            assert np.array_equal(A.view(np.uint32), ref_a.view(np.uint32))
            d8, q8a = orc.q8_quantize(A)
            assert np.array_equal(d8.view(np.uint32), ad.view(np.uint32)) and np.array_equal(q8a, aq)


def test_gemv_q4r_f32in_rejects(gemv):
    W = _q4r(gemv, 4, 64, 1)
    x = torch.zeros(128, dtype=torch.float32, device=DEV)
    y = torch.zeros(4, dtype=torch.float32, device=DEV)
    a = torch.zeros(2, dtype=torch.float32, device=DEV)
    for args in [(W, x, y, None, 4, 48), (W, x, y, None, 4, 32 * 513), (W, x[1:], y, None, 4, 64),
                 (W, x, y, None, -1, 64), (W, x, y, a, 3, 64), (W, x, None, None, 4, 64)]:
        with pytest.raises(ft_hip.FtHipError):
            gemv.gemv_q4r_f32in(*args)


def test_shared_mlp_two_launches(gemv, orc):
    """The shared MLP from its f32 input in two launches (gate|up from x with act,
    down from act, each with its q8 in the launch) gives the bits of the
    reference's four (quantize_q8, gate|up GEMV, gelu_mul_q8, down GEMV) with
    the gate|up GEMV at the lanes per row of the launch with act."""
    (gu_rows, H), (_, I) = moe_synth.DENSE["shared_gate_up"], moe_synth.DENSE["shared_down"]
    Wgu = moe_synth.dense_weights(gemv, "shared_gate_up")
    Wdn = moe_synth.dense_weights(gemv, "shared_down")
    x = torch.from_numpy(np.random.default_rng(12).standard_normal(H).astype(np.float32)).to(DEV)
    slots = torch.zeros(1, dtype=torch.int32, device=DEV)
    ygu, y4 = torch.zeros(gu_rows, dtype=torch.float32, device=DEV), torch.zeros(H, dtype=torch.float32, device=DEV)
    q8a = torch.zeros(I // 32 * 40, dtype=torch.uint8, device=DEV)
    gemv.set_gemv_lanes(32)  # the lanes per row the gate|up launch with act takes
    try:
        gemv.gemv_grouped_slots(Wgu, 0, 0, slots, None, 1, q8_dev(gemv, x), 0, ygu, gu_rows, gu_rows, H)
    finally:
        gemv.set_gemv_lanes(0)
    gemv.gelu_mul_q8(ygu, q8a, I, 1)
    gemv.gemv_grouped_slots(Wdn, 0, 0, slots, None, 1, q8a, 0, y4, H, H, I)
    gu2, y2 = torch.zeros_like(ygu), torch.zeros_like(y4)
    act = torch.zeros(I, dtype=torch.float32, device=DEV)
    gemv.gemv_q4r_f32in(Wgu, x, gu2, act, gu_rows, H)
    gemv.gemv_q4r_f32in(Wdn, act, y2, None, H, I)
    assert np.array_equal(host(gu2).view(np.uint32), host(ygu).view(np.uint32))
    assert np.array_equal(host(y2).view(np.uint32), host(y4).view(np.uint32))
    assert np.all(np.isfinite(host(y2)))
