"""GPU parity tests of the fused whole-stack kernel (ft_hip_moe_stack_fused).

Per layer, each stage is checked against the CPU oracle on the kernel's own
input to that stage (teacher forcing, from the kernel's debug record):
top-k ids and weights and the GELU*up q8 blocks bit-exact; gate|up sums and
the layer output within max|d| <= 1e-3 * ||ref||_2. The repack to the fused
layout is checked byte for byte against the oracle's q4_0 rows. The input
RMS norm (ft_hip_set_input_norm) is covered the same way: its scale enters
the logits (ids and weights still bit-exact) and the gate|up sums.
"""
import contextlib

import numpy as np
import pytest
import torch

import ft_hip
import moe_synth

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def unpack_fused_expert(buf, H, I):
    """Invert the fused layout on the host -> (gate|up q4_0 rows [2I, H*18/32], down q4_0 rows [H, I*18/32])."""
    nb, nbj = H // 32, I // 32
    gu = np.zeros((2 * I, nb, 18), np.uint8)
    tile = nb * 1152
    for jb in range(nbj):
        T = buf[jb * tile:(jb + 1) * tile]
        sc = T[:nb * 128].reshape(nb, 64, 2)
        qs = T[nb * 128:].reshape(nb, 64, 16)
        rows = np.r_[np.arange(32) + 32 * jb, I + 32 * jb + np.arange(32)]
        gu[rows, :, :2] = sc.transpose(1, 0, 2)
        gu[rows, :, 2:] = qs.transpose(1, 0, 2)
    dn = np.zeros((H, nbj, 18), np.uint8)
    base = nbj * tile
    dt = nbj * 288
    for jt in range(H // 16):
        T = buf[base + jt * dt: base + (jt + 1) * dt]
        sc = T[:nbj * 32].reshape(nbj, 16, 2)
        qs = T[nbj * 32:].reshape(nbj, 16, 16)
        dn[jt * 16:(jt + 1) * 16, :, :2] = sc.transpose(1, 0, 2)
        dn[jt * 16:(jt + 1) * 16, :, 2:] = qs.transpose(1, 0, 2)
    return gu.reshape(2 * I, -1), dn.reshape(H, -1)


@pytest.fixture(scope="module")
def stack(gemv):
    m = moe_synth.SyntheticMoE(gemv, moe_synth.GEMMA, n_layers=4)
    return moe_synth.FusedStack(m)


def test_fused_pack_is_lossless(gemv, orc, stack):
    m = stack.m
    H, I = m.shape.hidden, m.shape.inter
    eb = stack.expert_bytes
    assert eb == moe_synth.algorithmic_expert_bytes(m.shape)  # exactly q4_0's byte count
    for l, e in [(0, 0), (1, 77), (3, 127)]:
        buf = host(stack.banks[(l * m.shape.n_experts + e) * eb:(l * m.shape.n_experts + e + 1) * eb])
        gu, dn = unpack_fused_expert(buf, H, I)
        assert np.array_equal(gu, orc.gen_q4_rows(orc.tensor_key(1, l, e, orc.T_GU), 0, 2 * I, H, 0.02))
        assert np.array_equal(dn, orc.gen_q4_rows(orc.tensor_key(1, l, e, orc.T_DN), 0, H, I, 0.02))
    r = host(stack.routers[2]).reshape(H // 16, m.shape.n_experts, 16)
    ref = host(m.routers[2])
    assert np.array_equal(r.transpose(1, 0, 2).reshape(m.shape.n_experts, H), ref)


@contextlib.contextmanager
def input_norm(gemv, on):
    gemv.set_input_norm(on)
    try:
        yield
    finally:
        gemv.set_input_norm(0)


def route(orc, Wr, x, bias, K, norm):
    """The oracle's routing of one token: R-order logits, times the input RMS
    norm's scale when on, + bias; top-k and softmax."""
    lg = orc.router_logits(Wr, x)
    if norm:
        lg = (lg * orc.rms_inv(x)).astype(np.float32)
    if bias is not None:
        lg = (lg + bias).astype(np.float32)
    return orc.topk_softmax(lg, K)


def _run_debug(stack, token, norm=False):
    m = stack.m
    s = m.shape
    H, I, E, K, L = s.hidden, s.inter, s.n_experts, s.top_k, m.L
    x = m.hidden(token)
    out = torch.zeros_like(x)
    ids = torch.zeros(L * K, dtype=torch.int32, device=DEV)
    wts = torch.zeros(L * K, dtype=torch.float32, device=DEV)
    dbg_gu = torch.zeros(L * K * 2 * I, dtype=torch.float32, device=DEV)
    dbg_act = torch.zeros(L * K * (I // 32) * 40, dtype=torch.uint8, device=DEV)
    dbg_x = torch.zeros((L + 1) * H, dtype=torch.float32, device=DEV)
    with input_norm(m.g, norm):
        stack.run(x, out, ids, wts, dbg_gu, dbg_act, dbg_x)
    stack.check()
    return dict(x=host(x), out=host(out), ids=host(ids).reshape(L, K), wts=host(wts).reshape(L, K),
                gu=host(dbg_gu).reshape(L, K, 2 * I), act=host(dbg_act).reshape(L, K, I // 32, 40),
                xs=host(dbg_x).reshape(L + 1, H))


@pytest.fixture(scope="module")
def zstack(gemv):
    """Zipf(1.1)-skewed routing (BASELINE config 3's router bias)."""
    m = moe_synth.SyntheticMoE(gemv, moe_synth.GEMMA, n_layers=4, zipf_s=1.1)
    return moe_synth.FusedStack(m)


def test_fused_stack_stages_teacher_forced(gemv, orc, stack):
    _check_teacher_forced(orc, stack, 0)


def test_fused_zipf_stages_teacher_forced(gemv, orc, zstack):
    _check_teacher_forced(orc, zstack, 1)


def test_fused_norm_stages_teacher_forced(gemv, orc, stack):
    _check_teacher_forced(orc, stack, 4, norm=True)


def test_fused_zipf_norm_stages_teacher_forced(gemv, orc, zstack):
    _check_teacher_forced(orc, zstack, 5, norm=True)


def test_fused_norm_prefetch_does_not_change_results(gemv, zstack):
    with input_norm(gemv, 1):
        a = _run_plain(zstack, 6, 1)
        b = _run_plain(zstack, 6, 0)
    for u, v in zip(a, b):
        assert np.array_equal(u.view(np.uint32), v.view(np.uint32))


def test_fused_zipf_prefetch_does_not_change_results(gemv, zstack):
    a = _run_plain(zstack, 2, 1)
    b = _run_plain(zstack, 2, 0)
    for u, v in zip(a, b):
        assert np.array_equal(u.view(np.uint32), v.view(np.uint32))


def _table_record(stack, l, e):
    """Record (l, e) of the refined-prediction table -> (values [E, I] dequantized, scales [E, I/32])."""
    s = stack.m.shape
    E, nbj = s.n_experts, s.inter // 32
    rec = E * nbj * 36
    b = host(stack.pred[(l * E + e) * rec:(l * E + e + 1) * rec])
    q = b[:E * nbj * 32].view(np.int8).reshape(E, nbj, 32).astype(np.float64)
    d = b[E * nbj * 32:].view(np.float32).reshape(E, nbj)
    return (q * d[:, :, None].astype(np.float64)).reshape(E, -1), d


@pytest.mark.parametrize("l,e", [(0, 0), (0, 77), (2, 127)])
def test_fused_predictor_table(gemv, stack, l, e):
    """Record (l, e) of the refined-prediction table is R_{l+1} D_{l,e}
    quantized per 32 columns: against the f64 product of the model's router
    and the expert's down rows (read back from the fused banks and
    dequantized independently), each value within half a quantization step
    (and the rounding of v/d) plus the f32 sum's error bound n*u*sum|r*d|,
    and each block's scale within that bound of its amax / 127."""
    from test_oracle import unpack_q4
    m = stack.m
    s = m.shape
    H, I, E = s.hidden, s.inter, s.n_experts
    eb = stack.expert_bytes
    _, dn = unpack_fused_expert(host(stack.banks[(l * E + e) * eb:(l * E + e + 1) * eb]), H, I)
    nib, d4 = unpack_q4(dn, I)
    D = (nib.astype(np.float64) - 8) * np.repeat(d4.astype(np.float64), 32, axis=1)  # [H, I]
    R = host(m.routers[l + 1]).astype(np.float64)                                      # [E, H]
    ref, mag = R @ D, np.abs(R) @ np.abs(D)
    gam = H * 2.0 ** -24
    got, d = _table_record(stack, l, e)
    step = np.repeat(d.astype(np.float64), 32, axis=1)
    assert np.all(np.abs(got - ref) <= 0.5 * step * (1 + 1e-5) + gam * mag)
    amax = np.abs(ref).reshape(E, I // 32, 32).max(axis=2)
    bmag = mag.reshape(E, I // 32, 32).max(axis=2)
    assert np.all(np.abs(d - amax / 127) <= gam * bmag / 127 + 1e-7 * amax)
    assert np.all(d > 0)


def _run_pred(stack, token, pred, prefetch=1):
    saved = stack.pred
    stack.pred = saved if pred else None
    try:
        return _run_plain(stack, token, prefetch)
    finally:
        stack.pred = saved


@pytest.mark.parametrize("which,norm", [("uniform", False), ("zipf", True)])
def test_fused_predictor_does_not_change_results(gemv, stack, zstack, which, norm):
    """The refined prediction only decides which unit group holds which
    expert: outputs, ids and weights are bit-identical with it, with the
    early routing's prediction alone, and with no prefetch."""
    st = stack if which == "uniform" else zstack
    with input_norm(gemv, norm):
        for token in (31, 32):
            a = _run_pred(st, token, True)
            b = _run_pred(st, token, False)
            c = _run_pred(st, token, False, prefetch=0)
            for u, v, w in zip(a, b, c):
                assert np.array_equal(u.view(np.uint32), v.view(np.uint32))
                assert np.array_equal(u.view(np.uint32), w.view(np.uint32))


def test_fused_predictor_layer_mismatch_rejected(gemv, stack):
    """A table built for fewer layers than the launch runs is refused before
    the launch (FT_HIP_E_SHAPE); building one for 2 layers of the same banks
    works, and clearing it (None) returns to the early routing."""
    m = stack.m
    s = m.shape
    small = torch.empty(gemv.fused_predictor_bytes(s.hidden, s.inter, s.n_experts, 2), dtype=torch.uint8,
                        device=DEV)
    gemv.fused_build_predictor(stack.banks, stack.routers, s.hidden, s.inter, s.n_experts, 2, small)
    x = m.hidden(0)
    gemv.fused_set_predictor(small, 2)
    try:
        with pytest.raises(ft_hip.FtHipError) as ei:
            gemv.moe_stack_fused(x, torch.zeros_like(x), s.hidden, s.inter, s.n_experts, s.top_k, m.L, stack.banks,
                                 stack.routers, m.bias, None, None, None, stack.ws)
        assert ei.value.code == ft_hip.E_SHAPE
        with pytest.raises(ft_hip.FtHipError):
            gemv.fused_set_predictor(small[1:], 2)  # not 16-byte aligned
    finally:
        gemv.fused_set_predictor(None)
    stack.check()


def _misses(stack, token, pred, norm=False):
    """Held experts not routed, summed over unit groups and the predicted
    layers 1..L-1, from the debug trace: expert unit u (tile 0, workgroup u)
    records per layer whether its held expert was routed (slot 10 of row
    l+1; layer 0 holds nothing)."""
    m = stack.m
    nw = stack.n_workgroups()
    tr = torch.zeros(nw * (m.L + 1) * 32, dtype=torch.int64, device=DEV)
    x = m.hidden(token)
    saved = stack.pred
    stack.pred = saved if pred else None
    try:
        with input_norm(m.g, norm):
            stack.run(x, torch.zeros_like(x), trace=tr)
        stack.check()
    finally:
        stack.pred = saved
    t = host(tr).reshape(nw, m.L + 1, 32)
    return int(t[:m.shape.top_k, 2:, 10].sum())


@pytest.mark.parametrize("which,norm", [("uniform", False), ("zipf", True)])
def test_fused_predictor_removes_misses(gemv, stack, zstack, which, norm):
    """With the table nearly every held expert is routed: at most 3.5 % of
    the 8 tokens x 3 predicted layers x 8 unit groups miss (measured: 1 and
    4 of 192; the early routing alone misses 10-20 of them). Under the input
    norm the table's logits take x_l's norm scale for x_{l+1}'s, which with
    the Zipf bias decides a few close ranks."""
    st = stack if which == "uniform" else zstack
    n = 8 * (st.m.L - 1) * st.m.shape.top_k
    with_t = sum(_misses(st, 40 + i, True, norm) for i in range(8))
    without = sum(_misses(st, 40 + i, False, norm) for i in range(8))
    print(f"misses with the table {with_t}/{n}, early routing alone {without}/{n}")
    assert with_t <= 0.035 * n


def _weights_diag(orc, Wr, x, bias, K, got, want):
    """Which scale of the logits reproduces the kernel's weights (a failure report)."""
    lg = orc.router_logits(Wr, x)
    ir = orc.rms_inv(x)
    hits = []
    for k in range(-4, 5):
        c = ir
        for _ in range(abs(k)):
            c = np.nextafter(c, np.float32(np.inf if k > 0 else -np.inf), dtype=np.float32)
        v = (lg * c).astype(np.float32)
        if bias is not None:
            v = (v + bias).astype(np.float32)
        if np.array_equal(orc.topk_softmax(v, K)[1].view(np.uint32), got.view(np.uint32)):
            hits.append(k)
    return f"got {got.tolist()} want {want.tolist()} inv_r {float(ir)!r}; ulp offsets of inv_r that match: {hits}"


def _check_teacher_forced(orc, stack, token, norm=False):
    m = stack.m
    s = m.shape
    H, I, E, K, L = s.hidden, s.inter, s.n_experts, s.top_k, m.L
    r = _run_debug(stack, token, norm)
    assert np.array_equal(r["xs"][0], r["x"])
    assert np.array_equal(r["xs"][L], r["out"])
    for l in range(L):
        xl = r["xs"][l]
        Wr = host(m.routers[l])
        bias = None if m.bias is None else host(m.bias[l])
        ids, wts = route(orc, Wr, xl, bias, K, norm)
        assert np.array_equal(r["ids"][l], ids), f"layer {l}"
        assert np.array_equal(r["wts"][l].view(np.uint32), wts.view(np.uint32)), \
            f"layer {l}: " + _weights_diag(orc, Wr, xl, bias, K, r["wts"][l], wts)
        gu_b, dn_b = {}, {}
        for e in ids:
            b = host(m.bank_of(l, int(e)))
            gu_b[int(e)], dn_b[int(e)] = b[:m.gu_bytes], b[m.gu_bytes:]
        ref = orc.moe_layer(xl, Wr, gu_b, dn_b, H, I, K, bias=bias, layout=1, input_norm=norm)
        assert np.array_equal(ref["ids"], ids) and np.array_equal(ref["wts"].view(np.uint32), wts.view(np.uint32))
        out_ref = xl.astype(np.float64).copy()
        for p in range(K):
            yg = ref["y_gu"][p]
            assert np.max(np.abs(r["gu"][l, p] - yg)) <= 1e-3 * np.linalg.norm(yg), (l, p)
            # GELU*up -> q8 on the kernel's own gate|up sums: bit-exact
            _, d, q = orc.gelu_mul_q8(r["gu"][l, p], I)
            blk = r["act"][l, p]
            assert np.array_equal(blk[:, :4].copy().view(np.float32)[:, 0].view(np.uint32), d.view(np.uint32))
            assert np.array_equal(blk[:, 8:].copy().view(np.int8).ravel(), q)
            assert np.array_equal(blk[:, 4:8].copy().view(np.int32)[:, 0], q.reshape(-1, 32).astype(np.int32).sum(1))
            # down projection from the kernel's own q8 activations
            ydn = orc.gemv_q8(dn_b[int(ids[p])], H, d, q, I, layout=1)
            out_ref += np.float64(wts[p]) * ydn.astype(np.float64)
        dx = r["xs"][l + 1].astype(np.float64) - xl
        dref = out_ref - xl
        assert np.max(np.abs(dx - dref)) <= 1e-3 * np.linalg.norm(dref), f"layer {l}"


@pytest.mark.parametrize("norm", [False, True])
def test_fused_matches_launch_by_launch(gemv, stack, norm):
    """Per layer, the launch-by-launch path on the fused kernel's layer input
    picks the same experts with the same weights; outputs agree to 1e-3."""
    m = stack.m
    s = m.shape
    r = _run_debug(stack, 3, norm)
    ws = m.workspace(1)
    for l in range(m.L):
        x = torch.from_numpy(r["xs"][l]).to(DEV)
        xo = torch.zeros_like(x)
        ids = torch.zeros(s.top_k, dtype=torch.int32, device=DEV)
        wts = torch.zeros(s.top_k, dtype=torch.float32, device=DEV)
        with input_norm(gemv, norm):
            m.layer(l, x, xo, ids, wts, ws)
        assert np.array_equal(host(ids), r["ids"][l])
        assert np.array_equal(host(wts), r["wts"][l])
        d_ref = host(xo) - r["xs"][l]
        d = r["xs"][l + 1] - r["xs"][l]
        assert np.max(np.abs(d - d_ref)) <= 1e-3 * np.linalg.norm(d_ref)


def test_fused_repeatable_bit_for_bit(gemv, stack):
    """Fixed summation orders and no atomics: repeated launches (advancing
    epochs on one workspace) give identical bits."""
    m = stack.m
    x = m.hidden(5)
    outs = []
    for _ in range(3):
        o = torch.zeros_like(x)
        ids = torch.zeros(m.L * m.shape.top_k, dtype=torch.int32, device=DEV)
        stack.run(x, o, ids)
        outs.append((host(o), host(ids)))
    stack.check()
    for o, i in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0][0].view(np.uint32))
        assert np.array_equal(i, outs[0][1])


def _run_plain(stack, token, prefetch):
    m = stack.m
    x = m.hidden(token)
    o = torch.zeros_like(x)
    ids = torch.zeros(m.L * m.shape.top_k, dtype=torch.int32, device=DEV)
    wts = torch.zeros(m.L * m.shape.top_k, dtype=torch.float32, device=DEV)
    stack.m.g.fused_set_prefetch(prefetch)
    try:
        stack.run(x, o, ids, wts)
        stack.check()
    finally:
        stack.m.g.fused_set_prefetch(1)
    return host(o), host(ids), host(wts)


@pytest.mark.parametrize("token", [11, 12, 13])
def test_fused_prefetch_does_not_change_results(gemv, stack, token):
    """Prediction only decides which unit group holds which expert and what
    is streamed ahead: outputs, ids and weights are bit-identical with and
    without it (hits and misses both occur over these tokens)."""
    a = _run_plain(stack, token, 1)
    b = _run_plain(stack, token, 0)
    for u, v in zip(a, b):
        assert np.array_equal(u.view(np.uint32), v.view(np.uint32))


@pytest.mark.parametrize("n_layers", [1, 2, 3])
def test_fused_short_stacks(gemv, orc, n_layers):
    """Stacks too short to predict (1 layer), predicting one layer ahead only
    (2), and an odd layer count (3): same results as the launch-by-launch
    layers on the fused kernel's own layer inputs."""
    m = moe_synth.SyntheticMoE(gemv, moe_synth.GEMMA, n_layers=n_layers)
    st = moe_synth.FusedStack(m)
    r = _run_debug(st, 21 + n_layers)
    s = m.shape
    ws = m.workspace(1)
    for l in range(m.L):
        x = torch.from_numpy(r["xs"][l]).to(DEV)
        xo = torch.zeros_like(x)
        ids = torch.zeros(s.top_k, dtype=torch.int32, device=DEV)
        wts = torch.zeros(s.top_k, dtype=torch.float32, device=DEV)
        m.layer(l, x, xo, ids, wts, ws)
        assert np.array_equal(host(ids), r["ids"][l])
        assert np.array_equal(host(wts), r["wts"][l])
        d_ref = host(xo) - r["xs"][l]
        d = r["xs"][l + 1] - r["xs"][l]
        assert np.max(np.abs(d - d_ref)) <= 1e-3 * np.linalg.norm(d_ref)
    assert np.array_equal(r["xs"][m.L], r["out"])


def test_fused_rejects_bad_shapes(gemv, stack):
    m = stack.m
    s = m.shape
    x = m.hidden(0)
    with pytest.raises(ft_hip.FtHipError) as ei:
        gemv.moe_stack_fused(x, x, 2880, s.inter, s.n_experts, s.top_k, m.L, stack.banks, stack.routers, None,
                             None, None, None, stack.ws)
    assert ei.value.code == ft_hip.E_SHAPE
    small = torch.zeros(64, dtype=torch.uint8, device=DEV)
    with pytest.raises(ft_hip.FtHipError) as ei:
        gemv.moe_stack_fused(x, x, s.hidden, s.inter, s.n_experts, s.top_k, m.L, stack.banks, stack.routers,
                             None, None, None, None, small)
    assert ei.value.code == ft_hip.E_SHAPE


def test_fused_abort_poisons_workspace_until_init(gemv, stack):
    """A wait that gives up (forced from the host with a spin limit of 0, so
    the first incomplete poll aborts; every workgroup still exits normally)
    records the abort and marks the outputs: x_out all NaN, ids -1, weights
    NaN. The workspace then stays poisoned -- later launches compute nothing
    and mark their outputs the same way -- until ft_hip_fused_workspace_init,
    after which results match a clean run bit for bit."""
    m = stack.m
    K, L = m.shape.top_k, m.L
    x = m.hidden(7)
    ref = torch.zeros_like(x)
    stack.run(x, ref)
    stack.check()

    def marked(o, ids, wts):
        return (bool(torch.all(torch.isnan(o))) and bool(torch.all(ids == -1))
                and bool(torch.all(torch.isnan(wts))))

    gemv.fused_set_spin_limit(0)
    try:
        o = torch.full_like(x, 7.0)
        ids = torch.zeros(L * K, dtype=torch.int32, device=DEV)
        wts = torch.zeros(L * K, dtype=torch.float32, device=DEV)
        stack.run(x, o, ids, wts)
        torch.cuda.synchronize()
    finally:
        gemv.fused_set_spin_limit(1 << 21)
    with pytest.raises(ft_hip.FtHipError) as ei:
        stack.check()
    assert ei.value.code == ft_hip.E_TIMEOUT
    assert marked(o, ids, wts)
    o = torch.full_like(x, 7.0)
    ids = torch.zeros(L * K, dtype=torch.int32, device=DEV)
    wts = torch.zeros(L * K, dtype=torch.float32, device=DEV)
    stack.run(x, o, ids, wts)  # poisoned workspace: nothing computed, outputs marked
    torch.cuda.synchronize()
    assert marked(o, ids, wts)
    with pytest.raises(ft_hip.FtHipError):
        stack.check()
    stack.reset()
    o = torch.zeros_like(x)
    stack.run(x, o)
    stack.check()
    assert np.array_equal(host(o).view(np.uint32), host(ref).view(np.uint32))


@pytest.mark.parametrize("which,norm", [("uniform", False), ("uniform", True), ("zipf", False), ("zipf", True)])
def test_fused_plain_build_matches_debug_build(gemv, orc, stack, zstack, which, norm):
    """The build bench.py times (no debug pointers: the <..., false>
    instantiation) against the debug build whose stages the teacher-forced
    tests check: x_out, ids and weights bit-identical on the same tokens; and
    the plain run's per-layer routing equals the oracle's on the debug run's
    layer inputs."""
    st = stack if which == "uniform" else zstack
    m = st.m
    K, L = m.shape.top_k, m.L
    for token in (30, 31, 32):
        r = _run_debug(st, token, norm)
        x = m.hidden(token)
        o = torch.zeros_like(x)
        ids = torch.zeros(L * K, dtype=torch.int32, device=DEV)
        wts = torch.zeros(L * K, dtype=torch.float32, device=DEV)
        with input_norm(gemv, norm):
            st.run(x, o, ids, wts)
        st.check()
        o, ids, wts = host(o), host(ids).reshape(L, K), host(wts).reshape(L, K)
        assert np.array_equal(o.view(np.uint32), r["out"].view(np.uint32)), token
        assert np.array_equal(ids, r["ids"]), token
        assert np.array_equal(wts.view(np.uint32), r["wts"].view(np.uint32)), token
        for l in range(L):
            bias = None if m.bias is None else host(m.bias[l])
            ie, we = route(orc, host(m.routers[l]), r["xs"][l], bias, K, norm)
            assert np.array_equal(ids[l], ie), (token, l)
            assert np.array_equal(wts[l].view(np.uint32), we.view(np.uint32)), (token, l)


def _epoch(ws):
    torch.cuda.synchronize()
    return int(ws[:4].view(torch.int32).cpu().numpy()[0]) & 0xFFFFFFFF


def test_fused_epoch_guard_reinitialises_before_wrap(gemv, stack):
    """Launches across the 2^32 limit of the hand-over tags: with the epoch
    set so that two launches fit below 2^32, the third is preceded by a
    re-initialisation of the workspace (epoch back to 1), and every launch
    gives the first one's bits."""
    m = stack.m
    K, L = m.shape.top_k, m.L
    step = 4 * (L + 1)
    x = m.hidden(13)
    stack.reset()
    ref, ref_ids = torch.zeros_like(x), torch.zeros(L * K, dtype=torch.int32, device=DEV)
    stack.run(x, ref, ref_ids)
    stack.check()
    start = 2 ** 32 - 1 - 2 * step
    gemv.fused_workspace_set_epoch(stack.ws, start)
    assert _epoch(stack.ws) == start
    seen = []
    for i in range(4):
        o, ids = torch.zeros_like(x), torch.zeros(L * K, dtype=torch.int32, device=DEV)
        stack.run(x, o, ids)
        stack.check()
        seen.append(_epoch(stack.ws))
        assert np.array_equal(host(o).view(np.uint32), host(ref).view(np.uint32)), i
        assert torch.equal(ids, ref_ids), i
    assert seen == [start + step, 2 ** 32 - 1, 1 + step, 1 + 2 * step]


def test_fused_kernel_refuses_untracked_epoch_near_wrap(gemv, stack):
    """An epoch close to 2^32 that this context did not set (written to the
    workspace behind the guard's back) is refused by the kernel: outputs
    marked (NaN, ids -1), the status names the cause, and after
    ft_hip_fused_workspace_init the stack runs normally again."""
    m = stack.m
    K, L = m.shape.top_k, m.L
    x = m.hidden(14)
    stack.reset()
    ref, ref_ids = torch.zeros_like(x), torch.zeros(L * K, dtype=torch.int32, device=DEV)
    stack.run(x, ref, ref_ids)
    stack.check()
    stack.reset()
    stack.ws[:4].view(torch.int32)[0] = -2  # epoch 0xFFFFFFFE
    o, ids = torch.zeros_like(x), torch.zeros(L * K, dtype=torch.int32, device=DEV)
    stack.run(x, o, ids)
    with pytest.raises(ft_hip.FtHipError) as ei:
        stack.check()
    assert "2^32" in str(ei.value)
    assert np.all(np.isnan(host(o))) and np.all(host(ids) == -1)
    stack.reset()
    stack.run(x, o, ids)
    stack.check()
    assert np.array_equal(host(o).view(np.uint32), host(ref).view(np.uint32))
    assert torch.equal(ids, ref_ids)


def test_fused_many_launches_full_stack(gemv):
    """Regression test for lost hand-overs: 600 consecutive launches of the
    production build on one workspace over the full 30-layer stack (the
    bench's configuration), epochs advancing every launch, prediction on.
    The workspace status is checked every 100 launches (a lost hand-over
    shows as an aborted bounded wait), and every token's output and routing
    must equal its first launch bit for bit."""
    m = moe_synth.SyntheticMoE(gemv, moe_synth.GEMMA)
    st = moe_synth.FusedStack(m)
    K, L = m.shape.top_k, m.L
    toks = [m.hidden(t) for t in range(8)]
    outs = torch.zeros((600, m.shape.hidden), dtype=torch.float32, device=DEV)
    ids = torch.zeros((600, L * K), dtype=torch.int32, device=DEV)
    gemv.fused_set_prefetch(1)
    for i in range(600):
        st.run(toks[i % 8], outs[i], ids[i])
        if i % 100 == 99:
            st.check()
    o, d = host(outs), host(ids)
    for i in range(8, 600):
        assert np.array_equal(o[i].view(np.uint32), o[i % 8].view(np.uint32)), i
        assert np.array_equal(d[i], d[i % 8]), i
    assert np.all(np.isfinite(o))
    del st, m
    torch.cuda.empty_cache()


def test_fused_cooperative_launch_matches_plain(gemv, stack):
    """The cooperative launch mode gives the plain launch's bits."""
    m = stack.m
    x = m.hidden(11)
    res = []
    for coop in (0, 1, 0):
        o = torch.zeros_like(x)
        ids = torch.zeros(m.L * m.shape.top_k, dtype=torch.int32, device=DEV)
        gemv.fused_set_cooperative(coop)
        try:
            stack.run(x, o, ids)
            stack.check()
        finally:
            gemv.fused_set_cooperative(0)
        res.append((host(o), host(ids)))
    for o, i in res[1:]:
        assert np.array_equal(o.view(np.uint32), res[0][0].view(np.uint32))
        assert np.array_equal(i, res[0][1])
    with pytest.raises(ft_hip.FtHipError):
        gemv.fused_set_cooperative(2)
