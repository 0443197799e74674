"""CPU tests that pin the oracle (oracle/ft_oracle.cpp) before it is trusted.

The reference ships no golden vectors (its tests generate data inline with
xorshift32), so each oracle function is pinned by (a) the reference's own
test assertions, reproduced on the same xorshift inputs, and (b) checks that
the mathematics fixes: closed-form cases, independent numpy formulations of
the integer arithmetic, IEEE library routines (numpy float16 / float32
division), and f64 brute force. Each check is chosen so that a plausible slip
(swapped nibbles, wrong rounding mode, dropped offset, wrong index) fails.
"""
import math

import numpy as np
import pytest

from cases import nonfinite_q8_blocks


def xorshift_row(n, seed, add_golden=True):
    """ft-core/src/q4_0.rs:166-177 (pseudo_row); add_golden=False gives the
    closure used by q4r_matches_q4 (:333-337) and ft-cuda/tests/*.rs."""
    s = (seed + 0x9E3779B9) & 0xFFFFFFFF if add_golden else seed & 0xFFFFFFFF
    out = np.empty(n, np.float32)
    umax = np.float32(4294967295.0)
    for i in range(n):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        out[i] = (np.float32(s) / umax) * np.float32(2.0) - np.float32(1.0)
    return out


def unpack_q4(q, k):
    """Independent numpy unpacking of q4_0 rows -> (nibbles [n, k] u8, d [n, k/32] f32)."""
    q = np.asarray(q, np.uint8).reshape(-1, k // 32, 18)
    d = q[:, :, :2].copy().view(np.float16).astype(np.float32)[:, :, 0]
    qs = q[:, :, 2:]
    nib = np.concatenate([qs & 0xF, qs >> 4], axis=2)  # [n, nb, 32]: lo nibbles are 0..15
    return nib.reshape(q.shape[0], k), d


# ---------------------------------------------------------------------------
# The reference's own tests, on the reference's own inputs
# ---------------------------------------------------------------------------

def test_ref_roundtrip_error_is_small(orc):
    """ft-core/src/q4_0.rs:179-189"""
    row = xorshift_row(256, 7)
    back = orc.dequantize_row(orc.quantize_row(row), 256)
    assert np.all(np.abs(row - back) < 0.15)


def test_ref_gemv_matches_f32_reference(orc):
    """ft-core/src/q4_0.rs:191-215"""
    k, n = 512, 16
    x = xorshift_row(k, 1)
    w = np.zeros((n, orc.row_bytes(k)), np.uint8)
    wf = np.zeros((n, k), np.float32)
    for r in range(n):
        w[r] = orc.quantize_row(xorshift_row(k, 100 + r))
        wf[r] = orc.dequantize_row(w[r], k)
    y = orc.gemv(w, x, n)
    ref = (wf * x).sum(axis=1)
    assert np.all(np.abs(y - ref) < 0.15)


def test_ref_avx2_matches_scalar(orc):
    """ft-core/src/q4_0.rs:217-231"""
    k = 4096
    row = orc.quantize_row(xorshift_row(k, 42))
    d, qs = orc.q8_quantize(xorshift_row(k, 7))
    a = orc.dot_scalar(row, d, qs, k)
    b = orc.dot_avx2(row, d, qs, k)
    assert abs(a - b) < 1e-2 * (1.0 + abs(a))


def test_ref_q4r_matches_q4(orc):
    """ft-core/src/q4_0.rs:329-358 (the same xorshift stream, seed 0xC0DE)."""
    k, n = 2816, 8
    vals = xorshift_row(n * k + k, 0xC0DE, add_golden=False)
    w = orc.quantize_row(vals[: n * k].reshape(n, k))
    wr = orc.repack_q4r(w, k)
    d, qs = orc.q8_quantize(vals[n * k:])
    y1 = orc.gemv_q8(w, n, d, qs, k, layout=0)
    y2 = orc.gemv_q8(wr, n, d, qs, k, layout=1)
    assert np.all(np.abs(y1 - y2) < 1e-3 * (1.0 + np.abs(y1)))
    # stronger: the arithmetic is identical, so the bits are
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))


# ---------------------------------------------------------------------------
# q4_0 quantiser (ft-core/src/q4_0.rs:20-40)
# ---------------------------------------------------------------------------

def test_q4_scale_is_f16_rne_of_signed_max_over_minus8(orc):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((64, 32)) * 0.02).astype(np.float32)
    q = orc.quantize_row(x)
    for r in range(64):
        i = int(np.argmax(np.abs(x[r])))  # first occurrence of the largest magnitude
        d = np.float32(x[r, i]) / np.float32(-8.0)
        expect = np.array([d], np.float32).astype(np.float16).view(np.uint16)[0]
        assert int(q[r, 0]) | (int(q[r, 1]) << 8) == int(expect)


def test_q4_nibble_placement_single_spike(orc):
    """A lone spike at position p must come back at p: pins byte i = q_i | q_{i+16}<<4."""
    for p in range(32):
        x = np.zeros(32, np.float32)
        x[p] = -3.0  # maxv = -3 -> d = 0.375, the spike maps to q = 0 -> (0-8)*d = -3
        back = orc.dequantize_row(orc.quantize_row(x), 32)
        expect = np.zeros(32, np.float32)
        expect[p] = -3.0
        assert np.array_equal(back, expect), p


def test_q4_rounding_closed_form(orc):
    """maxv = -8 gives d = 1, id = 1, so q = clamp(trunc(x + 8.5), 0, 15)."""
    x = np.array([-8.0, 0.4, 0.5, -0.5, -0.6, 6.49, 6.5, 7.9, 3.0, -7.5, 1.2, -1.2, 2.5, -2.5, 4.99, 5.5]
                 + [0.0] * 16, np.float32)
    q = orc.quantize_row(x)
    nib, d = unpack_q4(q, 32)
    assert d[0, 0] == 1.0
    expect = np.clip(np.trunc(x.astype(np.float64) + 8.5), 0, 15).astype(np.uint8)
    assert np.array_equal(nib[0], expect)
    assert list(expect[:8]) == [0, 8, 9, 8, 7, 14, 15, 15]


def test_q4_amax_tie_first_occurrence_wins(orc):
    a = orc.quantize_row(np.array([0.5, -0.5] + [0.0] * 30, np.float32))
    b = orc.quantize_row(np.array([-0.5, 0.5] + [0.0] * 30, np.float32))
    # first: maxv = +0.5 -> d = -0.0625 (f16 0xAC00); second: maxv = -0.5 -> d = +0.0625 (0x2C00)
    assert (int(a[0]) | (int(a[1]) << 8)) == 0xAC00 and (int(b[0]) | (int(b[1]) << 8)) == 0x2C00
    assert (a[2] & 0xF) == 0                            # +0.5*(-16)+8.5 = 0.5 -> 0
    assert (a[3] & 0xF) == 15                           # -0.5*(-16)+8.5 = 16.5 -> 16 -> clamp 15
    assert (b[2] & 0xF) == 0 and (b[3] & 0xF) == 15


def test_q4_zero_block(orc):
    q = orc.quantize_row(np.zeros(32, np.float32))
    # d = 0.0 / -8.0 = -0.0 (f16 0x8000); id = 0, so q = trunc(8.5) = 8 everywhere
    assert q[0] == 0x00 and q[1] == 0x80 and np.all(q[2:] == 0x88)


# ---------------------------------------------------------------------------
# q8 activation quantiser (ft-core/src/q4_0.rs:62-78)
# ---------------------------------------------------------------------------

def test_q8_scale_is_ieee_amax_over_127(orc):
    rng = np.random.default_rng(2)
    x = rng.standard_normal(32 * 500).astype(np.float32) * np.float32(3.0)
    d, _ = orc.q8_quantize(x)
    amax = np.abs(x.reshape(-1, 32)).max(axis=1)
    assert np.array_equal(d, amax / np.float32(127.0))


def test_q8_rounds_half_away_from_zero(orc):
    """amax = 127 gives d = inv = 1, so q = round_half_away(v). RNE would give 2, -2, 0, 0, 126."""
    x = np.array([127.0, 2.5, -2.5, 0.5, -0.5, 126.5, -126.5, 1.5, -1.5, 0.49, -0.51, 3.0] + [0.0] * 20,
                 np.float32)
    d, qs = orc.q8_quantize(x)
    assert d[0] == 1.0
    assert list(qs[:12]) == [127, 3, -3, 1, -1, 127, -127, 2, -2, 0, -1, 3]


def test_q8_nonfinite_blocks_follow_rust_semantics(orc):
    x, de, qe = nonfinite_q8_blocks()
    d, qs = orc.q8_quantize(x)
    assert np.array_equal(d.view(np.uint32), de.view(np.uint32)), (d, de)
    assert np.array_equal(qs, qe), (qs.reshape(-1, 32)[:, :6], qe.reshape(-1, 32)[:, :6])


def test_q8_zero_block_and_error_bound(orc):
    x = np.concatenate([np.zeros(32, np.float32),
                        np.random.default_rng(3).standard_normal(32 * 200).astype(np.float32)])
    d, qs = orc.q8_quantize(x)
    assert d[0] == 0.0 and np.all(qs[:32] == 0)
    deq = qs.astype(np.float64) * np.repeat(d, 32).astype(np.float64)
    assert np.all(np.abs(deq - x) <= np.repeat(d, 32) * 0.5000001 + 1e-30)
    assert np.all(np.abs(qs) <= 127)


# ---------------------------------------------------------------------------
# the dot (ft-core/src/q4_0.rs:105-160)
# ---------------------------------------------------------------------------

def _rand_case(orc, k, seed, n=4):
    rng = np.random.default_rng(seed)
    w = orc.quantize_row((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    d8, qs8 = orc.q8_quantize(rng.standard_normal(k).astype(np.float32))
    return w, d8, qs8


@pytest.mark.parametrize("k", [32, 64, 704, 2816, 4096])
def test_block_dots_equal_numpy_integer_sum(orc, k):
    w, d8, qs8 = _rand_case(orc, k, k)
    got = orc.block_dots(w, qs8, k)
    nib, _ = unpack_q4(w, k)
    expect = ((nib.astype(np.int64) - 8) * qs8.astype(np.int64)).reshape(w.shape[0], k // 32, 32).sum(axis=2)
    assert np.array_equal(got, expect)


@pytest.mark.parametrize("k", [64, 704, 2816, 4096])
def test_dot_avx2_close_to_f64_bruteforce(orc, k):
    w, d8, qs8 = _rand_case(orc, k, 10 + k)
    nib, d4 = unpack_q4(w, k)
    wf = (nib.astype(np.float64) - 8) * np.repeat(d4, 32, axis=1)
    xf = qs8.astype(np.float64) * np.repeat(d8, 32).astype(np.float64)
    for r in range(w.shape[0]):
        exact = float(wf[r] @ xf)
        mag = float(np.abs(wf[r] * xf).sum())
        got = orc.dot_avx2(w[r], d8, qs8, k)
        assert abs(got - exact) <= 1e-5 * mag + 1e-12


def test_dot_avx2_exact_when_arithmetic_is_exact(orc):
    """Scales that are powers of two make every partial exact: the f32 result must
    equal the integer closed form, whatever the summation order."""
    k = 2816
    rng = np.random.default_rng(5)
    x = rng.integers(-127, 128, k).astype(np.float32)
    x[::32] = 127.0                                  # amax = 127 -> d8 = 1
    wv = rng.integers(-8, 8, k).astype(np.float32) * np.float32(0.0625)
    wv[::32] = -0.5                                  # maxv = -0.5 -> d4 = 1/16
    w = orc.quantize_row(wv)
    d8, qs8 = orc.q8_quantize(x)
    assert np.all(d8 == 1.0)
    nib, d4 = unpack_q4(w, k)
    assert np.all(d4 == 0.0625)
    exact = float(((nib[0].astype(np.int64) - 8) * qs8.astype(np.int64)).sum()) * 0.0625
    assert orc.dot_avx2(w[0] if w.ndim > 1 else w, d8, qs8, k) == exact
    assert orc.dot_scalar(w[0] if w.ndim > 1 else w, d8, qs8, k) == exact


def test_gemv_threads_do_not_change_bits(orc):
    k, n = 2816, 300
    rng = np.random.default_rng(6)
    w = orc.quantize_row((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    d8, qs8 = orc.q8_quantize(rng.standard_normal(k).astype(np.float32))
    y1 = orc.gemv_q8(w, n, d8, qs8, k, threads=1)
    y8 = orc.gemv_q8(w, n, d8, qs8, k, threads=8)
    assert np.array_equal(y1.view(np.uint32), y8.view(np.uint32))


@pytest.mark.parametrize("k", [704, 2816, 4096])
def test_q4r_layout_and_bit_identity(orc, k):
    w, d8, qs8 = _rand_case(orc, k, 20 + k, n=3)
    wr = orc.repack_q4r(w, k)
    nb = k // 32
    so = orc.q4r_scales_bytes(k)
    assert wr.shape[1] == so + nb * 16 and so % 16 == 0
    src = w.reshape(3, nb, 18)
    assert np.array_equal(wr[:, :2 * nb].reshape(3, nb, 2), src[:, :, :2])
    assert np.all(wr[:, 2 * nb:so] == 0)
    assert np.array_equal(wr[:, so:].reshape(3, nb, 16), src[:, :, 2:])
    for r in range(3):
        a = orc.dot_avx2(w[r], d8, qs8, k)
        b = orc.dot_q4r_avx2(wr[r], d8, qs8, k)
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32)
        assert orc.dot_scalar(w[r], d8, qs8, k) == orc.dot_q4r_scalar(wr[r], d8, qs8, k)


# ---------------------------------------------------------------------------
# GELU (ft-model/src/lib.rs:435-437) on the host libm's tanhf
# ---------------------------------------------------------------------------

_LIBM = None


def libm_f32(name):
    """The host libm's f32 function `name` through ctypes (the function Rust's
    f32 method calls on Linux), independent of the oracle library."""
    global _LIBM
    if _LIBM is None:
        import ctypes
        _LIBM = ctypes.CDLL("libm.so.6")
    f = getattr(_LIBM, name)
    import ctypes
    f.restype, f.argtypes = ctypes.c_float, [ctypes.c_float]
    return f


def test_gelu_special_values_and_accuracy(orc):
    L = orc.lib()
    assert L.orc_gelu_tanh(0.0) == 0.0
    assert L.orc_gelu_tanh(10.0) == 10.0
    g = L.orc_gelu_tanh(-10.0)
    assert g == 0.0 and math.copysign(1.0, g) == -1.0
    rng = np.random.default_rng(8)
    for g in rng.standard_normal(5000).astype(np.float32) * 2:
        a = np.float32(L.orc_gelu_tanh(float(g)))
        ref = 0.5 * float(g) * (1 + math.tanh(0.7978845608 * (float(g) + 0.044715 * float(g) ** 3)))
        # 1 + t cancels for negative g: its f32 rounding (~6e-8 absolute) is scaled by 0.5*|g|
        assert abs(float(a) - ref) <= 4e-7 * abs(ref) + 1.2e-7 * abs(float(g))


def test_gelu_mul_q8_composition(orc):
    """act[j] = gelu(gu[j]) * gu[I + j] (gate rows first), each f32 op of
    ft-model/src/lib.rs:436 rounded in order with libm's tanhf, then q8."""
    I = 704
    rng = np.random.default_rng(9)
    gu = rng.standard_normal(2 * I).astype(np.float32)
    act, d, qs = orc.gelu_mul_q8(gu, I)
    tanhf = libm_f32("tanhf")
    f = np.float32
    expect = np.empty(I, np.float32)
    for j in range(I):
        g = gu[j]
        inner = g + ((f(0.044715) * g) * g) * g
        t = f(tanhf(float(f(0.7978845608) * inner)))
        expect[j] = ((f(0.5) * g) * (f(1.0) + t)) * gu[I + j]
    assert np.array_equal(act, expect)
    d2, q2 = orc.q8_quantize(expect)
    assert np.array_equal(d, d2) and np.array_equal(qs, q2)


# ---------------------------------------------------------------------------
# grouped activations and expert reductions of Q4Gemv's batched surface
# ---------------------------------------------------------------------------

SPECIAL = np.array([0.0, -0.0, 1.0, -1.0, 88.0, -88.0, 104.0, -104.0, 1e-40, -1e-40, 3.4e38, -3.4e38,
                    np.inf, -np.inf, np.nan], np.float32)


def test_silu_mul_grouped_is_cpu_expression_with_libm_expf(orc):
    """ft-bench/src/bin/decode.rs:300: g / (1.0 + (-g).exp()) * up, each f32 op
    rounded in order, exp = libm's expf (called here through ctypes, the
    arithmetic in numpy f32): a sign slip (exp(g)), a contraction or another
    order changes bits on these inputs."""
    I = 64
    rng = np.random.default_rng(21)
    g = np.concatenate([SPECIAL, (rng.standard_normal(3 * I - SPECIAL.size) * 6).astype(np.float32)])
    up = (rng.standard_normal(3 * I) * 3).astype(np.float32)
    gu = np.concatenate([g.reshape(3, I), up.reshape(3, I)], axis=1)
    out = orc.silu_mul_grouped(gu, I)
    expf = libm_f32("expf")
    f = np.float32
    with np.errstate(all="ignore"):
        t = np.array([expf(float(-v)) for v in g], np.float32)
        expect = ((g / (f(1.0) + t)) * up).reshape(3, I)
    assert np.array_equal(out.view(np.uint32), expect.view(np.uint32))
    # closed forms: silu(0) = 0, silu(+inf) * up = inf * up, large negative g -> -0 * up
    assert out[0, 0] == 0.0 and np.isnan(out[0, 14])
    assert np.isposinf(out[0, 12]) == (up[12] > 0)


def test_gelu_mul_grouped_equals_gelu_mul_q8_activation(orc):
    """Per expert the f32 activation of gelu_mul_q8 (pinned above against libm's tanhf)."""
    I = 96
    rng = np.random.default_rng(22)
    gu = (rng.standard_normal((5, 2 * I)) * 3).astype(np.float32)
    gu[0, :SPECIAL.size] = SPECIAL
    out = orc.gelu_mul_grouped(gu, I)
    for e in range(5):
        act, _, _ = orc.gelu_mul_q8(gu[e], I)
        assert np.array_equal(out[e].view(np.uint32), act.view(np.uint32))


def test_reduce_expert_weighted_order_and_no_contraction(orc):
    """out + sum_e (w[e] * y[e]): exact on small integers; experts summed in
    order (1e8, -1e8, 1 gives 1, reversed it gives 0); the product rounded
    before the add (an fma would keep (1+2^-12)^2's low bits)."""
    rng = np.random.default_rng(23)
    y = rng.integers(-50, 50, (6, 40)).astype(np.float32)
    w = np.array([0.5, 2, 1, 0.25, 4, 1], np.float32)
    out0 = rng.integers(-9, 9, 40).astype(np.float32)
    assert np.array_equal(orc.reduce_expert_weighted(y, w, out0), out0 + (y * w[:, None]).sum(axis=0))
    yo = np.array([[1e8], [-1e8], [1.0]], np.float32)
    assert orc.reduce_expert_weighted(yo, np.ones(3, np.float32), np.zeros(1, np.float32))[0] == 1.0
    assert orc.reduce_expert_weighted(yo[::-1], np.ones(3, np.float32), np.zeros(1, np.float32))[0] == 0.0
    a = np.float32(1 + 2.0 ** -12)
    r = orc.reduce_expert_weighted(np.array([[-1.0], [a]], np.float32), np.array([1.0, a], np.float32),
                                   np.zeros(1, np.float32))[0]
    assert r == np.float32(a * a) - np.float32(1.0) and r != np.float32(2.0 ** -11 + 2.0 ** -24)
    # no experts: out unchanged; f64 agreement on random data
    assert np.array_equal(orc.reduce_expert_weighted(np.zeros((0, 40), np.float32), np.zeros(0, np.float32),
                                                     out0), out0)
    yr = rng.standard_normal((8, 512)).astype(np.float32)
    wr = rng.random(8).astype(np.float32)
    ref = (yr.astype(np.float64) * wr[:, None]).sum(axis=0)
    assert np.max(np.abs(orc.reduce_expert_weighted(yr, wr, np.zeros(512, np.float32)) - ref)) <= 1e-5


def test_reduce_weighted_order_and_scale(orc):
    """out + a * (sum_e y[e]): experts summed in order, then one product, then the add."""
    rng = np.random.default_rng(24)
    y = rng.integers(-50, 50, (5, 33)).astype(np.float32)
    out0 = rng.integers(-9, 9, 33).astype(np.float32)
    assert np.array_equal(orc.reduce_weighted(y, 0.5, out0), out0 + np.float32(0.5) * y.sum(axis=0))
    yo = np.array([[1e8], [-1e8], [1.0]], np.float32)
    assert orc.reduce_weighted(yo, 3.0, np.zeros(1, np.float32))[0] == 3.0
    assert orc.reduce_weighted(yo[::-1], 3.0, np.zeros(1, np.float32))[0] == 0.0
    # a * s rounded before the add: out = 1, a = 1 + 2^-12, s = 1 + 2^-12
    a = np.float32(1 + 2.0 ** -12)
    r = orc.reduce_weighted(np.array([[a]], np.float32), a, np.array([-1.0], np.float32))[0]
    assert r == np.float32(a * a) - np.float32(1.0)


# ---------------------------------------------------------------------------
# router logits (R-order), top-k, combine
# ---------------------------------------------------------------------------

def test_router_logits_f64_and_exact_integer_case(orc):
    E, H = 128, 2816
    rng = np.random.default_rng(10)
    W = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    x = rng.standard_normal(H).astype(np.float32)
    lg = orc.router_logits(W, x)
    ref = W.astype(np.float64) @ x.astype(np.float64)
    mag = np.abs(W.astype(np.float64)) @ np.abs(x.astype(np.float64))
    assert np.all(np.abs(lg - ref) <= 1e-6 * mag)
    # integer-valued inputs: every partial sum is exact, so the order cannot matter
    Wi = rng.integers(-50, 51, (E, H)).astype(np.float32)
    xi = rng.integers(-50, 51, H).astype(np.float32)
    assert np.array_equal(orc.router_logits(Wi, xi), (Wi.astype(np.int64) @ xi.astype(np.int64)).astype(np.float32))
    bias = rng.standard_normal(E).astype(np.float32)
    assert np.array_equal(orc.router_logits(Wi, xi, bias),
                          (Wi.astype(np.int64) @ xi.astype(np.int64)).astype(np.float32) + bias)


def test_router_logits_order_is_chunked_not_sequential(orc):
    """A case where the R-order and a plain left-to-right sum give different f32 bits,
    with the R-order value predicted by hand: chunk 0 holds 2^24 and 1s that a
    left-to-right sum would absorb one by one, but the chunk's own fma chain
    absorbs them too; group/chunk sums add exactly."""
    H = 128
    W = np.zeros((1, H), np.float32)
    x = np.zeros(H, np.float32)
    W[0, 0], x[0] = 1.0, 16777216.0          # chunk 0: 2^24
    W[0, 1], x[1] = 1.0, 1.0                 # 2^24 + 1 -> 2^24 (absorbed, RNE)
    W[0, 16:32] = 1.0                        # chunk 1 (group 1): sixteen 1s = 16
    x[16:32] = 1.0
    lg = orc.router_logits(W, x)
    assert lg[0] == np.float32(16777216.0 + 16.0)


def test_topk_matches_stable_argsort_and_f64_softmax(orc):
    rng = np.random.default_rng(11)
    for trial in range(50):
        E, k = 128, 8
        lg = rng.standard_normal(E).astype(np.float32)
        if trial % 5 == 0:  # force ties
            lg[rng.integers(0, E, 20)] = lg[3]
        ids, w = orc.topk_softmax(lg, k)
        order = np.argsort(-lg.astype(np.float64), kind="stable")[:k]
        assert np.array_equal(ids, order)
        ex = np.exp(lg[order].astype(np.float64) - float(lg[order[0]]))
        assert np.allclose(w, ex / ex.sum(), rtol=2e-6, atol=1e-9)
        assert abs(float(w.astype(np.float64).sum()) - 1.0) < 1e-5


def test_topk_ties_prefer_lower_index(orc):
    lg = np.zeros(16, np.float32)
    lg[[2, 5, 9]] = 1.0
    ids, w = orc.topk_softmax(lg, 4)
    assert list(ids) == [2, 5, 9, 0]
    ids, _ = orc.topk_softmax(np.full(10, -3.0, np.float32), 3)
    assert list(ids) == [0, 1, 2]


def test_topk_nan_sorts_last_and_signed_zeros_tie(orc):
    """The reference panics on a NaN logit (partial_cmp().unwrap()); this build
    ranks NaN after every number, NaNs among themselves by index. -0.0 == 0.0,
    so they tie and the lower index goes first."""
    lg = np.array([np.nan, -5.0, np.nan, 0.0, -0.0, -np.inf, 2.0], np.float32)
    ids, w = orc.topk_softmax(lg, 7)
    assert list(ids) == [6, 3, 4, 1, 5, 0, 2]
    lg = np.array([-0.0, 0.0, np.nan], np.float32)
    ids, _ = orc.topk_softmax(lg, 2)
    assert list(ids) == [0, 1]


def test_topk_expert_scale(orc):
    lg = np.array([3.0, 1.0, 2.0, 0.0], np.float32)
    es = np.array([2.0, 1.0, 0.5, 1.0], np.float32)
    ids, w = orc.topk_softmax(lg, 2, es)
    ids0, w0 = orc.topk_softmax(lg, 2)
    assert list(ids) == [0, 2]
    assert w[0] == w0[0] * 2.0 and w[1] == w0[1] * 0.5


def test_combine_exact_and_f64(orc):
    rng = np.random.default_rng(12)
    y = rng.standard_normal((8, 2816)).astype(np.float32)
    w = rng.random(8).astype(np.float32)
    x = rng.standard_normal(2816).astype(np.float32)
    out = orc.combine(y, w, x)
    ref = x.astype(np.float64) + (y.astype(np.float64) * w.astype(np.float64)[:, None]).sum(axis=0)
    assert np.allclose(out, ref, rtol=0, atol=2e-6 * np.abs(ref).max())
    # power-of-two weights and small integers: exact
    yi = rng.integers(-100, 100, (8, 64)).astype(np.float32)
    wi = np.array([0.5, 0.25, 1, 2, 0.125, 4, 1, 0.5], np.float32)
    assert np.array_equal(orc.combine(yi, wi), (yi * wi[:, None]).sum(axis=0))


# ---------------------------------------------------------------------------
# the layer composition (ft-model/src/lib.rs:1609-1653)
# ---------------------------------------------------------------------------

def test_moe_layer_stages_match_f64_composition(orc):
    H, I, E, k = 256, 64, 16, 4
    rng = np.random.default_rng(13)
    x = rng.standard_normal(H).astype(np.float32)
    W_r = (rng.standard_normal((E, H)) * 0.1).astype(np.float32)
    gu = {e: orc.quantize_row((rng.standard_normal((2 * I, H)) * 0.02).astype(np.float32)) for e in range(E)}
    dn = {e: orc.quantize_row((rng.standard_normal((H, I)) * 0.02).astype(np.float32)) for e in range(E)}
    r = orc.moe_layer(x, W_r, gu, dn, H, I, k)
    ids, wts = orc.topk_softmax(orc.router_logits(W_r, x), k)
    assert np.array_equal(r["ids"], ids) and np.array_equal(r["wts"], wts)
    d8, q8 = orc.q8_quantize(x)
    xf = q8.astype(np.float64) * np.repeat(d8, 32)
    out = x.astype(np.float64).copy()
    for p, e in enumerate(ids):
        nib, d4 = unpack_q4(gu[e], H)
        ygu = ((nib.astype(np.float64) - 8) * np.repeat(d4, 32, axis=1)) @ xf
        assert np.allclose(r["y_gu"][p], ygu, rtol=0, atol=1e-5 * np.abs(ygu).max())
        # down projection from the oracle's own act quants (teacher forced)
        af = r["act_qs"][p].astype(np.float64) * np.repeat(r["act_d"][p], 32)
        nib, d4 = unpack_q4(dn[e], I)
        ydn = ((nib.astype(np.float64) - 8) * np.repeat(d4, 32, axis=1)) @ af
        assert np.allclose(r["y_dn"][p], ydn, rtol=0, atol=1e-5 * np.abs(ydn).max() + 1e-12)
        out += float(wts[p]) * r["y_dn"][p].astype(np.float64)
    assert np.allclose(r["x_out"], out, rtol=0, atol=1e-5 * np.abs(out).max())
    # q4r banks give bit-identical results
    r2 = orc.moe_layer(x, W_r, {e: orc.repack_q4r(v, H) for e, v in gu.items()},
                       {e: orc.repack_q4r(v, I) for e, v in dn.items()}, H, I, k, layout=1)
    assert np.array_equal(r2["x_out"], r["x_out"])


def test_rms_inv_closed_forms(orc):
    """The input RMS norm's scale: f64 closed form 1/sqrt(mean(x^2) + 1e-6) to
    f32 accuracy; exact on a constant power-of-two vector (every partial sum
    exact); and its sum of squares is the R-order router dot of x with itself."""
    rng = np.random.default_rng(21)
    for H in (128, 2816, 4096):
        x = (rng.standard_normal(H) * rng.uniform(0.1, 30)).astype(np.float32)
        ir = orc.rms_inv(x)
        ref = 1.0 / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6)
        assert abs(float(ir) - ref) <= 4e-7 * ref, H
        ss = orc.router_logits(x[None, :], x)[0]
        assert ir == np.float32(1.0) / np.sqrt(ss / np.float32(H) + np.float32(1e-6))
    x = np.full(2816, 0.25, np.float32)  # ss = 176 exactly, mean = 1/16
    assert orc.rms_inv(x) == np.float32(1.0) / np.sqrt(np.float32(0.0625) + np.float32(1e-6))
    assert np.isclose(orc.rms_inv(np.zeros(256, np.float32)), 1000.0, rtol=1e-6)


def test_moe_layer_input_norm_is_layer_on_rmsnorm_x(orc):
    """input_norm runs the layer on rmsnorm(x): against the plain layer on
    u = x * inv_r (u quantized itself), the routing is the same and the MoE
    update agrees to rounding; scaling x by any c > 0 leaves the update of the
    normed layer unchanged up to rounding (the norm removes the scale); and
    the logits are the plain logits times inv_r, bit for bit."""
    H, I, E, k = 256, 64, 16, 4
    rng = np.random.default_rng(17)
    x = (rng.standard_normal(H) * 3.0).astype(np.float32)
    W_r = (rng.standard_normal((E, H)) * 0.1).astype(np.float32)
    gu = {e: orc.repack_q4r(orc.quantize_row((rng.standard_normal((2 * I, H)) * 0.02).astype(np.float32)), H)
          for e in range(E)}
    dn = {e: orc.repack_q4r(orc.quantize_row((rng.standard_normal((H, I)) * 0.02).astype(np.float32)), I)
          for e in range(E)}
    ir = orc.rms_inv(x)
    rn = orc.moe_layer(x, W_r, gu, dn, H, I, k, layout=1, input_norm=True)
    assert np.array_equal(rn["logits"].view(np.uint32), (orc.router_logits(W_r, x) * ir).astype(np.float32).view(np.uint32))
    u = (x * ir).astype(np.float32)
    ru = orc.moe_layer(u, W_r, gu, dn, H, I, k, layout=1)
    assert np.array_equal(rn["ids"], ru["ids"])
    assert np.allclose(rn["wts"], ru["wts"], rtol=1e-5, atol=0)
    dn_ = rn["x_out"].astype(np.float64) - x
    du = ru["x_out"].astype(np.float64) - u
    assert np.max(np.abs(dn_ - du)) <= 2e-2 * np.linalg.norm(du)
    for c in (0.125, 7.0):
        rc = orc.moe_layer((x * np.float32(c)).astype(np.float32), W_r, gu, dn, H, I, k, layout=1, input_norm=True)
        assert np.array_equal(rc["ids"], rn["ids"])
        dc = rc["x_out"].astype(np.float64) - (x * np.float32(c))
        assert np.max(np.abs(dc - dn_)) <= 2e-2 * np.linalg.norm(dn_)
    # off: identical bits to the layer without the argument
    r0 = orc.moe_layer(x, W_r, gu, dn, H, I, k, layout=1, input_norm=False)
    r1 = orc.moe_layer(x, W_r, gu, dn, H, I, k, layout=1)
    assert np.array_equal(r0["x_out"].view(np.uint32), r1["x_out"].view(np.uint32))


def test_moe_layer_missing_expert_raises(orc):
    H, I, E, k = 128, 32, 4, 2
    x = np.ones(H, np.float32)
    W_r = np.zeros((E, H), np.float32)
    with pytest.raises(KeyError):
        orc.moe_layer(x, W_r, {}, {}, H, I, k)


# ---------------------------------------------------------------------------
# seeded generator
# ---------------------------------------------------------------------------

def test_generator_moments_and_determinism(orc):
    key = orc.tensor_key(1, 0, 0, orc.T_GU)
    v = orc.gen_values(key, 0, 1 << 20, 0.02).astype(np.float64)
    assert abs(v.mean()) < 1e-4 and abs(v.std() - 0.02) < 2e-4
    assert np.abs(v).max() <= 0.02 * math.sqrt(3) * 2 + 1e-9  # Irwin-Hall(4) support: +-2*sqrt(3) sigma
    assert np.array_equal(orc.gen_values(key, 1000, 10, 0.02), orc.gen_values(key, 0, 1010, 0.02)[1000:])
    assert orc.tensor_key(1, 0, 0, orc.T_GU) != orc.tensor_key(1, 0, 1, orc.T_GU)
    rows = orc.gen_q4_rows(key, 3, 2, 64, 0.02)
    vals = orc.gen_values(key, 3 * 64, 2 * 64, 0.02).reshape(2, 64)
    assert np.array_equal(rows, orc.quantize_row(vals))
