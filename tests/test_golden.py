"""The oracle against the frozen vectors in tests/golden/moe_tiny.npz.

The reference ships no fixture files (its tests build inline xorshift32
data: ft-core/src/q4_0.rs:162-358, ft-cuda/tests/*.rs), so the
fixtures were written once by tests/golden/make_golden.py from the oracle
and are checked here bit-for-bit: a later change to the oracle that moves any
bit of any stage fails this file. Each stage is also checked against what
the mathematics fixes, independently of the oracle's code.
"""
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "moe_tiny.npz")


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint8)


def test_fixture_complete(gold):
    for k in ("q4_x", "q4_bytes", "q8_x", "q8_d", "q8_qs", "dot_w_q4r", "dot_blocks", "dot_y", "gelu_gu",
              "gelu_act", "gelu_d", "gelu_qs", "layer_shape", "layer_x", "layer_Wr", "layer_bank", "layer_bias",
              "layer_ids", "layer_wts", "layer_x_out", "layerb_ids", "layerb_x_out"):
        assert k in gold, k


def test_quantize_row_reproduces_golden(orc, gold):
    assert np.array_equal(orc.quantize_row(gold["q4_x"]), gold["q4_bytes"])
    # dequantised values are within one step |d| of the inputs (half a step,
    # except where x/d ~ +8 clamps q from 16 to 15), d rounded to f16
    deq = orc.dequantize_row(gold["q4_bytes"], 64)
    d = np.abs(gold["q4_bytes"].reshape(4, 2, 18)[:, :, :2].copy().view(np.float16).astype(np.float32))
    err = np.abs(deq - gold["q4_x"]).reshape(4, 2, 32).max(axis=2)
    assert np.all(err <= d[:, :, 0] * 1.002 + 1e-6)
    assert np.all(deq[1, :32] == 0) and deq[1, 40] == 3.0


def test_q8_reproduces_golden(orc, gold):
    d, qs = orc.q8_quantize(gold["q8_x"])
    assert np.array_equal(bits(d), bits(gold["q8_d"]))
    assert np.array_equal(qs, gold["q8_qs"])
    # closed form: d = amax/127 in f32, q = round-half-away(x/d) for the exact-tie block
    x = gold["q8_x"].reshape(-1, 32)
    assert np.array_equal(gold["q8_d"], (np.abs(x).max(axis=1) / np.float32(127)).astype(np.float32))
    assert list(gold["q8_qs"][32:38]) == [127, 3, -3, 1, -1, 127]


def test_block_dots_and_gemv_reproduce_golden(orc, gold):
    w = gold["dot_w_q4r"]
    k = 2816
    # q4r -> q4_0 rows for the integer dot: scales region then 16-byte blocks
    nb = k // 32
    sb = orc.q4r_scales_bytes(k)
    q4 = np.zeros((8, nb * 18), np.uint8)
    for r in range(8):
        q4[r].reshape(nb, 18)[:, :2] = w[r, :nb * 2].reshape(nb, 2)
        q4[r].reshape(nb, 18)[:, 2:] = w[r, sb:].reshape(nb, 16)
    dots = orc.block_dots(q4, gold["q8_qs"], k)
    assert np.array_equal(dots, gold["dot_blocks"])
    # textbook integer sum of (q - 8) * q8 per block
    qv = np.zeros((8, k), np.int64)
    b = q4.reshape(8, nb, 18)[:, :, 2:].astype(np.int64)
    qv.reshape(8, nb, 32)[:, :, :16] = (b & 15) - 8
    qv.reshape(8, nb, 32)[:, :, 16:] = (b >> 4) - 8
    ref = (qv * gold["q8_qs"].astype(np.int64)).reshape(8, nb, 32).sum(axis=2)
    assert np.array_equal(dots, ref)
    y = orc.gemv_q8(w, 8, gold["q8_d"], gold["q8_qs"], k, layout=1)
    assert np.array_equal(bits(y), bits(gold["dot_y"]))


def test_gelu_q8_reproduces_golden(orc, gold):
    act, d, qs = orc.gelu_mul_q8(gold["gelu_gu"], 704)
    assert np.array_equal(bits(act), bits(gold["gelu_act"]))
    assert np.array_equal(bits(d), bits(gold["gelu_d"]))
    assert np.array_equal(qs, gold["gelu_qs"])
    # GELU-tanh in f64 agrees to f32 rounding scale
    g, u = gold["gelu_gu"][:704].astype(np.float64), gold["gelu_gu"][704:].astype(np.float64)
    ref = 0.5 * g * (1 + np.tanh(0.7978845608 * (g + 0.044715 * g ** 3))) * u
    assert np.max(np.abs(act - ref)) <= 1e-5 * np.max(np.abs(ref))


@pytest.mark.parametrize("tag", ["layer_", "layerb_"])
def test_layer_reproduces_golden(orc, gold, tag):
    H, I, E, K = (int(v) for v in gold["layer_shape"])
    bank = gold["layer_bank"]
    gb = 2 * I * orc.q4r_row_bytes(H)
    gu = {e: bank[e, :gb] for e in range(E)}
    dn = {e: bank[e, gb:] for e in range(E)}
    bias = gold["layer_bias"] if tag == "layerb_" else None
    r = orc.moe_layer(gold["layer_x"], gold["layer_Wr"], gu, dn, H, I, K, bias=bias, layout=1)
    for key in ("logits", "ids", "wts", "act_d", "act_qs", "x_out"):
        assert np.array_equal(bits(r[key]), bits(gold[tag + key])), key
    # logits in f64 agree; the chosen experts are the stable argsort's
    lg64 = gold["layer_Wr"].astype(np.float64) @ gold["layer_x"].astype(np.float64)
    if bias is not None:
        lg64 = lg64 + bias
    assert np.max(np.abs(r["logits"] - lg64)) < 1e-5
    assert list(r["ids"]) == list(np.argsort(-r["logits"], kind="stable")[:K])
