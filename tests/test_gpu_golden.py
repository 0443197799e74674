"""The HIP path against the frozen vectors in tests/golden/moe_tiny.npz.

Bit-exact: q8 quants, per-block int32 dots, GELU*up q8 (libm tanhf),
top-k ids and weights. f32 outputs: max|dy| <= 1e-3 * ||y_ref||_2 (the
north-star tolerance), and the layer's residual output within 1e-5 of
||x_out - x||.
"""
import os

import numpy as np
import pytest
import torch

import ft_hip

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "moe_tiny.npz")


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def q8_wire(d, qs):
    nb = len(d)
    b = np.zeros((nb, 40), np.uint8)
    b[:, 0:4] = d.astype(np.float32).view(np.uint8).reshape(nb, 4)
    b[:, 4:8] = qs.reshape(nb, 32).astype(np.int32).sum(axis=1).astype(np.int32).view(np.uint8).reshape(nb, 4)
    b[:, 8:40] = qs.view(np.uint8).reshape(nb, 32)
    return b.ravel()


def q8_split(buf, nb):
    b = np.ascontiguousarray(buf).view(np.uint8).reshape(nb, 40)
    return b[:, 0:4].copy().view(np.float32)[:, 0], b[:, 8:40].copy().view(np.int8).ravel()


def test_q8_matches_golden(gemv, gold):
    x = gold["q8_x"]
    q8 = torch.zeros(len(x) // 32 * 40, dtype=torch.uint8, device=DEV)
    gemv.quantize_q8(dev(x), 0, q8, len(x), 1)
    d, qs = q8_split(host(q8), len(x) // 32)
    assert np.array_equal(d.view(np.uint32), gold["q8_d"].view(np.uint32))
    assert np.array_equal(qs, gold["q8_qs"])


def test_block_dots_and_gemv_match_golden(gemv, gold):
    k, n = 2816, 8
    w = gold["dot_w_q4r"]
    bank = dev(w.ravel())
    eb = w.size
    q8 = dev(q8_wire(gold["q8_d"], gold["q8_qs"]))
    slots = dev(np.zeros(1, np.int32))
    dots = torch.zeros(n * (k // 32), dtype=torch.int32, device=DEV)
    gemv.block_dots(bank, eb, 0, slots, None, 1, q8, k // 32, dots, n, k, ft_hip.LAYOUT_Q4R)
    assert np.array_equal(host(dots).reshape(n, k // 32), gold["dot_blocks"])
    y = torch.zeros(n, dtype=torch.float32, device=DEV)
    gemv.gemv_grouped_slots(bank, eb, 0, slots, None, 1, q8, k // 32, y, n, n, k, ft_hip.LAYOUT_Q4R)
    y, ref = host(y), gold["dot_y"]
    assert np.max(np.abs(y - ref)) <= 1e-3 * np.linalg.norm(ref)
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref))


def test_gelu_q8_matches_golden(gemv, gold):
    q8 = torch.zeros(704 // 32 * 40, dtype=torch.uint8, device=DEV)
    gemv.gelu_mul_q8(dev(gold["gelu_gu"]), q8, 704, 1)
    d, qs = q8_split(host(q8), 704 // 32)
    assert np.array_equal(d.view(np.uint32), gold["gelu_d"].view(np.uint32))
    assert np.array_equal(qs, gold["gelu_qs"])


@pytest.mark.parametrize("tag", ["layer_", "layerb_"])
def test_layer_matches_golden(gemv, gold, tag):
    H, I, E, K = (int(v) for v in gold["layer_shape"])
    bank = gold["layer_bank"]
    x = gold["layer_x"]
    bias = dev(gold["layer_bias"]) if tag == "layerb_" else None
    ws = torch.zeros(gemv.moe_layer_workspace_bytes(1, H, I, E, K), dtype=torch.uint8, device=DEV)
    ids = torch.zeros(K, dtype=torch.int32, device=DEV)
    wts = torch.zeros(K, dtype=torch.float32, device=DEV)
    out = torch.zeros(H, dtype=torch.float32, device=DEV)
    gemv.moe_layer(dev(x), out, 1, H, I, E, K, dev(gold["layer_Wr"]), bias, None, dev(bank.ravel()),
                   bank.shape[1], ft_hip.LAYOUT_Q4R, ids, wts, ws)
    assert np.array_equal(host(ids), gold[tag + "ids"])
    assert np.array_equal(host(wts).view(np.uint32), gold[tag + "wts"].view(np.uint32))
    o, ref = host(out), gold[tag + "x_out"]
    assert np.max(np.abs(o - ref)) <= 1e-5 * np.linalg.norm(ref - x)
    assert np.max(np.abs(o - ref)) <= 1e-3 * np.linalg.norm(ref)
