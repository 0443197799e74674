"""The rest of Q4Gemv's batched-MoE surface, bit-exact against the oracle.

silu_mul_grouped, gelu_mul_grouped, reduce_expert_weighted and
reduce_weighted (ft-cuda/src/lib.rs:1009-1094; kernels q4.cu:169-192,
:289-314), and gemv_grouped_q8 / gemv_grouped_q8_idx (lib.rs:926-957,
:772-804) over q4_0 banks. The last test runs the reference bench's grouped
MoE layer call for call (ft-bench/src/bin/decode.rs:272-277): quantize_q8 ->
gemv_grouped_q8 (one activation shared by the experts, q8_stride_blocks 0)
-> silu_mul_grouped -> quantize_q8 -> gemv_grouped_q8 -> reduce_weighted,
each stage teacher-forced on the GPU's own input to it.
"""
import numpy as np
import pytest
import torch

import ft_hip

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


SPECIAL = np.array([0.0, -0.0, 1.0, -1.0, 88.0, -88.0, 104.0, -104.0, 1e-40, -1e-40, 3.4e38, -3.4e38,
                    np.inf, -np.inf, np.nan], np.float32)


def _gu(n, inter, seed, scale):
    rng = np.random.default_rng(seed)
    gu = (rng.standard_normal((n, 2 * inter)) * scale).astype(np.float32)
    gu[0, :SPECIAL.size] = SPECIAL
    gu[0, inter:inter + SPECIAL.size] = SPECIAL[::-1]
    return gu


@pytest.mark.parametrize("n,inter", [(1, 704), (8, 704), (3, 14336), (5, 96)])
def test_silu_mul_grouped_bit_exact(gemv, orc, n, inter):
    gu = _gu(n, inter, 31 + n, 6.0)
    out = torch.full((n, inter), 7.0, dtype=torch.float32, device=DEV)
    gemv.silu_mul_grouped(dev(gu), out, inter, n)
    assert np.array_equal(bits(host(out)), bits(orc.silu_mul_grouped(gu, inter)))


def test_silu_mul_grouped_value_sweep(gemv, orc):
    """2^20 gate values spread over every binade (expf's reduction branches,
    overflow and underflow, subnormals), up = 1 and up = -3.5."""
    rng = np.random.default_rng(32)
    g = rng.integers(0, 2 ** 32, 2 ** 20, dtype=np.uint64).astype(np.uint32).view(np.float32)
    inter = 2 ** 19
    gu = np.empty((2, 2 * inter), np.float32)
    gu[:, :inter] = g.reshape(2, inter)
    gu[0, inter:] = 1.0
    gu[1, inter:] = -3.5
    out = torch.zeros((2, inter), dtype=torch.float32, device=DEV)
    gemv.silu_mul_grouped(dev(gu), out, inter, 2)
    assert np.array_equal(bits(host(out)), bits(orc.silu_mul_grouped(gu, inter)))


@pytest.mark.parametrize("n,inter", [(8, 704), (2, 14336)])
def test_gelu_mul_grouped_bit_exact(gemv, orc, n, inter):
    gu = _gu(n, inter, 41 + n, 4.0)
    out = torch.zeros((n, inter), dtype=torch.float32, device=DEV)
    gemv.gelu_mul_grouped(dev(gu), out, inter, n)
    assert np.array_equal(bits(host(out)), bits(orc.gelu_mul_grouped(gu, inter)))


@pytest.mark.parametrize("n,hidden", [(8, 2816), (2, 4096), (1, 100), (0, 64), (40, 3000)])
def test_reduce_expert_weighted_bit_exact(gemv, orc, n, hidden):
    rng = np.random.default_rng(51 + n)
    y = rng.standard_normal((n, hidden)).astype(np.float32)
    w = rng.random(n).astype(np.float32)
    out0 = rng.standard_normal(hidden).astype(np.float32)
    out = dev(out0.copy())
    gemv.reduce_expert_weighted(dev(y) if n else dev(np.zeros(1, np.float32)), dev(w) if n else
                                dev(np.zeros(1, np.float32)), out, hidden, n)
    assert np.array_equal(bits(host(out)), bits(orc.reduce_expert_weighted(y, w, out0)))


@pytest.mark.parametrize("n,hidden,a", [(8, 2816, 0.125), (3, 4096, -1.75), (0, 64, 2.0), (17, 1000, 0.3)])
def test_reduce_weighted_bit_exact(gemv, orc, n, hidden, a):
    rng = np.random.default_rng(61 + n)
    y = rng.standard_normal((n, hidden)).astype(np.float32)
    out0 = rng.standard_normal(hidden).astype(np.float32)
    out = dev(out0.copy())
    gemv.reduce_weighted(dev(y) if n else dev(np.zeros(1, np.float32)), out, a, hidden, n)
    assert np.array_equal(bits(host(out)), bits(orc.reduce_weighted(y, a, out0)))


def _q4_0_bank(orc, n_experts, hidden, inter, seed):
    """n_experts experts of q4_0 rows: gate|up [2I x H] then down [H x I]."""
    rng = np.random.default_rng(seed)
    gu = orc.quantize_row((rng.standard_normal((n_experts * 2 * inter, hidden)) * 0.02).astype(np.float32))
    dn = orc.quantize_row((rng.standard_normal((n_experts * hidden, inter)) * 0.02).astype(np.float32))
    gu = gu.reshape(n_experts, 2 * inter, -1)
    dn = dn.reshape(n_experts, hidden, -1)
    bank = np.concatenate([gu.reshape(n_experts, -1), dn.reshape(n_experts, -1)], axis=1)
    return bank, gu, dn


def q8_of(buf, n, nb):
    b = np.ascontiguousarray(buf).view(np.uint8).reshape(n, nb, 40)
    return b[:, :, 0:4].copy().view(np.float32)[:, :, 0], b[:, :, 8:40].copy().view(np.int8).reshape(n, nb * 32)


def test_gemv_grouped_q8_idx_block_dots_and_sums(gemv, orc):
    """gemv_grouped_q8_idx over a q4_0 bank: entry e = expert slots[e] on q8 row
    x_idx[e]; its sums within tolerance of the oracle's AVX2-order GEMV and its
    block dots (same inner loop, block-dot dump) equal the oracle's."""
    E, H, I = 6, 512, 96
    bank, gu, _ = _q4_0_bank(orc, E, H, I, 71)
    eb = bank.shape[1]
    rng = np.random.default_rng(72)
    x = rng.standard_normal((3, H)).astype(np.float32)
    q8 = torch.zeros(3 * (H // 32) * 40, dtype=torch.uint8, device=DEV)
    gemv.quantize_q8(dev(x), H, q8, H, 3)
    slots = np.array([4, 0, 4, 2, 5], np.int32)
    xi = np.array([2, 0, 1, 1, 2], np.int32)
    y = torch.zeros((5, 2 * I), dtype=torch.float32, device=DEV)
    gemv.gemv_grouped_q8_idx(dev(bank.ravel()), eb, 0, dev(slots), dev(xi), 5, q8, H // 32, y, 2 * I, 2 * I, H)
    Y = host(y)
    d8, qs8 = q8_of(host(q8), 3, H // 32)
    for e in range(5):
        ref = orc.gemv_q8(gu[slots[e]], 2 * I, d8[xi[e]], qs8[xi[e]], H)
        assert np.max(np.abs(Y[e] - ref)) <= 1e-3 * np.linalg.norm(ref), e
    dots = torch.zeros((5, 2 * I, H // 32), dtype=torch.int32, device=DEV)
    gemv.block_dots(dev(bank.ravel()), eb, 0, dev(slots), dev(xi), 5, q8, H // 32, dots, 2 * I, H,
                    layout=ft_hip.LAYOUT_Q4_0)
    D = host(dots)
    for e in range(5):
        assert np.array_equal(D[e], orc.block_dots(gu[slots[e]], qs8[xi[e]], H)), e


def test_decode_bench_grouped_layer_call_for_call(gemv, orc):
    """ft-bench/src/bin/decode.rs:272-277, the reference's grouped MoE layer, on
    this surface with the same arguments: the shared activation
    (q8_stride_blocks 0), SiLU*up, the act q8 and the down GEMV, then
    out += ew * sum of the expert outputs. Every integer stage bit-exact on
    the GPU's own input, f32 GEMV outputs within tolerance."""
    E, H, I, n = 10, 1024, 256, 4
    bank, gu, dn = _q4_0_bank(orc, E, H, I, 81)
    eb, gu_bytes = bank.shape[1], gu.shape[1] * gu.shape[2]
    rng = np.random.default_rng(82)
    x = rng.standard_normal(H).astype(np.float32)
    slots = np.array([7, 2, 9, 4], np.int32)
    ew = np.float32(1.0 / n)
    out0 = rng.standard_normal(H).astype(np.float32)
    cache, g_slots = dev(bank.ravel()), dev(slots)
    x_q8 = torch.zeros((H // 32) * 40, dtype=torch.uint8, device=DEV)
    y_gu = torch.zeros((n, 2 * I), dtype=torch.float32, device=DEV)
    act = torch.zeros((n, I), dtype=torch.float32, device=DEV)
    act_q8 = torch.zeros(n * (I // 32) * 40, dtype=torch.uint8, device=DEV)
    y_dn = torch.zeros((n, H), dtype=torch.float32, device=DEV)
    out = dev(out0.copy())
    gemv.quantize_q8(dev(x), 0, x_q8, H, 1)
    gemv.gemv_grouped_q8(cache, eb, 0, g_slots, n, x_q8, 0, y_gu, 2 * I, 2 * I, H)
    gemv.silu_mul_grouped(y_gu, act, I, n)
    gemv.quantize_q8(act, I, act_q8, I, n)
    gemv.gemv_grouped_q8(cache, eb, gu_bytes, g_slots, n, act_q8, I // 32, y_dn, H, H, I)
    gemv.reduce_weighted(y_dn, out, ew, H, n)
    d8, qs8 = q8_of(host(x_q8), 1, H // 32)
    od, oq = orc.q8_quantize(x)
    assert np.array_equal(d8[0], od) and np.array_equal(qs8[0], oq)
    YG, ACT, YD = host(y_gu), host(act), host(y_dn)
    ad, aq = q8_of(host(act_q8), n, I // 32)
    for p in range(n):
        ref = orc.gemv_q8(gu[slots[p]], 2 * I, od, oq, H)
        assert np.max(np.abs(YG[p] - ref)) <= 1e-3 * np.linalg.norm(ref), p
        assert np.array_equal(bits(ACT[p]), bits(orc.silu_mul_grouped(YG[p], I)[0])), p
        rd, rq = orc.q8_quantize(ACT[p])
        assert np.array_equal(ad[p], rd) and np.array_equal(aq[p], rq), p
        ref_dn = orc.gemv_q8(dn[slots[p]], H, ad[p], aq[p], I)
        assert np.max(np.abs(YD[p] - ref_dn)) <= 1e-3 * np.linalg.norm(ref_dn), p
    assert np.array_equal(bits(host(out)), bits(orc.reduce_weighted(YD, ew, out0)))
