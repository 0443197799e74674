"""The Zipf-skewed routing configuration: its router
bias scale is calibrated so that routing follows Zipf(1.1) popularity.

Calibration target: the share of routed (token, expert) pairs that land on a
layer's 8 most popular experts equals the Zipf(1.1) mass of the top 8 of 128
ranks (0.5668). A per-rank match is impossible at the top (an expert is
chosen at most once per token, while Zipf(1.1) gives rank 1 alone 22.6 % of
the mass), so the check pins the top-8 share and the ordering of the
selection rates.
"""
import numpy as np
import pytest

import moe_synth

S = 1.1


def test_host_generator_matches_oracle(orc):
    """The numpy generator used by the calibration is the device/oracle one."""
    for cfg, l, e, t, sigma in [(1, 0, 0, moe_synth.T_ROUTER, 0.02), (1, 3, 5, moe_synth.T_HIDDEN, 1.0),
                                (5, 31, 0, moe_synth.T_ROUTER, 0.02)]:
        key = moe_synth.tensor_key(cfg, l, e, t)
        assert key == orc.tensor_key(cfg, l, e, t)
        a = moe_synth.gen_values_np(key, 4096, moe_synth.gen_scale(sigma))
        b = orc.gen_values(key, 0, 4096, sigma)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_zipf_mass():
    p = np.arange(1, 129, dtype=np.float64) ** -S
    assert moe_synth.zipf_mass(128, 8, S) == pytest.approx(p[:8].sum() / p.sum())
    assert moe_synth.zipf_mass(128, 8, S) == pytest.approx(0.5668, abs=1e-4)
    assert moe_synth.zipf_mass(128, 128, S) == pytest.approx(1.0)


def test_calibrated_tau_reproduces():
    tau = moe_synth.calibrate_zipf_tau(moe_synth.GEMMA, S)
    assert tau == pytest.approx(moe_synth.ZIPF_TAU[(moe_synth.GEMMA.name, S)], abs=0.005)


def test_zipf_share_all_layers():
    """Over all 30 layers of the configuration (other tokens than the
    calibration's), the top-8 share is Zipf's mass; without the bias it is
    the uniform 8/128; the old uncalibrated scale 0.02*sqrt(H) overshoots."""
    g = moe_synth.GEMMA
    target = moe_synth.zipf_mass(g.n_experts, g.top_k, S)
    tau = moe_synth.ZIPF_TAU[(g.name, S)]
    share = moe_synth.zipf_top_share(g, g.n_layers, S, tau, n_tokens=128)
    assert abs(share - target) < 0.015
    assert moe_synth.zipf_top_share(g, 4, S, 0.0, n_tokens=128) == pytest.approx(8 / 128, abs=0.02)
    assert moe_synth.zipf_top_share(g, 4, S, 0.02 * np.sqrt(g.hidden), n_tokens=128) > target + 0.04


def test_zipf_selection_rate_falls_with_rank():
    """Selection rate per popularity rank, pooled over 8 layers: decreasing
    in rank bands (1-4 > 5-16 > 17-64 > 65-128), as Zipf orders them."""
    g = moe_synth.GEMMA
    H, E, k = g.hidden, g.n_experts, g.top_k
    tau = moe_synth.ZIPF_TAU[(g.name, S)]
    xs = np.stack([moe_synth.gen_values_np(moe_synth.tensor_key(g.cfg_id, 0, t, moe_synth.T_HIDDEN), H,
                                           moe_synth.gen_scale(1.0)) for t in range(128)]).astype(np.float64)
    xs /= np.sqrt((xs * xs).mean(axis=1, keepdims=True) + 1e-6)
    ranks = moe_synth.zipf_ranks(g, 8)
    bias = moe_synth.zipf_router_bias(g, 8, S)
    rate = np.zeros(E)
    for l in range(8):
        W = moe_synth.gen_values_np(moe_synth.tensor_key(g.cfg_id, l, 0, moe_synth.T_ROUTER), E * H,
                                    moe_synth.gen_scale(0.02)).reshape(E, H).astype(np.float64)
        top = np.argsort(-(xs @ W.T + bias[l][None, :]), axis=1, kind="stable")[:, :k]
        np.add.at(rate, ranks[l][top].ravel() - 1, 1.0)
    rate /= 8 * 128
    bands = [rate[0:4].mean(), rate[4:16].mean(), rate[16:64].mean(), rate[64:128].mean()]
    assert all(a > b for a, b in zip(bands, bands[1:])), bands
    assert rate.sum() == pytest.approx(k)
