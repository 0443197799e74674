"""ft_hip_moe_layer_noalloc (the layer on the library's own scratch array,
for callers that cannot allocate) against ft_hip_moe_layer with a caller
workspace: same kernels, so the same bits -- routing ids and weights and
x_out -- on two calls in a row, the second with fewer tokens (the scratch
keeps the first call's contents), with and without the input norm; a shape
whose scratch would exceed FT_HIP_NOALLOC_SCRATCH_BYTES is refused before
any GPU work. Both calls go through the C ABI (ctypes)."""
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


@pytest.fixture(scope="module")
def layer(gemv):
    return moe_synth.SyntheticMoE(gemv, moe_synth.GEMMA, n_layers=1, zipf_s=1.1)


def _both(gemv, m, x, n, norm):
    s = m.shape
    E, K = s.n_experts, s.top_k
    bank = m.banks[:E * m.expert_bytes]
    args = (n, s.hidden, s.inter, E, K, m.routers[0], m.layer_bias(0), None, bank, m.expert_bytes, m.layout)
    ref = [torch.zeros((n, s.hidden), dtype=torch.float32, device=DEV),
           torch.zeros(n * K, dtype=torch.int32, device=DEV), torch.zeros(n * K, dtype=torch.float32, device=DEV)]
    got = [torch.full((n, s.hidden), 7.0, dtype=torch.float32, device=DEV),
           torch.full((n * K,), -5, dtype=torch.int32, device=DEV),
           torch.full((n * K,), 7.0, dtype=torch.float32, device=DEV)]
    ws = torch.zeros(gemv.moe_layer_workspace_bytes(n, s.hidden, s.inter, E, K), dtype=torch.uint8, device=DEV)
    gemv.set_input_norm(norm)
    try:
        gemv.moe_layer(x, ref[0], *args, ref[1], ref[2], ws)
        gemv.moe_layer_noalloc(x, got[0], *args, got[1], got[2])
    finally:
        gemv.set_input_norm(0)
    return [host(t) for t in ref], [host(t) for t in got]


@pytest.mark.parametrize("norm", [0, 1])
def test_noalloc_matches_workspace_layer(gemv, layer, norm):
    m = layer
    H = m.shape.hidden
    for n in (12, 5):  # the second call smaller than the first
        x = torch.empty((n, H), dtype=torch.float32, device=DEV)
        for t in range(n):
            m.hidden(100 + 17 * n + t, x[t])
        ref, got = _both(gemv, m, x, n, norm)
        assert np.array_equal(got[1], ref[1]), n
        assert np.array_equal(got[2].view(np.uint32), ref[2].view(np.uint32)), n
        assert np.array_equal(got[0].view(np.uint32), ref[0].view(np.uint32)), n


def test_noalloc_rejects_oversized_shape(gemv, layer):
    m = layer
    s = m.shape
    n = 512  # y of n*top_k pairs alone is 46 MB > the 8 MiB scratch
    assert gemv.moe_layer_workspace_bytes(n, s.hidden, s.inter, s.n_experts, s.top_k) > ft_hip.NOALLOC_SCRATCH_BYTES
    x = torch.zeros((n, s.hidden), dtype=torch.float32, device=DEV)
    ids = torch.zeros(n * s.top_k, dtype=torch.int32, device=DEV)
    wts = torch.zeros(n * s.top_k, dtype=torch.float32, device=DEV)
    with pytest.raises(ft_hip.FtHipError) as ei:
        gemv.moe_layer_noalloc(x, x, n, s.hidden, s.inter, s.n_experts, s.top_k, m.routers[0], None, None,
                               m.banks, m.expert_bytes, m.layout, ids, wts)
    assert ei.value.code == ft_hip.E_SHAPE
    assert "scratch" in str(ei.value)


def test_noalloc_rejects_wrapping_n_seqs(gemv, layer):
    """n_seqs = 2^61 + 1 with top_k 4: n_seqs * top_k wraps in 64 bits; the
    shape is refused by division before any size or offset is formed (no
    kernel runs: the pointers are never dereferenced)."""
    m = layer
    s = m.shape
    x = torch.zeros(s.hidden, dtype=torch.float32, device=DEV)
    ids = torch.zeros(4, dtype=torch.int32, device=DEV)
    wts = torch.zeros(4, dtype=torch.float32, device=DEV)
    with pytest.raises(ft_hip.FtHipError) as ei:
        gemv.moe_layer_noalloc(x, x, (1 << 61) + 1, s.hidden, s.inter, s.n_experts, 4, m.routers[0], None, None,
                               m.banks, m.expert_bytes, m.layout, ids, wts)
    assert ei.value.code == ft_hip.E_SHAPE
