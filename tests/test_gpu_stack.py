"""ft_hip_moe_stack: L launch-by-launch layers in one call, each layer's
router head computed by the previous layer's down launch (k_gemv_down_head,
k_gemv_gu_act<HEAD>). Its states, ids and weights must equal L calls of
ft_hip_moe_layer bit for bit (the same R-order logits, norm scale and q8(x),
ft-model/src/lib.rs:1406-1476 per layer), on shapes that fold (16*k*lanes
threads per down workgroup: 256, 512, 1024) and on one that does not."""
import numpy as np
import pytest
import torch

import ft_hip
import moe_synth

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _layer_by_layer(m, x, B, expert_scale=None):
    s = m.shape
    k = s.top_k
    ws = m.workspace(B)
    ids = torch.zeros((m.L, B * k), dtype=torch.int32, device=DEV)
    wts = torch.zeros((m.L, B * k), dtype=torch.float32, device=DEV)
    cur = x.clone()
    for l in range(m.L):
        nxt = torch.zeros_like(cur)
        bank = m.banks[l * s.n_experts * m.expert_bytes:(l + 1) * s.n_experts * m.expert_bytes]
        m.g.moe_layer(cur, nxt, B, s.hidden, s.inter, s.n_experts, k, m.routers[l], m.layer_bias(l),
                      None if expert_scale is None else expert_scale[l], bank, m.expert_bytes, m.layout, ids[l],
                      wts[l], ws)
        cur = nxt
    torch.cuda.synchronize()
    return cur, ids, wts


def _stack(m, x, B, expert_scale=None):
    s = m.shape
    k = s.top_k
    ws = m.stack_workspace(B)
    ids = torch.full((m.L, B * k), -7, dtype=torch.int32, device=DEV)
    wts = torch.zeros((m.L, B * k), dtype=torch.float32, device=DEV)
    out = torch.zeros_like(x)
    m.g.moe_stack(x, out, B, s.hidden, s.inter, s.n_experts, k, m.L, m.routers, m.bias, expert_scale, m.banks,
                  m.expert_bytes, m.layout, ids, wts, ws)
    torch.cuda.synchronize()
    return out, ids, wts


def _same(a, b):
    return np.array_equal(a.cpu().numpy().view(np.uint32), b.cpu().numpy().view(np.uint32))


# (hidden, inter, n_experts, top_k, layers, layout, zipf): down workgroups of
# 16*k*lanes threads = 512 (large-expert rows, 16 lanes), 256 (k=2, 8 lanes),
# 1024 (k=8, 8 lanes), 1024 (k=4, 16 lanes); the Gemma shape does not fold
# (its 128 experts' partials exceed the gate|up launch's LDS budget) and
# adds a router bias.
CASES = [
    (4096, 8192, 8, 2, 3, ft_hip.LAYOUT_Q4R, None),
    (1024, 512, 16, 2, 4, ft_hip.LAYOUT_Q4_0, None),
    (1024, 512, 16, 8, 3, ft_hip.LAYOUT_Q4R, None),
    (2048, 8192, 16, 4, 3, ft_hip.LAYOUT_Q4R, None),
    (2816, 704, 128, 8, 3, ft_hip.LAYOUT_Q4R, 1.1),
]


@pytest.mark.parametrize("norm", [1, 0])
@pytest.mark.parametrize("H,I,E,K,L,layout,zipf", CASES)
@pytest.mark.parametrize("B", [1, 3])
def test_stack_equals_layers(gemv, H, I, E, K, L, layout, zipf, B, norm):
    shape = moe_synth.Shape(f"t{H}x{I}x{E}", H, I, E, K, L, 1)
    m = moe_synth.SyntheticMoE(gemv, shape, layout=layout)
    if zipf is not None:
        m.bias = torch.from_numpy(moe_synth.zipf_router_bias(shape, L, zipf, tau=0.895)).to(DEV)
    x = torch.stack([m.hidden(t) for t in range(B)])
    gemv.set_input_norm(norm)
    try:
        ref, rid, rwt = _layer_by_layer(m, x, B)
        out, ids, wts = _stack(m, x, B)
    finally:
        gemv.set_input_norm(0)
    assert torch.equal(ids, rid)
    assert _same(wts, rwt)
    assert _same(out, ref)
    assert torch.isfinite(out).all()


def test_stack_expert_scale_and_no_fold(gemv):
    """Per-layer expert scales reach the routing weights of every layer; a shape
    whose down workgroup would need 2048 threads (k = 8 with 16 lanes) runs
    layer by layer inside the call, with the same bits."""
    for H, I, E, K in [(2048, 8192, 16, 2), (1024, 8192, 16, 8)]:
        shape = moe_synth.Shape(f"s{H}x{I}x{K}", H, I, E, K, 3, 1)
        m = moe_synth.SyntheticMoE(gemv, shape)
        B = 2
        x = torch.stack([m.hidden(t) for t in range(B)])
        es = (torch.arange(3 * E, dtype=torch.float32, device=DEV).view(3, E) * 0.01 + 0.5).contiguous()
        ref, rid, rwt = _layer_by_layer(m, x, B, es)
        out, ids, wts = _stack(m, x, B, es)
        assert torch.equal(ids, rid)
        assert _same(wts, rwt)
        assert _same(out, ref)


def test_stack_rejects(gemv):
    shape = moe_synth.Shape("r", 1024, 512, 16, 2, 2, 1)
    m = moe_synth.SyntheticMoE(gemv, shape)
    x = m.hidden(0).view(1, -1)
    ws = m.stack_workspace(1)
    ids = torch.zeros((2, 2), dtype=torch.int32, device=DEV)
    wts = torch.zeros((2, 2), dtype=torch.float32, device=DEV)
    s = m.shape
    with pytest.raises(ft_hip.FtHipError) as ei:
        gemv.moe_stack(x, x.clone(), 1, s.hidden, s.inter, s.n_experts, s.top_k, 2, m.routers, None, None, m.banks,
                       m.expert_bytes, m.layout, ids, wts, ws[:ws.numel() - 256])
    assert ei.value.code == ft_hip.E_SHAPE
    with pytest.raises(ft_hip.FtHipError) as ei:
        gemv.moe_stack(x, x.clone(), 1, s.hidden, s.inter, s.n_experts, s.top_k, 0, m.routers, None, None, m.banks,
                       m.expert_bytes, m.layout, ids, wts, ws)
    assert ei.value.code == ft_hip.E_SHAPE
