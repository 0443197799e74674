"""Expert banks loaded from a GGUF file (ft_hip_load_expert_banks_gguf, the
counterpart of ft-model's bank construction, ft-model/src/lib.rs:570-609)
and a layer run on them with the file's router and expert scales
(lib.rs:506-514, :531): the bank bytes equal the file's q4_0 rows (as is, or
repacked to q4r losslessly), and the layer's routing and q8 stages match the
oracle run on the same file-derived inputs."""
import numpy as np
import pytest
import torch

import ft_hip
from cases import q4r_to_q4_0
from test_gguf import expert_file

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
H, I, E, K, L = 256, 64, 8, 2, 2


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("layout", [ft_hip.LAYOUT_Q4_0, ft_hip.LAYOUT_Q4R])
def test_banks_from_gguf_bytes(gemv, tmp_path, layout):
    path, raw, _ = expert_file(tmp_path, H=H, I=I, E=E, L=L, seed=5)
    g = ft_hip.Gguf(path)
    rbh, rbi = ft_hip.row_bytes(H, layout), ft_hip.row_bytes(I, layout)
    gu_bytes = 2 * I * rbh
    eb = gu_bytes + H * rbi + 48  # spare bytes per expert: the loader must honour expert_bytes
    banks = torch.full((L * E * eb,), 0x5A, dtype=torch.uint8, device=DEV)
    gemv.load_expert_banks_gguf(g, 0, L, H, I, E, banks, eb, layout)
    b = host(banks).reshape(L, E, eb)
    for l in range(L):
        gu, dn = raw[l][0].reshape(E, 2 * I, -1), raw[l][1].reshape(E, H, -1)
        for e in range(E):
            got_gu = b[l, e, :gu_bytes].reshape(2 * I, rbh)
            got_dn = b[l, e, gu_bytes:gu_bytes + H * rbi].reshape(H, rbi)
            if layout == ft_hip.LAYOUT_Q4R:
                got_gu, got_dn = q4r_to_q4_0(got_gu, 2 * I, H), q4r_to_q4_0(got_dn, H, I)
            assert np.array_equal(got_gu.reshape(2 * I, -1), gu[e])
            assert np.array_equal(got_dn.reshape(H, -1), dn[e])
            assert np.all(b[l, e, gu_bytes + H * rbi:] == 0x5A)  # the spare bytes are untouched
    # one layer of a file loaded alone (layer0 = 1)
    one = torch.zeros(E * eb, dtype=torch.uint8, device=DEV)
    gemv.load_expert_banks_gguf(g, 1, 1, H, I, E, one, eb, layout)
    assert np.array_equal(host(one).reshape(E, eb)[:, :gu_bytes + H * rbi], b[1, :, :gu_bytes + H * rbi])


def test_banks_from_gguf_rejects(gemv, tmp_path):
    path, _, _ = expert_file(tmp_path, H=H, I=I, E=E, L=L, seed=6)
    g = ft_hip.Gguf(path)
    eb = 2 * I * ft_hip.row_bytes(H, ft_hip.LAYOUT_Q4R) + H * ft_hip.row_bytes(I, ft_hip.LAYOUT_Q4R)
    banks = torch.zeros(L * E * eb, dtype=torch.uint8, device=DEV)
    for args, code in [((0, 3, H, I, E), ft_hip.E_NOT_FOUND),   # layer 2 is not in the file
                       ((0, 1, H, 2 * I, E), ft_hip.E_SHAPE),   # wrong inter: dims differ
                       ((0, 1, H, I, E + 1), ft_hip.E_SHAPE)]:  # wrong expert count
        with pytest.raises(ft_hip.FtHipError) as ei:
            gemv.load_expert_banks_gguf(g, *args, banks, eb * 4)
        assert ei.value.code == code
    with pytest.raises(ft_hip.FtHipError) as ei:
        gemv.load_expert_banks_gguf(g, 0, 1, H, I, E, banks, eb - 16)
    assert ei.value.code == ft_hip.E_SHAPE


def test_layer_on_gguf_weights(gemv, orc, tmp_path):
    """One layer per file layer, on banks, router and expert scales from the
    file, against the oracle on the same inputs: ids bit-exact, x_out within
    1e-3 * ||y||_2."""
    path, raw, _ = expert_file(tmp_path, H=H, I=I, E=E, L=L, seed=7)
    g = ft_hip.Gguf(path)
    eb = 2 * I * ft_hip.row_bytes(H, ft_hip.LAYOUT_Q4R) + H * ft_hip.row_bytes(I, ft_hip.LAYOUT_Q4R)
    banks = torch.zeros(L * E * eb, dtype=torch.uint8, device=DEV)
    gemv.load_expert_banks_gguf(g, 0, L, H, I, E, banks, eb, ft_hip.LAYOUT_Q4R)
    ws = torch.empty(ft_hip.Q4Gemv.moe_layer_workspace_bytes(1, H, I, E, K), dtype=torch.uint8, device=DEV)
    rng = np.random.default_rng(1)
    gemv.set_input_norm(1)
    try:
        _layers_vs_oracle(gemv, orc, g, raw, banks, eb, ws, rng)
    finally:
        gemv.set_input_norm(0)


def _layers_vs_oracle(gemv, orc, g, raw, banks, eb, ws, rng):
    for l in range(L):
        Wr = g.router_f32(l, H, E)
        es = g.to_f32(f"blk.{l}.ffn_down_exps.scale")
        x = (rng.standard_normal(H) * 4).astype(np.float32)
        xo = torch.zeros(H, dtype=torch.float32, device=DEV)
        ids = torch.zeros(K, dtype=torch.int32, device=DEV)
        wts = torch.zeros(K, dtype=torch.float32, device=DEV)
        gemv.moe_layer(torch.from_numpy(x).to(DEV), xo, 1, H, I, E, K, torch.from_numpy(Wr).to(DEV), None,
                       torch.from_numpy(es).to(DEV), banks[l * E * eb:(l + 1) * E * eb], eb, ft_hip.LAYOUT_Q4R,
                       ids, wts, ws)
        gu, dn = raw[l][0].reshape(E, -1), raw[l][1].reshape(E, -1)
        ref = orc.moe_layer(x, Wr, {e: gu[e] for e in range(E)}, {e: dn[e] for e in range(E)}, H, I, K,
                            expert_scale=es, layout=0, input_norm=True)
        assert np.array_equal(host(ids), ref["ids"])
        assert np.array_equal(host(wts).view(np.uint32), ref["wts"].view(np.uint32))
        y = ref["x_out"] - x
        assert np.max(np.abs(host(xo) - ref["x_out"])) <= 1e-3 * np.linalg.norm(y)
