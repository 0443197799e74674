"""CPU tests of the C-ABI boundary: the library loads, exports every symbol
that include/ft_hip.h declares, and turns violated shape preconditions into
FT_HIP_E_SHAPE (where the reference panics, e.g. ft-cuda/src/lib.rs:171-173)
before it touches a GPU. No compute entry point is called with valid inputs.
"""
import ctypes
import os
import re

import pytest

import ft_hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "ft_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ft_hip_\w+)\s*\(", text)))


def test_every_declared_symbol_is_exported_and_bound():
    L = ft_hip.lib()
    names = declared_symbols()
    assert len(names) >= 19
    for n in names:
        assert hasattr(L, n), n
        assert n in ft_hip.SIGNATURES, n


def test_version_and_sizes():
    L = ft_hip.lib()
    assert L.ft_hip_version() >= 100
    assert ft_hip.row_bytes(2816, ft_hip.LAYOUT_Q4_0) == 1584
    assert ft_hip.row_bytes(704, ft_hip.LAYOUT_Q4R) == 400       # 44 B of scales padded to 48, + 352
    assert ft_hip.row_bytes(2816, ft_hip.LAYOUT_Q4R) == 1584
    assert ft_hip.q4r_scales_bytes(704) == 48
    assert ft_hip.row_bytes(33, ft_hip.LAYOUT_Q4_0) == -1
    assert L.ft_hip_moe_layer_workspace_bytes(1, 2816, 704, 128, 8) > 0


def test_create_without_gpu_reports_device_error():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    ctx = ctypes.c_void_p()
    rc = ft_hip.lib().ft_hip_create(0, ctypes.byref(ctx))
    assert rc == ft_hip.E_DEVICE
    assert b"device" in ft_hip.lib().ft_hip_last_error()
    with pytest.raises(ft_hip.FtHipError):
        ft_hip.Q4Gemv(0)


def _err(rc):
    return rc, ft_hip.lib().ft_hip_last_error().decode()


def test_shape_errors_are_reported_before_any_gpu_call():
    L = ft_hip.lib()
    P = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    rc, msg = _err(L.ft_hip_quantize_q8(None, None, P, 0, P, 33, 1))
    assert rc == ft_hip.E_SHAPE and "multiple of 32" in msg
    rc, _ = _err(L.ft_hip_quantize_q8(None, None, P, 16, P, 32, 1))   # x_stride < k
    assert rc == ft_hip.E_SHAPE
    rc, _ = _err(L.ft_hip_quantize_q8(None, None, P, 0, P, 64, 1))    # valid shape, null ctx
    assert rc == ft_hip.E_INVALID
    rc, _ = _err(L.ft_hip_gemv_q4_grouped_ptr(None, None, P, 0, None, 1, P, 0, P, 10, 20, 100, 1))
    assert rc == ft_hip.E_SHAPE                                          # k = 100
    rc, _ = _err(L.ft_hip_gemv_q4_grouped_ptr(None, None, P, 0, None, 2, P, 0, P, 10, 20, 128, 1))
    assert rc == ft_hip.E_SHAPE                                          # y_stride < n_rows
    rc, _ = _err(L.ft_hip_gemv_q4_grouped_ptr(None, None, P, 0, None, 1, P, 0, P, 20, 20, 128, 7))
    assert rc == ft_hip.E_INVALID                                        # layout 7
    rc, _ = _err(L.ft_hip_gemv_q4_grouped_slots(None, None, ctypes.c_void_p(0x1008), 1600, 0, P, None, 1, P, 0,
                                                P, 20, 20, 128, 1))
    assert rc == ft_hip.E_SHAPE                                          # q4r base not 16-B aligned
    rc, _ = _err(L.ft_hip_router_logits(None, None, P, P, None, P, 2880, 128, 1))
    assert rc == ft_hip.E_SHAPE                                          # dim % 128
    rc, _ = _err(L.ft_hip_topk_router(None, None, P, None, P, P, 2048, 8, 1))
    assert rc == ft_hip.E_SHAPE                                          # e_count > 1024
    rc, _ = _err(L.ft_hip_topk_router(None, None, P, None, P, P, 128, 33, 1))
    assert rc == ft_hip.E_SHAPE                                          # k > 32
    rc, _ = _err(L.ft_hip_gelu_mul_q8(None, None, P, P, 700, 1))
    assert rc == ft_hip.E_SHAPE
    rc, _ = _err(L.ft_hip_moe_layer(None, None, P, P, 1, 2816, 704, 128, 8, P, None, None, P, 100, 1, P, P, P,
                                    1 << 30))
    assert rc == ft_hip.E_SHAPE                                          # expert_bytes too small
    ws = L.ft_hip_moe_layer_workspace_bytes(1, 2816, 704, 128, 8)
    rc, _ = _err(L.ft_hip_moe_layer(None, None, P, P, 1, 2816, 704, 128, 8, P, None, None, P, 1 << 30, 1, P, P,
                                    P, ws - 1))
    assert rc == ft_hip.E_SHAPE                                          # workspace too small


def test_huge_n_seqs_cannot_wrap_the_shape_checks():
    """A huge n_seqs (2^61 + 1 with top_k 4: the pair count wraps in 64 bits)
    is rejected by division, and the workspace sizes of such shapes are 0."""
    L = ft_hip.lib()
    P = ctypes.c_void_p(16)
    huge = (1 << 61) + 1
    rc, msg = _err(L.ft_hip_moe_layer(None, None, P, P, huge, 2816, 704, 128, 4, P, None, None, P, 1 << 30, 1, P,
                                      P, P, 1 << 30))
    assert rc == ft_hip.E_SHAPE and "n_seqs" in msg
    rc, _ = _err(L.ft_hip_moe_layer(None, None, P, P, 65535 // 4 + 1, 2816, 704, 128, 4, P, None, None, P, 1 << 30,
                                    1, P, P, P, 1 << 30))
    assert rc == ft_hip.E_SHAPE
    for fn in ("ft_hip_moe_layer_workspace_bytes", "ft_hip_moe_stack_workspace_bytes",
               "ft_hip_moe_layer_grouped_workspace_bytes"):
        assert getattr(L, fn)(huge, 2816, 704, 128, 4) == 0, fn
        assert getattr(L, fn)(16383, 2816, 704, 128, 4) > 0, fn
    assert L.ft_hip_moe_layer_workspace_bytes(1, 1 << 40, 704, 128, 8) == 0


def test_new_surface_shape_errors():
    """silu/gelu_mul_grouped and the expert reductions reject bad shapes before any GPU call."""
    L = ft_hip.lib()
    P = ctypes.c_void_p(16)
    for fn in (L.ft_hip_silu_mul_grouped, L.ft_hip_gelu_mul_grouped):
        assert _err(fn(None, None, P, P, 0, 4))[0] == ft_hip.E_SHAPE          # inter 0
        assert _err(fn(None, None, P, P, 64, -1))[0] == ft_hip.E_SHAPE        # negative n_experts
        assert _err(fn(None, None, P, P, 1 << 40, 1 << 20))[0] == ft_hip.E_SHAPE  # inter * n too large
        assert _err(fn(None, None, None, P, 64, 4))[0] == ft_hip.E_INVALID
    assert _err(L.ft_hip_reduce_expert_weighted(None, None, P, P, P, 0, 4))[0] == ft_hip.E_SHAPE
    assert _err(L.ft_hip_reduce_expert_weighted(None, None, P, P, P, 64, 70000))[0] == ft_hip.E_SHAPE
    assert _err(L.ft_hip_reduce_expert_weighted(None, None, P, None, P, 64, 4))[0] == ft_hip.E_INVALID
    assert _err(L.ft_hip_reduce_weighted(None, None, P, P, 1.0, -5, 4))[0] == ft_hip.E_SHAPE
    assert _err(L.ft_hip_reduce_weighted(None, None, P, None, 1.0, 64, 4))[0] == ft_hip.E_INVALID


def test_fused_workgroups_formula():
    """K*max(I/32, H/128) expert units, two group units (each with half of
    the experts' router sums), a pred unit and a refiner unit per R-order group."""
    assert ft_hip.Q4Gemv.fused_workgroups(2816, 704, 128, 8) == 8 * 22 + 4 * 8
    assert ft_hip.Q4Gemv.fused_workgroups(2816, 352, 128, 4) == 4 * 22 + 4 * 8
    assert ft_hip.Q4Gemv.fused_workgroups(4096, 512, 64, 2) == 2 * 32 + 4 * 8
    assert ft_hip.Q4Gemv.fused_workgroups(2816, 700, 128, 8) == -1


def test_fused_predictor_sizes_and_errors():
    """The refined-prediction table: (L-1) * E records of E x I/32 blocks of
    36 B; bad shapes and null arguments are refused before any GPU call."""
    L = ft_hip.lib()
    P = ctypes.c_void_p(16)
    assert ft_hip.Q4Gemv.fused_predictor_bytes(2816, 704, 128, 30) == 29 * 128 * 128 * 22 * 36
    assert ft_hip.Q4Gemv.fused_predictor_bytes(2816, 704, 128, 1) == 0
    assert ft_hip.Q4Gemv.fused_predictor_bytes(2816, 700, 128, 4) == -1
    assert ft_hip.Q4Gemv.fused_predictor_bytes(2816, 704, 128, 0) == -1
    need = ft_hip.Q4Gemv.fused_predictor_bytes(2816, 704, 128, 4)
    assert _err(L.ft_hip_fused_build_predictor(None, None, P, P, 2880, 704, 128, 4, P, need))[0] == ft_hip.E_SHAPE
    assert _err(L.ft_hip_fused_build_predictor(None, None, P, P, 2816, 704, 128, 4, P, need - 1))[0] == ft_hip.E_SHAPE
    assert _err(L.ft_hip_fused_build_predictor(None, None, P, P, 2816, 704, 128, 4, P, need))[0] == ft_hip.E_INVALID
    assert _err(L.ft_hip_fused_set_predictor(None, P, need, 4))[0] == ft_hip.E_INVALID
