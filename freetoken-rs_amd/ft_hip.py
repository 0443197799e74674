"""Python host binding of libfthip.so (include/ft_hip.h) over ctypes.

`Q4Gemv` mirrors the reference's ft_cuda::Q4Gemv (ft-cuda/src/lib.rs:69-150):
same method names, same argument meaning, device buffers owned by the caller
(torch tensors on the GPU here), launches asynchronous on a stream. Where the
reference panics on a violated shape (assert!), these methods raise
FtHipError carrying the library's status code and message.

PyTorch is used only for device memory and streams. There is no CPU fallback:
if libfthip.so is missing or no gfx950 GPU is present, construction fails.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libfthip.so")

OK, E_INVALID, E_SHAPE, E_DEVICE, E_LAUNCH, E_TIMEOUT = 0, -1, -2, -3, -4, -5
E_IO, E_FORMAT, E_NOT_FOUND = -6, -7, -8
NOALLOC_SCRATCH_BYTES = 8 << 20  # FT_HIP_NOALLOC_SCRATCH_BYTES
Q8_BLK = 40
LAYOUT_Q4_0, LAYOUT_Q4R = 0, 1

_lib = None

# Exported symbols and their signatures (kept in step with include/ft_hip.h).
_P, _I, _I64, _U64, _F, _SZ = (ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint64,
                               ctypes.c_float, ctypes.c_size_t)
SIGNATURES = {
    "ft_hip_version": (_I, []),
    "ft_hip_last_error": (ctypes.c_char_p, []),
    "ft_hip_create": (_I, [_I, ctypes.POINTER(_P)]),
    "ft_hip_destroy": (_I, [_P]),
    "ft_hip_row_bytes": (_I64, [_I, _I64]),
    "ft_hip_q4r_scales_bytes": (_I64, [_I64]),
    "ft_hip_quantize_q8": (_I, [_P, _P, _P, _I64, _P, _I64, _I64]),
    "ft_hip_gemv_q4_grouped_ptr": (_I, [_P, _P, _P, _U64, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I]),
    "ft_hip_gemv_q4_grouped_slots": (_I, [_P, _P, _P, _U64, _U64, _P, _P, _I64, _P, _I64, _P, _I64, _I64,
                                          _I64, _I]),
    "ft_hip_q4q8_block_dots": (_I, [_P, _P, _P, _U64, _U64, _P, _P, _I64, _P, _I64, _P, _I64, _I64, _I]),
    "ft_hip_gelu_mul_q8": (_I, [_P, _P, _P, _P, _I64, _I64]),
    "ft_hip_silu_mul_grouped": (_I, [_P, _P, _P, _P, _I64, _I64]),
    "ft_hip_gelu_mul_grouped": (_I, [_P, _P, _P, _P, _I64, _I64]),
    "ft_hip_reduce_expert_weighted": (_I, [_P, _P, _P, _P, _P, _I64, _I64]),
    "ft_hip_reduce_weighted": (_I, [_P, _P, _P, _P, ctypes.c_float, _I64, _I64]),
    "ft_hip_gemv_gate_up_act": (_I, [_P, _P, _P, _U64, _P, _I64, _I64, _P, _I64, _I64, _I, _P, _P]),
    "ft_hip_gemv_q4r_f32in": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64]),
    "ft_hip_router_logits": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64]),
    "ft_hip_topk_router": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64]),
    "ft_hip_reduce_pairs_weighted": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64]),
    "ft_hip_repack_rows": (_I, [_P, _P, _P, _I, _P, _I, _I64, _I64]),
    "ft_hip_gen_values": (_I, [_P, _P, _U64, _I64, _I64, _F, _P]),
    "ft_hip_gen_q4_rows": (_I, [_P, _P, _U64, _I64, _I64, _I64, _F, _P, _I]),
    "ft_hip_moe_layer_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I64]),
    "ft_hip_moe_layer": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _U64, _I, _P, _P,
                              _P, _SZ]),
    "ft_hip_moe_layer_noalloc": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _U64, _I, _P,
                                      _P]),
    "ft_hip_moe_stack_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I64]),
    "ft_hip_moe_stack": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _U64, _I, _P,
                              _P, _P, _SZ]),
    "ft_hip_moe_layer_grouped_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I64]),
    "ft_hip_moe_layer_grouped": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P,
                                      _SZ, _P, _P]),
    "ft_hip_moe_stack_grouped_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64, _I64, _I64]),
    "ft_hip_moe_stack_grouped": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P,
                                      _P, _P, _P, _SZ]),
    "ft_hip_fused_expert_bytes": (_I64, [_I64, _I64]),
    "ft_hip_fused_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64]),
    "ft_hip_fused_workgroups": (ctypes.c_int, [_I64, _I64, _I64, _I64]),
    "ft_hip_fused_set_spin_limit": (_I, [_P, _I]),
    "ft_hip_fused_set_prefetch": (_I, [_P, _I]),
    "ft_hip_fused_set_cooperative": (_I, [_P, _I]),
    "ft_hip_fused_predictor_bytes": (_I64, [_I64, _I64, _I64, _I64]),
    "ft_hip_fused_build_predictor": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _SZ]),
    "ft_hip_fused_set_predictor": (_I, [_P, _P, _SZ, _I64]),
    "ft_hip_set_input_norm": (_I, [_P, _I]),
    "ft_hip_set_grouped_mfma_min": (_I, [_P, _I]),
    "ft_hip_set_gemv_lanes": (_I, [_P, _I]),
    "ft_hip_stream_read": (_I, [_P, _P, _P, _U64, _P, _I]),
    "ft_hip_set_block_dot_record": (_I, [_P, _P, _P]),
    "ft_hip_set_layer_record": (_I, [_P, _P, _P, _P, _P, _P, _P]),
    "ft_hip_fused_workspace_init": (_I, [_P, _P, _P, _SZ]),
    "ft_hip_fused_workspace_set_epoch": (_I, [_P, _P, _P, ctypes.c_uint32]),
    "ft_hip_pack_experts_fused": (_I, [_P, _P, _P, _I, _U64, _P, _I64, _I64, _I64]),
    "ft_hip_pack_router_fused": (_I, [_P, _P, _P, _P, _I64, _I64, _I64]),
    "ft_hip_moe_stack_fused": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P,
                                    _SZ, _P, _P, _P, _P]),
    "ft_hip_fused_status": (_I, [_P, _P, ctypes.POINTER(_I)]),
    "ft_gguf_open": (_I, [ctypes.c_char_p, ctypes.POINTER(_P)]),
    "ft_gguf_close": (_I, [_P]),
    "ft_gguf_version": (ctypes.c_uint32, [_P]),
    "ft_gguf_data_start": (_U64, [_P]),
    "ft_gguf_n_kv": (_I64, [_P]),
    "ft_gguf_n_tensors": (_I64, [_P]),
    "ft_gguf_kv_key": (_I, [_P, _I64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_uint32)]),
    "ft_gguf_meta_type": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32)]),
    "ft_gguf_meta_u64": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(_U64)]),
    "ft_gguf_meta_f32": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(_F)]),
    "ft_gguf_meta_str": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(_P), ctypes.POINTER(_U64)]),
    "ft_gguf_meta_array": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(_U64)]),
    "ft_gguf_meta_array_u64": (_I, [_P, ctypes.c_char_p, _U64, ctypes.POINTER(_U64)]),
    "ft_gguf_meta_array_bool": (_I, [_P, ctypes.c_char_p, _U64, ctypes.POINTER(_I)]),
    "ft_gguf_meta_array_str": (_I, [_P, ctypes.c_char_p, _U64, ctypes.POINTER(_P), ctypes.POINTER(_U64)]),
    "ft_gguf_tensor_name": (_I, [_P, _I64, ctypes.POINTER(ctypes.c_char_p)]),
    "ft_gguf_tensor_info": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(_U64),
                                 ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(_U64), ctypes.POINTER(_U64)]),
    "ft_gguf_tensor_data": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(_P), ctypes.POINTER(_U64)]),
    "ft_gguf_tensor_to_f32": (_I, [_P, ctypes.c_char_p, _P, _U64]),
    "ft_gguf_router_f32": (_I, [_P, _I64, _I64, _I64, _P]),
    "ft_hip_load_expert_banks_gguf": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _U64, _I]),
}


class FtHipError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"ft_hip error {code}: {msg}")
        self.code = code


def lib():
    """Load libfthip.so; raise if it has not been built (no fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FtHipError(E_DEVICE, f"{LIB_PATH} is missing: run freetoken-rs_amd/build.py")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc):
    if rc != OK:
        raise FtHipError(rc, lib().ft_hip_last_error().decode())
    return rc


def row_bytes(k, layout=LAYOUT_Q4_0):
    return lib().ft_hip_row_bytes(layout, k)


def q4r_scales_bytes(k):
    return lib().ft_hip_q4r_scales_bytes(k)


def _ptr(t):
    """Raw device pointer of a tensor (None -> NULL)."""
    if t is None:
        return None
    return ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    if stream is None:
        import torch
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


class Q4Gemv:
    """Counterpart of ft_cuda::Q4Gemv on one gfx950 device."""

    def __init__(self, device=0):
        self._ctx = ctypes.c_void_p()
        check(lib().ft_hip_create(device, ctypes.byref(self._ctx)))
        self.device = device

    def close(self):
        if self._ctx:
            lib().ft_hip_destroy(self._ctx)
            self._ctx = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- ft-cuda/src/lib.rs:898-921 --
    def quantize_q8(self, x, x_stride, q8, k, n, stream=None):
        check(lib().ft_hip_quantize_q8(self._ctx, _stream(stream), _ptr(x), x_stride, _ptr(q8), k, n))

    # -- ft-cuda/src/lib.rs:593-623 (q4_0) and :736-767 (q4r) --
    def gemv_grouped_ptr(self, bases, bank_off, x_idx, n_entries, q8, q8_stride_blocks, y, y_stride,
                         n_rows, k, layout=LAYOUT_Q4R, stream=None):
        check(lib().ft_hip_gemv_q4_grouped_ptr(self._ctx, _stream(stream), _ptr(bases), bank_off, _ptr(x_idx),
                                               n_entries, _ptr(q8), q8_stride_blocks, _ptr(y), y_stride, n_rows,
                                               k, layout))

    def gemv_grouped_q8_ptr(self, bases, bank_off, x_idx, n_entries, q8, q8_stride_blocks, y, y_stride,
                            n_rows, k, stream=None):
        self.gemv_grouped_ptr(bases, bank_off, x_idx, n_entries, q8, q8_stride_blocks, y, y_stride, n_rows, k,
                              LAYOUT_Q4_0, stream)

    def gemv_q4r_ptr(self, bases, bank_off, x_idx, n_entries, q8, q8_stride_blocks, y, y_stride, n_rows, k,
                     stream=None):
        self.gemv_grouped_ptr(bases, bank_off, x_idx, n_entries, q8, q8_stride_blocks, y, y_stride, n_rows, k,
                              LAYOUT_Q4R, stream)

    # -- ft-cuda/src/lib.rs:926-957, :772-804 (q4_0) and :699-732 (q4r) --
    def gemv_grouped_slots(self, cache, expert_bytes, bank_off, slots, x_idx, n_entries, q8, q8_stride_blocks,
                           y, y_stride, n_rows, k, layout=LAYOUT_Q4R, stream=None):
        check(lib().ft_hip_gemv_q4_grouped_slots(self._ctx, _stream(stream), _ptr(cache), expert_bytes, bank_off,
                                                 _ptr(slots), _ptr(x_idx), n_entries, _ptr(q8), q8_stride_blocks,
                                                 _ptr(y), y_stride, n_rows, k, layout))

    def gemv_grouped_q8(self, cache, expert_bytes, bank_off, slots, n_experts, q8, q8_stride_blocks, y,
                        y_stride, n_rows, k, stream=None):
        self.gemv_grouped_slots(cache, expert_bytes, bank_off, slots, None, n_experts, q8, q8_stride_blocks, y,
                                y_stride, n_rows, k, LAYOUT_Q4_0, stream)

    def gemv_grouped_q8_idx(self, cache, expert_bytes, bank_off, slots, x_idx, n_entries, q8, q8_stride_blocks,
                            y, y_stride, n_rows, k, stream=None):
        self.gemv_grouped_slots(cache, expert_bytes, bank_off, slots, x_idx, n_entries, q8, q8_stride_blocks, y,
                                y_stride, n_rows, k, LAYOUT_Q4_0, stream)

    def gemv_q4r_idx(self, cache, expert_bytes, bank_off, slots, x_idx, n_entries, q8, q8_stride_blocks, y,
                     y_stride, n_rows, k, stream=None):
        self.gemv_grouped_slots(cache, expert_bytes, bank_off, slots, x_idx, n_entries, q8, q8_stride_blocks, y,
                                y_stride, n_rows, k, LAYOUT_Q4R, stream)

    def block_dots(self, cache, expert_bytes, bank_off, slots, x_idx, n_entries, q8, q8_stride_blocks, out,
                   n_rows, k, layout=LAYOUT_Q4R, stream=None):
        check(lib().ft_hip_q4q8_block_dots(self._ctx, _stream(stream), _ptr(cache), expert_bytes, bank_off,
                                           _ptr(slots), _ptr(x_idx), n_entries, _ptr(q8), q8_stride_blocks,
                                           _ptr(out), n_rows, k, layout))

    # -- ft-cuda/src/lib.rs:354-374 --
    def gemv_q4r_f32in(self, w, x, y, act, n_rows, k, stream=None):
        """y = w . q8(x), the q8 of the f32 row x computed in the launch; act (or
        None): for a gate|up matrix, also gelu_tanh(gate) * up per column."""
        check(lib().ft_hip_gemv_q4r_f32in(self._ctx, _stream(stream), _ptr(w), _ptr(x), _ptr(y), _ptr(act), n_rows,
                                          k))

    def gelu_mul_q8(self, gu, q8, inter, n, stream=None):
        check(lib().ft_hip_gelu_mul_q8(self._ctx, _stream(stream), _ptr(gu), _ptr(q8), inter, n))

    # -- ft-cuda/src/lib.rs:1009-1094: grouped activations and expert reductions --
    def silu_mul_grouped(self, gu, out, inter, n_experts, stream=None):
        check(lib().ft_hip_silu_mul_grouped(self._ctx, _stream(stream), _ptr(gu), _ptr(out), inter, n_experts))

    def gelu_mul_grouped(self, gu, out, inter, n_experts, stream=None):
        check(lib().ft_hip_gelu_mul_grouped(self._ctx, _stream(stream), _ptr(gu), _ptr(out), inter, n_experts))

    def reduce_expert_weighted(self, y, wts, out, hidden, n_experts, stream=None):
        check(lib().ft_hip_reduce_expert_weighted(self._ctx, _stream(stream), _ptr(y), _ptr(wts), _ptr(out), hidden,
                                                  n_experts))

    def reduce_weighted(self, y, out, a, hidden, n_experts, stream=None):
        check(lib().ft_hip_reduce_weighted(self._ctx, _stream(stream), _ptr(y), _ptr(out), float(a), hidden,
                                           n_experts))

    # -- ft-model/src/lib.rs:1584-1593 (gate|up GEMV then gelu_mul_q8), one launch --
    def gemv_gate_up_act(self, bank, expert_bytes, slots, n_pairs, x_div, q8x, hidden, inter, q8_act,
                         layout=LAYOUT_Q4R, in_scale=None, stream=None):
        check(lib().ft_hip_gemv_gate_up_act(self._ctx, _stream(stream), _ptr(bank), expert_bytes, _ptr(slots),
                                            n_pairs, x_div, _ptr(q8x), hidden, inter, layout, _ptr(in_scale),
                                            _ptr(q8_act)))

    # -- ft-cuda/src/lib.rs:674-694 --
    def gemv_f32_rows_dev(self, w, x, y, dim, n_rows, n_seqs, bias=None, stream=None):
        check(lib().ft_hip_router_logits(self._ctx, _stream(stream), _ptr(w), _ptr(x), _ptr(bias), _ptr(y), dim,
                                         n_rows, n_seqs))

    # -- ft-cuda/src/lib.rs:472-494 --
    def topk_router_dev(self, logits, expert_scale, ids, wts, e_count, k, n_seqs, stream=None):
        check(lib().ft_hip_topk_router(self._ctx, _stream(stream), _ptr(logits), _ptr(expert_scale), _ptr(ids),
                                       _ptr(wts), e_count, k, n_seqs))

    # -- ft-cuda/src/lib.rs:808-829 --
    def reduce_pairs_weighted(self, y, wts, seq_of, out, hidden, n_pairs, n_seqs, stream=None):
        check(lib().ft_hip_reduce_pairs_weighted(self._ctx, _stream(stream), _ptr(y), _ptr(wts), _ptr(seq_of),
                                                 _ptr(out), hidden, n_pairs, n_seqs))

    # -- setup: ft-core/src/q4_0.rs:248-258 on the device --
    def repack_rows(self, src, src_layout, dst, dst_layout, n_rows, k, stream=None):
        check(lib().ft_hip_repack_rows(self._ctx, _stream(stream), _ptr(src), src_layout, _ptr(dst), dst_layout,
                                       n_rows, k))

    def gen_values(self, key, start, n, scale, out, stream=None):
        check(lib().ft_hip_gen_values(self._ctx, _stream(stream), key, start, n, scale, _ptr(out)))

    def gen_q4_rows(self, key, row0, n_rows, k, scale, out, layout=LAYOUT_Q4R, stream=None):
        check(lib().ft_hip_gen_q4_rows(self._ctx, _stream(stream), key, row0, n_rows, k, scale, _ptr(out), layout))

    # -- the whole layer (ft-model/src/lib.rs:1406-1476 composition) --
    @staticmethod
    def moe_layer_workspace_bytes(n_seqs, hidden, inter, n_experts, top_k):
        return lib().ft_hip_moe_layer_workspace_bytes(n_seqs, hidden, inter, n_experts, top_k)

    def moe_layer(self, x, x_out, n_seqs, hidden, inter, n_experts, top_k, router_w, router_bias, expert_scale,
                  bank, expert_bytes, layout, ids, wts, workspace, stream=None):
        check(lib().ft_hip_moe_layer(self._ctx, _stream(stream), _ptr(x), _ptr(x_out), n_seqs, hidden, inter,
                                     n_experts, top_k, _ptr(router_w), _ptr(router_bias), _ptr(expert_scale),
                                     _ptr(bank), expert_bytes, layout, _ptr(ids), _ptr(wts), _ptr(workspace),
                                     workspace.numel() * workspace.element_size()))

    def moe_layer_noalloc(self, x, x_out, n_seqs, hidden, inter, n_experts, top_k, router_w, router_bias,
                          expert_scale, bank, expert_bytes, layout, ids, wts, stream=None):
        """moe_layer on the library's own scratch (no workspace; allocates nothing)."""
        check(lib().ft_hip_moe_layer_noalloc(self._ctx, _stream(stream), _ptr(x), _ptr(x_out), n_seqs, hidden,
                                             inter, n_experts, top_k, _ptr(router_w), _ptr(router_bias),
                                             _ptr(expert_scale), _ptr(bank), expert_bytes, layout, _ptr(ids),
                                             _ptr(wts)))

    @staticmethod
    def moe_stack_workspace_bytes(n_seqs, hidden, inter, n_experts, top_k):
        return lib().ft_hip_moe_stack_workspace_bytes(n_seqs, hidden, inter, n_experts, top_k)

    def moe_stack(self, x_in, x_out, n_seqs, hidden, inter, n_experts, top_k, n_layers, routers, router_bias,
                  expert_scale, banks, expert_bytes, layout, ids, wts, workspace, stream=None):
        """n_layers launch-by-launch layers in one call (ft_hip_moe_stack); ids/wts [L][n_seqs*top_k]."""
        check(lib().ft_hip_moe_stack(self._ctx, _stream(stream), _ptr(x_in), _ptr(x_out), n_seqs, hidden, inter,
                                     n_experts, top_k, n_layers, _ptr(routers), _ptr(router_bias),
                                     _ptr(expert_scale), _ptr(banks), expert_bytes, layout, _ptr(ids), _ptr(wts),
                                     _ptr(workspace), workspace.numel() * workspace.element_size()))

    # -- grouped batched layer (ft-model/src/lib.rs:1507-1606) --
    @staticmethod
    def moe_layer_grouped_workspace_bytes(n_seqs, hidden, inter, n_experts, top_k):
        return lib().ft_hip_moe_layer_grouped_workspace_bytes(n_seqs, hidden, inter, n_experts, top_k)

    def moe_layer_grouped(self, x, x_out, n_seqs, hidden, inter, n_experts, top_k, router_w, router_bias,
                          expert_scale, bank, ids, wts, workspace, dbg_gu=None, dbg_act=None, stream=None):
        check(lib().ft_hip_moe_layer_grouped(self._ctx, _stream(stream), _ptr(x), _ptr(x_out), n_seqs, hidden,
                                             inter, n_experts, top_k, _ptr(router_w), _ptr(router_bias),
                                             _ptr(expert_scale), _ptr(bank), _ptr(ids), _ptr(wts), _ptr(workspace),
                                             workspace.numel() * workspace.element_size(), _ptr(dbg_gu),
                                             _ptr(dbg_act)))

    @staticmethod
    def moe_stack_grouped_workspace_bytes(max_seqs, hidden, inter, n_experts, top_k, n_layers):
        return lib().ft_hip_moe_stack_grouped_workspace_bytes(max_seqs, hidden, inter, n_experts, top_k, n_layers)

    def moe_stack_grouped(self, x_in, x_out, n_seqs, max_seqs, hidden, inter, n_experts, top_k, n_layers, banks,
                          routers, router_bias, expert_scale, ids, wts, workspace, stream=None):
        check(lib().ft_hip_moe_stack_grouped(self._ctx, _stream(stream), _ptr(x_in), _ptr(x_out), n_seqs, max_seqs,
                                             hidden, inter, n_experts, top_k, n_layers, _ptr(banks), _ptr(routers),
                                             _ptr(router_bias), _ptr(expert_scale), _ptr(ids), _ptr(wts),
                                             _ptr(workspace), workspace.numel() * workspace.element_size()))

    # -- fused whole-stack path --
    @staticmethod
    def fused_expert_bytes(hidden, inter):
        return lib().ft_hip_fused_expert_bytes(hidden, inter)

    @staticmethod
    def fused_workspace_bytes(hidden, inter, n_experts, top_k):
        return lib().ft_hip_fused_workspace_bytes(hidden, inter, n_experts, top_k)

    @staticmethod
    def fused_workgroups(hidden, inter, n_experts, top_k):
        return lib().ft_hip_fused_workgroups(hidden, inter, n_experts, top_k)

    def fused_set_spin_limit(self, polls):
        check(lib().ft_hip_fused_set_spin_limit(self._ctx, polls))

    def fused_set_cooperative(self, on):
        """Fused kernel: cooperative launch (1) or plain launch (0, the default)."""
        check(lib().ft_hip_fused_set_cooperative(self._ctx, int(on)))

    def fused_set_prefetch(self, on):
        """1: stream early-routed experts ahead (default); 0: load each layer's experts once routed."""
        check(lib().ft_hip_fused_set_prefetch(self._ctx, int(on)))

    @staticmethod
    def fused_predictor_bytes(hidden, inter, n_experts, n_layers):
        return lib().ft_hip_fused_predictor_bytes(hidden, inter, n_experts, n_layers)

    def fused_build_predictor(self, banks, routers, hidden, inter, n_experts, n_layers, table, stream=None):
        """Refined-prediction table M = R_{l+1} D_{l,e} from fused banks and routers (setup)."""
        check(lib().ft_hip_fused_build_predictor(self._ctx, _stream(stream), _ptr(banks), _ptr(routers), hidden, inter,
                                                 n_experts, n_layers, _ptr(table),
                                                 0 if table is None else table.numel() * table.element_size()))

    def fused_set_predictor(self, table, n_layers=0):
        """Later fused launches prefetch the refined prediction from `table` (None: early routing only)."""
        check(lib().ft_hip_fused_set_predictor(self._ctx, _ptr(table),
                                               0 if table is None else table.numel() * table.element_size(),
                                               n_layers))

    def set_input_norm(self, on):
        """1: the layer entry points run on rmsnorm(x) (logits and gate|up sums times
        1/sqrt(mean(x*x) + 1e-6)); 0 (default): on x as given."""
        check(lib().ft_hip_set_input_norm(self._ctx, int(on)))

    def set_layer_record(self, x=None, q8x=None, gu=None, act=None, gu_dots=None, dn_dots=None):
        """Test hook: stage records of the launch-by-launch layer path (see the
        header); all None turns it off."""
        check(lib().ft_hip_set_layer_record(self._ctx, _ptr(x), _ptr(q8x), _ptr(gu), _ptr(act), _ptr(gu_dots),
                                            _ptr(dn_dots)))

    def set_block_dot_record(self, gu_dots, dn_dots):
        """Test hook: record every int32 block dot of the grouped / fused
        kernels into two int32 tensors (None, None: off)."""
        check(lib().ft_hip_set_block_dot_record(self._ctx, _ptr(gu_dots), _ptr(dn_dots)))

    def set_grouped_mfma_min(self, n_tokens):
        """moe_layer_grouped: experts with >= n_tokens tokens take the MFMA kernels (0, the default:
        all MFMA from 4 pairs per expert on, else all dot4)."""
        check(lib().ft_hip_set_grouped_mfma_min(self._ctx, int(n_tokens)))

    def stream_read(self, buf, out, n_workgroups, nbytes=None, stream=None):
        """Read all of `buf` (or its first nbytes) once; out: uint32[n_workgroups]."""
        n = buf.numel() * buf.element_size() if nbytes is None else nbytes
        check(lib().ft_hip_stream_read(self._ctx, _stream(stream), _ptr(buf), n, _ptr(out), int(n_workgroups)))

    def set_gemv_lanes(self, lanes_per_row):
        """q4r GEMV lanes per row: 0 automatic (the default), 8, 16, 32 or 64."""
        check(lib().ft_hip_set_gemv_lanes(self._ctx, int(lanes_per_row)))

    def fused_workspace_init(self, ws, stream=None):
        check(lib().ft_hip_fused_workspace_init(self._ctx, _stream(stream), _ptr(ws), ws.numel() * ws.element_size()))

    def fused_workspace_set_epoch(self, ws, epoch, stream=None):
        """Test hook: the workspace's epoch (device and this context's wrap guard)."""
        check(lib().ft_hip_fused_workspace_set_epoch(self._ctx, _stream(stream), _ptr(ws), int(epoch)))

    def pack_experts_fused(self, src, src_layout, src_expert_bytes, dst, n_experts, hidden, inter, stream=None):
        check(lib().ft_hip_pack_experts_fused(self._ctx, _stream(stream), _ptr(src), src_layout, src_expert_bytes,
                                              _ptr(dst), n_experts, hidden, inter))

    def load_expert_banks_gguf(self, gguf, layer0, n_layers, hidden, inter, n_experts, banks, expert_bytes,
                               layout=LAYOUT_Q4R, stream=None):
        """Expert banks of a GGUF file's layers into the device tensor `banks`."""
        check(lib().ft_hip_load_expert_banks_gguf(self._ctx, _stream(stream), gguf.handle, layer0, n_layers, hidden,
                                                  inter, n_experts, _ptr(banks), expert_bytes, layout))

    def pack_router_fused(self, src, dst, n_layers, n_experts, hidden, stream=None):
        check(lib().ft_hip_pack_router_fused(self._ctx, _stream(stream), _ptr(src), _ptr(dst), n_layers, n_experts,
                                             hidden))

    def moe_stack_fused(self, x_in, x_out, hidden, inter, n_experts, top_k, n_layers, banks, routers, bias,
                        expert_scale, ids, wts, ws, dbg_gu=None, dbg_act=None, dbg_x=None, dbg_trace=None,
                        stream=None):
        check(lib().ft_hip_moe_stack_fused(self._ctx, _stream(stream), _ptr(x_in), _ptr(x_out), hidden, inter,
                                           n_experts, top_k, n_layers, _ptr(banks), _ptr(routers), _ptr(bias),
                                           _ptr(expert_scale), _ptr(ids), _ptr(wts), _ptr(ws),
                                           ws.numel() * ws.element_size(), _ptr(dbg_gu), _ptr(dbg_act),
                                           _ptr(dbg_x), _ptr(dbg_trace)))

    def fused_status(self, ws):
        """Raise FtHipError(E_TIMEOUT) if a fused launch on `ws` gave up a wait (sync first)."""
        ab = ctypes.c_int(0)
        check(lib().ft_hip_fused_status(self._ctx, _ptr(ws), ctypes.byref(ab)))


class TensorInfo:
    """One entry of a GGUF tensor table (ft_gguf::TensorInfo)."""

    def __init__(self, dims, ggml_type, offset, nbytes):
        self.dims, self.ggml_type, self.offset, self.nbytes = dims, ggml_type, offset, nbytes

    def __repr__(self):
        return f"TensorInfo(dims={self.dims}, ggml_type={self.ggml_type}, offset={self.offset}, nbytes={self.nbytes})"


class Gguf:
    """A local GGUF v2/v3 file through ft_gguf_* (mirrors ft_gguf::Gguf:
    open, meta, tensors, tensor, tensor_data). Host only."""

    def __init__(self, path):
        h = _P()
        check(lib().ft_gguf_open(os.fsencode(path), ctypes.byref(h)))
        self.handle = h
        L = lib()
        self.version = L.ft_gguf_version(h)
        self.data_start = L.ft_gguf_data_start(h)
        self.meta = {}
        for i in range(L.ft_gguf_n_kv(h)):
            key, ty = ctypes.c_char_p(), ctypes.c_uint32()
            check(L.ft_gguf_kv_key(h, i, ctypes.byref(key), ctypes.byref(ty)))
            self.meta[key.value.decode()] = self._value(key.value, ty.value)
        self.tensors = {}
        for i in range(L.ft_gguf_n_tensors(h)):
            name = ctypes.c_char_p()
            check(L.ft_gguf_tensor_name(h, i, ctypes.byref(name)))
            nd, ty = ctypes.c_uint32(), ctypes.c_uint32()
            dims, off, nb = (_U64 * 8)(), _U64(), _U64()
            check(L.ft_gguf_tensor_info(h, name.value, ctypes.byref(nd), dims, ctypes.byref(ty), ctypes.byref(off),
                                        ctypes.byref(nb)))
            self.tensors[name.value.decode()] = TensorInfo(list(dims[:nd.value]), ty.value, off.value, nb.value)

    def _str(self, fn, *args):
        p, n = _P(), _U64()
        check(fn(self.handle, *args, ctypes.byref(p), ctypes.byref(n)))
        return ctypes.string_at(p.value, n.value).decode() if n.value else ""

    def _value(self, key, ty):
        L = lib()
        if ty in (0, 1, 2, 3, 4, 5, 10, 11):
            v = _U64()
            rc = L.ft_gguf_meta_u64(self.handle, key, ctypes.byref(v))
            return v.value if rc == OK else ("negative", ty)
        if ty == 6:
            v = _F()
            check(L.ft_gguf_meta_f32(self.handle, key, ctypes.byref(v)))
            return v.value
        if ty == 8:
            return self._str(L.ft_gguf_meta_str, key)
        if ty == 9:
            et, n = ctypes.c_uint32(), _U64()
            check(L.ft_gguf_meta_array(self.handle, key, ctypes.byref(et), ctypes.byref(n)))
            out = []
            for i in range(n.value):
                if et.value == 8:
                    out.append(self._str(L.ft_gguf_meta_array_str, key, i))
                elif et.value == 7:
                    b = _I()
                    check(L.ft_gguf_meta_array_bool(self.handle, key, i, ctypes.byref(b)))
                    out.append(bool(b.value))
                else:
                    v = _U64()
                    rc = L.ft_gguf_meta_array_u64(self.handle, key, i, ctypes.byref(v))
                    out.append(v.value if rc == OK else None)
            return out
        return ("type", ty)

    def tensor(self, name):
        if name not in self.tensors:
            raise FtHipError(E_NOT_FOUND, f"tensor {name} not found")
        return self.tensors[name]

    def tensor_data(self, name):
        """The tensor's bytes (a read-only numpy view of the mapping)."""
        import numpy as np
        p, n = _P(), _U64()
        check(lib().ft_gguf_tensor_data(self.handle, name.encode(), ctypes.byref(p), ctypes.byref(n)))
        buf = (ctypes.c_uint8 * n.value).from_address(p.value)
        a = np.frombuffer(buf, dtype=np.uint8)
        a.flags.writeable = False
        return a

    def to_f32(self, name):
        import numpy as np
        n = int(np.prod(self.tensor(name).dims))
        out = np.zeros(n, np.float32)
        check(lib().ft_gguf_tensor_to_f32(self.handle, name.encode(), out.ctypes.data_as(_P), n))
        return out

    def router_f32(self, layer, hidden, n_experts):
        import numpy as np
        out = np.zeros((n_experts, hidden), np.float32)
        check(lib().ft_gguf_router_f32(self.handle, layer, hidden, n_experts, out.ctypes.data_as(_P)))
        return out

    def close(self):
        if self.handle:
            lib().ft_gguf_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
