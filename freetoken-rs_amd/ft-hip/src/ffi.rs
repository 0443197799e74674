//! Raw declarations of libfthip's C ABI (`include/ft_hip.h`), one `extern`
//! item per exported symbol, argument for argument: `int` <-> `c_int`,
//! `int64_t` <-> `i64`, `uint64_t` <-> `u64`, `size_t` <-> `usize`, pointers
//! keep their constness. `tests/test_rust_crate.py` checks this file
//! against the header. Device pointers are raw addresses from the ROCm
//! allocator; streams are `hipStream_t` handles as `*mut c_void`.
#![allow(non_camel_case_types, clippy::too_many_arguments)]

use std::os::raw::{c_char, c_int, c_void};

/// Opaque library context (`ft_hip_ctx`), created by `ft_hip_create`.
#[repr(C)]
pub struct FtHipCtx {
    _private: [u8; 0],
}

/// Opaque handle of an open GGUF file (`ft_gguf`), created by `ft_gguf_open`.
#[repr(C)]
pub struct FtGguf {
    _private: [u8; 0],
}

pub const FT_HIP_OK: c_int = 0;
pub const FT_HIP_E_INVALID: c_int = -1;
pub const FT_HIP_E_SHAPE: c_int = -2;
pub const FT_HIP_E_DEVICE: c_int = -3;
pub const FT_HIP_E_LAUNCH: c_int = -4;
pub const FT_HIP_E_TIMEOUT: c_int = -5;
pub const FT_HIP_E_IO: c_int = -6;
pub const FT_HIP_E_FORMAT: c_int = -7;
pub const FT_HIP_E_NOT_FOUND: c_int = -8;
pub const FT_Q8_BLK: usize = 40;
pub const FT_LAYOUT_Q4_0: c_int = 0;
pub const FT_LAYOUT_Q4R: c_int = 1;
pub const FT_HIP_NOALLOC_SCRATCH_BYTES: usize = 8 << 20;

#[link(name = "fthip")]
extern "C" {
    pub fn ft_hip_version() -> c_int;
    pub fn ft_hip_last_error() -> *const c_char;
    pub fn ft_hip_create(device: c_int, out: *mut *mut FtHipCtx) -> c_int;
    pub fn ft_hip_destroy(ctx: *mut FtHipCtx) -> c_int;
    pub fn ft_hip_row_bytes(layout: c_int, k: i64) -> i64;
    pub fn ft_hip_q4r_scales_bytes(k: i64) -> i64;
    pub fn ft_hip_quantize_q8(ctx: *mut FtHipCtx, stream: *mut c_void, x: *const f32, x_stride: i64, q8: *mut c_void, k: i64, n: i64) -> c_int;
    pub fn ft_hip_gemv_q4_grouped_ptr(ctx: *mut FtHipCtx, stream: *mut c_void, bases: *const u64, bank_off: u64, x_idx: *const i32, n_entries: i64, q8: *const c_void, q8_stride_blocks: i64, y: *mut f32, y_stride: i64, n_rows: i64, k: i64, layout: c_int) -> c_int;
    pub fn ft_hip_gemv_q4_grouped_slots(ctx: *mut FtHipCtx, stream: *mut c_void, base: *const c_void, expert_bytes: u64, bank_off: u64, slots: *const i32, x_idx: *const i32, n_entries: i64, q8: *const c_void, q8_stride_blocks: i64, y: *mut f32, y_stride: i64, n_rows: i64, k: i64, layout: c_int) -> c_int;
    pub fn ft_hip_q4q8_block_dots(ctx: *mut FtHipCtx, stream: *mut c_void, base: *const c_void, expert_bytes: u64, bank_off: u64, slots: *const i32, x_idx: *const i32, n_entries: i64, q8: *const c_void, q8_stride_blocks: i64, out: *mut i32, n_rows: i64, k: i64, layout: c_int) -> c_int;
    pub fn ft_hip_gelu_mul_q8(ctx: *mut FtHipCtx, stream: *mut c_void, gu: *const f32, q8: *mut c_void, inter: i64, n: i64) -> c_int;
    pub fn ft_hip_silu_mul_grouped(ctx: *mut FtHipCtx, stream: *mut c_void, gu: *const f32, out: *mut f32, inter: i64, n_experts: i64) -> c_int;
    pub fn ft_hip_gelu_mul_grouped(ctx: *mut FtHipCtx, stream: *mut c_void, gu: *const f32, out: *mut f32, inter: i64, n_experts: i64) -> c_int;
    pub fn ft_hip_reduce_expert_weighted(ctx: *mut FtHipCtx, stream: *mut c_void, y: *const f32, wts: *const f32, out: *mut f32, hidden: i64, n_experts: i64) -> c_int;
    pub fn ft_hip_reduce_weighted(ctx: *mut FtHipCtx, stream: *mut c_void, y: *const f32, out: *mut f32, a: f32, hidden: i64, n_experts: i64) -> c_int;
    pub fn ft_hip_gemv_gate_up_act(ctx: *mut FtHipCtx, stream: *mut c_void, base: *const c_void, expert_bytes: u64, slots: *const i32, n_pairs: i64, x_div: i64, q8x: *const c_void, hidden: i64, inter: i64, layout: c_int, in_scale: *const f32, q8_act: *mut c_void) -> c_int;
    pub fn ft_hip_gemv_q4r_f32in(ctx: *mut FtHipCtx, stream: *mut c_void, w: *const c_void, x: *const f32, y: *mut f32, act: *mut f32, n_rows: i64, k: i64) -> c_int;
    pub fn ft_hip_router_logits(ctx: *mut FtHipCtx, stream: *mut c_void, w: *const f32, x: *const f32, bias: *const f32, y: *mut f32, dim: i64, n_rows: i64, n_seqs: i64) -> c_int;
    pub fn ft_hip_topk_router(ctx: *mut FtHipCtx, stream: *mut c_void, logits: *const f32, expert_scale: *const f32, ids: *mut i32, wts: *mut f32, e_count: i64, k: i64, n_seqs: i64) -> c_int;
    pub fn ft_hip_reduce_pairs_weighted(ctx: *mut FtHipCtx, stream: *mut c_void, y: *const f32, wts: *const f32, seq_of: *const i32, out: *mut f32, hidden: i64, n_pairs: i64, n_seqs: i64) -> c_int;
    pub fn ft_hip_repack_rows(ctx: *mut FtHipCtx, stream: *mut c_void, src: *const c_void, src_layout: c_int, dst: *mut c_void, dst_layout: c_int, n_rows: i64, k: i64) -> c_int;
    pub fn ft_hip_gen_values(ctx: *mut FtHipCtx, stream: *mut c_void, key: u64, start: i64, n: i64, scale: f32, out: *mut f32) -> c_int;
    pub fn ft_hip_gen_q4_rows(ctx: *mut FtHipCtx, stream: *mut c_void, key: u64, row0: i64, n_rows: i64, k: i64, scale: f32, out: *mut c_void, layout: c_int) -> c_int;
    pub fn ft_hip_set_block_dot_record(ctx: *mut FtHipCtx, gu_dots: *mut i32, dn_dots: *mut i32) -> c_int;
    pub fn ft_hip_set_layer_record(
        ctx: *mut FtHipCtx,
        x: *mut f32,
        q8x: *mut c_void,
        gu: *mut f32,
        act: *mut c_void,
        gu_dots: *mut i32,
        dn_dots: *mut i32,
    ) -> c_int;
    pub fn ft_hip_moe_layer_workspace_bytes(n_seqs: i64, hidden: i64, inter: i64, n_experts: i64, top_k: i64) -> usize;
    pub fn ft_hip_moe_layer(ctx: *mut FtHipCtx, stream: *mut c_void, x: *const f32, x_out: *mut f32, n_seqs: i64, hidden: i64, inter: i64, n_experts: i64, top_k: i64, router_w: *const f32, router_bias: *const f32, expert_scale: *const f32, bank: *const c_void, expert_bytes: u64, layout: c_int, ids: *mut i32, wts: *mut f32, workspace: *mut c_void, workspace_bytes: usize) -> c_int;
    pub fn ft_hip_moe_layer_noalloc(ctx: *mut FtHipCtx, stream: *mut c_void, x: *const f32, x_out: *mut f32, n_seqs: i64, hidden: i64, inter: i64, n_experts: i64, top_k: i64, router_w: *const f32, router_bias: *const f32, expert_scale: *const f32, bank: *const c_void, expert_bytes: u64, layout: c_int, ids: *mut i32, wts: *mut f32) -> c_int;
    pub fn ft_hip_moe_stack_workspace_bytes(n_seqs: i64, hidden: i64, inter: i64, n_experts: i64, top_k: i64) -> usize;
    pub fn ft_hip_moe_stack(ctx: *mut FtHipCtx, stream: *mut c_void, x_in: *const f32, x_out: *mut f32, n_seqs: i64, hidden: i64, inter: i64, n_experts: i64, top_k: i64, n_layers: i64, routers: *const f32, router_bias: *const f32, expert_scale: *const f32, banks: *const c_void, expert_bytes: u64, layout: c_int, ids: *mut i32, wts: *mut f32, workspace: *mut c_void, workspace_bytes: usize) -> c_int;
    pub fn ft_hip_moe_layer_grouped_workspace_bytes(n_seqs: i64, hidden: i64, inter: i64, n_experts: i64, top_k: i64) -> usize;
    pub fn ft_hip_moe_layer_grouped(ctx: *mut FtHipCtx, stream: *mut c_void, x: *const f32, x_out: *mut f32, n_seqs: i64, hidden: i64, inter: i64, n_experts: i64, top_k: i64, router_w: *const f32, router_bias: *const f32, expert_scale: *const f32, bank: *const c_void, ids: *mut i32, wts: *mut f32, workspace: *mut c_void, workspace_bytes: usize, dbg_gu: *mut f32, dbg_act: *mut c_void) -> c_int;
    pub fn ft_hip_moe_stack_grouped_workspace_bytes(max_seqs: i64, hidden: i64, inter: i64, n_experts: i64, top_k: i64, n_layers: i64) -> usize;
    pub fn ft_hip_moe_stack_grouped(ctx: *mut FtHipCtx, stream: *mut c_void, x_in: *const f32, x_out: *mut f32, n_seqs: i64, max_seqs: i64, hidden: i64, inter: i64, n_experts: i64, top_k: i64, n_layers: i64, banks: *const c_void, routers: *const f32, router_bias: *const f32, expert_scale: *const f32, ids: *mut i32, wts: *mut f32, workspace: *mut c_void, workspace_bytes: usize) -> c_int;
    pub fn ft_hip_set_grouped_mfma_min(ctx: *mut FtHipCtx, n_tokens: c_int) -> c_int;
    pub fn ft_hip_set_gemv_lanes(ctx: *mut FtHipCtx, lanes_per_row: c_int) -> c_int;
    pub fn ft_hip_stream_read(ctx: *mut FtHipCtx, stream: *mut c_void, buf: *const c_void, bytes: u64, out: *mut u32, n_workgroups: c_int) -> c_int;
    pub fn ft_hip_set_input_norm(ctx: *mut FtHipCtx, on: c_int) -> c_int;
    pub fn ft_hip_fused_expert_bytes(hidden: i64, inter: i64) -> i64;
    pub fn ft_hip_fused_workspace_bytes(hidden: i64, inter: i64, n_experts: i64, top_k: i64) -> usize;
    pub fn ft_hip_fused_workgroups(hidden: i64, inter: i64, n_experts: i64, top_k: i64) -> c_int;
    pub fn ft_hip_fused_workspace_init(ctx: *mut FtHipCtx, stream: *mut c_void, workspace: *mut c_void, workspace_bytes: usize) -> c_int;
    pub fn ft_hip_fused_workspace_set_epoch(ctx: *mut FtHipCtx, stream: *mut c_void, workspace: *mut c_void, epoch: u32) -> c_int;
    pub fn ft_hip_pack_experts_fused(ctx: *mut FtHipCtx, stream: *mut c_void, src: *const c_void, src_layout: c_int, src_expert_bytes: u64, dst: *mut c_void, n_experts: i64, hidden: i64, inter: i64) -> c_int;
    pub fn ft_hip_pack_router_fused(ctx: *mut FtHipCtx, stream: *mut c_void, src: *const f32, dst: *mut f32, n_layers: i64, n_experts: i64, hidden: i64) -> c_int;
    pub fn ft_hip_moe_stack_fused(ctx: *mut FtHipCtx, stream: *mut c_void, x_in: *const f32, x_out: *mut f32, hidden: i64, inter: i64, n_experts: i64, top_k: i64, n_layers: i64, banks: *const c_void, routers: *const f32, bias: *const f32, expert_scale: *const f32, ids: *mut i32, wts: *mut f32, workspace: *mut c_void, workspace_bytes: usize, dbg_gu: *mut f32, dbg_act: *mut c_void, dbg_x: *mut f32, dbg_trace: *mut u64) -> c_int;
    pub fn ft_hip_fused_set_spin_limit(ctx: *mut FtHipCtx, polls: c_int) -> c_int;
    pub fn ft_hip_fused_set_prefetch(ctx: *mut FtHipCtx, on: c_int) -> c_int;
    pub fn ft_hip_fused_set_cooperative(ctx: *mut FtHipCtx, on: c_int) -> c_int;
    pub fn ft_hip_fused_predictor_bytes(hidden: i64, inter: i64, n_experts: i64, n_layers: i64) -> i64;
    pub fn ft_hip_fused_build_predictor(ctx: *mut FtHipCtx, stream: *mut c_void, banks: *const c_void, routers: *const f32, hidden: i64, inter: i64, n_experts: i64, n_layers: i64, table: *mut c_void, table_bytes: usize) -> c_int;
    pub fn ft_hip_fused_set_predictor(ctx: *mut FtHipCtx, table: *const c_void, table_bytes: usize, n_layers: i64) -> c_int;
    pub fn ft_hip_fused_status(ctx: *mut FtHipCtx, workspace: *mut c_void, aborted: *mut c_int) -> c_int;
    pub fn ft_gguf_open(path: *const c_char, out: *mut *mut FtGguf) -> c_int;
    pub fn ft_gguf_close(g: *mut FtGguf) -> c_int;
    pub fn ft_gguf_version(g: *const FtGguf) -> u32;
    pub fn ft_gguf_data_start(g: *const FtGguf) -> u64;
    pub fn ft_gguf_n_kv(g: *const FtGguf) -> i64;
    pub fn ft_gguf_n_tensors(g: *const FtGguf) -> i64;
    pub fn ft_gguf_kv_key(g: *const FtGguf, i: i64, key: *mut *const c_char, value_type: *mut u32) -> c_int;
    pub fn ft_gguf_meta_type(g: *const FtGguf, key: *const c_char, value_type: *mut u32) -> c_int;
    pub fn ft_gguf_meta_u64(g: *const FtGguf, key: *const c_char, out: *mut u64) -> c_int;
    pub fn ft_gguf_meta_f32(g: *const FtGguf, key: *const c_char, out: *mut f32) -> c_int;
    pub fn ft_gguf_meta_str(g: *const FtGguf, key: *const c_char, s: *mut *const c_char, len: *mut u64) -> c_int;
    pub fn ft_gguf_meta_array(g: *const FtGguf, key: *const c_char, elem_type: *mut u32, n: *mut u64) -> c_int;
    pub fn ft_gguf_meta_array_u64(g: *const FtGguf, key: *const c_char, i: u64, out: *mut u64) -> c_int;
    pub fn ft_gguf_meta_array_bool(g: *const FtGguf, key: *const c_char, i: u64, out: *mut c_int) -> c_int;
    pub fn ft_gguf_meta_array_str(g: *const FtGguf, key: *const c_char, i: u64, s: *mut *const c_char, len: *mut u64) -> c_int;
    pub fn ft_gguf_tensor_name(g: *const FtGguf, i: i64, name: *mut *const c_char) -> c_int;
    pub fn ft_gguf_tensor_info(g: *const FtGguf, name: *const c_char, n_dims: *mut u32, dims: *mut u64, ggml_type: *mut u32, offset: *mut u64, nbytes: *mut u64) -> c_int;
    pub fn ft_gguf_tensor_data(g: *const FtGguf, name: *const c_char, data: *mut *const c_void, nbytes: *mut u64) -> c_int;
    pub fn ft_gguf_tensor_to_f32(g: *const FtGguf, name: *const c_char, out: *mut f32, n: u64) -> c_int;
    pub fn ft_gguf_router_f32(g: *const FtGguf, layer: i64, hidden: i64, n_experts: i64, out: *mut f32) -> c_int;
    pub fn ft_hip_load_expert_banks_gguf(ctx: *mut FtHipCtx, stream: *mut c_void, g: *const FtGguf, layer0: i64, n_layers: i64, hidden: i64, inter: i64, n_experts: i64, banks: *mut c_void, expert_bytes: u64, layout: c_int) -> c_int;
}
