//! `ft_hip::Q4Gemv`: the MoE expert-FFN operators of `ft_cuda::Q4Gemv`
//! (ft-cuda/src/lib.rs:69-150) on an MI355X, over libfthip's C ABI.
//!
//! Method names and argument meaning follow the reference, so ft-model's GPU
//! expert section (ft-model/src/lib.rs:1397-1476, :1507-1606) switches
//! backend call for call. Differences, all from the boundary:
//! - buffers are raw device addresses from the ROCm allocator (`DevPtr`) in
//!   place of cudarc's `CudaSlice<T>`, and streams are `hipStream_t` handles
//!   (`Stream`); the caller owns every buffer;
//! - shape preconditions that the reference `assert!`s come back as `Err`
//!   carrying the library's message (`FT_HIP_E_SHAPE`), driver and launch
//!   failures as `Err` too (the reference's `?`);
//! - q8 activation blocks are the library's 40-byte {f32 d; i32 qsum;
//!   i8 qs[32]} (the reference stores d*qsum as f32 in the second word).
//! One context per device, used by one thread at a time (as Model owns its
//! Q4Gemv on one worker thread, ft-model/src/bin/serve.rs:635-636).

pub mod ffi;

use anyhow::{bail, Result};
use std::ffi::CStr;
use std::os::raw::c_void;

/// A device address (the value cudarc's `DevicePtr` exposes).
pub type DevPtr = u64;

/// A `hipStream_t`; `Stream::NULL` is the null stream.
#[derive(Clone, Copy, Debug)]
pub struct Stream(pub *mut c_void);
impl Stream {
    pub const NULL: Stream = Stream(std::ptr::null_mut());
}

/// Weight row layout of a bank: ggml q4_0 rows or the q4r repack
/// (ft-core/src/q4_0.rs:1-16, :234-258).
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum Layout {
    Q4_0,
    Q4r,
}
impl Layout {
    fn raw(self) -> i32 {
        match self {
            Layout::Q4_0 => ffi::FT_LAYOUT_Q4_0,
            Layout::Q4r => ffi::FT_LAYOUT_Q4R,
        }
    }
}

/// Bytes per 32-element q8 activation block.
pub const Q8_BLK: usize = ffi::FT_Q8_BLK;

fn check(rc: i32) -> Result<()> {
    if rc == ffi::FT_HIP_OK {
        return Ok(());
    }
    let msg = unsafe { CStr::from_ptr(ffi::ft_hip_last_error()) };
    bail!("ft-hip error {rc}: {}", msg.to_string_lossy())
}

fn p<T>(a: DevPtr) -> *const T {
    a as usize as *const T
}
fn pm<T>(a: DevPtr) -> *mut T {
    a as usize as *mut T
}
fn opt<T>(a: Option<DevPtr>) -> *const T {
    a.map_or(std::ptr::null(), |v| p(v))
}

pub struct Q4Gemv {
    ctx: *mut ffi::FtHipCtx,
}

impl Q4Gemv {
    /// `Q4Gemv::new` (ft-cuda/src/lib.rs:111-150): binds `device` (gfx950 only).
    pub fn new(device: i32) -> Result<Self> {
        let mut ctx = std::ptr::null_mut();
        check(unsafe { ffi::ft_hip_create(device, &mut ctx) })?;
        Ok(Self { ctx })
    }

    /// `quantize_q8` (ft-cuda/src/lib.rs:898-921), arithmetic of ft-core's
    /// `Q8Vec::quantize` (ft-core/src/q4_0.rs:62-78): n rows of k, `x_stride`
    /// floats apart (0 shares one row).
    pub fn quantize_q8(&self, s: Stream, x: DevPtr, x_stride: usize, q8: DevPtr, k: usize, n: usize) -> Result<()> {
        check(unsafe { ffi::ft_hip_quantize_q8(self.ctx, s.0, p(x), x_stride as i64, pm(q8), k as i64, n as i64) })
    }

    /// `quantize_q8_view` (ft-cuda/src/lib.rs:871-894): the same over a row view.
    pub fn quantize_q8_view(&self, s: Stream, x: DevPtr, x_stride: usize, q8: DevPtr, k: usize, n: usize) -> Result<()> {
        self.quantize_q8(s, x, x_stride, q8, k, n)
    }

    /// `gemv_grouped_q8_ptr` (ft-cuda/src/lib.rs:593-623): y[e] = W_e q8[x_idx[e]]
    /// with W_e at bases[e] + bank_off, q4_0 rows.
    #[allow(clippy::too_many_arguments)]
    pub fn gemv_grouped_q8_ptr(&self, s: Stream, bases: DevPtr, bank_off: usize, x_idx: Option<DevPtr>,
                               n_entries: usize, q8: DevPtr, q8_stride_blocks: usize, y: DevPtr, y_stride: usize,
                               n_rows: usize, k: usize) -> Result<()> {
        check(unsafe {
            ffi::ft_hip_gemv_q4_grouped_ptr(self.ctx, s.0, p(bases), bank_off as u64, opt(x_idx), n_entries as i64,
                                            p(q8), q8_stride_blocks as i64, pm(y), y_stride as i64, n_rows as i64,
                                            k as i64, ffi::FT_LAYOUT_Q4_0)
        })
    }

    /// `gemv_q4r_ptr` (ft-cuda/src/lib.rs:736-767): as gemv_grouped_q8_ptr over q4r rows.
    #[allow(clippy::too_many_arguments)]
    pub fn gemv_q4r_ptr(&self, s: Stream, bases: DevPtr, bank_off: usize, x_idx: Option<DevPtr>, n_entries: usize,
                        q8: DevPtr, q8_stride_blocks: usize, y: DevPtr, y_stride: usize, n_rows: usize,
                        k: usize) -> Result<()> {
        check(unsafe {
            ffi::ft_hip_gemv_q4_grouped_ptr(self.ctx, s.0, p(bases), bank_off as u64, opt(x_idx), n_entries as i64,
                                            p(q8), q8_stride_blocks as i64, pm(y), y_stride as i64, n_rows as i64,
                                            k as i64, ffi::FT_LAYOUT_Q4R)
        })
    }

    /// `gemv_grouped_q8` / `gemv_grouped_q8_idx` / `gemv_q4r_idx`
    /// (ft-cuda/src/lib.rs:926-957, :772-804, :699-732): entry e's weights at
    /// base + slots[e]*expert_bytes + bank_off.
    #[allow(clippy::too_many_arguments)]
    pub fn gemv_grouped_slots(&self, s: Stream, base: DevPtr, expert_bytes: usize, bank_off: usize, slots: DevPtr,
                              x_idx: Option<DevPtr>, n_entries: usize, q8: DevPtr, q8_stride_blocks: usize,
                              y: DevPtr, y_stride: usize, n_rows: usize, k: usize, layout: Layout) -> Result<()> {
        check(unsafe {
            ffi::ft_hip_gemv_q4_grouped_slots(self.ctx, s.0, p(base), expert_bytes as u64, bank_off as u64, p(slots),
                                              opt(x_idx), n_entries as i64, p(q8), q8_stride_blocks as i64, pm(y),
                                              y_stride as i64, n_rows as i64, k as i64, layout.raw())
        })
    }

    /// `gemv_grouped_q8` (ft-cuda/src/lib.rs:926-957): y[e] = W_{slots[e]} q8[e]
    /// over q4_0 rows at cache + slots[e]*expert_bytes + bank_off;
    /// q8_stride_blocks = 0 shares one activation row across the experts.
    #[allow(clippy::too_many_arguments)]
    pub fn gemv_grouped_q8(&self, s: Stream, cache: DevPtr, expert_bytes: usize, bank_off: usize, slots: DevPtr,
                           n_experts: usize, q8: DevPtr, q8_stride_blocks: usize, y: DevPtr, y_stride: usize,
                           n_rows: usize, k: usize) -> Result<()> {
        self.gemv_grouped_slots(s, cache, expert_bytes, bank_off, slots, None, n_experts, q8, q8_stride_blocks, y,
                                y_stride, n_rows, k, Layout::Q4_0)
    }

    /// `gemv_grouped_q8_idx` (ft-cuda/src/lib.rs:772-804): as gemv_grouped_q8,
    /// entry e reading q8 row x_idx[e].
    #[allow(clippy::too_many_arguments)]
    pub fn gemv_grouped_q8_idx(&self, s: Stream, cache: DevPtr, expert_bytes: usize, bank_off: usize, slots: DevPtr,
                               x_idx: DevPtr, n_entries: usize, q8: DevPtr, q8_stride_blocks: usize, y: DevPtr,
                               y_stride: usize, n_rows: usize, k: usize) -> Result<()> {
        self.gemv_grouped_slots(s, cache, expert_bytes, bank_off, slots, Some(x_idx), n_entries, q8,
                                q8_stride_blocks, y, y_stride, n_rows, k, Layout::Q4_0)
    }

    /// `silu_mul_grouped` (ft-cuda/src/lib.rs:1053-1072): out[e] = silu(gate)*up,
    /// bit-exact with the CPU expression of ft-bench/src/bin/decode.rs:300.
    pub fn silu_mul_grouped(&self, s: Stream, gu: DevPtr, out: DevPtr, inter: usize, n_experts: usize) -> Result<()> {
        check(unsafe { ffi::ft_hip_silu_mul_grouped(self.ctx, s.0, p(gu), pm(out), inter as i64, n_experts as i64) })
    }

    /// `gelu_mul_grouped` (ft-cuda/src/lib.rs:1009-1028): out[e] = gelu_tanh(gate)*up
    /// (ft-model/src/lib.rs:435-437).
    pub fn gelu_mul_grouped(&self, s: Stream, gu: DevPtr, out: DevPtr, inter: usize, n_experts: usize) -> Result<()> {
        check(unsafe { ffi::ft_hip_gelu_mul_grouped(self.ctx, s.0, p(gu), pm(out), inter as i64, n_experts as i64) })
    }

    /// `reduce_expert_weighted` (ft-cuda/src/lib.rs:1031-1050): out += sum_e wts[e] * y[e].
    pub fn reduce_expert_weighted(&self, s: Stream, y: DevPtr, wts: DevPtr, out: DevPtr, hidden: usize,
                                  n_experts: usize) -> Result<()> {
        check(unsafe {
            ffi::ft_hip_reduce_expert_weighted(self.ctx, s.0, p(y), p(wts), pm(out), hidden as i64, n_experts as i64)
        })
    }

    /// `reduce_weighted` (ft-cuda/src/lib.rs:1075-1094): out += a * sum_e y[e].
    pub fn reduce_weighted(&self, s: Stream, y: DevPtr, out: DevPtr, a: f32, hidden: usize,
                           n_experts: usize) -> Result<()> {
        check(unsafe { ffi::ft_hip_reduce_weighted(self.ctx, s.0, p(y), pm(out), a, hidden as i64, n_experts as i64) })
    }

    /// `gemv_q4r_idx` (ft-cuda/src/lib.rs:699-732).
    #[allow(clippy::too_many_arguments)]
    pub fn gemv_q4r_idx(&self, s: Stream, base: DevPtr, expert_bytes: usize, bank_off: usize, slots: DevPtr,
                        x_idx: Option<DevPtr>, n_entries: usize, q8: DevPtr, q8_stride_blocks: usize, y: DevPtr,
                        y_stride: usize, n_rows: usize, k: usize) -> Result<()> {
        self.gemv_grouped_slots(s, base, expert_bytes, bank_off, slots, x_idx, n_entries, q8, q8_stride_blocks, y,
                                y_stride, n_rows, k, Layout::Q4r)
    }

    /// `gelu_mul_q8` (ft-cuda/src/lib.rs:354-374): gelu_tanh(gate)*up, then q8
    /// (ft-model/src/lib.rs:435-437; tanh bit-identical to glibc's tanhf).
    pub fn gelu_mul_q8(&self, s: Stream, gu: DevPtr, q8: DevPtr, inter: usize, n: usize) -> Result<()> {
        check(unsafe { ffi::ft_hip_gelu_mul_q8(self.ctx, s.0, p(gu), pm(q8), inter as i64, n as i64) })
    }

    /// `gemv_f32_rows_dev` (ft-cuda/src/lib.rs:674-694): router logits in the
    /// library's R-order, plus bias.
    #[allow(clippy::too_many_arguments)]
    pub fn gemv_f32_rows_dev(&self, s: Stream, w: DevPtr, x: DevPtr, bias: Option<DevPtr>, y: DevPtr, dim: usize,
                             n_rows: usize, n_seqs: usize) -> Result<()> {
        check(unsafe {
            ffi::ft_hip_router_logits(self.ctx, s.0, p(w), p(x), opt(bias), pm(y), dim as i64, n_rows as i64,
                                      n_seqs as i64)
        })
    }

    /// `topk_router_dev` (ft-cuda/src/lib.rs:472-494): top-k (ties to the
    /// lower index) and softmax over the chosen, times expert_scale.
    #[allow(clippy::too_many_arguments)]
    pub fn topk_router_dev(&self, s: Stream, logits: DevPtr, expert_scale: Option<DevPtr>, ids: DevPtr, wts: DevPtr,
                           e_count: usize, k: usize, n_seqs: usize) -> Result<()> {
        check(unsafe {
            ffi::ft_hip_topk_router(self.ctx, s.0, p(logits), opt(expert_scale), pm(ids), pm(wts), e_count as i64,
                                    k as i64, n_seqs as i64)
        })
    }

    /// `reduce_pairs_weighted` (ft-cuda/src/lib.rs:808-829).
    #[allow(clippy::too_many_arguments)]
    pub fn reduce_pairs_weighted(&self, s: Stream, y: DevPtr, wts: DevPtr, seq_of: DevPtr, out: DevPtr,
                                 hidden: usize, n_pairs: usize, n_seqs: usize) -> Result<()> {
        check(unsafe {
            ffi::ft_hip_reduce_pairs_weighted(self.ctx, s.0, p(y), p(wts), p(seq_of), pm(out), hidden as i64,
                                              n_pairs as i64, n_seqs as i64)
        })
    }

    /// Dense q4r GEMV from an f32 row, its q8 computed in the launch
    /// (`quantize_q8` + `gemv_q4r_idx`); with `act`, a gate|up matrix whose
    /// launch also stores gelu_tanh(gate) * up per column, the f32 of
    /// `gelu_mul_q8` (ft-model/src/lib.rs:1368-1395).
    #[allow(clippy::too_many_arguments)]
    pub fn gemv_q4r_f32in(&self, s: Stream, w: DevPtr, x: DevPtr, y: DevPtr, act: Option<DevPtr>, n_rows: usize,
                          k: usize) -> Result<()> {
        let a: *mut f32 = match act {
            Some(v) => pm(v),
            None => std::ptr::null_mut(),
        };
        check(unsafe { ffi::ft_hip_gemv_q4r_f32in(self.ctx, s.0, p(w), p(x), pm(y), a, n_rows as i64, k as i64) })
    }

    /// Gate|up GEMV with GELU*up and q8 in one launch (the `gemv_q4r_ptr` +
    /// `gelu_mul_q8` pair of ft-model/src/lib.rs:1584-1593).
    #[allow(clippy::too_many_arguments)]
    pub fn gemv_gate_up_act(&self, s: Stream, base: DevPtr, expert_bytes: usize, slots: DevPtr, n_pairs: usize,
                            x_div: usize, q8x: DevPtr, hidden: usize, inter: usize, layout: Layout,
                            in_scale: Option<DevPtr>, q8_act: DevPtr) -> Result<()> {
        check(unsafe {
            ffi::ft_hip_gemv_gate_up_act(self.ctx, s.0, p(base), expert_bytes as u64, p(slots), n_pairs as i64,
                                         x_div as i64, p(q8x), hidden as i64, inter as i64, layout.raw(),
                                         opt(in_scale), pm(q8_act))
        })
    }

    pub fn moe_layer_workspace_bytes(n_seqs: usize, hidden: usize, inter: usize, n_experts: usize, top_k: usize) -> usize {
        unsafe {
            ffi::ft_hip_moe_layer_workspace_bytes(n_seqs as i64, hidden as i64, inter as i64, n_experts as i64,
                                                  top_k as i64)
        }
    }

    /// One expert-FFN layer for n_seqs tokens (ft-model/src/lib.rs:1406-1476
    /// with device routing): x_out = x + combine, ids/wts the routing.
    #[allow(clippy::too_many_arguments)]
    pub fn moe_layer(&self, s: Stream, x: DevPtr, x_out: DevPtr, n_seqs: usize, hidden: usize, inter: usize,
                     n_experts: usize, top_k: usize, router_w: DevPtr, router_bias: Option<DevPtr>,
                     expert_scale: Option<DevPtr>, bank: DevPtr, expert_bytes: usize, layout: Layout, ids: DevPtr,
                     wts: DevPtr, workspace: DevPtr, workspace_bytes: usize) -> Result<()> {
        check(unsafe {
            ffi::ft_hip_moe_layer(self.ctx, s.0, p(x), pm(x_out), n_seqs as i64, hidden as i64, inter as i64,
                                  n_experts as i64, top_k as i64, p(router_w), opt(router_bias), opt(expert_scale),
                                  p(bank), expert_bytes as u64, layout.raw(), pm(ids), pm(wts), pm(workspace),
                                  workspace_bytes)
        })
    }

    /// `moe_layer` on the library's own scratch (no workspace, no allocation).
    #[allow(clippy::too_many_arguments)]
    pub fn moe_layer_noalloc(&self, s: Stream, x: DevPtr, x_out: DevPtr, n_seqs: usize, hidden: usize, inter: usize,
                             n_experts: usize, top_k: usize, router_w: DevPtr, router_bias: Option<DevPtr>,
                             expert_scale: Option<DevPtr>, bank: DevPtr, expert_bytes: usize, layout: Layout,
                             ids: DevPtr, wts: DevPtr) -> Result<()> {
        check(unsafe {
            ffi::ft_hip_moe_layer_noalloc(self.ctx, s.0, p(x), pm(x_out), n_seqs as i64, hidden as i64, inter as i64,
                                          n_experts as i64, top_k as i64, p(router_w), opt(router_bias),
                                          opt(expert_scale), p(bank), expert_bytes as u64, layout.raw(), pm(ids),
                                          pm(wts))
        })
    }

    pub fn moe_stack_workspace_bytes(n_seqs: usize, hidden: usize, inter: usize, n_experts: usize,
                                     top_k: usize) -> usize {
        unsafe {
            ffi::ft_hip_moe_stack_workspace_bytes(n_seqs as i64, hidden as i64, inter as i64, n_experts as i64,
                                                  top_k as i64)
        }
    }

    /// The MoE sections of every layer of the decode stack (ft-model/src/lib.rs:778-1056) on the
    /// launch-by-launch path: moe_layer for each layer, two launches per layer after the first.
    #[allow(clippy::too_many_arguments)]
    pub fn moe_stack(&self, s: Stream, x_in: DevPtr, x_out: DevPtr, n_seqs: usize, hidden: usize, inter: usize,
                     n_experts: usize, top_k: usize, n_layers: usize, routers: DevPtr, router_bias: Option<DevPtr>,
                     expert_scale: Option<DevPtr>, banks: DevPtr, expert_bytes: usize, layout: Layout, ids: DevPtr,
                     wts: DevPtr, workspace: DevPtr, workspace_bytes: usize) -> Result<()> {
        check(unsafe {
            ffi::ft_hip_moe_stack(self.ctx, s.0, p(x_in), pm(x_out), n_seqs as i64, hidden as i64, inter as i64,
                                  n_experts as i64, top_k as i64, n_layers as i64, p(routers), opt(router_bias),
                                  opt(expert_scale), p(banks), expert_bytes as u64, layout.raw(), pm(ids), pm(wts),
                                  pm(workspace), workspace_bytes)
        })
    }

    pub fn moe_layer_grouped_workspace_bytes(n_seqs: usize, hidden: usize, inter: usize, n_experts: usize,
                                             top_k: usize) -> usize {
        unsafe {
            ffi::ft_hip_moe_layer_grouped_workspace_bytes(n_seqs as i64, hidden as i64, inter as i64,
                                                          n_experts as i64, top_k as i64)
        }
    }

    /// The batched pair section (ft-model/src/lib.rs:1507-1606) with pairs
    /// grouped by expert; `bank` is one layer in the fused layout.
    #[allow(clippy::too_many_arguments)]
    pub fn moe_layer_grouped(&self, s: Stream, x: DevPtr, x_out: DevPtr, n_seqs: usize, hidden: usize, inter: usize,
                             n_experts: usize, top_k: usize, router_w: DevPtr, router_bias: Option<DevPtr>,
                             expert_scale: Option<DevPtr>, bank: DevPtr, ids: DevPtr, wts: DevPtr, workspace: DevPtr,
                             workspace_bytes: usize) -> Result<()> {
        check(unsafe {
            ffi::ft_hip_moe_layer_grouped(self.ctx, s.0, p(x), pm(x_out), n_seqs as i64, hidden as i64,
                                          inter as i64, n_experts as i64, top_k as i64, p(router_w),
                                          opt(router_bias), opt(expert_scale), p(bank), pm(ids), pm(wts),
                                          pm(workspace), workspace_bytes, std::ptr::null_mut(), std::ptr::null_mut())
        })
    }

    pub fn moe_stack_grouped_workspace_bytes(max_seqs: usize, hidden: usize, inter: usize, n_experts: usize,
                                             top_k: usize, n_layers: usize) -> usize {
        unsafe {
            ffi::ft_hip_moe_stack_grouped_workspace_bytes(max_seqs as i64, hidden as i64, inter as i64,
                                                          n_experts as i64, top_k as i64, n_layers as i64)
        }
    }

    /// All layers of a forward_batch step (ft-model/src/lib.rs:1151-1154,
    /// :1507-1606) for n_seqs <= max_seqs tokens, on one workspace sized for
    /// max_seqs; `banks` holds the layers' fused-layout banks back to back.
    #[allow(clippy::too_many_arguments)]
    pub fn moe_stack_grouped(&self, s: Stream, x_in: DevPtr, x_out: DevPtr, n_seqs: usize, max_seqs: usize,
                             hidden: usize, inter: usize, n_experts: usize, top_k: usize, n_layers: usize,
                             banks: DevPtr, routers: DevPtr, router_bias: Option<DevPtr>,
                             expert_scale: Option<DevPtr>, ids: Option<DevPtr>, wts: Option<DevPtr>,
                             workspace: DevPtr, workspace_bytes: usize) -> Result<()> {
        check(unsafe {
            ffi::ft_hip_moe_stack_grouped(self.ctx, s.0, p(x_in), pm(x_out), n_seqs as i64, max_seqs as i64,
                                          hidden as i64, inter as i64, n_experts as i64, top_k as i64,
                                          n_layers as i64, p(banks), p(routers), opt(router_bias), opt(expert_scale),
                                          ids.map_or(std::ptr::null_mut(), pm), wts.map_or(std::ptr::null_mut(), pm),
                                          pm(workspace), workspace_bytes)
        })
    }

    /// The whole L-layer section for one token in one launch (the graphed
    /// token of ft-model/src/lib.rs:1059-1121); Gemma shape.
    #[allow(clippy::too_many_arguments)]
    pub fn moe_stack_fused(&self, s: Stream, x_in: DevPtr, x_out: DevPtr, hidden: usize, inter: usize,
                           n_experts: usize, top_k: usize, n_layers: usize, banks: DevPtr, routers: DevPtr,
                           bias: Option<DevPtr>, expert_scale: Option<DevPtr>, ids: Option<DevPtr>,
                           wts: Option<DevPtr>, workspace: DevPtr, workspace_bytes: usize) -> Result<()> {
        let opt_m = |a: Option<DevPtr>| a.map_or(std::ptr::null_mut(), |v| v as usize as *mut _);
        check(unsafe {
            ffi::ft_hip_moe_stack_fused(self.ctx, s.0, p(x_in), pm(x_out), hidden as i64, inter as i64,
                                        n_experts as i64, top_k as i64, n_layers as i64, p(banks), p(routers),
                                        opt(bias), opt(expert_scale), opt_m(ids), opt_m(wts), pm(workspace),
                                        workspace_bytes, std::ptr::null_mut(), std::ptr::null_mut(),
                                        std::ptr::null_mut(), std::ptr::null_mut())
        })
    }

    /// Bytes of the fused kernel's refined-prediction table for n_layers layers.
    pub fn fused_predictor_bytes(hidden: usize, inter: usize, n_experts: usize, n_layers: usize) -> Option<usize> {
        let n = unsafe { ffi::ft_hip_fused_predictor_bytes(hidden as i64, inter as i64, n_experts as i64, n_layers as i64) };
        if n < 0 { None } else { Some(n as usize) }
    }

    /// Build the refined-prediction table (M = R_{l+1} D_{l,e}) from fused banks and routers (setup).
    #[allow(clippy::too_many_arguments)]
    pub fn fused_build_predictor(&self, s: Stream, banks: DevPtr, routers: DevPtr, hidden: usize, inter: usize,
                                 n_experts: usize, n_layers: usize, table: DevPtr, table_bytes: usize) -> Result<()> {
        check(unsafe {
            ffi::ft_hip_fused_build_predictor(self.ctx, s.0, p(banks), p(routers), hidden as i64, inter as i64,
                                              n_experts as i64, n_layers as i64, pm(table), table_bytes)
        })
    }

    /// Later fused launches prefetch the refined prediction (None: the early routing's alone).
    pub fn fused_set_predictor(&self, table: Option<(DevPtr, usize)>, n_layers: usize) -> Result<()> {
        let (t, n) = table.map_or((std::ptr::null(), 0), |(t, n)| (p(t), n));
        check(unsafe { ffi::ft_hip_fused_set_predictor(self.ctx, t, n, n_layers as i64) })
    }

    /// After synchronising the stream: Err if a fused launch on `workspace`
    /// gave up a bounded wait (its outputs are NaN / id -1).
    pub fn fused_status(&self, workspace: DevPtr) -> Result<bool> {
        let mut aborted = 0;
        let rc = unsafe { ffi::ft_hip_fused_status(self.ctx, pm(workspace), &mut aborted) };
        if rc == ffi::FT_HIP_E_TIMEOUT {
            return Ok(true);
        }
        check(rc)?;
        Ok(aborted != 0)
    }

    pub fn set_input_norm(&self, on: bool) -> Result<()> {
        check(unsafe { ffi::ft_hip_set_input_norm(self.ctx, on as i32) })
    }

    /// The expert banks of layers `layer0..layer0 + n_layers` of a GGUF file
    /// into device `banks` (ft-model/src/lib.rs:570-609): expert (l, e) at
    /// ((l - layer0) * n_experts + e) * expert_bytes, gate|up rows then down
    /// rows in `layout`. Synchronises `s`.
    pub fn load_expert_banks_gguf(&self, s: Stream, g: &Gguf, layer0: usize, n_layers: usize, hidden: usize,
                                  inter: usize, n_experts: usize, banks: DevPtr, expert_bytes: usize,
                                  layout: Layout) -> Result<()> {
        check(unsafe {
            ffi::ft_hip_load_expert_banks_gguf(self.ctx, s.0, g.h, layer0 as i64, n_layers as i64, hidden as i64,
                                               inter as i64, n_experts as i64, pm(banks), expert_bytes as u64,
                                               layout.raw())
        })
    }
}

/// One entry of a GGUF tensor table (`ft_gguf::TensorInfo`).
#[derive(Debug, Clone, PartialEq)]
pub struct TensorInfo {
    /// ne[0] is the contiguous (row/k) dimension, ggml order.
    pub dims: Vec<u64>,
    pub ggml_type: u32,
    /// byte offset within the data section
    pub offset: u64,
    pub nbytes: u64,
}

/// A local GGUF v2/v3 file, mapped read-only (`ft_gguf::Gguf`,
/// ft-gguf/src/lib.rs:141-206): header, metadata and tensor table parsed at
/// `open`, tensor bytes borrowed from the mapping.
pub struct Gguf {
    h: *mut ffi::FtGguf,
}

fn cstr(s: &str) -> Result<std::ffi::CString> {
    Ok(std::ffi::CString::new(s)?)
}

impl Gguf {
    pub fn open(path: impl AsRef<std::path::Path>) -> Result<Self> {
        let p = cstr(&path.as_ref().to_string_lossy())?;
        let mut h = std::ptr::null_mut();
        check(unsafe { ffi::ft_gguf_open(p.as_ptr(), &mut h) })?;
        Ok(Self { h })
    }

    pub fn tensor(&self, name: &str) -> Result<TensorInfo> {
        let n = cstr(name)?;
        let (mut nd, mut ty, mut off, mut nb) = (0u32, 0u32, 0u64, 0u64);
        let mut dims = [0u64; 8];
        check(unsafe {
            ffi::ft_gguf_tensor_info(self.h, n.as_ptr(), &mut nd, dims.as_mut_ptr(), &mut ty, &mut off, &mut nb)
        })?;
        Ok(TensorInfo { dims: dims[..nd as usize].to_vec(), ggml_type: ty, offset: off, nbytes: nb })
    }

    pub fn tensor_data(&self, name: &str) -> Result<&[u8]> {
        let n = cstr(name)?;
        let mut data: *const c_void = std::ptr::null();
        let mut nb = 0u64;
        check(unsafe { ffi::ft_gguf_tensor_data(self.h, n.as_ptr(), &mut data, &mut nb) })?;
        // from_raw_parts needs a non-null pointer even for an empty slice
        if data.is_null() || nb == 0 {
            return Ok(&[]);
        }
        Ok(unsafe { std::slice::from_raw_parts(data as *const u8, nb as usize) })
    }

    /// `Value::as_u64` of a metadata value.
    pub fn meta_u64(&self, key: &str) -> Result<u64> {
        let k = cstr(key)?;
        let mut v = 0u64;
        check(unsafe { ffi::ft_gguf_meta_u64(self.h, k.as_ptr(), &mut v) })?;
        Ok(v)
    }

    pub fn meta_f32(&self, key: &str) -> Result<f32> {
        let k = cstr(key)?;
        let mut v = 0f32;
        check(unsafe { ffi::ft_gguf_meta_f32(self.h, k.as_ptr(), &mut v) })?;
        Ok(v)
    }

    pub fn meta_str(&self, key: &str) -> Result<String> {
        let k = cstr(key)?;
        let (mut s, mut n) = (std::ptr::null(), 0u64);
        check(unsafe { ffi::ft_gguf_meta_str(self.h, k.as_ptr(), &mut s, &mut n) })?;
        if s.is_null() || n == 0 {
            return Ok(String::new());
        }
        let b = unsafe { std::slice::from_raw_parts(s as *const u8, n as usize) };
        Ok(String::from_utf8_lossy(b).into_owned())
    }

    /// ft-model's to_f32 (ft-model/src/lib.rs:128-151) of an f32, f16 or q4_0 tensor.
    pub fn to_f32(&self, name: &str) -> Result<Vec<f32>> {
        let n: u64 = self.tensor(name)?.dims.iter().product();
        let mut out = vec![0f32; n as usize];
        let c = cstr(name)?;
        check(unsafe { ffi::ft_gguf_tensor_to_f32(self.h, c.as_ptr(), out.as_mut_ptr(), n) })?;
        Ok(out)
    }

    /// The router of `layer` with its scale and hidden^-1/2 folded in
    /// (ft-model/src/lib.rs:506-514), [n_experts][hidden].
    pub fn router_f32(&self, layer: usize, hidden: usize, n_experts: usize) -> Result<Vec<f32>> {
        let mut out = vec![0f32; hidden * n_experts];
        check(unsafe {
            ffi::ft_gguf_router_f32(self.h, layer as i64, hidden as i64, n_experts as i64, out.as_mut_ptr())
        })?;
        Ok(out)
    }
}

impl Drop for Gguf {
    fn drop(&mut self) {
        unsafe {
            ffi::ft_gguf_close(self.h);
        }
    }
}

impl Drop for Q4Gemv {
    fn drop(&mut self) {
        unsafe {
            ffi::ft_hip_destroy(self.ctx);
        }
    }
}
