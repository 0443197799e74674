/* ft_hip.h -- C ABI of the MI355X (gfx950) MoE expert-FFN decode library.
 *
 * This is the drop-in boundary for freeToken-rs's GPU expert section. Each
 * entry point names the reference interface it replaces (paths relative to
 * the freeToken-rs repository root). Conventions, mirroring ft_cuda::Q4Gemv
 * (ft-cuda/src/lib.rs:69-150):
 *   - the caller owns every device buffer; no entry point allocates device
 *     memory during a launch (ft-cuda/src/lib.rs:989-990), so launches can be
 *     captured into a HIP graph;
 *   - launches are asynchronous on the given stream (a hipStream_t passed as
 *     void*; NULL is the null stream) and never synchronise the host;
 *   - where the reference panics on a violated shape precondition
 *     (assert!, e.g. ft-cuda/src/lib.rs:171-173), these entry points return
 *     FT_HIP_E_SHAPE before touching the GPU, and ft_hip_last_error() names
 *     the violated condition. Runtime failures return FT_HIP_E_LAUNCH (the
 *     reference's Err via `?`, lib.rs:184);
 *   - one context is used by one host thread at a time (the reference keeps
 *     Model and its Q4Gemv on one worker thread, ft-model/src/bin/serve.rs:635).
 *
 * Data formats:
 *   q4_0 rows : ggml block_q4_0, 18 B per 32 weights {f16 d; u8 qs[16]},
 *               byte i = q_i | q_{i+16} << 4, w = (q - 8) * d
 *               (ft-core/src/q4_0.rs:1-16).
 *   q4r rows  : [nb f16 scales, zero-padded to 16 B][nb x 16 B qs]
 *               (ft-core/src/q4_0.rs:234-258).
 *   q8 blocks : FT_Q8_BLK = 40 B per 32 activations {f32 d; i32 qsum; i8 qs[32]}.
 *               The reference's 40-B block is {f32 d; f32 d*sum(qs); i8 qs[32]}
 *               (ft-cuda/src/q4.cu:316-320); this build keeps the exact integer
 *               sum so the -8 offset folds out in integer arithmetic. q8 buffers
 *               are only produced and consumed by this library.
 */
#ifndef FT_HIP_H
#define FT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FT_HIP_OK 0
#define FT_HIP_E_INVALID (-1) /* null pointer or bad enum value */
#define FT_HIP_E_SHAPE (-2)   /* a shape precondition does not hold */
#define FT_HIP_E_DEVICE (-3)  /* no usable gfx950 device */
#define FT_HIP_E_LAUNCH (-4)  /* HIP runtime or launch failure */
#define FT_HIP_E_TIMEOUT (-5) /* the fused kernel's bounded wait expired */
#define FT_HIP_E_IO (-6)      /* a file could not be opened or mapped */
#define FT_HIP_E_FORMAT (-7)  /* a malformed or unsupported file or value */
#define FT_HIP_E_NOT_FOUND (-8) /* no such tensor, metadata key or index */

#define FT_Q8_BLK 40

/* weight row layouts */
#define FT_LAYOUT_Q4_0 0
#define FT_LAYOUT_Q4R 1

typedef struct ft_hip_ctx ft_hip_ctx;

/* Library version (major*10000 + minor*100 + patch). */
int ft_hip_version(void);

/* Message of the last failing call on this host thread ("" if none). */
const char* ft_hip_last_error(void);

/* Replaces Q4Gemv::new (ft-cuda/src/lib.rs:111-150): binds `device`, checks
 * that it is gfx950 and records its compute-unit count. */
int ft_hip_create(int device, ft_hip_ctx** out);
int ft_hip_destroy(ft_hip_ctx* ctx);

/* Byte sizes of one row of k weights (ft-core/src/q4_0.rs:13-16, :238-245).
 * Return -1 if k is not a multiple of 32. */
int64_t ft_hip_row_bytes(int layout, int64_t k);
int64_t ft_hip_q4r_scales_bytes(int64_t k);

/* Replaces Q4Gemv::quantize_q8 / quantize_q8_view (ft-cuda/src/lib.rs:898-921,
 * :871-894) with the arithmetic of ft-core's Q8Vec::quantize
 * (ft-core/src/q4_0.rs:62-78: d = amax/127, round half away from zero).
 * x: [n, x_stride] f32 (x_stride 0 shares one vector), q8: [n, k/32] blocks. */
int ft_hip_quantize_q8(ft_hip_ctx* ctx, void* stream, const float* x, int64_t x_stride,
                       void* q8, int64_t k, int64_t n);

/* Grouped q4 x q8 GEMV over per-entry weight pointers. Replaces
 * gemv_grouped_q8_ptr (ft-cuda/src/lib.rs:593-623, layout q4_0) and
 * gemv_q4r_ptr (ft-cuda/src/lib.rs:736-767, layout q4r).
 *   bases   : device u64 [n_entries], entry e's weights at bases[e] + bank_off
 *   x_idx   : device i32 [n_entries] (entry e reads q8 row x_idx[e]) or NULL
 *             (entry e reads q8 row e)
 *   q8 row r starts at q8 + r * q8_stride_blocks * 40 (stride 0 shares one)
 *   y[e * y_stride + row] = dot(W_e[row], q8 row)  for row < n_rows */
int ft_hip_gemv_q4_grouped_ptr(ft_hip_ctx* ctx, void* stream, const uint64_t* bases,
                               uint64_t bank_off, const int32_t* x_idx, int64_t n_entries,
                               const void* q8, int64_t q8_stride_blocks, float* y,
                               int64_t y_stride, int64_t n_rows, int64_t k, int layout);

/* Same over a slot-indexed bank: entry e's weights at
 * base + slots[e] * expert_bytes + bank_off. Replaces gemv_grouped_q8
 * (ft-cuda/src/lib.rs:926-957), gemv_grouped_q8_idx (:772-804) and
 * gemv_q4r_idx (:699-732). */
int ft_hip_gemv_q4_grouped_slots(ft_hip_ctx* ctx, void* stream, const void* base,
                                 uint64_t expert_bytes, uint64_t bank_off, const int32_t* slots,
                                 const int32_t* x_idx, int64_t n_entries, const void* q8,
                                 int64_t q8_stride_blocks, float* y, int64_t y_stride,
                                 int64_t n_rows, int64_t k, int layout);

/* Test entry (no reference counterpart): dumps the per-(entry, row, block)
 * int32 dots sum_i (q4_i - 8) * q8_i computed by the same device routine the
 * GEMVs use. out: [n_entries, n_rows, k/32] i32. Addressing as _slots. */
int ft_hip_q4q8_block_dots(ft_hip_ctx* ctx, void* stream, const void* base,
                           uint64_t expert_bytes, uint64_t bank_off, const int32_t* slots,
                           const int32_t* x_idx, int64_t n_entries, const void* q8,
                           int64_t q8_stride_blocks, int32_t* out, int64_t n_rows, int64_t k,
                           int layout);

/* Replaces gelu_mul_q8 (ft-cuda/src/lib.rs:354-374; kernel q4.cu:255-287):
 * act = gelu_tanh(gu[:, j]) * gu[:, inter + j] (ft-model/src/lib.rs:435-437),
 * then Q8Vec::quantize. gu: [n, 2*inter] f32, q8: [n, inter/32] blocks.
 * tanh returns the bits of glibc's tanhf, which Rust's f32::tanh calls on
 * Linux (a restatement of its fdlibm algorithm in IEEE basic operations). */
int ft_hip_gelu_mul_q8(ft_hip_ctx* ctx, void* stream, const float* gu, void* q8, int64_t inter,
                       int64_t n);

/* Replaces silu_mul_grouped (ft-cuda/src/lib.rs:1053-1072; kernel q4.cu:169-179):
 * out[e][j] = (g / (1 + expf(-g))) * gu[e][inter + j], g = gu[e][j], for
 * e < n_experts, j < inter; gu [n_experts][2*inter] f32, out [n_experts][inter].
 * The f32 expression of the reference's CPU twin (ft-bench/src/bin/decode.rs:300),
 * one rounding per operation, with glibc's expf: bit-exact with it. */
int ft_hip_silu_mul_grouped(ft_hip_ctx* ctx, void* stream, const float* gu, float* out, int64_t inter,
                            int64_t n_experts);

/* Replaces gelu_mul_grouped (ft-cuda/src/lib.rs:1009-1028; kernel q4.cu:289-300):
 * out[e][j] = gelu_tanh(gu[e][j]) * gu[e][inter + j] with ft-model's CPU GELU
 * (ft-model/src/lib.rs:435-437; glibc's tanhf), the f32 activations
 * ft_hip_gelu_mul_q8 quantizes. Shapes as ft_hip_silu_mul_grouped. */
int ft_hip_gelu_mul_grouped(ft_hip_ctx* ctx, void* stream, const float* gu, float* out, int64_t inter,
                            int64_t n_experts);

/* Replaces reduce_expert_weighted (ft-cuda/src/lib.rs:1031-1050; kernel
 * q4.cu:303-314): out[i] = out[i] + s, s = sum over e = 0..n_experts-1 (in
 * order, from 0) of wts[e] * y[e][i]; y [n_experts][hidden], wts [n_experts],
 * one rounding per operation (the pair combine's f32 order,
 * ft-model/src/lib.rs:1634-1646). n_experts = 0 leaves out unchanged. */
int ft_hip_reduce_expert_weighted(ft_hip_ctx* ctx, void* stream, const float* y, const float* wts,
                                  float* out, int64_t hidden, int64_t n_experts);

/* Replaces reduce_weighted (ft-cuda/src/lib.rs:1075-1094; kernel q4.cu:182-192):
 * out[i] = out[i] + a * s, s = sum over e (in order, from 0) of y[e][i], one
 * rounding per operation (the reference kernel's expression order without
 * contraction). */
int ft_hip_reduce_weighted(ft_hip_ctx* ctx, void* stream, const float* y, float* out, float a,
                           int64_t hidden, int64_t n_experts);

/* Gate|up GEMV and the activation in one launch: replaces gemv_q4r_ptr over
 * the gate|up rows followed by gelu_mul_q8 (ft-model/src/lib.rs:1584-1593;
 * ft-cuda/src/lib.rs:354-374). Pair p runs expert slots[p] (gate|up rows
 * [2I x H] at base + slots[p]*expert_bytes, in `layout`) against q8 row
 * p / x_div of q8x ([*, H/32] blocks); the gate and up sums are multiplied by
 * in_scale[p / x_div] when in_scale is not NULL (the input RMS norm).
 * q8_act: [n_pairs, I/32] blocks of gelu_tanh(gate) * up, the arithmetic of
 * ft_hip_gelu_mul_q8; the f32 gate and up sums run in 4 lane chains per row
 * (lane s: blocks s, s+4, ...; ft_hip_gemv_q4_grouped_slots uses 8), so
 * they may differ from that GEMV's in the last bits. */
int ft_hip_gemv_gate_up_act(ft_hip_ctx* ctx, void* stream, const void* base, uint64_t expert_bytes,
                            const int32_t* slots, int64_t n_pairs, int64_t x_div, const void* q8x,
                            int64_t hidden, int64_t inter, int layout, const float* in_scale,
                            void* q8_act);

/* A dense q4r GEMV from an f32 input row, its q8 computed in the same launch
 * with the bits of ft_hip_quantize_q8; the shared MLP's chain (ft-model/src/
 * lib.rs:1368-1395: quantize_q8, gemv_q4r gate|up, gelu_mul_q8, gemv_q4r
 * down; ft-cuda/src/lib.rs:329-374, :736-767) then runs as two launches:
 *   gate|up: x [k] -> y [2I] gate and up sums, act [I] f32 = gelu_tanh(gate)
 *     * up, the f32 that gelu_mul_q8 quantizes (replaces quantize_q8 +
 *     gemv_q4r_idx + the f32 half of gelu_mul_q8);
 *   down: x = act, act NULL (replaces the q8 half of gelu_mul_q8 +
 *     gemv_q4r_idx).
 * y[r] = row r of w ([n_rows x k] q4r) against q8(x), with the sums of
 * ft_hip_gemv_q4_grouped_slots (one entry, that q8) at the same lanes per
 * row bit for bit: the 16, 32 or 64 lanes that GEMV takes, except with act
 * (unless ft_hip_set_gemv_lanes forces them) 32 for rows up to 256 blocks;
 * where that GEMV takes 8 lanes (65,536 rows and more, or forced), 16, 32 or
 * 64 by row length (sums within rounding of its). act:
 * NULL, or for a gate|up matrix (n_rows = 2I, even) its [n_rows/2] outputs.
 * w and x 16-byte aligned; k <= 16384. */
int ft_hip_gemv_q4r_f32in(ft_hip_ctx* ctx, void* stream, const void* w, const float* x, float* y,
                          float* act, int64_t n_rows, int64_t k);

/* Replaces gemv_f32_rows_dev (ft-cuda/src/lib.rs:674-694): router logits
 * y[s][e] = sum_i W[e][i] * x[s][i] in this library's R-order (chunks of 16
 * elements by fma, 8 groups of dim/128 chunks, summed in order), plus bias[e]
 * if bias is not NULL. dim must be a multiple of 128. */
int ft_hip_router_logits(ft_hip_ctx* ctx, void* stream, const float* w, const float* x,
                         const float* bias, float* y, int64_t dim, int64_t n_rows,
                         int64_t n_seqs);

/* Replaces topk_router_dev (ft-cuda/src/lib.rs:472-494): per sequence, top-k
 * logits (ties: lower expert index first), weights exp(l - lmax)/sum over the
 * top-k, times expert_scale[e] (NULL = 1). e_count <= 1024, k <= 32. */
int ft_hip_topk_router(ft_hip_ctx* ctx, void* stream, const float* logits,
                       const float* expert_scale, int32_t* ids, float* wts, int64_t e_count,
                       int64_t k, int64_t n_seqs);

/* Replaces reduce_pairs_weighted (ft-cuda/src/lib.rs:808-829):
 * out[s][i] += sum over pairs p with seq_of[p] == s, in p order, of
 * wts[p] * y[p][i] (products rounded, then summed from 0, as the CPU pair
 * combine of ft-model/src/lib.rs:1641-1646). */
int ft_hip_reduce_pairs_weighted(ft_hip_ctx* ctx, void* stream, const float* y,
                                 const float* wts, const int32_t* seq_of, float* out,
                                 int64_t hidden, int64_t n_pairs, int64_t n_seqs);

/* Row layout conversion on the device (setup, not the hot path): the
 * reference repacks q4_0 banks to q4r at load (ft-model/src/lib.rs:570-609,
 * ft-core/src/q4_0.rs:248-258). src and dst hold n_rows rows of k weights. */
int ft_hip_repack_rows(ft_hip_ctx* ctx, void* stream, const void* src, int src_layout,
                       void* dst, int dst_layout, int64_t n_rows, int64_t k);

/* Measurement utility (no reference counterpart; the reference's own
 * bandwidth line is ft-bench's "cpu q4_0 gemv GB/s", ft-bench/src/main.rs:
 * 77-114): reads `bytes` (16-byte aligned) of device memory at buf once with
 * n_workgroups 256-thread workgroups (grid-stride, four 16-byte loads in
 * flight per thread) and writes each workgroup's XOR of what it read to
 * out[n_workgroups]. Its rate is the achievable HBM read bandwidth the GEMV
 * kernels are compared with, and its known byte count calibrates the
 * profiler's FETCH_SIZE counter. */
int ft_hip_stream_read(ft_hip_ctx* ctx, void* stream, const void* buf, uint64_t bytes, uint32_t* out,
                       int n_workgroups);

/* Seeded synthetic inputs (no reference counterpart; the reference's synthetic
 * bench uses templated weights, ft-bench/src/bin/decode.rs:111-116).
 * Value i of the tensor with key `key`: Irwin-Hall(4) over the 16-bit fields of
 * splitmix64(key + (i+1)*0x9E3779B97F4A7C15), centred, times `scale`.
 * gen_values writes n f32 values starting at index `start`; gen_q4_rows writes
 * rows [row0, row0 + n_rows) of a seeded [*, k] matrix quantized to q4_0
 * (ft-core/src/q4_0.rs:20-40) in `layout`. */
int ft_hip_gen_values(ft_hip_ctx* ctx, void* stream, uint64_t key, int64_t start, int64_t n,
                      float scale, float* out);
int ft_hip_gen_q4_rows(ft_hip_ctx* ctx, void* stream, uint64_t key, int64_t row0,
                       int64_t n_rows, int64_t k, float scale, void* out, int layout);

/* Test hook (no reference counterpart): while set, ft_hip_moe_layer_grouped,
 * ft_hip_moe_stack_fused and ft_hip_gemv_q4_grouped_ptr/_slots run
 * instantiations of their kernels that also store every per-block int32 dot
 * sum_i (q4_i - 8) * q8_i their production inner loops compute (v_dot4 and
 * int8 MFMA alike; the production instantiations are unchanged), into
 *   grouped: gu_dots [n_seqs*top_k pairs][2*inter rows][hidden/32 blocks],
 *            dn_dots [pairs][hidden rows][inter/32 blocks], pair p = s*top_k + k;
 *   fused:   gu_dots [n_layers][top_k slots][2*inter][hidden/32],
 *            dn_dots [n_layers][top_k][hidden][inter/32] (with the dbg_* record on);
 *   gemv:    gu_dots [n_entries][n_rows][k/32] (dn_dots unused).
 * Rows are the expert's gate rows then up rows (gate|up) or its down rows.
 * Both NULL (the state after create) turns it off; give both or neither. */
int ft_hip_set_block_dot_record(ft_hip_ctx* ctx, int32_t* gu_dots, int32_t* dn_dots);

/* Test hook (no reference counterpart): while any pointer is set,
 * ft_hip_moe_layer, ft_hip_moe_layer_noalloc and ft_hip_moe_stack run
 * instantiations of the launch-by-launch layer kernels that also store the
 * stages they compute (the production instantiations are unchanged), per
 * layer l of the call (l = 0 for one layer), seq s and pair p = s*top_k + k:
 *   x       [l][s][hidden]             f32 layer input as the layer read it
 *   q8x     [l][s][hidden/32] x 40 B   its q8 blocks as the gate|up launch took them
 *   gu      [l][p][2*inter]            f32 gate sums then up sums as GELU takes them
 *                                      (times the input norm's scale when on)
 *   act     [l][p][inter/32] x 40 B    the activation's q8 blocks
 *   gu_dots [l][p][2*inter][hidden/32] int32 block dots of the gate|up rows
 *   dn_dots [l][p][hidden][inter/32]   int32 block dots of the down rows
 * ft_hip_gemv_gate_up_act stores gu and gu_dots of its pairs ([p][...]).
 * NULL pointers are skipped; all NULL (the state after create) turns it off. */
int ft_hip_set_layer_record(ft_hip_ctx* ctx, float* x, void* q8x, float* gu, void* act, int32_t* gu_dots,
                            int32_t* dn_dots);

/* One MoE expert-FFN layer for n_seqs tokens (the composition of
 * ft-model/src/lib.rs:1406-1476 with host routing replaced by device routing):
 *   logits = router(W_r, x) (+bias) -> top-k/softmax -> q8(x) -> grouped
 *   gate|up GEMV -> gelu*up -> q8 -> grouped down GEMV -> x_out = x + combine.
 * Three launches: logits with q8(x); gate|up with the top-k (n_experts <= 256)
 * and the activation; down with the combine (top_k dividing 32 and the k
 * activation rows of a token within 64 KB). Other shapes add a top-k launch
 * or a separate combine launch; the results are the same bits either way.
 * Expert e of this layer: gate|up rows [2I x H] at bank + e*expert_bytes,
 * down rows [H x I] right after them (gu_bytes = 2I * row_bytes(H)), both in
 * `layout`. x_out may equal x. workspace: device scratch of
 * ft_hip_moe_layer_workspace_bytes() bytes. ids/wts (device [n_seqs*k]) receive
 * the routing. */
size_t ft_hip_moe_layer_workspace_bytes(int64_t n_seqs, int64_t hidden, int64_t inter,
                                        int64_t n_experts, int64_t top_k);
int ft_hip_moe_layer(ft_hip_ctx* ctx, void* stream, const float* x, float* x_out,
                     int64_t n_seqs, int64_t hidden, int64_t inter, int64_t n_experts,
                     int64_t top_k, const float* router_w, const float* router_bias,
                     const float* expert_scale, const void* bank, uint64_t expert_bytes,
                     int layout, int32_t* ids, float* wts, void* workspace,
                     size_t workspace_bytes);

/* The n_layers-layer expert section of the launch-by-launch path:
 * ft_hip_moe_layer for each layer in turn, x_{l+1} = x_l + MoE_l(x_l) (the
 * MoE section of every layer of ft-model's decode stack, lib.rs:778-1056,
 * per-layer body :1406-1476). Where the shape allows (n_experts <= 256,
 * top_k dividing 32 with at most 8, the k activation rows of a token within
 * 64 KB), each layer's down launch also computes the next layer's router
 * partials, so layers after the first take two launches instead of three;
 * the results are those of the layer-by-layer calls, bit for bit, either way.
 * banks: the layers' banks back to back (layer l at l * n_experts *
 * expert_bytes, each as ft_hip_moe_layer's `bank`); routers [L][E][H];
 * router_bias and expert_scale [L][E] or NULL; ids/wts [L][n_seqs*top_k]
 * (device) receive the routing. x_in, x_out [n_seqs][H]. workspace: device
 * scratch of ft_hip_moe_stack_workspace_bytes() bytes. No allocation; the
 * launches can be captured in a HIP graph. */
size_t ft_hip_moe_stack_workspace_bytes(int64_t n_seqs, int64_t hidden, int64_t inter,
                                        int64_t n_experts, int64_t top_k);
int ft_hip_moe_stack(ft_hip_ctx* ctx, void* stream, const float* x_in, float* x_out,
                     int64_t n_seqs, int64_t hidden, int64_t inter, int64_t n_experts,
                     int64_t top_k, int64_t n_layers, const float* routers,
                     const float* router_bias, const float* expert_scale, const void* banks,
                     uint64_t expert_bytes, int layout, int32_t* ids, float* wts,
                     void* workspace, size_t workspace_bytes);

/* ft_hip_moe_layer without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference. Its
 * scratch is a library-owned device array of FT_HIP_NOALLOC_SCRATCH_BYTES per
 * GPU (resolved at ft_hip_create, held until the process ends); a shape whose
 * ft_hip_moe_layer_workspace_bytes() exceeds that returns FT_HIP_E_SHAPE.
 * The call itself allocates nothing. Every call on one GPU shares that
 * array: calls that overlap on one GPU (other streams, other contexts, other
 * host threads) race and must be serialised by the caller. Same kernels and
 * results as ft_hip_moe_layer. */
#define FT_HIP_NOALLOC_SCRATCH_BYTES (8 << 20)
int ft_hip_moe_layer_noalloc(ft_hip_ctx* ctx, void* stream, const float* x, float* x_out,
                             int64_t n_seqs, int64_t hidden, int64_t inter, int64_t n_experts,
                             int64_t top_k, const float* router_w, const float* router_bias,
                             const float* expert_scale, const void* bank, uint64_t expert_bytes,
                             int layout, int32_t* ids, float* wts);

/* One MoE layer for n_seqs decode tokens with the (token, expert) pairs
 * grouped by expert: replaces the batched pair section of
 * ft-model/src/lib.rs:1507-1606 (quantize_q8, gemv_q4r_ptr over every pair,
 * gelu_mul_q8, gemv_q4r_ptr, reduce_pairs_weighted), which re-reads an
 * expert's weights for each of its tokens; here each routed expert's weights
 * stream once for all of its tokens. bank: ONE layer's n_experts experts in
 * the fused layout (ft_hip_pack_experts_fused), 16-byte aligned; router_w:
 * [E][H] f32. ids/wts: [n_seqs][top_k] routing (written). Same arithmetic as
 * ft_hip_moe_layer: q8 quants, block dots, routing, GELU q8 and the combine
 * (slot order) are bit-identical; f32 GEMV sums may differ in order.
 * dbg_gu [n_seqs*top_k][2I] f32 and dbg_act [n_seqs*top_k][I/32][40] (NULL
 * in normal use) receive the gate|up sums and act q8 blocks per pair.
 * Shapes: hidden 2816 or 4096, inter a multiple of 32 up to 16384,
 * n_seqs*top_k <= 4096. */
size_t ft_hip_moe_layer_grouped_workspace_bytes(int64_t n_seqs, int64_t hidden, int64_t inter,
                                                int64_t n_experts, int64_t top_k);
int ft_hip_moe_layer_grouped(ft_hip_ctx* ctx, void* stream, const float* x, float* x_out, int64_t n_seqs,
                             int64_t hidden, int64_t inter, int64_t n_experts, int64_t top_k,
                             const float* router_w, const float* router_bias, const float* expert_scale,
                             const void* bank, int32_t* ids, float* wts, void* workspace,
                             size_t workspace_bytes, float* dbg_gu, void* dbg_act);

/* The n_layers-layer expert section for a batch of n_seqs decode tokens:
 * ft_hip_moe_layer_grouped for each layer in turn, x_{l+1} = x_l +
 * MoE_l(x_l) (the batched pair section of ft-model/src/lib.rs:1507-1606 for
 * every layer of a forward_batch step, :1151-1154). banks: the layers'
 * fused-layout banks back to back (layer l at l * n_experts *
 * ft_hip_fused_expert_bytes(hidden, inter), 16-byte aligned); routers
 * [L][E][H]; router_bias and expert_scale [L][E] or NULL; ids/wts
 * [L][n_seqs][top_k] routing record, or both NULL. x_in, x_out [n_seqs][H]
 * (x_out may equal x_in). The workspace, sized by
 * ft_hip_moe_stack_grouped_workspace_bytes(max_seqs, ...), serves every
 * batch of n_seqs <= max_seqs tokens, so a serving loop whose batch grows
 * and shrinks between steps keeps one workspace; each call's results are
 * those of the layer-by-layer calls on the same tokens, bit for bit. No
 * allocation; the launches can be captured in a HIP graph. */
size_t ft_hip_moe_stack_grouped_workspace_bytes(int64_t max_seqs, int64_t hidden, int64_t inter,
                                                int64_t n_experts, int64_t top_k, int64_t n_layers);
int ft_hip_moe_stack_grouped(ft_hip_ctx* ctx, void* stream, const float* x_in, float* x_out, int64_t n_seqs,
                             int64_t max_seqs, int64_t hidden, int64_t inter, int64_t n_experts, int64_t top_k,
                             int64_t n_layers, const void* banks, const float* routers, const float* router_bias,
                             const float* expert_scale, int32_t* ids, float* wts, void* workspace,
                             size_t workspace_bytes);

/* ft_hip_moe_layer_grouped: experts routed at least n_tokens tokens of the
 * batch take the int8 MFMA tile kernels (16 rows x 16 tokens per
 * v_mfma_i32_16x16x32_i8, one q4_0 block per instruction), the others the
 * v_dot4 kernels; results agree to f32 summation order (q8 quants, int32
 * block dots, routing and GELU q8 are the same). 0 (the default) = automatic:
 * every expert on the MFMA kernels when the batch has at least 4 (token,
 * expert) pairs per expert (n_seqs * top_k >= 4 * n_experts), else every
 * expert on the dot4 kernels; 1 = MFMA
 * for every expert. Rows longer than 1024 weights (inter > 1024) always take
 * the MFMA kernels. No reference counterpart (the reference runs one GEMV
 * per (token, expert) pair, ft-model/src/lib.rs:1507-1606). */
int ft_hip_set_grouped_mfma_min(ft_hip_ctx* ctx, int n_tokens);

/* ft_hip_gemv_q4_grouped_ptr/_slots on q4r rows: lanes per row of the GEMV
 * launch. 8 = 32 rows per 256-thread workgroup, each lane streaming its
 * blocks four at a time (the kernel for long launches); 16, 32 or 64 =
 * 256/lanes rows per workgroup, each lane loading all of its blocks (at most
 * 8) at once (for launches of a few MB, such as a decode step's dense
 * projections, that would otherwise leave CUs idle). 0 (the default) =
 * automatic: 8 when the launch has at least 2048 workgroups of 32 rows, else
 * the fewest lanes that give 1024 workgroups (64 when none does). The int32
 * block dots are the same; y differs by f32 summation order only. No
 * reference counterpart (gemv_q4r_grouped_*, ft-cuda/src/q4.cu:1466-1567,
 * runs one warp per row). */
int ft_hip_set_gemv_lanes(ft_hip_ctx* ctx, int lanes_per_row);

/* Input RMS norm of the layer entry points (ft_hip_moe_layer,
 * ft_hip_moe_layer_grouped, ft_hip_moe_stack_fused); off (0) after create.
 * On (1), each layer runs on rmsnorm(x) = x * inv_r with
 *   inv_r = 1 / sqrt(ss / H + 1e-6),  ss = x.x in the R-order of the router
 * (each op rounded once, f32), applied where the layer is linear in its
 * input: router logits = R-order(W_r, x) * inv_r (+ bias), gate|up sums
 * times inv_r before GELU*up. q8 quants and int32 dots stay those of x; the
 * residual stays x. Replaces the caller-side norms that feed the reference's
 * router and routed experts (rmsnorm_rows_dev, ft-model/src/lib.rs:1362-1365
 * and :1398-1399; unweighted here), which keeps a layer chain bounded. */
int ft_hip_set_input_norm(ft_hip_ctx* ctx, int on);

/* ---- fused whole-stack path (no single reference counterpart) ----
 * The reference runs the section as a sequence of launches per layer
 * (ft-model/src/lib.rs:1406-1476) and removes host launch cost with a CUDA
 * graph over the whole stack (forward_sample_graphed, ft-model/src/lib.rs:
 * 1062-1121). Here the L-layer section for one token is ONE persistent
 * kernel whose workgroups hand data to each other through tagged words
 * (plain launch by default, see ft_hip_fused_set_cooperative): device-side
 * routing, gate|up, GELU*up, q8, down and
 * combine for every layer, with the same arithmetic as the launch-by-launch
 * entry points (q8 quants, per-block int32 dots, router R-order and top-k are
 * bit-identical; f32 sums may differ in order).
 *
 * Workgroups: K*max(I/32, H/128) expert units (routed slot p, index j: the
 * gate|up rows of act block j and the down rows 128j..128j+127 of expert
 * ids[p]) plus 16 group units (two per R-order group of H/8 rows: combine,
 * the router sums of half of the experts, q8 of x), 8 prediction units
 * (layer l+2's router sums over x_{l+1}) and 8 refiner units (the
 * prediction of layer l+1, see ft_hip_fused_set_predictor) -- see
 * ft_hip_fused_workgroups. Supported shape: the Gemma expert section (hidden
 * 2816, inter 704, 128 experts, top-8), the one its tests cover; other
 * shapes return FT_HIP_E_SHAPE (use ft_hip_moe_layer).
 *
 * Fused expert layout (a lossless repack of q4_0, same byte count):
 *   expert = [gate|up tiles][down tiles];
 *   gate|up tile jb (I/32 tiles) = 64 rows (gate rows 32jb..32jb+31, then up
 *     rows I+32jb..): [H/32 blocks x 64 rows x f16 scale][H/32 x 64 x 16 B qs];
 *   down tile jt (H/16 tiles) = rows 16jt..16jt+15:
 *     [I/32 blocks x 16 rows x f16 scale][I/32 x 16 x 16 B qs].
 * Fused router layout: [L][H/16 chunks][E][16] f32. */
int64_t ft_hip_fused_expert_bytes(int64_t hidden, int64_t inter);
size_t ft_hip_fused_workspace_bytes(int64_t hidden, int64_t inter, int64_t n_experts, int64_t top_k);

/* Grid size of ft_hip_moe_stack_fused for this shape (-1 on a bad shape);
 * sizes the dbg_trace buffer. */
int ft_hip_fused_workgroups(int64_t hidden, int64_t inter, int64_t n_experts, int64_t top_k);

/* Zero a fused workspace and set its epoch; call once after allocating it,
 * and again after a launch reported FT_HIP_E_TIMEOUT.
 * Epoch guard: every launch advances the workspace's 32-bit epoch by
 * 4*(n_layers+1), and the hand-over tags of a launch must stay below 2^32.
 * For a workspace initialised through this context, ft_hip_moe_stack_fused
 * tracks the epoch and re-initialises the workspace on the launch stream
 * before a launch that would pass the limit (every ~2^32/(4*(L+1)) launches:
 * 34.6M for 30 layers); a workspace near the limit that this context did not
 * initialise is refused by the kernel, which ft_hip_fused_status reports. */
int ft_hip_fused_workspace_init(ft_hip_ctx* ctx, void* stream, void* workspace, size_t workspace_bytes);

/* Test hook (no reference counterpart): set an initialised workspace's epoch
 * (nonzero) on the device and in this context's epoch guard, so tests can run
 * launches across the 2^32 limit of the tags. */
int ft_hip_fused_workspace_set_epoch(ft_hip_ctx* ctx, void* stream, void* workspace, uint32_t epoch);

/* Repack n_experts expert banks (gate rows, up rows, down rows, each in
 * src_layout, src_expert_bytes apart) into the fused layout
 * (ft_hip_fused_expert_bytes apart). Setup only. */
int ft_hip_pack_experts_fused(ft_hip_ctx* ctx, void* stream, const void* src, int src_layout,
                              uint64_t src_expert_bytes, void* dst, int64_t n_experts, int64_t hidden,
                              int64_t inter);

/* Repack routers [n_layers][E][H] f32 into the fused router layout. */
int ft_hip_pack_router_fused(ft_hip_ctx* ctx, void* stream, const float* src, float* dst, int64_t n_layers,
                             int64_t n_experts, int64_t hidden);

/* Run the n_layers-layer section for one token: x_out = x_L where
 * x_{l+1} = x_l + MoE_l(x_l). banks: [n_layers][E] fused experts; routers:
 * fused [n_layers][H/16][E][16]; bias, expert_scale: [n_layers][E] or NULL;
 * ids/wts: [n_layers][top_k] routing record or NULL. One workspace serves one
 * launch at a time (launches on one stream may reuse it). dbg_* (NULL in
 * normal use) receive per-layer stage values for tests: dbg_gu
 * [L][K][2I] gate|up sums, dbg_act [L][K][I/32] q8 blocks, dbg_x [L+1][H];
 * dbg_trace [workgroups][L+1][32] u64 receives wall-clock stamps of each
 * workgroup's phases (row 0 = the prologue), the analogue of the
 * reference's per-section Profile counters (ft-model/src/lib.rs:252-296). */
int ft_hip_moe_stack_fused(ft_hip_ctx* ctx, void* stream, const float* x_in, float* x_out, int64_t hidden,
                           int64_t inter, int64_t n_experts, int64_t top_k, int64_t n_layers,
                           const void* banks, const float* routers, const float* bias,
                           const float* expert_scale, int32_t* ids, float* wts, void* workspace,
                           size_t workspace_bytes, float* dbg_gu, void* dbg_act, float* dbg_x,
                           uint64_t* dbg_trace);

/* Length of the fused kernel's bounded waits, in polls (default 2^21, about
 * a second): a wait that has not seen its data after this many polls gives up,
 * records the abort in the workspace and every workgroup exits. 0 makes the
 * first incomplete poll give up (tests of the abort path). No counterpart in
 * the reference, whose launch sequence has no cross-workgroup waits. */
int ft_hip_fused_set_spin_limit(ft_hip_ctx* ctx, int polls);

/* Fused kernel, 1 (default): while layer l finishes, every unit group streams
 * the tiles of the expert that early routing (layer l+1's router applied to
 * x_l) predicts, and only mispredicted experts are loaded after the true
 * routing of l+1; 0: each layer loads its routed experts once routed.
 * Results are identical either way. A performance choice with no reference
 * counterpart (the reference's SlotCache, ft-core/src/lib.rs:61-91, keeps
 * recently routed experts in device slots and copies misses over PCIe after
 * routing; it predicts nothing). */
int ft_hip_fused_set_prefetch(ft_hip_ctx* ctx, int on);

/* Refined prediction for the fused kernel's prefetch (no reference
 * counterpart; the reference predicts nothing). Layer l+1's router logits
 * are linear in x_{l+1} = x_l + sum_p w_p D_p a_p, so with the table
 * M_{l,e} = R_{l+1} D_{l,e} (E router rows x inter columns per expert, int8
 * per 32 columns with an f32 scale, [n_layers-1][E] records) the early
 * routing's 16 best experts (R_{l+1} x_l) are re-ranked by
 * R_{l+1} x_l + sum_p w_p M_p a_p as soon as layer l's act blocks are
 * published, and every unit group prefetches that prediction instead of the
 * early routing's. Results are identical with or without it: the prediction
 * only decides which unit group holds which expert.
 * Bytes of the table for these banks (-1 on a bad shape). */
int64_t ft_hip_fused_predictor_bytes(int64_t hidden, int64_t inter, int64_t n_experts, int64_t n_layers);

/* Build the table from fused-layout banks and fused-layout routers (those
 * ft_hip_moe_stack_fused takes), on `stream`. Setup only. */
int ft_hip_fused_build_predictor(ft_hip_ctx* ctx, void* stream, const void* banks, const float* routers,
                                 int64_t hidden, int64_t inter, int64_t n_experts, int64_t n_layers, void* table,
                                 size_t table_bytes);

/* Use `table` (built for n_layers layers of the banks later launches take)
 * in every later ft_hip_moe_stack_fused on this context; it must stay
 * allocated while set. NULL returns to the early routing's prediction (the
 * default). A launch with more layers than the table covers returns
 * FT_HIP_E_SHAPE. */
int ft_hip_fused_set_predictor(ft_hip_ctx* ctx, const void* table, size_t table_bytes, int64_t n_layers);

/* Fused kernel launch mode. 0 (default): a plain launch, whose workgroups
 * (one per CU, fewer than the device's CUs) are all resident only while no
 * kernel of another stream occupies CUs; the fastest mode for a device the
 * decode loop has to itself. 1: a cooperative launch, which the runtime
 * starts only with every workgroup resident, for callers that run other
 * kernels concurrently on other streams (the reference overlaps a copy
 * stream, ft-model/src/lib.rs:1425-1433; copies use DMA engines, not CUs,
 * and need no cooperative launch). ~19 us more per launch measured on
 * MI355X. Results are identical either way. No reference counterpart. */
int ft_hip_fused_set_cooperative(ft_hip_ctx* ctx, int on);

/* Host-synchronous check of a fused workspace after the stream has been
 * synchronised: FT_HIP_E_TIMEOUT (and *aborted = 1) if a launch gave up a
 * bounded wait, or was refused because its tags would have passed 2^32 (the
 * epoch guard above). Such a workspace stays poisoned -- later launches on it
 * do nothing but set x_out to NaN and the routing record to -1/NaN -- until
 * ft_hip_fused_workspace_init. */
int ft_hip_fused_status(ft_hip_ctx* ctx, void* workspace, int* aborted);

/* ---- local GGUF model files (ft-gguf/src/lib.rs:141-206) ----
 * ft_gguf_open maps a GGUF v2/v3 file read-only and parses its header,
 * metadata and tensor table (ft_gguf::Gguf::open): bad magic, other
 * versions, truncation, unknown value types and unsupported ggml tensor
 * types give FT_HIP_E_FORMAT (the reference's bail!s); a missing file
 * FT_HIP_E_IO. The data section starts at the header's end rounded up to
 * general.alignment (default 32). Strings returned point into the handle
 * (not NUL-terminated for values: use the length) and live until
 * ft_gguf_close. Host only; no GPU needed. Metadata value types follow the
 * GGUF spec: 0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32, 7 bool, 8 string,
 * 9 array, 10 u64, 11 i64, 12 f64. */
typedef struct ft_gguf ft_gguf;
int ft_gguf_open(const char* path, ft_gguf** out);
int ft_gguf_close(ft_gguf* g);
uint32_t ft_gguf_version(const ft_gguf* g);
uint64_t ft_gguf_data_start(const ft_gguf* g);
int64_t ft_gguf_n_kv(const ft_gguf* g);
int64_t ft_gguf_n_tensors(const ft_gguf* g);
/* metadata key i (file order) and its value type */
int ft_gguf_kv_key(const ft_gguf* g, int64_t i, const char** key, uint32_t* value_type);
int ft_gguf_meta_type(const ft_gguf* g, const char* key, uint32_t* value_type);
/* Value::as_u64 (ft-gguf/src/lib.rs:29-41): unsigned, or non-negative signed */
int ft_gguf_meta_u64(const ft_gguf* g, const char* key, uint64_t* out);
/* f32 values only (ft-model's mf, ft-model/src/lib.rs:57-62) */
int ft_gguf_meta_f32(const ft_gguf* g, const char* key, float* out);
int ft_gguf_meta_str(const ft_gguf* g, const char* key, const char** s, uint64_t* len);
int ft_gguf_meta_array(const ft_gguf* g, const char* key, uint32_t* elem_type, uint64_t* n);
int ft_gguf_meta_array_u64(const ft_gguf* g, const char* key, uint64_t i, uint64_t* out);
/* 1 for Bool(true), else 0 (ft-model's arr_b, ft-model/src/lib.rs:70-78) */
int ft_gguf_meta_array_bool(const ft_gguf* g, const char* key, uint64_t i, int* out);
int ft_gguf_meta_array_str(const ft_gguf* g, const char* key, uint64_t i, const char** s, uint64_t* len);
/* tensor i (file order); info of a named tensor (Gguf::tensor): dims[8]
 * (ne[0], the contiguous dimension, first; unused dims 1), ggml type, offset
 * in the data section and byte size from the type's block layout */
int ft_gguf_tensor_name(const ft_gguf* g, int64_t i, const char** name);
int ft_gguf_tensor_info(const ft_gguf* g, const char* name, uint32_t* n_dims, uint64_t* dims,
                        uint32_t* ggml_type, uint64_t* offset, uint64_t* nbytes);
/* Gguf::tensor_data: the tensor's bytes in the mapping (bounds-checked) */
int ft_gguf_tensor_data(const ft_gguf* g, const char* name, const void** data, uint64_t* nbytes);
/* ft-model's to_f32 (ft-model/src/lib.rs:128-151): f32, f16 or q4_0 tensor
 * of exactly n elements to f32 */
int ft_gguf_tensor_to_f32(const ft_gguf* g, const char* name, float* out, uint64_t n);
/* The router of `layer` as the expert section takes it: [n_experts][hidden]
 * f32 from blk.<layer>.ffn_gate_inp.weight with blk.<layer>.ffn_gate_inp.scale
 * and hidden^-1/2 folded in per column (ft-model/src/lib.rs:506-514). */
int ft_gguf_router_f32(const ft_gguf* g, int64_t layer, int64_t hidden, int64_t n_experts, float* out);
/* Expert banks of layers [layer0, layer0 + n_layers) from the file's q4_0
 * blk.<l>.ffn_gate_up_exps.weight [hidden, 2*inter, n_experts] and
 * blk.<l>.ffn_down_exps.weight [inter, hidden, n_experts] into device
 * `banks` (ft-model/src/lib.rs:570-609): expert (l, e) at
 * ((l - layer0) * n_experts + e) * expert_bytes, its 2*inter gate|up rows
 * then its hidden down rows, each row in `layout` (the reference repacks to
 * q4r on the host; here each tensor is uploaded once and repacked on the
 * device). Every tensor's type and dims are checked before any copy.
 * Allocates a device staging buffer of n_experts * max(tensor) bytes for the
 * call and synchronises `stream` before returning. */
int ft_hip_load_expert_banks_gguf(ft_hip_ctx* ctx, void* stream, const ft_gguf* g, int64_t layer0,
                                  int64_t n_layers, int64_t hidden, int64_t inter, int64_t n_experts,
                                  void* banks, uint64_t expert_bytes, int layout);

#ifdef __cplusplus
}
#endif

#endif /* FT_HIP_H */
