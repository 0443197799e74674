// ft_runtime.hpp -- host-side context, error reporting and launch checks
// shared by the library's translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <unordered_map>

#include "../../include/ft_hip.h"

// Where ft_hip_set_layer_record sends the launch-by-launch layer path's
// stage records (tests only); on = any of them set.
struct LayerRecord {
    bool on;
    float* x;
    uint8_t* q8x;
    float* gu;
    uint8_t* act;
    int32_t* gu_dots;
    int32_t* dn_dots;
};

struct ft_hip_ctx {
    int device;
    int num_cus;
    int num_xcds;
    int fused_spin_limit;  // polls before a fused-kernel wait gives up
    int fused_prefetch;    // fused kernel: stream predicted experts ahead (1) or not (0)
    int fused_cooperative; // fused kernel: cooperative launch (1) or plain (0)
    const void* fused_pred;      // fused kernel: refined-prediction table (ft_hip_fused_set_predictor), or null
    size_t fused_pred_bytes;     // its size
    int64_t fused_pred_layers;   // the n_layers it was built for
    int input_norm;        // layer entry points run on rmsnorm(x) (1) or x (0)
    int grouped_mfma_min;  // grouped layer: experts with at least this many tokens take the MFMA kernels (0: auto)
    int gemv_lanes;        // q4r GEMV lanes per row (ft_hip_set_gemv_lanes): 0 automatic, 8, 16, 32 or 64
    int32_t* rec_gu;       // test record of gate|up block dots (ft_hip_set_block_dot_record), or null
    int32_t* rec_dn;       // test record of down block dots, or null
    LayerRecord lrec;      // test record of the launch-by-launch layer path (ft_hip_set_layer_record)
    void* noalloc_scratch; // device address of this device's no-alloc scratch array (ft_hip_moe_layer_noalloc)
    // fused workspaces this context initialised -> their epoch after the launches it made (the wrap guard)
    std::unordered_map<const void*, uint64_t> fused_epochs;
    char arch[64];
};

namespace ft {
void clear_error();
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Status of the launch just issued: FT_HIP_OK, or FT_HIP_E_LAUNCH with the
// HIP error text.
int launch_status(const char* what);
// Router logits in the R-order, times in_scale[s] when given, + bias (shapes
// already checked by the caller).
int launch_router_logits(void* stream, const float* w, const float* x, const float* bias, const float* in_scale,
                         float* y, int64_t dim, int64_t n_rows, int64_t n_seqs);
// Router logits (+ the input norm's scale when norm) and q8(x) in one launch;
// needs n_rows * 16 >= dim / 32.
int launch_route_prep(void* stream, const float* w, const float* x, const float* bias, int norm, float* inv,
                      void* q8, float* y, int64_t dim, int64_t n_rows, int64_t n_seqs);
// Resolves the no-alloc scratch array's device address for ctx->device
// (current) into ctx->noalloc_scratch (ft_hip_ops.hip, beside the array).
int scratch_setup(ft_hip_ctx* ctx);
// Input RMS norm scale per seq: inv[s] = 1 / sqrt(R-order(x_s . x_s) / dim + 1e-6).
int launch_rms_inv(void* stream, const float* x, float* inv, int64_t dim, int64_t n_seqs);
}  // namespace ft

using ft::clear_error;
using ft::fail;
using ft::launch_status;
