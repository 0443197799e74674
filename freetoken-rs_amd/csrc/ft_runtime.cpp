// ft_runtime.cpp -- context creation (the counterpart of Q4Gemv::new,
// ft-cuda/src/lib.rs:111-150), thread-local error text, launch checks.
#include "ft_runtime.hpp"

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>

namespace ft {

static thread_local char g_err[512] = "";

void clear_error() { g_err[0] = 0; }

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

int launch_status(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(FT_HIP_E_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
    return FT_HIP_OK;
}

}  // namespace ft

extern "C" int ft_hip_version(void) { return 100; }

extern "C" const char* ft_hip_last_error(void) { return ft::g_err; }

extern "C" int ft_hip_create(int device, ft_hip_ctx** out) {
    clear_error();
    if (!out) return fail(FT_HIP_E_INVALID, "create: null out");
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0)
        return fail(FT_HIP_E_DEVICE, "create: no HIP device (%s)", e != hipSuccess ? hipGetErrorString(e) : "count 0");
    if (device < 0 || device >= n) return fail(FT_HIP_E_DEVICE, "create: device %d out of range [0, %d)", device, n);
    hipDeviceProp_t p;
    if ((e = hipGetDeviceProperties(&p, device)) != hipSuccess)
        return fail(FT_HIP_E_DEVICE, "create: %s", hipGetErrorString(e));
    if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return fail(FT_HIP_E_DEVICE, "create: device %d is %s; this library is built for gfx950 only", device,
                    p.gcnArchName);
    if ((e = hipSetDevice(device)) != hipSuccess) return fail(FT_HIP_E_DEVICE, "create: %s", hipGetErrorString(e));
    ft_hip_ctx* c = new (std::nothrow) ft_hip_ctx{};
    if (!c) return fail(FT_HIP_E_INVALID, "create: out of host memory");
    c->device = device;
    c->num_cus = p.multiProcessorCount;
    c->num_xcds = 8;  // MI355X: 8 XCDs of 32 CUs
    c->fused_spin_limit = 1 << 21;
    c->fused_prefetch = 1;
    c->fused_cooperative = 0;
    c->grouped_mfma_min = 0;  // automatic
    c->gemv_lanes = 0;        // automatic
    std::snprintf(c->arch, sizeof c->arch, "%s", p.gcnArchName);
    if (int rc = ft::scratch_setup(c)) {  // once per context, with its device current
        delete c;
        return rc;
    }
    *out = c;
    return FT_HIP_OK;
}

extern "C" int ft_hip_set_input_norm(ft_hip_ctx* ctx, int on) {
    clear_error();
    if (!ctx) return fail(FT_HIP_E_INVALID, "set_input_norm: null ctx");
    if (on != 0 && on != 1) return fail(FT_HIP_E_SHAPE, "set_input_norm: on=%d is not 0 or 1", on);
    ctx->input_norm = on;
    return FT_HIP_OK;
}

extern "C" int ft_hip_set_grouped_mfma_min(ft_hip_ctx* ctx, int n_tokens) {
    clear_error();
    if (!ctx) return fail(FT_HIP_E_INVALID, "set_grouped_mfma_min: null ctx");
    if (n_tokens < 0) return fail(FT_HIP_E_SHAPE, "set_grouped_mfma_min: n_tokens=%d < 0", n_tokens);
    ctx->grouped_mfma_min = n_tokens;
    return FT_HIP_OK;
}

extern "C" int ft_hip_set_gemv_lanes(ft_hip_ctx* ctx, int lanes_per_row) {
    clear_error();
    if (!ctx) return fail(FT_HIP_E_INVALID, "set_gemv_lanes: null ctx");
    if (lanes_per_row != 0 && lanes_per_row != 8 && lanes_per_row != 16 && lanes_per_row != 32 && lanes_per_row != 64)
        return fail(FT_HIP_E_SHAPE, "set_gemv_lanes: lanes_per_row=%d is not 0, 8, 16, 32 or 64", lanes_per_row);
    ctx->gemv_lanes = lanes_per_row;
    return FT_HIP_OK;
}

extern "C" int ft_hip_set_block_dot_record(ft_hip_ctx* ctx, int32_t* gu_dots, int32_t* dn_dots) {
    clear_error();
    if (!ctx) return fail(FT_HIP_E_INVALID, "set_block_dot_record: null ctx");
    if ((gu_dots == nullptr) != (dn_dots == nullptr))
        return fail(FT_HIP_E_INVALID, "set_block_dot_record: give both records or neither");
    ctx->rec_gu = gu_dots;
    ctx->rec_dn = dn_dots;
    return FT_HIP_OK;
}

extern "C" int ft_hip_set_layer_record(ft_hip_ctx* ctx, float* x, void* q8x, float* gu, void* act, int32_t* gu_dots,
                                       int32_t* dn_dots) {
    clear_error();
    if (!ctx) return fail(FT_HIP_E_INVALID, "set_layer_record: null ctx");
    LayerRecord& r = ctx->lrec;
    r.x = x;
    r.q8x = (uint8_t*)q8x;
    r.gu = gu;
    r.act = (uint8_t*)act;
    r.gu_dots = gu_dots;
    r.dn_dots = dn_dots;
    r.on = x || q8x || gu || act || gu_dots || dn_dots;
    return FT_HIP_OK;
}

extern "C" int ft_hip_destroy(ft_hip_ctx* ctx) {
    clear_error();
    delete ctx;
    return FT_HIP_OK;
}
