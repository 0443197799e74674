// ft_runtime.hpp -- host-side context, error reporting and launch checks
// shared by the library's translation units.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/ft_hip.h"

struct ft_hip_ctx {
    int device;
    int num_cus;
    int num_xcds;
    int fused_spin_limit;  // polls before a fused-kernel wait gives up
    int fused_prefetch;    // fused kernel: stream predicted experts ahead (1) or not (0)
    char arch[64];
};

namespace ft {
void clear_error();
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Status of the launch just issued: FT_HIP_OK, or FT_HIP_E_LAUNCH with the
// HIP error text.
int launch_status(const char* what);
}  // namespace ft

using ft::clear_error;
using ft::fail;
using ft::launch_status;
