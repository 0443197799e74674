// ft_device.hpp -- device-side building blocks shared by every kernel of the
// library: the q8 block format, the per-block integer dot, q8 quantisation,
// the q4_0 block quantiser, GELU and exp (libm-exact), and the seeded generator.
//
// The translation units that include this file are compiled with
// -ffp-contract=off, so a*b+c stays two roundings unless fmaf()/fma() is
// written out. That keeps every f32 expression the same as the Rust source it
// restates (Rust never contracts).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ft_libm.hpp"

namespace ft {

constexpr int QK = 32;
constexpr int Q8_BLK = 40;  // {f32 d; i32 qsum; i8 qs[32]}

__device__ __forceinline__ float h2f(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return (float)v;
}

__device__ __forceinline__ uint16_t f2h(float f) {
    _Float16 v = (_Float16)f;  // v_cvt_f16_f32: round to nearest even
    uint16_t h;
    __builtin_memcpy(&h, &v, 2);
    return h;
}

// sum_i q4u_i * q8_i over one 32-weight block. w holds the 16 packed bytes
// (byte i = q_i | q_{i+16} << 4, ft-core/src/q4_0.rs:2-3); a points at the 8
// dwords of the block's q8 values. v_dot4_i32_i8 treats both operands as
// signed bytes; nibbles 0..15 are non-negative, so the products are exact.
__device__ __forceinline__ int dot_q4u_q8(const uint4 w, const int* a) {
    int s = 0;
    s = __builtin_amdgcn_sdot4((int)(w.x & 0x0F0F0F0Fu), a[0], s, false);
    s = __builtin_amdgcn_sdot4((int)(w.y & 0x0F0F0F0Fu), a[1], s, false);
    s = __builtin_amdgcn_sdot4((int)(w.z & 0x0F0F0F0Fu), a[2], s, false);
    s = __builtin_amdgcn_sdot4((int)(w.w & 0x0F0F0F0Fu), a[3], s, false);
    s = __builtin_amdgcn_sdot4((int)((w.x >> 4) & 0x0F0F0F0Fu), a[4], s, false);
    s = __builtin_amdgcn_sdot4((int)((w.y >> 4) & 0x0F0F0F0Fu), a[5], s, false);
    s = __builtin_amdgcn_sdot4((int)((w.z >> 4) & 0x0F0F0F0Fu), a[6], s, false);
    s = __builtin_amdgcn_sdot4((int)((w.w >> 4) & 0x0F0F0F0Fu), a[7], s, false);
    return s;
}

// The exact per-block dot sum_i (q4_i - 8) * q8_i, with the -8 offset folded
// out through the block's integer q8 sum (|result| <= 32*15*127, exact).
__device__ __forceinline__ int block_dot(const uint4 w, const int* a, int qsum) {
    return dot_q4u_q8(w, a) - 8 * qsum;
}

// The same from two 16-byte halves of the q8 values (low: values 0..15,
// high: 16..31), for operands read from LDS as 16-byte vectors.
__device__ __forceinline__ int block_dot_v(const uint4 w, const uint4 lo, const uint4 hi, int qsum) {
    int s = 0;
    s = __builtin_amdgcn_sdot4((int)(w.x & 0x0F0F0F0Fu), (int)lo.x, s, false);
    s = __builtin_amdgcn_sdot4((int)(w.y & 0x0F0F0F0Fu), (int)lo.y, s, false);
    s = __builtin_amdgcn_sdot4((int)(w.z & 0x0F0F0F0Fu), (int)lo.z, s, false);
    s = __builtin_amdgcn_sdot4((int)(w.w & 0x0F0F0F0Fu), (int)lo.w, s, false);
    s = __builtin_amdgcn_sdot4((int)((w.x >> 4) & 0x0F0F0F0Fu), (int)hi.x, s, false);
    s = __builtin_amdgcn_sdot4((int)((w.y >> 4) & 0x0F0F0F0Fu), (int)hi.y, s, false);
    s = __builtin_amdgcn_sdot4((int)((w.z >> 4) & 0x0F0F0F0Fu), (int)hi.z, s, false);
    s = __builtin_amdgcn_sdot4((int)((w.w >> 4) & 0x0F0F0F0Fu), (int)hi.w, s, false);
    return s - 8 * qsum;
}

// ---------------------------------------------------------------------------
// q8 quantisation of one 32-value block held one value per lane in a 32-lane
// half of a wavefront (ft-core/src/q4_0.rs:62-78): d = amax/127 (IEEE
// division), inv = 1/d, q = clamp(round_half_away(v*inv), -127, 127).
// ---------------------------------------------------------------------------
// clamp(r, -127, 127) as i8 in Rust: a NaN product (inf*0 in a block that
// holds inf, 0*inf when amax/127 is subnormal, a NaN input) becomes 0, where
// fminf/fmaxf alone would return -127.
__device__ __forceinline__ float q8_clamp(float r) {
    return r == r ? fminf(127.0f, fmaxf(-127.0f, r)) : 0.0f;
}

struct Q8Lane {
    float d;
    int q;
    int qsum;
};

__device__ __forceinline__ Q8Lane q8_quantize_half(float v) {
    float a = fabsf(v);
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) a = fmaxf(a, __shfl_xor(a, off, 32));
    float d = a > 0.0f ? a / 127.0f : 0.0f;
    float inv = d > 0.0f ? 1.0f / d : 0.0f;
    float r = roundf(v * inv);
    r = q8_clamp(r);
    int q = (int)r;
    int s = q;
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) s += __shfl_xor(s, off, 32);
    return Q8Lane{d, q, s};
}

// Store a half-wave's block: lane 0 writes the header, every lane its byte.
__device__ __forceinline__ void q8_store_half(uint8_t* blk, int l, const Q8Lane& r) {
    if (l == 0) {
        reinterpret_cast<float*>(blk)[0] = r.d;
        reinterpret_cast<int*>(blk)[1] = r.qsum;
    }
    blk[8 + l] = (uint8_t)(int8_t)r.q;
}

// Lane-quad exchanges by DPP (quad_perm): a few cycles, unlike ds_bpermute.
__device__ __forceinline__ float quad_xor1(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));  // [1,0,3,2]
}
__device__ __forceinline__ float quad_xor2(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));  // [2,3,0,1]
}
__device__ __forceinline__ int quad_xor1i(int v) { return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false); }
__device__ __forceinline__ int quad_xor2i(int v) { return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false); }

// DPP moves by a fixed control: quad_perm broadcasts 0x00/0x55/0xAA/0xFF,
// 0x140 row_mirror, 0x141 row_half_mirror; every lane of the row must be
// active.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false);
}
// Lane l <-> lane l ^ 16 within each 32-lane half (ds_swizzle, bit mode:
// and 0x1F, or 0, xor 0x10).
__device__ __forceinline__ float swz_xor16_f(float v) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
}
__device__ __forceinline__ int swz_xor16_i(int v) { return __builtin_amdgcn_ds_swizzle(v, 0x401F); }
// lane ^ 4 (bit-mask mode: xor 4, and 0x1F)
__device__ __forceinline__ int swz_xor4_i(int v) { return __builtin_amdgcn_ds_swizzle(v, 0x101F); }

// All-lane max / sum over the 32 lanes of a half-wave (every one active):
// DPP within rows of 16 (quad xor 1, quad xor 2, half-row mirror, row
// mirror), then one swizzle across the two rows. Max is exact in any order;
// the sum is of integers.
__device__ __forceinline__ float half_max32(float a) {
    a = fmaxf(a, quad_xor1(a));
    a = fmaxf(a, quad_xor2(a));
    a = fmaxf(a, dpp_f<0x141>(a));
    a = fmaxf(a, dpp_f<0x140>(a));
    return fmaxf(a, swz_xor16_f(a));
}
__device__ __forceinline__ int half_sum32(int s) {
    s += quad_xor1i(s);
    s += quad_xor2i(s);
    s += dpp_i<0x141>(s);
    s += dpp_i<0x140>(s);
    return s + swz_xor16_i(s);
}

// q8 block of 32 values held one per lane by lanes 0..31 (all active), the
// arithmetic of q8_quantize_half (ft-core/src/q4_0.rs:62-78). Returns, in
// lane 4k, output word 2+k (the packed bytes of lanes 4k..4k+3); *d and
// *qsum are the same in every lane.
__device__ __forceinline__ uint32_t q8_quantize_lanes32(float v, float* d_out, int* qsum_out) {
    const float amax = half_max32(fabsf(v));
    const float d = amax > 0.0f ? amax / 127.0f : 0.0f;
    const float inv = d > 0.0f ? 1.0f / d : 0.0f;
    float r = roundf(v * inv);
    r = q8_clamp(r);
    const int q = (int)r;
    *d_out = d;
    *qsum_out = half_sum32(q);
    const int b = q & 0xFF;
    return (uint32_t)dpp_i<0x00>(b) | ((uint32_t)dpp_i<0x55>(b) << 8) | ((uint32_t)dpp_i<0xAA>(b) << 16) |
           ((uint32_t)dpp_i<0xFF>(b) << 24);
}

// A lane quad quantizes one 32-value block to q8 {d, qsum, qs[32]}
// (ft-core/src/q4_0.rs:62-78; the same arithmetic as q8_quantize_half): lane
// part (0..3) owns values 8*part..8*part+7 (a, b) and writes output words
// 2+2*part and 3+2*part; part 0 also writes d and qsum. All four lanes must be
// active.
__device__ __forceinline__ void quantize_block_quad_v(const float4 a, const float4 b, int part, uint32_t* out) {
    const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(x[i]));
    amax = fmaxf(amax, quad_xor1(amax));
    amax = fmaxf(amax, quad_xor2(amax));
    const float d = amax > 0.0f ? amax / 127.0f : 0.0f;
    const float inv = d > 0.0f ? 1.0f / d : 0.0f;
    int qsum = 0;
    uint32_t w0 = 0, w1 = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float r = roundf(x[i] * inv);
        r = q8_clamp(r);
        const int q = (int)r;
        qsum += q;
        const uint32_t byte = (uint32_t)(uint8_t)(int8_t)q << (8 * (i & 3));
        if (i < 4) w0 |= byte; else w1 |= byte;
    }
    qsum += quad_xor1i(qsum);
    qsum += quad_xor2i(qsum);
    out[2 + 2 * part] = w0;
    out[3 + 2 * part] = w1;
    if (part == 0) {
        out[0] = __float_as_uint(d);
        out[1] = (uint32_t)qsum;
    }
}

// The same, with the lane's 8 values read from the block at v.
__device__ __forceinline__ void quantize_block_quad(const float* v, int part, uint32_t* out) {
    const float4* v4 = reinterpret_cast<const float4*>(v);
    quantize_block_quad_v(v4[2 * part], v4[2 * part + 1], part, out);
}

// Router order as one unsigned compare: a larger key sorts first. Monotone
// float bits (larger logit first), then the complemented index (lower index
// first on equal values; -0 and +0 are equal); NaN below every number.
__device__ __forceinline__ uint64_t rank_key(float v, int i) {
    v = v + 0.0f;  // -0 -> +0: equal values tie on the index
    const uint32_t b = __float_as_uint(v);
    uint32_t mo = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    mo = v == v ? mo : 0u;  // NaN below -inf
    return ((uint64_t)mo << 32) | (0xFFFFFFFFu - (uint32_t)i);
}

// ---------------------------------------------------------------------------
// GELU and the softmax exp with the bits of the libm calls ft-core makes
// (f32::tanh, ft-model/src/lib.rs:436; f32::exp, :1495): restatements of
// glibc's tanhf / expf, swept against the host libm over every f32 input.
// ---------------------------------------------------------------------------
// expf for the routing weights. T: anything indexable by 0..31 holding
// libm::exp2_table() (libm::Exp2TableRef reads the constant table; a
// persistent kernel passes a copy in LDS so the lookup does not wait behind
// its own weight loads).
template <typename T>
__device__ __forceinline__ float expf_libm_t(float x, const T& tab) { return libm::expf_glibc_t(x, tab); }

__device__ __forceinline__ float expf_libm(float x) { return libm::expf_glibc(x); }

// gelu_tanh (ft-model/src/lib.rs:435-437), left to right, no contraction:
// 0.5*g*(1 + tanh(0.7978845608*(g + 0.044715*g*g*g))).
__device__ __forceinline__ float gelu_tanh(float g) {
    float c = 0.044715f * g;
    c = c * g;
    c = c * g;
    const float inner = g + c;
    const float t = libm::tanhf_glibc(0.7978845608f * inner);
    const float h = 0.5f * g;
    return h * (1.0f + t);
}

// ---------------------------------------------------------------------------
// Seeded generator (same definition as the host oracle): value i of a tensor
// is the centred sum of the four 16-bit fields of splitmix64's output, times
// `scale`.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

__device__ __forceinline__ float gen_value(uint64_t key, uint64_t i, float scale) {
    uint64_t h = mix64(key + (i + 1) * 0x9E3779B97F4A7C15ULL);
    int s = (int)(h & 0xFFFF) + (int)((h >> 16) & 0xFFFF) + (int)((h >> 32) & 0xFFFF) + (int)(h >> 48);
    return (float)(s - 131070) * scale;
}

// ggml q4_0 block quantiser (ft-core/src/q4_0.rs:20-40) of 32 values:
// writes the f16 scale bits and the 16 packed bytes (as 4 dwords).
__device__ __forceinline__ void quantize_block_q4_0(const float* xb, uint16_t& dh, uint4& qs) {
    float amax = 0.0f, maxv = 0.0f;
    for (int i = 0; i < QK; ++i) {
        float a = fabsf(xb[i]);
        if (a > amax) {
            amax = a;
            maxv = xb[i];
        }
    }
    float d = maxv / -8.0f;
    float id = (d != 0.0f) ? 1.0f / d : 0.0f;
    dh = f2h(d);
    uint32_t w[4] = {0, 0, 0, 0};
    for (int i = 0; i < QK / 2; ++i) {
        float t0 = xb[i] * id;
        float t1 = xb[i + QK / 2] * id;
        int q0 = (int)(t0 + 8.5f);
        int q1 = (int)(t1 + 8.5f);
        q0 = min(15, max(0, q0));
        q1 = min(15, max(0, q1));
        w[i >> 2] |= (uint32_t)(q0 | (q1 << 4)) << (8 * (i & 3));
    }
    qs = make_uint4(w[0], w[1], w[2], w[3]);
}

}  // namespace ft
