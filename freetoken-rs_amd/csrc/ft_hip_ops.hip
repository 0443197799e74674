// ft_hip_ops.hip -- the launch-by-launch kernels of the MoE expert-FFN decode
// section and their C ABI (include/ft_hip.h). Each kernel replaces one
// kernel of ft-cuda/src/q4.cu; the fused whole-stack path lives in
// ft_hip_fused.hip and reuses the device routines of ft_device.hpp.

#include "ft_device.hpp"
#include "ft_runtime.hpp"

#include <algorithm>

using namespace ft;

// lanes per row of the gate|up launch with the activation (k_gemv_gu_act):
// 4 lanes take 256-thread workgroups, so that a long layer's block-pairs
// (I/32 per pair) all run at once; measured faster than 8 on the
// large-expert shape
constexpr int GU_LANES = 4;

// ---------------------------------------------------------------------------
// Weight addressing shared by the grouped GEMV and the block-dot dump.
// ---------------------------------------------------------------------------
struct GemvArgs {
    const uint64_t* bases;     // per-entry base pointers, or NULL
    const uint8_t* base;       // slot form: base + slots[e] * expert_bytes
    uint64_t expert_bytes;
    const int32_t* slots;
    uint64_t bank_off;
    const int32_t* x_idx;      // per-entry q8 row, or NULL (row = e / x_div)
    int x_div;
    const uint8_t* q8;
    int64_t q8_stride_blocks;
    float* y;                  // GEMV output
    int32_t* dots;             // block-dot dump output (layer kernels: the REC record, or null)
    float* sums;               // layer record (REC): gate|up sums as GELU takes them, [pair][2*inter], or null
    uint8_t* x8rec;            // layer record (REC, head in the launch): q8 of x per seq, [seq][k/32][40], or null
    int64_t y_stride;
    int n_rows;
    int k;
    const float* xf;           // f32 input row of the short GEMV's XIN mode (k floats), quantized in the launch
    float* act;                // gate|up launch of the short GEMV (ACT): gelu_tanh(gate) * up per column
};

__device__ __forceinline__ const uint8_t* entry_base(const GemvArgs& a, int e) {
    // no slots: one dense matrix at base
    const uint8_t* p = a.bases ? reinterpret_cast<const uint8_t*>(a.bases[e])
                               : a.base + (a.slots ? (uint64_t)a.slots[e] * a.expert_bytes : 0);
    return p + a.bank_off;
}

__device__ __forceinline__ int entry_xrow(const GemvArgs& a, int e) {
    return a.x_idx ? a.x_idx[e] : e / a.x_div;
}

// Fetch block b of a row: its f32 scale and its 16 packed bytes.
template <int LAYOUT>
__device__ __forceinline__ void load_block(const uint8_t* wr, int b, int qs_off, float& d4, uint4& q) {
    if constexpr (LAYOUT == FT_LAYOUT_Q4R) {
        d4 = h2f(reinterpret_cast<const uint16_t*>(wr)[b]);
        q = *reinterpret_cast<const uint4*>(wr + qs_off + 16 * b);
    } else {
        // 18-byte blocks are only 2-byte aligned: nine u16 loads.
        const uint16_t* p = reinterpret_cast<const uint16_t*>(wr + 18 * b);
        d4 = h2f(p[0]);
        q.x = (uint32_t)p[1] | ((uint32_t)p[2] << 16);
        q.y = (uint32_t)p[3] | ((uint32_t)p[4] << 16);
        q.z = (uint32_t)p[5] | ((uint32_t)p[6] << 16);
        q.w = (uint32_t)p[7] | ((uint32_t)p[8] << 16);
    }
}

__host__ __device__ __forceinline__ int64_t row_bytes_of(int layout, int k) {
    int nb = k / 32;
    if (layout == FT_LAYOUT_Q4R) return (int64_t)((nb * 2 + 15) / 16 * 16) + (int64_t)nb * 16;
    return (int64_t)nb * 18;
}

// n words from src into LDS; a thread issues up to R loads before its first
// store, so a long row costs a few load latencies, not one per word.
template <int R = 16>
__device__ __forceinline__ void stage_words(const int* src, int n, int* lds) {
    const int t = threadIdx.x, nt = blockDim.x;
    for (int base = 0; base < n; base += R * nt) {
        int v[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int i = base + r * nt + t;
            v[r] = i < n ? src[i] : 0;
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int i = base + r * nt + t;
            if (i < n) lds[i] = v[r];
        }
    }
    __syncthreads();
}

// An entry's q8 activation row (nb blocks of 40 B) into LDS.
__device__ __forceinline__ void stage_q8(const GemvArgs& a, int e, int* lds) {
    stage_words(reinterpret_cast<const int*>(a.q8 + (int64_t)entry_xrow(a, e) * a.q8_stride_blocks * Q8_BLK),
                (a.k >> 5) * 10, lds);
}

// The q8 row of the f32 row x computed into LDS (nb blocks of 40 B, 4 lanes
// per block, 8 values each; the loads of two rounds issued before their
// arithmetic), with k_quantize_q8's arithmetic.
__device__ __forceinline__ void stage_f32_q8(const float* x, int nb, int* lds) {
    const float4* x4 = reinterpret_cast<const float4*>(x);
    for (int base = 0; base < nb * 4; base += 2 * 256) {
        float4 va[2], vb[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int i = base + h * 256 + (int)threadIdx.x, f = i < nb * 4 ? 2 * i : 0;
            va[h] = x4[f];
            vb[h] = x4[f + 1];
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int i = base + h * 256 + (int)threadIdx.x;
            if (i < nb * 4)  // whole quads: nb * 4 and the strides are multiples of 4
                quantize_block_quad_v(va[h], vb[h], i & 3, reinterpret_cast<uint32_t*>(lds + (i >> 2) * 10));
        }
    }
    __syncthreads();
}

// Top-k of E <= 256 logits sv (LDS) in the router's order (larger first,
// then lower index, NaN last), by a workgroup of at least E threads: one
// thread per logit, its rank the number of logits ahead of it, counted with
// the branch-free keys of rank_key (a total order: ranks are distinct); ranks
// < k go to selv/seli in rank order.
// Barriers inside; the caller reads selv/seli after it returns.
__device__ __forceinline__ void topk_rank_select(const float* sv, int E, int k, uint64_t* key, float* selv,
                                                 int* seli) {
    const int t = threadIdx.x;
    if (t < E) key[t] = rank_key(sv[t], t);
    __syncthreads();
    if (t < E) {
        const float v = sv[t];
        const uint64_t kt = key[t];
        int rank = 0;
        for (int i0 = 0; i0 < E; i0 += 16) {  // 16 keys per step, their LDS reads issued together
            uint64_t c[16];
#pragma unroll
            for (int q = 0; q < 16; ++q) c[q] = key[min(i0 + q, E - 1)];
#pragma unroll
            for (int q = 0; q < 16; ++q) rank += (i0 + q < E && c[q] > kt) ? 1 : 0;
        }
        if (rank < k) {
            selv[rank] = v;
            seli[rank] = t;
        }
    }
    __syncthreads();
}

// Softmax over the chosen (rank order): thread j < k computes
// exp(l_j - l_max); the sum runs in rank order from 0.0f (the same bits as
// one thread doing all); returns thread j's weight (times escale of its
// expert when given). One barrier inside.
__device__ __forceinline__ float topk_softmax(const float* selv, const int* seli, int k, const float* escale,
                                              float* exv) {
    const int t = threadIdx.x;
    if (t < k) exv[t] = expf_libm(selv[t] - selv[0]);
    __syncthreads();
    float w = 0.0f;
    if (t < k) {
        float denom = 0.0f;
        for (int j = 0; j < k; ++j) denom = denom + exv[j];
        w = exv[t] / denom;
        if (escale) w = w * escale[seli[t]];
    }
    return w;
}

// One row's share of a lane: lane `sub` of the row's LPR takes blocks sub,
// sub+LPR, ..., an fma chain in block order (four blocks' loads issued
// together: long rows are otherwise one load latency per block). The caller
// sums the LPR lanes by xor 1, 2, 4 (, 8).
template <int LAYOUT, int LPR = 8, bool REC = false>
__device__ __forceinline__ float gemv_row_part(const uint8_t* wr, int sub, int nb, const int* lds,
                                               int32_t* rec = nullptr) {
    const int qs_off = (nb * 2 + 15) / 16 * 16;
    float acc = 0.0f;
    int b = sub;
    for (; b + 3 * LPR < nb; b += 4 * LPR) {
        float d4[4];
        uint4 q[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) load_block<LAYOUT>(wr, b + LPR * u, qs_off, d4[u], q[u]);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int* xb = lds + (b + LPR * u) * 10;
            const float d8 = __int_as_float(xb[0]);
            const int diff = block_dot(q[u], xb + 2, xb[1]);
            if constexpr (REC) if (rec) rec[b + LPR * u] = diff;
            acc = fmaf((float)diff, d4[u] * d8, acc);
        }
    }
    for (; b < nb; b += LPR) {
        float d4;
        uint4 q;
        load_block<LAYOUT>(wr, b, qs_off, d4, q);
        const int* xb = lds + b * 10;
        const float d8 = __int_as_float(xb[0]);
        const int diff = block_dot(q, xb + 2, xb[1]);
        if constexpr (REC) if (rec) rec[b] = diff;
        acc = fmaf((float)diff, d4 * d8, acc);
    }
    return acc;
}

template <int LPR = 8>
__device__ __forceinline__ float sum_row_lanes(float acc) {
    acc += __shfl_xor(acc, 1);
    acc += __shfl_xor(acc, 2);
    if (LPR >= 8) acc += __shfl_xor(acc, 4);
    if (LPR >= 16) acc += __shfl_xor(acc, 8);
    return acc;
}

// Grouped GEMV (replaces gemv_q4r_grouped_ptr/_idx, q4.cu:1497-1567, and the
// v3 q4_0 variants, q4.cu:360-491, :1189-1241). A 256-thread workgroup owns 32
// rows of one entry: 8 lanes per row, lane s takes blocks s, s+8, ...; the
// activation sits in LDS. REC: every block's int32 dot is also stored to
// a.dots[e][row][block] (test record). Grid: (ceil(n_rows/32), n_entries).
template <int LAYOUT, bool REC>
__global__ __launch_bounds__(256) void k_gemv_q4_grouped(GemvArgs a) {
    extern __shared__ int lds[];
    const int e = blockIdx.y;
    stage_q8(a, e, lds);
    const int nb = a.k >> 5;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row = (blockIdx.x * 4 + wave) * 8 + (lane >> 3);
    const int sub = lane & 7;
    float acc = 0.0f;
    if (row < a.n_rows)
        acc = gemv_row_part<LAYOUT, 8, REC>(entry_base(a, e) + (int64_t)row * row_bytes_of(LAYOUT, a.k), sub, nb,
                                            lds, REC ? a.dots + ((int64_t)e * a.n_rows + row) * nb : nullptr);
    acc = sum_row_lanes(acc);
    if (row < a.n_rows && sub == 0) a.y[(int64_t)e * a.y_stride + row] = acc;
}

// Short-launch GEMV for q4r matrices whose k_gemv_q4_grouped grid would
// leave most CUs with one workgroup or none (the dense projections of a
// decode step: a few MB each, so the launch is one HBM latency long, not a
// bandwidth-long stream). LPR lanes per row (16, 32 or 64) and 256/LPR rows
// per workgroup multiply the workgroups; a lane's NBL blocks (sub, sub+LPR,
// ..., nb <= LPR*NBL) are all loaded before the activation row is staged, so
// the weight loads and the q8 staging share one latency. The lane's fma chain
// runs in block order and the LPR lanes are summed by xor 1, 2, ..., LPR/2.
// REC: every block's int32 dot is also stored to a.dots[e][row][block] (test
// record). XIN: the q8 activation from the q8 row a.q8 (0, the reference's
// gemv_q4r) or computed in the launch from the f32 row a.xf (1, its
// quantize_q8 then gemv_q4r). ACT (a gate|up matrix, n_rows = 2I): a
// workgroup takes RPW/2 gate rows c.. and the up rows I+c.. of the same
// columns, and also stores a.act[c] = gelu_tanh(gate) * up (the f32 of its
// gelu_mul_q8). Grid (ceil(n_rows / (256/LPR)), n_entries).
template <int LPR, int NBL, bool REC, int XIN = 0, bool ACT = false>
__global__ __launch_bounds__(256) void k_gemv_q4r_short(GemvArgs a) {
    extern __shared__ int lds[];
    constexpr int RPW = 256 / LPR;
    const int e = blockIdx.y;
    const int nb = a.k >> 5;
    const int qs_off = (nb * 2 + 15) / 16 * 16;
    const int lr = (int)threadIdx.x / LPR, half = a.n_rows >> 1;
    const int col = blockIdx.x * (RPW / 2) + lr % (RPW / 2);  // ACT: the row's column
    const int row = ACT ? (col < half ? (lr < RPW / 2 ? col : half + col) : a.n_rows) : blockIdx.x * RPW + lr;
    const int sub = (int)threadIdx.x % LPR;
    const bool live = row < a.n_rows;
    const uint8_t* wr = entry_base(a, e) + (int64_t)(live ? row : 0) * row_bytes_of(FT_LAYOUT_Q4R, a.k);
    float d4[NBL];
    uint4 q[NBL];
#pragma unroll
    for (int u = 0; u < NBL; ++u) {
        const int b = sub + LPR * u;
        if (live && b < nb) {
            load_block<FT_LAYOUT_Q4R>(wr, b, qs_off, d4[u], q[u]);
        } else {
            d4[u] = 0.0f;
            q[u] = make_uint4(0u, 0u, 0u, 0u);
        }
    }
    if constexpr (XIN == 0) stage_q8(a, e, lds);
    else stage_f32_q8(a.xf + (int64_t)entry_xrow(a, e) * a.k, nb, lds);
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < NBL; ++u) {
        const int b = sub + LPR * u;
        if (b < nb) {
            const int* xb = lds + b * 10;
            const float d8 = __int_as_float(xb[0]);
            const int diff = block_dot(q[u], xb + 2, xb[1]);
            if constexpr (REC) {
                if (live) a.dots[((int64_t)e * a.n_rows + row) * nb + b] = diff;
            }
            acc = fmaf((float)diff, d4[u] * d8, acc);
        }
    }
#pragma unroll
    for (int m = 1; m < LPR; m <<= 1) acc += __shfl_xor(acc, m);
    if (live && sub == 0) a.y[(int64_t)e * a.y_stride + row] = acc;
    if constexpr (ACT) {  // the rows' sums to the lanes of their columns
        __shared__ float rs[RPW];
        if (sub == 0) rs[lr] = acc;
        __syncthreads();
        const int c = blockIdx.x * (RPW / 2) + (int)threadIdx.x;
        if ((int)threadIdx.x < RPW / 2 && c < half)
            a.act[(int64_t)e * half + c] = gelu_tanh(rs[threadIdx.x]) * rs[RPW / 2 + threadIdx.x];
    }
}

// The head of a layer taken from the previous layer's down launch
// (k_gemv_down_head) instead of a launch of its own: the states x the layer
// runs on, and the R-order chunk partials part[s][c][e] of its router rows e
// < E and, at e = E, of x.x (16-element fma chains over chunk c of x_s).
struct HeadArgs {
    const float* x;     // [n_seqs][H]
    const float* part;  // [n_seqs][H/16][E+1]
    const float* bias;  // [E] or null
    int norm;           // input RMS norm on
};

// Prologue of a gate|up launch that computes its layer's head (HeadArgs):
// the group sums G[e][g] (the C = H/128 chunk partials of group g in order
// from 0.0f), each logit (groups in order from 0.0f, times the input norm's
// scale when on, then + bias) into sv, the norm's scale into *irs, and the
// q8 row of x_s into lds (4 lanes per block): k_route_prep's arithmetic, so
// its bits. The seq's partials are copied to hp (LDS, H/16 * (E+1) floats)
// with the thread's first q8 quad of x loaded alongside, so the prologue costs
// one load latency. Barriers inside; sv, lds and *irs are read after it
// returns.
__device__ __forceinline__ void head_prologue(const HeadArgs& h, int s, int H, int E, float* sv, int* lds, float* hp,
                                              float* hg, float* irs) {
    const int t = threadIdx.x, nt = blockDim.x;
    const int nch = H >> 4, C = H >> 7, EP = E + 1, nb = H >> 5;
    const float* xs = h.x + (int64_t)s * H;
    float4 xa = make_float4(0.f, 0.f, 0.f, 0.f), xb = xa;
    if (t < 4 * nb) {
        const float4* v = reinterpret_cast<const float4*>(xs + 32 * (t >> 2));
        xa = v[2 * (t & 3)];
        xb = v[2 * (t & 3) + 1];
    }
    stage_words(reinterpret_cast<const int*>(h.part + (int64_t)s * nch * EP), nch * EP,
                reinterpret_cast<int*>(hp));
    for (int q = t; q < 4 * nb; q += nt) {  // whole quads: nt and 4*nb are multiples of 4
        if (q != t) {
            const float4* v = reinterpret_cast<const float4*>(xs + 32 * (q >> 2));
            xa = v[2 * (q & 3)];
            xb = v[2 * (q & 3) + 1];
        }
        quantize_block_quad_v(xa, xb, q & 3, reinterpret_cast<uint32_t*>(lds + (q >> 2) * 10));
    }
    for (int q = t; q < 8 * EP; q += nt) {
        const int e = q >> 3, g = q & 7;
        const float* p = hp + g * C * EP + e;
        float acc = 0.0f;
        for (int c = 0; c < C; ++c) acc = acc + p[c * EP];
        hg[q] = acc;
    }
    __syncthreads();
    float ir = 1.0f;
    if (h.norm) {
        float ss = 0.0f;
        for (int g = 0; g < 8; ++g) ss = ss + hg[E * 8 + g];
        ir = 1.0f / sqrtf(ss / (float)H + 1e-6f);  // correctly rounded (HIP default)
    }
    for (int e = t; e < E; e += nt) {
        float tot = 0.0f;
        for (int g = 0; g < 8; ++g) tot = tot + hg[e * 8 + g];
        if (h.norm) tot = tot * ir;
        if (h.bias) tot = tot + h.bias[e];
        sv[e] = tot;
    }
    if (t == 0) *irs = ir;
    __syncthreads();
}

// Layer-record helpers of the REC instantiations (tests only).
// The q8 row of x_s that a head prologue left in LDS, stored by the seq's
// first workgroup (blockIdx.x 0 of pair s*div).
__device__ __forceinline__ void record_x8(const GemvArgs& a, int e, int s, int div, const int* lds,
                                          int jb = -1) {
    if (!a.x8rec || (jb < 0 ? (int)blockIdx.x : jb) != 0 || e != s * div) return;
    const int nw = (a.k >> 5) * 10;
    int* dst = reinterpret_cast<int*>(a.x8rec + (int64_t)s * (a.k >> 5) * Q8_BLK);
    for (int i = threadIdx.x; i < nw; i += blockDim.x) dst[i] = lds[i];
}
// Lane l < 32 of the tail: the scaled gate and up sums of act block blockIdx.x.
__device__ __forceinline__ void record_sums(const GemvArgs& a, int e, int inter, float gate, float up, int jb = -1,
                                            int tl = -1) {
    const int t = tl < 0 ? (int)threadIdx.x : tl;
    if (!a.sums || t >= 32) return;
    float* dst = a.sums + (int64_t)e * 2 * inter + (jb < 0 ? (int)blockIdx.x : jb) * 32 + t;
    dst[0] = gate;
    dst[inter] = up;
}

// Gate|up GEMV of one pair with GELU(gate)*up and its q8 block in the same
// launch (replaces gemv_q4r_grouped + gelu_mul_quantize_q8, q4.cu). A
// workgroup of 64*LPR threads owns gate rows 32j..32j+31 (the first LPR/2
// waves) and up rows I+32j.. (the others) of pair blockIdx.y, LPR lanes per
// row (gemv_row_part), and writes q8 block j of the pair's activation with
// k_gelu_mul_q8's arithmetic. LPR 8 gives k_gemv_q4_grouped's sums (and so
// the bits of the two launches); LPR 4 sums each row in 4 lane chains.
// Grid (I/32, n_pairs).
//
// TOPK: the routing of the pair's seq (top-div of the E <= 256 logits and
// their softmax, the arithmetic of k_topk_router) is computed by every
// workgroup from the logits, the expert of pair blockIdx.y taken from it, and
// ids/wts written by the seq's workgroup (0, s*div); without TOPK the pair's
// expert is a.slots[pair].
//
// HEAD (with TOPK): the logits, the input norm's scale and q8(x_s) come from
// head_prologue (HeadArgs: the previous layer's down launch left the router
// partials) instead of logits, in_scale and a.q8; the dynamic LDS then holds
// the q8 row and, after it, the seq's partials (H/16 * (E+1) floats).
//
// REC (test record, ft_hip_set_layer_record): the same arithmetic, and the
// workgroup also stores every int32 block dot of its rows to
// a.dots[pair][row][block], the scaled gate and up sums it hands to GELU to
// a.sums[pair][row], and (HEAD) the seq's first workgroup the q8 row of x it
// computed to a.x8rec[seq]; null pointers are skipped.
template <int LAYOUT, bool TOPK, int LPR = 8, bool HEAD = false, bool REC = false>
__global__ __launch_bounds__(64 * LPR, 24 / LPR) void k_gemv_gu_act(GemvArgs a, int inter, uint8_t* q8a,
                                                                  const float* in_scale, int div, const float* logits,
                                                                  const float* escale, int32_t* ids, float* wts,
                                                                  int E, HeadArgs h) {
    static_assert(TOPK || !HEAD, "the head's logits are ranked in the launch");
    extern __shared__ int lds[];
    __shared__ float gs[64];
    const int e = blockIdx.y, t = threadIdx.x;
    __shared__ float sv[TOPK ? 256 : 1], selv[TOPK ? 32 : 1];
    __shared__ int seli[TOPK ? 32 : 1];
    __shared__ uint64_t key[TOPK ? 256 : 1];
    __shared__ float exv[TOPK ? 32 : 1];
    __shared__ float hg[HEAD ? 8 * 257 : 1];
    __shared__ float irs;
    const int s = e / div;
    if constexpr (HEAD) {
        head_prologue(h, s, a.k, E, sv, lds, reinterpret_cast<float*>(lds + (a.k >> 5) * 10), hg, &irs);
        if (REC) record_x8(a, e, s, div, lds);
    } else {
        if (TOPK && t < E) sv[t] = logits[(int64_t)s * E + t];
        stage_q8(a, e, lds);  // its barrier also covers sv
    }
    int slot;
    if constexpr (TOPK) {
        topk_rank_select(sv, E, div, key, selv, seli);
        if (blockIdx.x == 0 && e == s * div) {  // the seq's writer (uniform per workgroup): the weights too
            const float w = topk_softmax(selv, seli, div, escale, exv);
            if (t < div) {
                ids[(int64_t)s * div + t] = seli[t];
                wts[(int64_t)s * div + t] = w;
            }
        }
        slot = seli[e - s * div];
    } else {
        slot = a.slots[e];
    }
    const uint8_t* eb = a.base + (uint64_t)slot * a.expert_bytes + a.bank_off;
    const int nb = a.k >> 5;
    // waves 0..LPR/2-1: gate rows, the others up rows, 64/LPR rows per wave
    const int lane = t & 63, wave = t >> 6;
    const bool up = wave >= LPR / 2;
    const int rl = (wave - (up ? LPR / 2 : 0)) * (64 / LPR) + lane / LPR, sub = lane % LPR;
    const int row = (up ? inter : 0) + (int)blockIdx.x * 32 + rl;
    int32_t* rec = REC && a.dots ? a.dots + ((int64_t)e * 2 * inter + row) * nb : nullptr;
    float acc = gemv_row_part<LAYOUT, LPR, REC>(eb + (int64_t)row * row_bytes_of(LAYOUT, a.k), sub, nb, lds, rec);
    acc = sum_row_lanes<LPR>(acc);
    if (sub == 0) gs[(up ? 32 : 0) + rl] = acc;
    __syncthreads();
    if (threadIdx.x < 64) {  // both half-waves compute block j; the first stores it
        const int l = threadIdx.x & 31;
        float gate = gs[l], up = gs[32 + l];
        if (HEAD ? h.norm != 0 : in_scale != nullptr) {
            const float sc = HEAD ? irs : in_scale[e / div];
            gate = gate * sc;
            up = up * sc;
        }
        if (REC) record_sums(a, e, inter, gate, up);
        const float v = gelu_tanh(gate) * up;
        const Q8Lane r = q8_quantize_half(v);
        if (threadIdx.x < 32) q8_store_half(q8a + ((int64_t)e * (inter >> 5) + blockIdx.x) * Q8_BLK, l, r);
    }
}

// Down GEMV of the k pairs of one seq with the residual combine of
// k_combine_residual in the same launch: a workgroup owns rows R*j..R*j+R-1
// (R = (256/LPR)/k) of all k pairs of seq s (the k q8 activation rows,
// contiguous, staged together) and computes out = x + ((0 + w0*y0) + w1*y1
// + ...) for them, pairs in order. LPR lanes per row: 8 is
// k_gemv_q4_grouped's arithmetic; 16 (long rows) sums each row's blocks in
// 16 lane chains instead, twice the workgroups. Grid (ceil(H/R), n_seqs).
// REC (test record): every int32 block dot also goes to a.dots[pair][row][block].
template <int LAYOUT, int LPR, bool REC = false>
__global__ __launch_bounds__(256) void k_gemv_down_combine(GemvArgs a, const float* wts, const float* x, float* out,
                                                           int k) {
    extern __shared__ int lds[];
    constexpr int NE = 256 / LPR;  // row entries per workgroup
    __shared__ float ys[NE];
    const int s = blockIdx.y, R = NE / k;
    const int nb = a.k >> 5;
    // up to 40 loads per thread in one batch: the k rows (36 words per thread
    // for two rows of 448 blocks) arrive in one load latency
    stage_words<40>(reinterpret_cast<const int*>(a.q8 + (int64_t)s * k * a.q8_stride_blocks * Q8_BLK), k * nb * 10,
                    lds);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int re = wave * (64 / LPR) + lane / LPR, sub = lane % LPR;  // row entry: pair kk, local row rl
    const int kk = re / R, rl = re - kk * R;
    const int row = (int)blockIdx.x * R + rl;
    float acc = 0.0f;
    if (row < a.n_rows) {
        int32_t* rec = REC && a.dots ? a.dots + ((int64_t)(s * k + kk) * a.n_rows + row) * nb : nullptr;
        acc = gemv_row_part<LAYOUT, LPR, REC>(entry_base(a, s * k + kk) + (int64_t)row * row_bytes_of(LAYOUT, a.k),
                                              sub, nb, lds + kk * nb * 10, rec);
    }
    acc = sum_row_lanes<LPR>(acc);
    if (sub == 0) ys[re] = acc;
    __syncthreads();
    const int i = (int)blockIdx.x * R + (int)threadIdx.x;
    if ((int)threadIdx.x < R && i < a.n_rows) {
        float h = 0.0f;
        for (int q = 0; q < k; ++q) {
            const float part = ys[q * R + threadIdx.x] * wts[(int64_t)s * k + q];
            h = h + part;
        }
        out[(int64_t)s * a.n_rows + i] = x[(int64_t)s * a.n_rows + i] + h;
    }
}

// k_gemv_down_combine for 16 rows of every pair of seq s per workgroup
// (16*k*LPR threads: the same per-row arithmetic, so the same bits), which
// then computes the next layer's head partials of those rows: they are R-order
// chunk c = blockIdx.x, and the workgroup writes part[s][c][e] = the
// 16-element fma chain (in row order, from 0.0f) of the next router's row e
// (wnext, [E][H]) with out, and part[s][c][E] = that of out with itself:
// k_route_prep's chunk partials P_c, for head_prologue in the next gate|up
// launch. Grid (H/16, n_seqs), NT = 16*k*LPR threads; E < NT.
// REC (test record): every int32 block dot also goes to a.dots[pair][row][block].
template <int LAYOUT, int LPR, int NT, bool REC = false>
__global__ __launch_bounds__(NT) void k_gemv_down_head(GemvArgs a, const float* wts, const float* x, float* out,
                                                      int k, const float* wnext, float* part, int E) {
    extern __shared__ int lds[];
    __shared__ float ys[NT / LPR];
    __shared__ float4 xs4[4];
    float* xs = reinterpret_cast<float*>(xs4);
    const int s = blockIdx.y, c = blockIdx.x, t = threadIdx.x;
    const int nb = a.k >> 5, H = a.n_rows;
    // this chunk of the next router's row t: loaded ahead of the GEMV when the
    // registers allow (up to 512 threads), else after it
    constexpr bool EARLY = NT <= 512;
    float4 wv[4];
    auto load_w = [&]() __attribute__((always_inline)) {
        if (t < E) {
            const float4* w4 = reinterpret_cast<const float4*>(wnext + (int64_t)t * H + 16 * c);
#pragma unroll
            for (int q = 0; q < 4; ++q) wv[q] = w4[q];
        }
    };
    if (EARLY) load_w();
    // the combine's operands (this row's x and the seq's pair weights), loaded
    // first: read only after the GEMV, they would add a load latency there
    constexpr int KW = NT / (16 * 8);  // k <= NT / (16 * LPR) <= NT / 128 pairs
    float xr = 0.0f, wk[KW];
    if (t < 16) {
        xr = x[(int64_t)s * H + c * 16 + t];
#pragma unroll
        for (int q = 0; q < KW; ++q) wk[q] = q < k ? wts[(int64_t)s * k + q] : 0.0f;
    }
    stage_words<40>(reinterpret_cast<const int*>(a.q8 + (int64_t)s * k * a.q8_stride_blocks * Q8_BLK), k * nb * 10,
                    lds);
    const int lane = t & 63, wave = t >> 6;
    const int re = wave * (64 / LPR) + lane / LPR, sub = lane % LPR;  // row entry: pair kk, local row rl
    const int kk = re >> 4, rl = re & 15;
    const int row = c * 16 + rl;
    int32_t* rec = REC && a.dots ? a.dots + ((int64_t)(s * k + kk) * H + row) * nb : nullptr;
    float acc = gemv_row_part<LAYOUT, LPR, REC>(entry_base(a, s * k + kk) + (int64_t)row * row_bytes_of(LAYOUT, a.k),
                                                sub, nb, lds + kk * nb * 10, rec);
    acc = sum_row_lanes<LPR>(acc);
    if (sub == 0) ys[re] = acc;
    if (!EARLY) load_w();
    __syncthreads();
    if (t < 16) {
        const int i = c * 16 + t;
        float hsum = 0.0f;
#pragma unroll
        for (int q = 0; q < KW; ++q) {
            const float p = ys[min(q, k - 1) * 16 + t] * wk[q];
            hsum = q < k ? hsum + p : hsum;
        }
        const float v = xr + hsum;
        out[(int64_t)s * H + i] = v;
        xs[t] = v;
    }
    __syncthreads();
    if (t <= E) {
        float p = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 b = xs4[q];
            const float4 w = t < E ? wv[q] : b;  // t == E: the self-dot
            p = fmaf(w.x, b.x, p);
            p = fmaf(w.y, b.y, p);
            p = fmaf(w.z, b.z, p);
            p = fmaf(w.w, b.w, p);
        }
        part[((int64_t)s * (H >> 4) + c) * (E + 1) + t] = p;
    }
}

// ---------------------------------------------------------------------------
// Long rows (q4r, nb = 64*BPL blocks: gate|up rows of 64 or 128 blocks, the
// large-expert shape's hidden 2048 or 4096): a wavefront owns whole rows, lane l
// blocks l, l+64, ... of each, so one load instruction of the wave is 1 KB of
// contiguous qs (and 128 B of scales), every row's loads are issued before
// any of its dots, and a lane's q8 operands are the same for every row of
// its entry (held in registers). Per row: acc = fma chain over the lane's
// blocks in block order, then the 64 lanes summed by an xor tree (32, 16, ...,
// 1). The int32 block dots are those of every other GEMV; the f32 order is
// this kernel's own, the same in every launch that uses it.
// ---------------------------------------------------------------------------
template <int BPL>
struct LongRow {
    uint4 q[BPL];
    uint32_t s[BPL];  // the aligned dword holding this lane's block scale and the neighbour lane's
};

template <int BPL>
__device__ __forceinline__ void long_row_load(const uint8_t* wr, int lane, LongRow<BPL>& r) {
    constexpr int NB = 64 * BPL, QS_OFF = (NB * 2 + 15) / 16 * 16;
#pragma unroll
    for (int i = 0; i < BPL; ++i) r.q[i] = *reinterpret_cast<const uint4*>(wr + QS_OFF + 16 * (lane + 64 * i));
#pragma unroll
    for (int i = 0; i < BPL; ++i) r.s[i] = *reinterpret_cast<const uint32_t*>(wr + ((2 * (lane + 64 * i)) & ~3));
}

// this lane's q8 operand blocks (lane + 64*i) of an activation row in LDS
template <int BPL>
struct LongAct {
    int w[BPL][10];
};
template <int BPL>
__device__ __forceinline__ void long_act_load(const int* lds, int lane, LongAct<BPL>& x) {
#pragma unroll
    for (int i = 0; i < BPL; ++i)
#pragma unroll
        for (int k = 0; k < 10; ++k) x.w[i][k] = lds[(lane + 64 * i) * 10 + k];
}

template <int BPL>
__device__ __forceinline__ float long_row_dot(const LongRow<BPL>& r, const LongAct<BPL>& x, int lane,
                                              int32_t* rec = nullptr) {
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < BPL; ++i) {
        const int diff = block_dot(r.q[i], x.w[i] + 2, x.w[i][1]);
        if (rec) rec[lane + 64 * i] = diff;  // test record (REC launches only pass one)
        const float d4 = h2f((uint16_t)(r.s[i] >> ((lane & 1) * 16)));
        acc = fmaf((float)diff, d4 * __int_as_float(x.w[i][0]), acc);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) acc += __shfl_xor(acc, m);
    return acc;
}

// k_gemv_gu_act for rows of 64*BPL blocks (q4r): the same work per (act
// block j, pair) unit and the same prologues (logits or head, top-k) and
// tail (GELU*up, q8). 256 threads per unit: wave w owns gate rows 32j+8w..+7
// and up rows I+32j+8w..+7, four rows in flight, a row's slot refilled with
// the row four later once its dots are done. The activation row's loads go
// out before the weights' (loads complete in order), their LDS stores after.
// UPB units per workgroup (256*UPB threads, grid (inter/32)*pairs/UPB):
// sub-group g takes unit blockIdx.x*UPB + g, act block j = unit % (inter/32)
// of pair unit / (inter/32), so the UPB units share their pair (inter/32 is a
// multiple of UPB) and the prologue is computed once for them; with UPB 1 the
// grid is (inter/32, pairs). REC: the test record of k_gemv_gu_act (block
// dots, sums, head q8 row).
template <bool TOPK, int BPL, bool HEAD = false, bool REC = false, int UPB = 1>
__global__ __launch_bounds__(256 * UPB, UPB == 1 ? 4 : 1) void k_gemv_gu_long(GemvArgs a, int inter, uint8_t* q8a,
                                                                             const float* in_scale, int div,
                                                                             const float* logits, const float* escale,
                                                                             int32_t* ids, float* wts, int E,
                                                                             HeadArgs h) {
    static_assert(TOPK || !HEAD, "the head's logits are ranked in the launch");
    // rows per wave, rows in flight (with one workgroup per CU, 3 measured faster than 2, 4 or 6:
    // large1 1438.7-1439.0 vs 1448.1-1448.5, 1443.3-1448.4 and 1466.9-1467.6 us/token, same box)
    constexpr int RPW = 16, RIF = UPB > 1 ? 3 : 4;
    extern __shared__ int lds[];
    __shared__ float gs[UPB][64];
    const int tw = threadIdx.x;  // thread of the workgroup (prologue)
    const int g = UPB > 1 ? tw >> 8 : 0, t = UPB > 1 ? tw & 255 : tw;  // sub-group, thread of the unit
    const int nblk = inter >> 5, unit = (int)blockIdx.x * UPB + g;
    const int jb = UPB > 1 ? unit % nblk : (int)blockIdx.x;   // act block
    const int e = UPB > 1 ? unit / nblk : (int)blockIdx.y;    // pair (the same for the workgroup's units)
    // the workgroup's first act block: the conditions below that guard
    // barriers depend on it, not on jb, so they are uniform per workgroup
    const int jw = UPB > 1 ? ((int)blockIdx.x * UPB) % nblk : (int)blockIdx.x;
    __shared__ float sv[TOPK ? 256 : 1], selv[TOPK ? 32 : 1];
    __shared__ int seli[TOPK ? 32 : 1];
    __shared__ uint64_t key[TOPK ? 256 : 1];
    __shared__ float exv[TOPK ? 32 : 1];
    __shared__ float hg[HEAD ? 8 * 257 : 1];
    __shared__ float irs;
    const int s = e / div;
    const int lane = t & 63, wave = t >> 6;
    constexpr int RB = (64 * BPL * 2 + 15) / 16 * 16 + 64 * BPL * 16;  // q4r row bytes
    LongRow<BPL> rr[RIF];
    const uint8_t* eb = nullptr;
    auto row_of = [&](int i) { return (i < 8 ? 0 : inter) + jb * 32 + 8 * wave + (i & 7); };
    auto load_row = [&](int i) __attribute__((always_inline)) {
        long_row_load<BPL>(eb + (int64_t)row_of(i) * RB, lane, rr[i % RIF]);
    };
    auto issue = [&](int slot) __attribute__((always_inline)) {
        eb = a.base + (uint64_t)slot * a.expert_bytes + a.bank_off;
#pragma unroll
        for (int i = 0; i < RIF; ++i) load_row(i);
    };
    if constexpr (HEAD) {
        head_prologue(h, s, a.k, E, sv, lds, reinterpret_cast<float*>(lds + (a.k >> 5) * 10), hg, &irs);
        if (REC) record_x8(a, e, s, div, lds, jw);  // every thread of the workgroup holding block 0
    } else {
        // the q8 row of x (10 words per block: 64*BPL*10 words, XW per thread)
        constexpr int XW = (64 * BPL * 10 + 256 * UPB - 1) / (256 * UPB);
        const int nw = (a.k >> 5) * 10;
        const int* src = reinterpret_cast<const int*>(a.q8 + (int64_t)entry_xrow(a, e) * a.q8_stride_blocks * Q8_BLK);
        int v[XW];
#pragma unroll
        for (int r = 0; r < XW; ++r) v[r] = tw + 256 * UPB * r < nw ? src[tw + 256 * UPB * r] : 0;
        if (TOPK && tw < E) sv[tw] = logits[(int64_t)s * E + tw];
        if constexpr (!TOPK) issue(a.slots[e]);  // the pair's expert is known: weights behind the q8 row
#pragma unroll
        for (int r = 0; r < XW; ++r)
            if (tw + 256 * UPB * r < nw) lds[tw + 256 * UPB * r] = v[r];
        __syncthreads();
    }
    if constexpr (TOPK) {
        topk_rank_select(sv, E, div, key, selv, seli);
        if (jw == 0 && e == s * div) {  // the seq's writer (uniform per workgroup; a barrier inside): the weights too
            const float w = topk_softmax(selv, seli, div, escale, exv);
            if (tw < div) {
                ids[(int64_t)s * div + tw] = seli[tw];
                wts[(int64_t)s * div + tw] = w;
            }
        }
        issue(seli[e - s * div]);
    }
    LongAct<BPL> xa;
    long_act_load<BPL>(lds, lane, xa);
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        int32_t* rec = REC && a.dots ? a.dots + ((int64_t)e * 2 * inter + row_of(i)) * (64 * BPL) : nullptr;
        const float acc = long_row_dot<BPL>(rr[i % RIF], xa, lane, rec);
        if (lane == 0) gs[g][(i < 8 ? 0 : 32) + 8 * wave + (i & 7)] = acc;
        if (i + RIF < RPW) load_row(i + RIF);
    }
    __syncthreads();
    if (t < 64) {  // both half-waves compute block j; the first stores it
        const int l = t & 31;
        float gate = gs[g][l], up = gs[g][32 + l];
        if (HEAD ? h.norm != 0 : in_scale != nullptr) {
            const float sc = HEAD ? irs : in_scale[e / div];
            gate = gate * sc;
            up = up * sc;
        }
        if (REC) record_sums(a, e, inter, gate, up, jb, t);
        const float v = gelu_tanh(gate) * up;
        const Q8Lane r = q8_quantize_half(v);
        if (t < 32) q8_store_half(q8a + ((int64_t)e * (inter >> 5) + jb) * Q8_BLK, l, r);
    }
}

// Block-dot dump: the same addressing and block_dot() as k_gemv_q4_grouped.
template <int LAYOUT>
__global__ __launch_bounds__(256) void k_block_dots(GemvArgs a) {
    extern __shared__ int lds[];
    const int e = blockIdx.y;
    stage_q8(a, e, lds);
    const int nb = a.k >> 5;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row = (blockIdx.x * 4 + wave) * 8 + (lane >> 3);
    const int sub = lane & 7;
    const int qs_off = (nb * 2 + 15) / 16 * 16;
    if (row >= a.n_rows) return;
    const uint8_t* wr = entry_base(a, e) + (int64_t)row * row_bytes_of(LAYOUT, a.k);
    int32_t* out = a.dots + ((int64_t)e * a.n_rows + row) * nb;
    for (int b = sub; b < nb; b += 8) {
        float d4;
        uint4 q;
        load_block<LAYOUT>(wr, b, qs_off, d4, q);
        const int* xb = lds + b * 10;
        out[b] = block_dot(q, xb + 2, xb[1]);
    }
}

// q8 quantisation (replaces quantize_q8_grouped, q4.cu:324-355, with the
// round-half-away rule of ft-core/src/q4_0.rs:73). 32 lanes per block.
__global__ __launch_bounds__(256) void k_quantize_q8(const float* x, int64_t x_stride, uint8_t* q8,
                                                     int nb, int64_t n) {
    const int64_t g = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 5;
    const int l = threadIdx.x & 31;
    const bool ok = g < n * nb;
    const int64_t gg = ok ? g : 0;
    const int64_t e = gg / nb, b = gg % nb;
    const float v = x[e * x_stride + b * 32 + l];
    const Q8Lane r = q8_quantize_half(v);
    if (ok) q8_store_half(q8 + (e * nb + b) * Q8_BLK, l, r);
}

// Fused gelu_tanh(gate)*up -> q8 (replaces gelu_mul_q8, q4.cu:255-287).
// in_scale (input RMS norm, or null): pair e's gate and up sums are first
// multiplied by in_scale[e / div].
__global__ __launch_bounds__(256) void k_gelu_mul_q8(const float* gu, uint8_t* q8, int inter, int64_t n,
                                                     const float* in_scale, int div) {
    const int nb = inter >> 5;
    const int64_t g = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 5;
    const int l = threadIdx.x & 31;
    const bool ok = g < n * nb;
    const int64_t gg = ok ? g : 0;
    const int64_t e = gg / nb, b = gg % nb;
    const int j = (int)b * 32 + l;
    float gate = gu[e * 2 * inter + j];
    float up = gu[e * 2 * inter + inter + j];
    if (in_scale) {
        const float sc = in_scale[e / div];
        gate = gate * sc;
        up = up * sc;
    }
    const float v = gelu_tanh(gate) * up;
    const Q8Lane r = q8_quantize_half(v);
    if (ok) q8_store_half(q8 + (e * nb + b) * Q8_BLK, l, r);
}

// s = ((0 + p[0]) + p[1]) + ... + p[n-1] (each add rounded, in order), with
// the LDS reads issued eight at a time ahead of their adds
__device__ __forceinline__ float group_sum(const float* p, int n) {
    float s = 0.0f;
    int c = 0;
    for (; c + 8 <= n; c += 8) {
        float v[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] = p[c + q];
#pragma unroll
        for (int q = 0; q < 8; ++q) s = s + v[q];
    }
    for (; c < n; ++c) s = s + p[c];
    return s;
}

// R-order dot w.xs of one workgroup (the value is returned in thread 0):
// thread c computes chunk partials P_c (16-element fma chains), threads 0..7
// sum their group's chunks in order, thread 0 sums the 8 groups in order.
__device__ __forceinline__ float rorder_dot(const float* w, const float* xs, int dim, float* P, float* G) {
    const int l = threadIdx.x;
    const int nch = dim >> 4;
    for (int c = l; c < nch; c += blockDim.x) {
        const float4* w4 = reinterpret_cast<const float4*>(w + 16 * c);
        const float4* x4 = reinterpret_cast<const float4*>(xs + 16 * c);
        float p = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 a = w4[q], b = x4[q];
            p = fmaf(a.x, b.x, p);
            p = fmaf(a.y, b.y, p);
            p = fmaf(a.z, b.z, p);
            p = fmaf(a.w, b.w, p);
        }
        P[c] = p;
    }
    __syncthreads();
    const int C = dim >> 7;
    if (l < 8) G[l] = group_sum(P + l * C, C);
    __syncthreads();
    float t = 0.0f;
    if (l == 0)
        for (int g = 0; g < 8; ++g) t = t + G[g];
    return t;
}

// Router logits in the R-order (replaces gemv_f32_rows, q4.cu:1153-1174),
// times in_scale[s] (input RMS norm) when given, then + bias.
// Grid (n_rows, n_seqs), one 256-thread workgroup per logit.
// Grouped activations of Q4Gemv's batched surface, one thread per output:
// gu [n][2*inter] (gate then up), out [n][inter].
// SiLU*up: the CPU expression of ft-bench/src/bin/decode.rs:300,
// g / (1 + expf(-g)) * up, one rounding per op, glibc's expf (restated in
// ft_libm.hpp): bit-exact with it (replaces silu_mul_grouped, q4.cu:169-179).
// GELU*up: gelu_tanh of ft-model/src/lib.rs:435-437 (replaces
// gelu_mul_grouped, q4.cu:289-300).
template <bool SILU>
__global__ __launch_bounds__(256) void k_act_mul_grouped(const float* gu, float* out, int64_t inter, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n * inter) return;
    const int64_t e = i / inter, j = i - e * inter;
    const float g = gu[e * 2 * inter + j], up = gu[e * 2 * inter + inter + j];
    float a;
    if constexpr (SILU) {
        const float t = expf_libm(-g);
        const float den = 1.0f + t;
        a = g / den;  // correctly rounded (HIP default)
    } else {
        a = gelu_tanh(g);
    }
    out[i] = a * up;
}

// Weighted reductions over experts (replace reduce_expert_weighted,
// q4.cu:303-314, and reduce_weighted, q4.cu:182-192): one thread per i,
// experts in order from 0.0f, one rounding per op:
//   W: out[i] = out[i] + sum_e (w[e] * y[e][i]);  else out[i] = out[i] + a * sum_e y[e][i].
template <bool W>
__global__ __launch_bounds__(256) void k_reduce_experts(const float* y, const float* w, float a, float* out,
                                                        int64_t hidden, int n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= hidden) return;
    float s = 0.0f;
    for (int e = 0; e < n; ++e) {
        const float v = y[(int64_t)e * hidden + i];
        if constexpr (W) {
            const float part = w[e] * v;
            s = s + part;
        } else {
            s = s + v;
        }
    }
    if constexpr (W) {
        out[i] = out[i] + s;
    } else {
        const float as = a * s;
        out[i] = out[i] + as;
    }
}

__global__ __launch_bounds__(256) void k_router_logits(const float* W, const float* x, const float* bias,
                                                      const float* in_scale, float* y, int dim, int n_rows) {
    extern __shared__ float P[];  // dim/16 chunk partials
    __shared__ float G[8];
    const int e = blockIdx.x, s = blockIdx.y;
    float t = rorder_dot(W + (int64_t)e * dim, x + (int64_t)s * dim, dim, P, G);
    if (threadIdx.x == 0) {
        if (in_scale) t = t * in_scale[s];
        if (bias) t = t + bias[e];
        y[(int64_t)s * n_rows + e] = t;
    }
}

// The head of a layer in one launch (grid (n_rows, n_seqs), one workgroup per
// logit): router logits as k_router_logits, with the input RMS norm's scale
// computed by each workgroup for its seq (the same R-order self-dot as
// k_rms_inv, so the same bits) when norm is set; workgroup (e, s) with e <
// ceil(nb/16) also quantizes blocks 16e..16e+15 of x_s to q8 (the
// arithmetic of k_quantize_q8) and e == 0 stores inv[s].
__global__ __launch_bounds__(256) void k_route_prep(const float* W, const float* x, const float* bias, int norm,
                                                   float* inv, uint8_t* q8, float* y, int dim, int n_rows) {
    extern __shared__ float P[];  // 2 * dim/16 chunk partials
    __shared__ float G[8], G2[16];
    __shared__ float irs;
    const int e = blockIdx.x, s = blockIdx.y, l = threadIdx.x;
    const float* xs = x + (int64_t)s * dim;
    // this lane's part of the q8 block it quantizes at the end, loaded with
    // the first loads (one load latency for the launch, not two)
    const int nb = dim >> 5, b = e * 16 + (l >> 2);
    const bool qz = e * 16 < nb && l < 64 && b < nb;  // quads of blocks beyond nb idle
    float4 qa = make_float4(0.f, 0.f, 0.f, 0.f), qb = qa;
    if (qz) {
        const float4* v4 = reinterpret_cast<const float4*>(xs + 32 * b);
        qa = v4[2 * (l & 3)];
        qb = v4[2 * (l & 3) + 1];
    }
    const float bv = bias && l == 0 ? bias[e] : 0.0f;  // the logit's bias, loaded with them
    float t;
    if (norm) {  // both R-order dots in one pass: x.x (P) and w.x (Q), each in its own order
        const float* w = W + (int64_t)e * dim;
        float* Q = P + (dim >> 4);
        for (int c = l; c < (dim >> 4); c += blockDim.x) {
            const float4* w4 = reinterpret_cast<const float4*>(w + 16 * c);
            const float4* x4 = reinterpret_cast<const float4*>(xs + 16 * c);
            float p = 0.0f, q = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float4 a = w4[k], b = x4[k];
                p = fmaf(b.x, b.x, p);
                p = fmaf(b.y, b.y, p);
                p = fmaf(b.z, b.z, p);
                p = fmaf(b.w, b.w, p);
                q = fmaf(a.x, b.x, q);
                q = fmaf(a.y, b.y, q);
                q = fmaf(a.z, b.z, q);
                q = fmaf(a.w, b.w, q);
            }
            P[c] = p;
            Q[c] = q;
        }
        __syncthreads();
        const int C = dim >> 7;
        if (l < 16) G2[l] = group_sum((l < 8 ? P : Q) + (l & 7) * C, C);
        __syncthreads();
        t = 0.0f;
        if (l == 0) {
            float ss = 0.0f;
            for (int g = 0; g < 8; ++g) ss = ss + G2[g];
            for (int g = 0; g < 8; ++g) t = t + G2[8 + g];
            irs = 1.0f / sqrtf(ss / (float)dim + 1e-6f);  // correctly rounded (HIP default)
        }
    } else {
        t = rorder_dot(W + (int64_t)e * dim, xs, dim, P, G);
    }
    const float ir = norm ? irs : 1.0f;
    if (l == 0) {
        if (norm) t = t * ir;
        if (bias) t = t + bv;
        y[(int64_t)s * n_rows + e] = t;
        if (norm && e == 0) inv[s] = ir;
    }
    if (qz) quantize_block_quad_v(qa, qb, l & 3, reinterpret_cast<uint32_t*>(q8 + ((int64_t)s * nb + b) * Q8_BLK));
}

// k_route_prep for EG logits per workgroup (batched decode): workgroup
// (eg, s) computes logits EG*eg..EG*eg+EG-1 of seq s, each in the R-order as
// k_route_prep (the same bits), reading each chunk of x once for the EG
// router rows and the self-dot; and quantizes q8 blocks [eg*Q, eg*Q+Q) of
// x_s, Q = ceil(nb / gridDim.x). e == 0's workgroup stores inv[s].
// Grid (n_rows/EG, n_seqs), 256 threads.
template <int EG>
__global__ __launch_bounds__(256) void k_route_prep_n(const float* W, const float* x, const float* bias, int norm,
                                                      float* inv, uint8_t* q8, float* y, int dim, int n_rows) {
    extern __shared__ float P[];  // [EG+1][dim/16] chunk partials: the EG logits', then x.x
    __shared__ float G[EG + 1][8], tot[EG + 1];
    const int eg = blockIdx.x, s = blockIdx.y, l = threadIdx.x;
    const int nch = dim >> 4;
    const float* xs = x + (int64_t)s * dim;
    const float* w0 = W + (int64_t)eg * EG * dim;
    const float bv = bias && l < EG ? bias[eg * EG + l] : 0.0f;  // the logit's bias, loaded with the chunks
    for (int c = l; c < nch; c += blockDim.x) {
        const float4* x4 = reinterpret_cast<const float4*>(xs + 16 * c);
        float4 xv[4], wv[EG][4];
#pragma unroll
        for (int k = 0; k < 4; ++k) xv[k] = x4[k];
#pragma unroll
        for (int j = 0; j < EG; ++j)
#pragma unroll
            for (int k = 0; k < 4; ++k) wv[j][k] = reinterpret_cast<const float4*>(w0 + (int64_t)j * dim + 16 * c)[k];
        // every value held at once here: the loads are all issued before the
        // chains (the scheduler otherwise interleaved them, a load latency
        // per few loads)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            asm volatile("" : "+v"(xv[k].x), "+v"(xv[k].y), "+v"(xv[k].z), "+v"(xv[k].w));
#pragma unroll
            for (int j = 0; j < EG; ++j)
                asm volatile("" : "+v"(wv[j][k].x), "+v"(wv[j][k].y), "+v"(wv[j][k].z), "+v"(wv[j][k].w));
        }
        float pe[EG], ps = 0.0f;
#pragma unroll
        for (int j = 0; j < EG; ++j) {
            float p = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float4 a = wv[j][k], b = xv[k];
                p = fmaf(a.x, b.x, p);
                p = fmaf(a.y, b.y, p);
                p = fmaf(a.z, b.z, p);
                p = fmaf(a.w, b.w, p);
            }
            pe[j] = p;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float4 b = xv[k];
            ps = fmaf(b.x, b.x, ps);
            ps = fmaf(b.y, b.y, ps);
            ps = fmaf(b.z, b.z, ps);
            ps = fmaf(b.w, b.w, ps);
        }
#pragma unroll
        for (int j = 0; j < EG; ++j) P[j * nch + c] = pe[j];
        P[EG * nch + c] = ps;
    }
    __syncthreads();
    const int C = dim >> 7;
    if (l < 8 * (EG + 1)) G[l >> 3][l & 7] = group_sum(P + (l >> 3) * nch + (l & 7) * C, C);
    __syncthreads();
    if (l < EG + 1) {
        float t = 0.0f;
        for (int g = 0; g < 8; ++g) t = t + G[l][g];
        tot[l] = t;
    }
    __syncthreads();
    if (l < EG) {
        const float ir = norm ? 1.0f / sqrtf(tot[EG] / (float)dim + 1e-6f) : 1.0f;  // correctly rounded
        const int e = eg * EG + l;
        float t = tot[l];
        if (norm) t = t * ir;
        if (bias) t = t + bv;
        y[(int64_t)s * n_rows + e] = t;
        if (norm && e == 0) inv[s] = ir;
    }
    const int nb = dim >> 5, Q = (nb + gridDim.x - 1) / gridDim.x, b = eg * Q + (l >> 2);
    if ((l >> 2) < Q && b < nb)
        quantize_block_quad(xs + 32 * b, l & 3, reinterpret_cast<uint32_t*>(q8 + ((int64_t)s * nb + b) * Q8_BLK));
}

// k_route_prep_n for SQ seqs per workgroup as well (larger batches): workgroup
// (eg, sg) computes logits EG*eg..+EG-1 of seqs SQ*sg..+SQ-1, each in the
// R-order as k_route_prep (the same bits), holding the EG router chunks in
// registers across the SQ seqs, so the router is read n_seqs/SQ times
// instead of n_seqs; and quantizes q8 blocks [eg*Q, eg*Q+Q) of each of its
// seqs, Q = ceil(nb / gridDim.x). Workgroup eg == 0 stores inv of its seqs.
// Grid (n_rows/EG, n_seqs/SQ), 256 threads.
template <int EG, int SQ>
__global__ __launch_bounds__(256) void k_route_prep_m(const float* W, const float* x, const float* bias, int norm,
                                                      float* inv, uint8_t* q8, float* y, int dim, int n_rows) {
    extern __shared__ float P[];  // [SQ][EG+1][nch + 1] chunk partials: the EG logits', then x.x
    __shared__ float G[SQ * (EG + 1) * 8], tot[SQ * (EG + 1)];
    const int eg = blockIdx.x, s0 = blockIdx.y * SQ, l = threadIdx.x;
    const int nch = dim >> 4, ps = nch + 1;  // odd row stride: the group sums' lanes read different banks
    const float* w0 = W + (int64_t)eg * EG * dim;
    const float bv = bias && l < SQ * EG ? bias[eg * EG + l % EG] : 0.0f;  // loaded with the chunks
    for (int c = l; c < nch; c += blockDim.x) {
        // every load of the chunk issued before the first fma (one load
        // latency), then the chains: each (logit, seq) partial and each seq's
        // x.x over the 16 elements in order
        float4 wv[EG][4], xv[SQ][4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
#pragma unroll
            for (int j = 0; j < EG; ++j) wv[j][k] = reinterpret_cast<const float4*>(w0 + (int64_t)j * dim + 16 * c)[k];
#pragma unroll
            for (int q = 0; q < SQ; ++q) xv[q][k] = reinterpret_cast<const float4*>(x + (int64_t)(s0 + q) * dim + 16 * c)[k];
        }
        // every value held at once here: the loads cannot be sunk towards
        // their first use (the scheduler otherwise interleaved them with the
        // chains, one load latency per few loads)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
#pragma unroll
            for (int j = 0; j < EG; ++j)
                asm volatile("" : "+v"(wv[j][k].x), "+v"(wv[j][k].y), "+v"(wv[j][k].z), "+v"(wv[j][k].w));
#pragma unroll
            for (int q = 0; q < SQ; ++q)
                asm volatile("" : "+v"(xv[q][k].x), "+v"(xv[q][k].y), "+v"(xv[q][k].z), "+v"(xv[q][k].w));
        }
#pragma unroll
        for (int q = 0; q < SQ; ++q) {
            float* Pq = P + q * (EG + 1) * ps;
#pragma unroll
            for (int j = 0; j < EG; ++j) {
                float p = 0.0f;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float4 a = wv[j][k], b = xv[q][k];
                    p = fmaf(a.x, b.x, p);
                    p = fmaf(a.y, b.y, p);
                    p = fmaf(a.z, b.z, p);
                    p = fmaf(a.w, b.w, p);
                }
                Pq[j * ps + c] = p;
            }
            float pss = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float4 b = xv[q][k];
                pss = fmaf(b.x, b.x, pss);
                pss = fmaf(b.y, b.y, pss);
                pss = fmaf(b.z, b.z, pss);
                pss = fmaf(b.w, b.w, pss);
            }
            Pq[EG * ps + c] = pss;
        }
    }
    __syncthreads();
    const int C = dim >> 7;
    for (int i = l; i < SQ * (EG + 1) * 8; i += blockDim.x) G[i] = group_sum(P + (i >> 3) * ps + (i & 7) * C, C);
    __syncthreads();
    if (l < SQ * (EG + 1)) {
        float t = 0.0f;
        for (int g = 0; g < 8; ++g) t = t + G[l * 8 + g];
        tot[l] = t;
    }
    __syncthreads();
    if (l < SQ * EG) {
        const int q = l / EG, jj = l - q * EG;
        const float ir = norm ? 1.0f / sqrtf(tot[q * (EG + 1) + EG] / (float)dim + 1e-6f) : 1.0f;  // correctly rounded
        const int e = eg * EG + jj, s = s0 + q;
        float t = tot[q * (EG + 1) + jj];
        if (norm) t = t * ir;
        if (bias) t = t + bv;
        y[(int64_t)s * n_rows + e] = t;
        if (norm && e == 0) inv[s] = ir;
    }
    const int nb = dim >> 5, Q = (nb + gridDim.x - 1) / gridDim.x;
    for (int i = l; i < SQ * Q * 4; i += blockDim.x) {  // whole quads: 4 consecutive lanes per block
        const int q = i / (Q * 4), rem = i - q * Q * 4, b = eg * Q + (rem >> 2);
        if (b < nb)
            quantize_block_quad(x + (int64_t)(s0 + q) * dim + 32 * b, rem & 3,
                                reinterpret_cast<uint32_t*>(q8 + ((int64_t)(s0 + q) * nb + b) * Q8_BLK));
    }
}

// Scale of the input RMS norm per seq: inv[s] = 1 / sqrt(ss / dim + 1e-6),
// ss = x_s.x_s in the R-order, each op rounded once. Grid n_seqs.
__global__ __launch_bounds__(256) void k_rms_inv(const float* x, float* inv, int dim) {
    extern __shared__ float P[];
    __shared__ float G[8];
    const int s = blockIdx.x;
    const float* xs = x + (int64_t)s * dim;
    const float ss = rorder_dot(xs, xs, dim, P, G);
    if (threadIdx.x == 0) inv[s] = 1.0f / sqrtf(ss / (float)dim + 1e-6f);  // correctly rounded (HIP default)
}

// (value, index) order of the router: larger logit first, then lower index;
// NaN after every number (the reference's sort would panic on one).
__device__ __forceinline__ bool topk_better(float v1, int i1, float v2, int i2, int E) {
    if (i2 >= E) return i1 < E;
    if (i1 >= E) return false;
    const bool n1 = !(v1 == v1), n2 = !(v2 == v2);
    if (n1 != n2) return n2;
    if (!n1) {
        if (v1 > v2) return true;
        if (v1 < v2) return false;
    }
    return i1 < i2;
}

// Top-k + softmax over the chosen (replaces topk_router, q4.cu:1297-1349;
// order and weights of ft-model/src/lib.rs:1487-1504). One workgroup per seq.
__global__ __launch_bounds__(256) void k_topk_router(const float* logits, const float* escale, int32_t* ids,
                                                     float* wts, int E, int k) {
    __shared__ float sv[1024];
    __shared__ uint8_t taken[1024];
    __shared__ float rv[256];
    __shared__ int ri[256];
    __shared__ float selv[32];
    __shared__ int seli[32];
    const int s = blockIdx.x, t = threadIdx.x;
    for (int i = t; i < E; i += 256) {
        sv[i] = logits[(int64_t)s * E + i];
        taken[i] = 0;
    }
    __syncthreads();
    if (E <= 256) {
        __shared__ uint64_t key[256];
        topk_rank_select(sv, E, k, key, selv, seli);
    }
    for (int j = 0; E > 256 && j < k; ++j) {
        float bv = 0.0f;
        int bi = E;
        for (int i = t; i < E; i += 256)
            if (!taken[i] && topk_better(sv[i], i, bv, bi, E)) {
                bv = sv[i];
                bi = i;
            }
        rv[t] = bv;
        ri[t] = bi;
        __syncthreads();
        for (int h = 128; h > 0; h >>= 1) {
            if (t < h && topk_better(rv[t + h], ri[t + h], rv[t], ri[t], E)) {
                rv[t] = rv[t + h];
                ri[t] = ri[t + h];
            }
            __syncthreads();
        }
        if (t == 0) {
            selv[j] = rv[0];
            seli[j] = ri[0];
            taken[ri[0]] = 1;
        }
        __syncthreads();
    }
    __shared__ float exv[32];
    const float w = topk_softmax(selv, seli, k, escale, exv);
    if (t < k) {
        ids[(int64_t)s * k + t] = seli[t];
        wts[(int64_t)s * k + t] = w;
    }
}

// out[s][i] += sum_{p: seq_of[p]==s} wts[p]*y[p][i] (replaces
// reduce_pairs_weighted, q4.cu:419-434; CPU order of ft-model/src/lib.rs:1641-1646).
__global__ __launch_bounds__(256) void k_reduce_pairs(const float* y, const float* wts, const int32_t* seq_of,
                                                      float* out, int hidden, int n_pairs) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int s = blockIdx.y;
    if (i >= hidden) return;
    float acc = 0.0f;
    for (int p = 0; p < n_pairs; ++p)
        if (seq_of[p] == s) {
            const float part = y[(int64_t)p * hidden + i] * wts[p];
            acc = acc + part;
        }
    out[(int64_t)s * hidden + i] = out[(int64_t)s * hidden + i] + acc;
}

// Residual combine over contiguous per-seq pairs [s*k, s*k+k):
// out[s][i] = x[s][i] + ((0 + w0*y0) + w1*y1 + ...). out may alias x.
__global__ __launch_bounds__(256) void k_combine_residual(const float* y, const float* wts, const float* x,
                                                          float* out, int hidden, int k) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int s = blockIdx.y;
    if (i >= hidden) return;
    float acc = 0.0f;
    for (int p = s * k; p < s * k + k; ++p) {
        const float part = y[(int64_t)p * hidden + i] * wts[p];
        acc = acc + part;
    }
    out[(int64_t)s * hidden + i] = x[(int64_t)s * hidden + i] + acc;
}

// Row layout conversion, one thread per (row, block).
__global__ __launch_bounds__(256) void k_repack(const uint8_t* src, int sl, uint8_t* dst, int dl, int64_t n_rows,
                                                int k) {
    const int nb = k >> 5;
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n_rows * nb) return;
    const int64_t r = g / nb;
    const int b = (int)(g % nb);
    const int qs_off = (nb * 2 + 15) / 16 * 16;
    const uint8_t* s = src + r * row_bytes_of(sl, k);
    uint8_t* d = dst + r * row_bytes_of(dl, k);
    const uint8_t* sq = sl == FT_LAYOUT_Q4R ? s + qs_off + 16 * b : s + 18 * b + 2;
    const uint8_t* ss = sl == FT_LAYOUT_Q4R ? s + 2 * b : s + 18 * b;
    uint8_t* dq = dl == FT_LAYOUT_Q4R ? d + qs_off + 16 * b : d + 18 * b + 2;
    uint8_t* ds = dl == FT_LAYOUT_Q4R ? d + 2 * b : d + 18 * b;
    ds[0] = ss[0];
    ds[1] = ss[1];
    for (int i = 0; i < 16; ++i) dq[i] = sq[i];
    if (dl == FT_LAYOUT_Q4R && b == nb - 1)  // zero the scale padding
        for (int i = 2 * nb; i < qs_off; ++i) d[i] = 0;
}

// Read-only stream over n16 16-byte words (the achievable HBM read rate):
// grid-stride, each thread with four 16-byte loads in flight per step; the
// XOR of everything a workgroup read goes to out[blockIdx.x] so no load is
// dead code.
__global__ __launch_bounds__(256) void k_stream_read(const uint4* buf, uint64_t n16, uint32_t* out) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t acc = 0;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        uint4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = buf[i + u * stride];
#pragma unroll
        for (int u = 0; u < 4; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += stride) {
        const uint4 v = buf[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    __shared__ uint32_t red[4];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

__global__ __launch_bounds__(256) void k_gen_values(uint64_t key, int64_t start, int64_t n, float scale, float* out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = gen_value(key, (uint64_t)(start + i), scale);
}

// Seeded q4_0 rows, one thread per (row, block), written in `layout`.
__global__ __launch_bounds__(256) void k_gen_q4_rows(uint64_t key, int64_t row0, int64_t n_rows, int k, float scale,
                                                     uint8_t* out, int layout) {
    const int nb = k >> 5;
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n_rows * nb) return;
    const int64_t r = g / nb;
    const int b = (int)(g % nb);
    float v[QK];
    const uint64_t base = (uint64_t)(row0 + r) * (uint64_t)k + (uint64_t)b * QK;
    for (int i = 0; i < QK; ++i) v[i] = gen_value(key, base + i, scale);
    uint16_t dh;
    uint4 qs;
    quantize_block_q4_0(v, dh, qs);
    uint8_t* row = out + r * row_bytes_of(layout, k);
    if (layout == FT_LAYOUT_Q4R) {
        const int qs_off = (nb * 2 + 15) / 16 * 16;
        reinterpret_cast<uint16_t*>(row)[b] = dh;
        *reinterpret_cast<uint4*>(row + qs_off + 16 * b) = qs;
        if (b == nb - 1)
            for (int i = 2 * nb; i < qs_off; ++i) row[i] = 0;
    } else {
        uint16_t* p = reinterpret_cast<uint16_t*>(row + 18 * b);
        p[0] = dh;
        const uint32_t w[4] = {qs.x, qs.y, qs.z, qs.w};
        for (int i = 0; i < 4; ++i) {
            p[1 + 2 * i] = (uint16_t)(w[i] & 0xFFFF);
            p[2 + 2 * i] = (uint16_t)(w[i] >> 16);
        }
    }
}

// ===========================================================================
// C ABI
// ===========================================================================
static inline hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }

static int check_layout(int layout) {
    if (layout != FT_LAYOUT_Q4_0 && layout != FT_LAYOUT_Q4R)
        return fail(FT_HIP_E_INVALID, "unknown layout %d", layout);
    return FT_HIP_OK;
}

extern "C" int64_t ft_hip_row_bytes(int layout, int64_t k) {
    if (k <= 0 || k % 32) return -1;
    if (layout != FT_LAYOUT_Q4_0 && layout != FT_LAYOUT_Q4R) return -1;
    return row_bytes_of(layout, (int)k);
}

extern "C" int64_t ft_hip_q4r_scales_bytes(int64_t k) {
    if (k <= 0 || k % 32) return -1;
    return (k / 32 * 2 + 15) / 16 * 16;
}

extern "C" int ft_hip_quantize_q8(ft_hip_ctx* ctx, void* stream, const float* x, int64_t x_stride, void* q8,
                                  int64_t k, int64_t n) {
    clear_error();
    if (k <= 0 || k % 32) return fail(FT_HIP_E_SHAPE, "quantize_q8: k=%lld must be a positive multiple of 32", (long long)k);
    if (n < 0 || x_stride < 0) return fail(FT_HIP_E_SHAPE, "quantize_q8: negative n or x_stride");
    if (x_stride != 0 && x_stride < k) return fail(FT_HIP_E_SHAPE, "quantize_q8: x_stride < k");
    if (!ctx || !x || !q8) return fail(FT_HIP_E_INVALID, "quantize_q8: null argument");
    if (n == 0) return FT_HIP_OK;
    const int nb = (int)(k / 32);
    const int64_t threads = n * nb * 32;
    hipLaunchKernelGGL(k_quantize_q8, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, S(stream), x, x_stride,
                       (uint8_t*)q8, nb, n);
    return launch_status("quantize_q8");
}

// Lanes per row of a q4r GEMV launch: 0 for k_gemv_q4_grouped (8 lanes, 32
// rows per workgroup), else 16/32/64 for k_gemv_q4r_short. Automatic (knob 0):
// launches of at least 2048 workgroups of 32 rows stream at full rate on the
// 8-lane kernel; smaller ones take the fewest lanes per row that give 1024
// workgroups (64 when none does), with at most 8 blocks per lane.
static int short_lanes(const ft_hip_ctx* ctx, int layout, int64_t n_rows, int64_t n_entries, int nb) {
    if (layout != FT_LAYOUT_Q4R) return 0;
    const int force = ctx->gemv_lanes;
    if (force == 8) return 0;
    if (force) return nb <= 8 * force ? force : 0;
    if ((n_rows + 31) / 32 * n_entries >= 2048) return 0;
    for (int lpr : {16, 32, 64})
        if (nb <= 8 * lpr && (n_rows + 256 / lpr - 1) / (256 / lpr) * n_entries >= 1024) return lpr;
    return nb <= 8 * 64 ? 64 : 0;
}

// The long-row gate|up kernel (k_gemv_gu_long) takes q4r banks whose
// gate|up rows are 64 or 128 blocks (BPL = blocks per lane = 1, 2); 0 = the
// other kernels.
static int gu_long_bpl(int layout, int64_t hidden) {
    return layout == FT_LAYOUT_Q4R && (hidden == 2048 || hidden == 4096) ? (int)(hidden / 2048) : 0;
}
// Launches of (inter/32, pairs) units: four units per workgroup (one per
// CU: the workgroups then spread evenly, 224 for the large-expert layer's
// 896 units, instead of 3 or 4 of the 256-thread form per CU) when 4 divides
// inter/32 and the layer has at least 128 such workgroups.
template <bool TOPK, bool HEAD, bool REC = false>
static void launch_gu_long_r(int bpl, dim3 grid, size_t lds, hipStream_t st, const GemvArgs& a, int inter,
                             uint8_t* q8a, const float* in_scale, int div, const float* logits, const float* escale,
                             int32_t* ids, float* wts, int E, const HeadArgs& h) {
    if (bpl == 2 && grid.x % 4 == 0 && grid.x * grid.y / 4 >= 128) {
        hipLaunchKernelGGL((k_gemv_gu_long<TOPK, 2, HEAD, REC, 4>), dim3(grid.x * grid.y / 4), dim3(1024), lds, st, a,
                           inter, q8a, in_scale, div, logits, escale, ids, wts, E, h);
        return;
    }
    if (bpl == 1)
        hipLaunchKernelGGL((k_gemv_gu_long<TOPK, 1, HEAD, REC>), grid, dim3(256), lds, st, a, inter, q8a, in_scale,
                           div, logits, escale, ids, wts, E, h);
    else
        hipLaunchKernelGGL((k_gemv_gu_long<TOPK, 2, HEAD, REC>), grid, dim3(256), lds, st, a, inter, q8a, in_scale,
                           div, logits, escale, ids, wts, E, h);
}
// rec: the record instantiation (a layer record is set)
template <bool TOPK, bool HEAD>
static void launch_gu_long(int bpl, dim3 grid, size_t lds, hipStream_t st, const GemvArgs& a, int inter, uint8_t* q8a,
                           const float* in_scale, int div, const float* logits, const float* escale, int32_t* ids,
                           float* wts, int E, const HeadArgs& h, bool rec = false) {
    if (rec)
        launch_gu_long_r<TOPK, HEAD, true>(bpl, grid, lds, st, a, inter, q8a, in_scale, div, logits, escale, ids, wts,
                                           E, h);
    else
        launch_gu_long_r<TOPK, HEAD, false>(bpl, grid, lds, st, a, inter, q8a, in_scale, div, logits, escale, ids,
                                            wts, E, h);
}

// The gate|up launch with the activation, k_gemv_gu_act<LAYOUT, TOPK,
// GU_LANES, HEAD> or its record instantiation.
template <bool TOPK, bool HEAD>
static void launch_gu_act(int layout, bool rec, dim3 grid, size_t lds, hipStream_t st, const GemvArgs& a, int inter,
                          uint8_t* q8a, const float* in_scale, int div, const float* logits, const float* escale,
                          int32_t* ids, float* wts, int E, const HeadArgs& h) {
    auto kern = layout == FT_LAYOUT_Q4R
                    ? (rec ? k_gemv_gu_act<FT_LAYOUT_Q4R, TOPK, GU_LANES, HEAD, true>
                           : k_gemv_gu_act<FT_LAYOUT_Q4R, TOPK, GU_LANES, HEAD, false>)
                    : (rec ? k_gemv_gu_act<FT_LAYOUT_Q4_0, TOPK, GU_LANES, HEAD, true>
                           : k_gemv_gu_act<FT_LAYOUT_Q4_0, TOPK, GU_LANES, HEAD, false>);
    hipLaunchKernelGGL(kern, grid, dim3(64 * GU_LANES), lds, st, a, inter, q8a, in_scale, div, logits, escale, ids,
                       wts, E, h);
}

template <int LPR, bool REC, int XIN = 0, bool ACT = false>
static void launch_short_rec(int nbl, dim3 grid, size_t lds, hipStream_t s, const GemvArgs& a) {
    if (nbl <= 2) hipLaunchKernelGGL((k_gemv_q4r_short<LPR, 2, REC, XIN, ACT>), grid, dim3(256), lds, s, a);
    else if (nbl <= 4) hipLaunchKernelGGL((k_gemv_q4r_short<LPR, 4, REC, XIN, ACT>), grid, dim3(256), lds, s, a);
    else hipLaunchKernelGGL((k_gemv_q4r_short<LPR, 8, REC, XIN, ACT>), grid, dim3(256), lds, s, a);
}

template <int LPR, int XIN = 0, bool ACT = false>
static void launch_short(bool rec, int nbl, dim3 grid, size_t lds, hipStream_t s, const GemvArgs& a) {
    if (rec) launch_short_rec<LPR, true, XIN, ACT>(nbl, grid, lds, s, a);
    else launch_short_rec<LPR, false, XIN, ACT>(nbl, grid, lds, s, a);
}

template <int LPR>
static void launch_short_f32in(bool rec, bool act, int nbl, dim3 grid, size_t lds, hipStream_t s, const GemvArgs& a) {
    if (act) launch_short<LPR, 1, true>(rec, nbl, grid, lds, s, a);
    else launch_short<LPR, 1, false>(rec, nbl, grid, lds, s, a);
}

static int gemv_common(ft_hip_ctx* ctx, void* stream, GemvArgs& a, int64_t n_entries, int64_t n_rows, int64_t k,
                       int layout, bool dots, const char* name) {
    if (k <= 0 || k % 32) return fail(FT_HIP_E_SHAPE, "%s: k=%lld must be a positive multiple of 32", name, (long long)k);
    if (k > 32 * 4096) return fail(FT_HIP_E_SHAPE, "%s: k=%lld exceeds 131072", name, (long long)k);
    if (n_rows < 0 || n_entries < 0) return fail(FT_HIP_E_SHAPE, "%s: negative n_rows or n_entries", name);
    if (n_rows > (1 << 30) || n_entries > 65535) return fail(FT_HIP_E_SHAPE, "%s: n_rows or n_entries too large", name);
    if (!dots && a.y_stride < n_rows && n_entries > 1)
        return fail(FT_HIP_E_SHAPE, "%s: y_stride=%lld < n_rows=%lld", name, (long long)a.y_stride, (long long)n_rows);
    if (a.q8_stride_blocks < 0) return fail(FT_HIP_E_SHAPE, "%s: negative q8_stride_blocks", name);
    if (int rc = check_layout(layout)) return rc;
    if (layout == FT_LAYOUT_Q4R && !a.bases &&
        ((reinterpret_cast<uintptr_t>(a.base) | a.expert_bytes | a.bank_off) & 15))
        return fail(FT_HIP_E_SHAPE, "%s: q4r banks need 16-byte aligned base, expert_bytes and bank_off", name);
    if (!ctx || !a.q8 || (!dots && !a.y) || (dots && !a.dots)) return fail(FT_HIP_E_INVALID, "%s: null argument", name);
    if (!a.bases && (!a.base || !a.slots)) return fail(FT_HIP_E_INVALID, "%s: null weight addressing", name);
    if (n_entries == 0 || n_rows == 0) return FT_HIP_OK;
    a.n_rows = (int)n_rows;
    a.k = (int)k;
    const size_t lds = (size_t)(k / 32) * Q8_BLK;
    dim3 grid((unsigned)((n_rows + 31) / 32), (unsigned)n_entries);
    if (dots) {
        if (layout == FT_LAYOUT_Q4R) hipLaunchKernelGGL(k_block_dots<FT_LAYOUT_Q4R>, grid, dim3(256), lds, S(stream), a);
        else hipLaunchKernelGGL(k_block_dots<FT_LAYOUT_Q4_0>, grid, dim3(256), lds, S(stream), a);
        return launch_status(name);
    }
    // a block-dot record (ft_hip_set_block_dot_record, tests only) selects the
    // instantiations that also store the dots
    const bool rec = ctx->rec_gu != nullptr;
    a.dots = ctx->rec_gu;
    const int nb = (int)(k / 32);
    if (const int lpr = short_lanes(ctx, layout, n_rows, n_entries, nb)) {
        const int nbl = (nb + lpr - 1) / lpr;
        const dim3 g2((unsigned)((n_rows + 256 / lpr - 1) / (256 / lpr)), (unsigned)n_entries);
        if (lpr == 16) launch_short<16>(rec, nbl, g2, lds, S(stream), a);
        else if (lpr == 32) launch_short<32>(rec, nbl, g2, lds, S(stream), a);
        else launch_short<64>(rec, nbl, g2, lds, S(stream), a);
    } else if (layout == FT_LAYOUT_Q4R) {
        hipLaunchKernelGGL((rec ? k_gemv_q4_grouped<FT_LAYOUT_Q4R, true> : k_gemv_q4_grouped<FT_LAYOUT_Q4R, false>),
                           grid, dim3(256), lds, S(stream), a);
    } else {
        hipLaunchKernelGGL((rec ? k_gemv_q4_grouped<FT_LAYOUT_Q4_0, true> : k_gemv_q4_grouped<FT_LAYOUT_Q4_0, false>),
                           grid, dim3(256), lds, S(stream), a);
    }
    return launch_status(name);
}

extern "C" int ft_hip_gemv_q4_grouped_ptr(ft_hip_ctx* ctx, void* stream, const uint64_t* bases, uint64_t bank_off,
                                          const int32_t* x_idx, int64_t n_entries, const void* q8,
                                          int64_t q8_stride_blocks, float* y, int64_t y_stride, int64_t n_rows,
                                          int64_t k, int layout) {
    clear_error();
    if (!bases) return fail(FT_HIP_E_INVALID, "gemv_q4_grouped_ptr: null bases");
    GemvArgs a{};
    a.bases = bases;
    a.bank_off = bank_off;
    a.x_idx = x_idx;
    a.x_div = 1;
    a.q8 = (const uint8_t*)q8;
    a.q8_stride_blocks = q8_stride_blocks;
    a.y = y;
    a.y_stride = y_stride;
    return gemv_common(ctx, stream, a, n_entries, n_rows, k, layout, false, "gemv_q4_grouped_ptr");
}

extern "C" int ft_hip_gemv_q4_grouped_slots(ft_hip_ctx* ctx, void* stream, const void* base, uint64_t expert_bytes,
                                            uint64_t bank_off, const int32_t* slots, const int32_t* x_idx,
                                            int64_t n_entries, const void* q8, int64_t q8_stride_blocks, float* y,
                                            int64_t y_stride, int64_t n_rows, int64_t k, int layout) {
    clear_error();
    GemvArgs a{};
    a.base = (const uint8_t*)base;
    a.expert_bytes = expert_bytes;
    a.slots = slots;
    a.bank_off = bank_off;
    a.x_idx = x_idx;
    a.x_div = 1;
    a.q8 = (const uint8_t*)q8;
    a.q8_stride_blocks = q8_stride_blocks;
    a.y = y;
    a.y_stride = y_stride;
    return gemv_common(ctx, stream, a, n_entries, n_rows, k, layout, false, "gemv_q4_grouped_slots");
}

extern "C" int ft_hip_gemv_q4r_f32in(ft_hip_ctx* ctx, void* stream, const void* w, const float* x, float* y,
                                     float* act, int64_t n_rows, int64_t k) {
    clear_error();
    const char* nm = "gemv_q4r_f32in";
    if (k <= 0 || k % 32 || k > 32 * 8 * 64)
        return fail(FT_HIP_E_SHAPE, "%s: k=%lld must be a positive multiple of 32 up to 16384", nm, (long long)k);
    if (n_rows < 0 || n_rows > (1 << 30)) return fail(FT_HIP_E_SHAPE, "%s: n_rows out of range", nm);
    if (act && n_rows % 2) return fail(FT_HIP_E_SHAPE, "%s: a gate|up matrix (act given) has an even n_rows", nm);
    if (!ctx || !w || !x || !y) return fail(FT_HIP_E_INVALID, "%s: null argument", nm);
    if ((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(x)) & 15)
        return fail(FT_HIP_E_SHAPE, "%s: w and x must be 16-byte aligned", nm);
    if (n_rows == 0) return FT_HIP_OK;
    GemvArgs a{};
    a.base = (const uint8_t*)w;  // no slots: the one matrix at base
    a.x_div = 1;
    a.xf = x;
    a.y = y;
    a.act = act;
    a.y_stride = n_rows;
    a.n_rows = (int)n_rows;
    a.k = (int)k;
    const bool rec = ctx->rec_gu != nullptr;  // the block-dot record (tests)
    a.dots = ctx->rec_gu;
    const int nb = (int)(k / 32);
    // the lanes the q8-input GEMV takes for this shape (the same sums, bit for
    // bit), or where that is the 8-lane kernel, the fewest that hold the row;
    // with act (unless forced) 32 where the row fits: 8 rows, 4 columns per
    // workgroup, so the GELU tail runs on half as many workgroups (Gemma's
    // shared gate|up: 7.50 vs 8.16 us at 64 lanes)
    int lpr = short_lanes(ctx, FT_LAYOUT_Q4R, n_rows, 1, nb);
    if (act && !ctx->gemv_lanes && nb <= 8 * 32) lpr = 32;
    if (!lpr) lpr = nb <= 8 * 16 ? 16 : (nb <= 8 * 32 ? 32 : 64);
    const int nbl = (nb + lpr - 1) / lpr;
    const dim3 grid((unsigned)((n_rows + 256 / lpr - 1) / (256 / lpr)), 1);
    const size_t lds = (size_t)nb * Q8_BLK;
    if (lpr == 16) launch_short_f32in<16>(rec, act != nullptr, nbl, grid, lds, S(stream), a);
    else if (lpr == 32) launch_short_f32in<32>(rec, act != nullptr, nbl, grid, lds, S(stream), a);
    else launch_short_f32in<64>(rec, act != nullptr, nbl, grid, lds, S(stream), a);
    return launch_status(nm);
}

extern "C" int ft_hip_q4q8_block_dots(ft_hip_ctx* ctx, void* stream, const void* base, uint64_t expert_bytes,
                                      uint64_t bank_off, const int32_t* slots, const int32_t* x_idx, int64_t n_entries,
                                      const void* q8, int64_t q8_stride_blocks, int32_t* out, int64_t n_rows,
                                      int64_t k, int layout) {
    clear_error();
    GemvArgs a{};
    a.base = (const uint8_t*)base;
    a.expert_bytes = expert_bytes;
    a.slots = slots;
    a.bank_off = bank_off;
    a.x_idx = x_idx;
    a.x_div = 1;
    a.q8 = (const uint8_t*)q8;
    a.q8_stride_blocks = q8_stride_blocks;
    a.dots = out;
    return gemv_common(ctx, stream, a, n_entries, n_rows, k, layout, true, "q4q8_block_dots");
}

extern "C" int ft_hip_gelu_mul_q8(ft_hip_ctx* ctx, void* stream, const float* gu, void* q8, int64_t inter, int64_t n) {
    clear_error();
    if (inter <= 0 || inter % 32) return fail(FT_HIP_E_SHAPE, "gelu_mul_q8: inter=%lld must be a positive multiple of 32", (long long)inter);
    if (n < 0) return fail(FT_HIP_E_SHAPE, "gelu_mul_q8: negative n");
    if (!ctx || !gu || !q8) return fail(FT_HIP_E_INVALID, "gelu_mul_q8: null argument");
    if (n == 0) return FT_HIP_OK;
    const int64_t threads = n * (inter / 32) * 32;
    hipLaunchKernelGGL(k_gelu_mul_q8, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, S(stream), gu,
                       (uint8_t*)q8, (int)inter, n, (const float*)nullptr, 1);
    return launch_status("gelu_mul_q8");
}

static int act_mul_grouped(bool silu, ft_hip_ctx* ctx, void* stream, const float* gu, float* out, int64_t inter,
                           int64_t n, const char* nm) {
    if (inter <= 0) return fail(FT_HIP_E_SHAPE, "%s: inter=%lld must be positive", nm, (long long)inter);
    if (n < 0) return fail(FT_HIP_E_SHAPE, "%s: negative n_experts", nm);
    if (n > 0 && inter > ((int64_t)1 << 40) / n) return fail(FT_HIP_E_SHAPE, "%s: inter * n_experts too large", nm);
    if (!ctx || !gu || !out) return fail(FT_HIP_E_INVALID, "%s: null argument", nm);
    if (n == 0) return FT_HIP_OK;
    const int64_t total = n * inter;
    hipLaunchKernelGGL(silu ? k_act_mul_grouped<true> : k_act_mul_grouped<false>,
                       dim3((unsigned)((total + 255) / 256)), dim3(256), 0, S(stream), gu, out, inter, n);
    return launch_status(nm);
}

extern "C" int ft_hip_silu_mul_grouped(ft_hip_ctx* ctx, void* stream, const float* gu, float* out, int64_t inter,
                                       int64_t n_experts) {
    clear_error();
    return act_mul_grouped(true, ctx, stream, gu, out, inter, n_experts, "silu_mul_grouped");
}

extern "C" int ft_hip_gelu_mul_grouped(ft_hip_ctx* ctx, void* stream, const float* gu, float* out, int64_t inter,
                                       int64_t n_experts) {
    clear_error();
    return act_mul_grouped(false, ctx, stream, gu, out, inter, n_experts, "gelu_mul_grouped");
}

static int reduce_experts(bool weighted, ft_hip_ctx* ctx, void* stream, const float* y, const float* wts, float a,
                          float* out, int64_t hidden, int64_t n, const char* nm) {
    if (hidden <= 0 || hidden > ((int64_t)1 << 34)) return fail(FT_HIP_E_SHAPE, "%s: hidden out of range", nm);
    if (n < 0 || n > 65535) return fail(FT_HIP_E_SHAPE, "%s: n_experts not in [0, 65535]", nm);
    if (!ctx || !y || !out || (weighted && !wts)) return fail(FT_HIP_E_INVALID, "%s: null argument", nm);
    hipLaunchKernelGGL(weighted ? k_reduce_experts<true> : k_reduce_experts<false>,
                       dim3((unsigned)((hidden + 255) / 256)), dim3(256), 0, S(stream), y, wts, a, out, hidden,
                       (int)n);
    return launch_status(nm);
}

extern "C" int ft_hip_reduce_expert_weighted(ft_hip_ctx* ctx, void* stream, const float* y, const float* wts,
                                             float* out, int64_t hidden, int64_t n_experts) {
    clear_error();
    return reduce_experts(true, ctx, stream, y, wts, 0.0f, out, hidden, n_experts, "reduce_expert_weighted");
}

extern "C" int ft_hip_reduce_weighted(ft_hip_ctx* ctx, void* stream, const float* y, float* out, float a,
                                      int64_t hidden, int64_t n_experts) {
    clear_error();
    return reduce_experts(false, ctx, stream, y, nullptr, a, out, hidden, n_experts, "reduce_weighted");
}

extern "C" int ft_hip_router_logits(ft_hip_ctx* ctx, void* stream, const float* w, const float* x, const float* bias,
                                    float* y, int64_t dim, int64_t n_rows, int64_t n_seqs) {
    clear_error();
    if (dim <= 0 || dim % 128) return fail(FT_HIP_E_SHAPE, "router_logits: dim=%lld must be a positive multiple of 128", (long long)dim);
    if (dim > 65536) return fail(FT_HIP_E_SHAPE, "router_logits: dim=%lld exceeds 65536", (long long)dim);
    if (n_rows < 0 || n_seqs < 0 || n_rows > 65535 || n_seqs > 65535)
        return fail(FT_HIP_E_SHAPE, "router_logits: n_rows/n_seqs out of range");
    if (!ctx || !w || !x || !y) return fail(FT_HIP_E_INVALID, "router_logits: null argument");
    return ft::launch_router_logits(stream, w, x, bias, nullptr, y, dim, n_rows, n_seqs);
}

namespace ft {
int launch_router_logits(void* stream, const float* w, const float* x, const float* bias, const float* in_scale,
                         float* y, int64_t dim, int64_t n_rows, int64_t n_seqs) {
    if (n_rows == 0 || n_seqs == 0) return FT_HIP_OK;
    hipLaunchKernelGGL(k_router_logits, dim3((unsigned)n_rows, (unsigned)n_seqs), dim3(256), (size_t)(dim / 16) * 4,
                       S(stream), w, x, bias, in_scale, y, (int)dim, (int)n_rows);
    return launch_status("router_logits");
}

int launch_route_prep(void* stream, const float* w, const float* x, const float* bias, int norm, float* inv,
                      void* q8, float* y, int64_t dim, int64_t n_rows, int64_t n_seqs) {
    if (n_rows == 0 || n_seqs == 0) return FT_HIP_OK;
    // every q8 block needs a workgroup: rows >= ceil(blocks / 16)
    if (n_rows * 16 < dim / 32) return fail(FT_HIP_E_SHAPE, "route_prep: %lld rows cannot quantize %lld blocks",
                                            (long long)n_rows, (long long)(dim / 32));
    // batches: EG logits per workgroup (each chunk of x read once for them),
    // when the rows split into groups that still cover the q8 blocks at up to
    // 64 per workgroup: 8 from 32 seqs (measured faster at 64), 4 from 16
    const int eg = n_seqs >= 32 ? 8 : (n_seqs >= 16 ? 4 : 1);
    // from 32 seqs also 4 seqs per workgroup (the router read n_seqs/4
    // times), when that still makes at least 128 workgroups (256 at 64 seqs
    // of 128 experts: 65.8-66.8 vs 66.2-67.2 us/token on two boxes; at 16
    // seqs 2 per workgroup measured no faster)
    constexpr int sq = 4;
    if (eg == 8 && n_rows % eg == 0 && n_seqs % sq == 0 && (n_rows / eg) * (n_seqs / sq) >= 128) {
        const size_t lds = sizeof(float) * (size_t)sq * (eg + 1) * (dim / 16 + 1);
        auto kern = k_route_prep_m<8, sq>;
        hipLaunchKernelGGL(kern, dim3((unsigned)(n_rows / eg), (unsigned)(n_seqs / sq)), dim3(256), lds, S(stream), w,
                           x, bias, norm, inv, (uint8_t*)q8, y, (int)dim, (int)n_rows);
        return launch_status("route_prep_m");
    }
    if (eg > 1 && n_rows % eg == 0 && (n_rows / eg) * 64 >= dim / 32) {
        hipLaunchKernelGGL(eg == 8 ? k_route_prep_n<8> : k_route_prep_n<4>, dim3((unsigned)(n_rows / eg),
                           (unsigned)n_seqs), dim3(256), (size_t)(dim / 16) * (eg + 1) * 4, S(stream), w, x, bias,
                           norm, inv, (uint8_t*)q8, y, (int)dim, (int)n_rows);
        return launch_status("route_prep_n");
    }
    hipLaunchKernelGGL(k_route_prep, dim3((unsigned)n_rows, (unsigned)n_seqs), dim3(256), (size_t)(dim / 16) * 8,
                       S(stream), w, x, bias, norm, inv, (uint8_t*)q8, y, (int)dim, (int)n_rows);
    return launch_status("route_prep");
}

int launch_rms_inv(void* stream, const float* x, float* inv, int64_t dim, int64_t n_seqs) {
    if (n_seqs == 0) return FT_HIP_OK;
    hipLaunchKernelGGL(k_rms_inv, dim3((unsigned)n_seqs), dim3(256), (size_t)(dim / 16) * 4, S(stream), x, inv,
                       (int)dim);
    return launch_status("rms_inv");
}
}  // namespace ft

extern "C" int ft_hip_gemv_gate_up_act(ft_hip_ctx* ctx, void* stream, const void* base, uint64_t expert_bytes,
                                       const int32_t* slots, int64_t n_pairs, int64_t x_div, const void* q8x,
                                       int64_t hidden, int64_t inter, int layout, const float* in_scale,
                                       void* q8_act) {
    clear_error();
    const char* nm = "gemv_gate_up_act";
    if (hidden <= 0 || hidden % 32 || hidden > 32 * 4096)
        return fail(FT_HIP_E_SHAPE, "%s: hidden=%lld must be a positive multiple of 32 up to 131072", nm, (long long)hidden);
    if (inter <= 0 || inter % 32) return fail(FT_HIP_E_SHAPE, "%s: inter=%lld must be a positive multiple of 32", nm, (long long)inter);
    if (n_pairs < 0 || n_pairs > 65535 || x_div <= 0) return fail(FT_HIP_E_SHAPE, "%s: n_pairs or x_div out of range", nm);
    if (int rc = check_layout(layout)) return rc;
    if (layout == FT_LAYOUT_Q4R && ((reinterpret_cast<uintptr_t>(base) | expert_bytes) & 15))
        return fail(FT_HIP_E_SHAPE, "%s: q4r banks need 16-byte aligned base and expert_bytes", nm);
    if ((int64_t)expert_bytes < 2 * inter * row_bytes_of(layout, (int)hidden))
        return fail(FT_HIP_E_SHAPE, "%s: expert_bytes too small for the gate|up rows", nm);
    if (!ctx || !base || !slots || !q8x || !q8_act) return fail(FT_HIP_E_INVALID, "%s: null argument", nm);
    if (n_pairs == 0) return FT_HIP_OK;
    GemvArgs a{};
    a.base = (const uint8_t*)base;
    a.expert_bytes = expert_bytes;
    a.slots = slots;
    a.x_div = (int)x_div;
    a.q8 = (const uint8_t*)q8x;
    a.q8_stride_blocks = hidden / 32;
    a.n_rows = (int)(2 * inter);
    a.k = (int)hidden;
    // the layer record (tests): the gate|up sums and block dots of the pairs
    const bool rec = ctx->lrec.on;
    a.sums = ctx->lrec.gu;
    a.dots = ctx->lrec.gu_dots;
    const dim3 grid((unsigned)(inter / 32), (unsigned)n_pairs);
    const size_t lds = (size_t)(hidden / 32) * Q8_BLK;
    if (const int bpl = gu_long_bpl(layout, hidden)) {
        launch_gu_long<false, false>(bpl, grid, lds, S(stream), a, (int)inter, (uint8_t*)q8_act, in_scale, (int)x_div,
                                     nullptr, nullptr, nullptr, nullptr, 0, HeadArgs{}, rec);
        return launch_status(nm);
    }
    launch_gu_act<false, false>(layout, rec, grid, lds, S(stream), a, (int)inter, (uint8_t*)q8_act, in_scale,
                                (int)x_div, nullptr, nullptr, nullptr, nullptr, 0, HeadArgs{});
    return launch_status(nm);
}

extern "C" int ft_hip_topk_router(ft_hip_ctx* ctx, void* stream, const float* logits, const float* expert_scale,
                                  int32_t* ids, float* wts, int64_t e_count, int64_t k, int64_t n_seqs) {
    clear_error();
    if (e_count <= 0 || e_count > 1024) return fail(FT_HIP_E_SHAPE, "topk_router: e_count=%lld not in [1, 1024]", (long long)e_count);
    if (k <= 0 || k > 32 || k > e_count) return fail(FT_HIP_E_SHAPE, "topk_router: k=%lld not in [1, min(32, e_count)]", (long long)k);
    if (n_seqs < 0 || n_seqs > 65535) return fail(FT_HIP_E_SHAPE, "topk_router: n_seqs out of range");
    if (!ctx || !logits || !ids || !wts) return fail(FT_HIP_E_INVALID, "topk_router: null argument");
    if (n_seqs == 0) return FT_HIP_OK;
    hipLaunchKernelGGL(k_topk_router, dim3((unsigned)n_seqs), dim3(256), 0, S(stream), logits, expert_scale, ids, wts,
                       (int)e_count, (int)k);
    return launch_status("topk_router");
}

extern "C" int ft_hip_reduce_pairs_weighted(ft_hip_ctx* ctx, void* stream, const float* y, const float* wts,
                                            const int32_t* seq_of, float* out, int64_t hidden, int64_t n_pairs,
                                            int64_t n_seqs) {
    clear_error();
    if (hidden <= 0 || n_pairs < 0 || n_seqs < 0 || n_seqs > 65535 || hidden > (1 << 30))
        return fail(FT_HIP_E_SHAPE, "reduce_pairs_weighted: bad hidden/n_pairs/n_seqs");
    if (!ctx || !y || !wts || !seq_of || !out) return fail(FT_HIP_E_INVALID, "reduce_pairs_weighted: null argument");
    if (n_seqs == 0) return FT_HIP_OK;
    hipLaunchKernelGGL(k_reduce_pairs, dim3((unsigned)((hidden + 255) / 256), (unsigned)n_seqs), dim3(256), 0,
                       S(stream), y, wts, seq_of, out, (int)hidden, (int)n_pairs);
    return launch_status("reduce_pairs_weighted");
}

extern "C" int ft_hip_repack_rows(ft_hip_ctx* ctx, void* stream, const void* src, int src_layout, void* dst,
                                  int dst_layout, int64_t n_rows, int64_t k) {
    clear_error();
    if (k <= 0 || k % 32 || n_rows < 0) return fail(FT_HIP_E_SHAPE, "repack_rows: bad k or n_rows");
    if (int rc = check_layout(src_layout)) return rc;
    if (int rc = check_layout(dst_layout)) return rc;
    if (!ctx || !src || !dst) return fail(FT_HIP_E_INVALID, "repack_rows: null argument");
    if (n_rows == 0) return FT_HIP_OK;
    const int64_t threads = n_rows * (k / 32);
    hipLaunchKernelGGL(k_repack, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, S(stream),
                       (const uint8_t*)src, src_layout, (uint8_t*)dst, dst_layout, n_rows, (int)k);
    return launch_status("repack_rows");
}

extern "C" int ft_hip_stream_read(ft_hip_ctx* ctx, void* stream, const void* buf, uint64_t bytes, uint32_t* out,
                                  int n_workgroups) {
    clear_error();
    if (!ctx || !buf || !out) return fail(FT_HIP_E_INVALID, "stream_read: null argument");
    if (bytes % 16 || (reinterpret_cast<uintptr_t>(buf) & 15))
        return fail(FT_HIP_E_SHAPE, "stream_read: buf and bytes must be 16-byte aligned");
    if (n_workgroups <= 0 || n_workgroups > 65536)
        return fail(FT_HIP_E_SHAPE, "stream_read: n_workgroups=%d not in 1..65536", n_workgroups);
    if (bytes == 0) return FT_HIP_OK;
    hipLaunchKernelGGL(k_stream_read, dim3((unsigned)n_workgroups), dim3(256), 0, S(stream),
                       reinterpret_cast<const uint4*>(buf), bytes / 16, out);
    return launch_status("stream_read");
}

extern "C" int ft_hip_gen_values(ft_hip_ctx* ctx, void* stream, uint64_t key, int64_t start, int64_t n, float scale,
                                 float* out) {
    clear_error();
    if (n < 0 || start < 0) return fail(FT_HIP_E_SHAPE, "gen_values: negative n or start");
    if (!ctx || !out) return fail(FT_HIP_E_INVALID, "gen_values: null argument");
    if (n == 0) return FT_HIP_OK;
    hipLaunchKernelGGL(k_gen_values, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, S(stream), key, start, n, scale, out);
    return launch_status("gen_values");
}

extern "C" int ft_hip_gen_q4_rows(ft_hip_ctx* ctx, void* stream, uint64_t key, int64_t row0, int64_t n_rows, int64_t k,
                                  float scale, void* out, int layout) {
    clear_error();
    if (k <= 0 || k % 32 || n_rows < 0 || row0 < 0) return fail(FT_HIP_E_SHAPE, "gen_q4_rows: bad k, row0 or n_rows");
    if (int rc = check_layout(layout)) return rc;
    if (!ctx || !out) return fail(FT_HIP_E_INVALID, "gen_q4_rows: null argument");
    if (n_rows == 0) return FT_HIP_OK;
    const int64_t threads = n_rows * (k / 32);
    hipLaunchKernelGGL(k_gen_q4_rows, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, S(stream), key, row0,
                       n_rows, (int)k, scale, (uint8_t*)out, layout);
    return launch_status("gen_q4_rows");
}

// ---------------------------------------------------------------------------
// One layer through the launch-by-launch kernels.
// ---------------------------------------------------------------------------
struct LayerWs {
    float* logits;
    uint8_t* q8x;
    uint8_t* q8a;
    float* ydn;
    float* inv;         // [B] input RMS norm scales
    size_t bytes;
};

static LayerWs layer_ws(void* base, int64_t B, int64_t H, int64_t I, int64_t E, int64_t K) {
    auto up = [](size_t v) { return (v + 255) / 256 * 256; };
    size_t off = 0;
    LayerWs w{};
    uint8_t* p = (uint8_t*)base;
    w.logits = (float*)(p + off); off += up(sizeof(float) * B * E);
    w.q8x = p + off; off += up((size_t)B * (H / 32) * Q8_BLK);
    w.q8a = p + off; off += up((size_t)B * K * (I / 32) * Q8_BLK);
    w.ydn = (float*)(p + off); off += up(sizeof(float) * B * K * H);
    w.inv = (float*)(p + off); off += up(sizeof(float) * B);
    w.bytes = off;
    return w;
}

// The shapes a layer entry point accepts, checked by division so that no
// product below can overflow: at most 65535 (seq, expert) pairs, rows of at
// most 131072 weights, at most 1024 experts.
static bool layer_shape_in_range(int64_t n_seqs, int64_t hidden, int64_t inter, int64_t n_experts, int64_t top_k) {
    return n_seqs >= 0 && top_k > 0 && n_seqs <= 65535 / top_k && hidden > 0 && hidden <= 32 * 4096 && inter > 0 &&
           inter <= 32 * 4096 && n_experts > 0 && n_experts <= 1024;
}

extern "C" size_t ft_hip_moe_layer_workspace_bytes(int64_t n_seqs, int64_t hidden, int64_t inter, int64_t n_experts,
                                                   int64_t top_k) {
    if (!layer_shape_in_range(n_seqs, hidden, inter, n_experts, top_k)) return 0;
    return layer_ws(nullptr, n_seqs, hidden, inter, n_experts, top_k).bytes;
}

// The scratch of ft_hip_moe_layer_noalloc: every call on a device shares
// this array (its contents are whatever the last call left; the layer writes
// every byte it reads first, so nothing needs clearing). Host code never
// names it directly: the device address comes from hipGetSymbolAddress at
// ft_hip_create (scratch_setup) and is kept in the context.
static __device__ __align__(256) uint8_t scratch[FT_HIP_NOALLOC_SCRATCH_BYTES];

namespace ft {
int scratch_setup(ft_hip_ctx* ctx) {
    // called by ft_hip_create with ctx->device current
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
        return fail(FT_HIP_E_DEVICE, "create: no address for the no-alloc scratch on device %d (%s)", ctx->device,
                    hipGetErrorString(e));
    ctx->noalloc_scratch = ptr;
    return FT_HIP_OK;
}
}  // namespace ft

// Lanes per row of the down launch with the combine (k_gemv_down_combine):
// 16 for rows of at least 256 blocks when k divides 16, else 8.
static int down_lanes(int64_t inter, int64_t top_k) { return inter / 32 >= 256 && 16 % top_k == 0 ? 16 : 8; }

// Whether a stack of layers can take each layer's head from the previous
// layer's down launch (k_gemv_down_head, then k_gemv_gu_act<HEAD>): the top-k
// runs in the gate|up launch, the down launch is the combined one, 16 rows
// of every pair (16*k*lanes threads) plus the E+1 partials fit one
// workgroup, and the gate|up launch's q8 row and partials fit 32 KB of LDS.
static bool head_fold_ok(int64_t hidden, int64_t inter, int64_t n_experts, int64_t top_k) {
    if (n_experts > 256 || 32 % top_k || top_k * (inter / 32) * Q8_BLK > 64 * 1024) return false;
    if ((hidden / 32) * Q8_BLK + (hidden / 16) * (n_experts + 1) * 4 > 32 * 1024) return false;  // the gate|up LDS
    const int64_t nt = 16 * top_k * down_lanes(inter, top_k);
    return nt >= 256 && nt <= 1024 && n_experts < nt;
}

// k_gemv_down_head for nt = 16*k*LPR threads (256, 512 or 1024)
template <int LAYOUT, int LPR, bool REC>
static void launch_down_head_r(int nt, dim3 grid, size_t lds, hipStream_t st, const GemvArgs& a, const float* wts,
                               const float* x, float* out, int k, const float* wnext, float* part, int E) {
    if (nt == 256)
        hipLaunchKernelGGL((k_gemv_down_head<LAYOUT, LPR, 256, REC>), grid, dim3(256), lds, st, a, wts, x, out, k,
                           wnext, part, E);
    else if (nt == 512)
        hipLaunchKernelGGL((k_gemv_down_head<LAYOUT, LPR, 512, REC>), grid, dim3(512), lds, st, a, wts, x, out, k,
                           wnext, part, E);
    else
        hipLaunchKernelGGL((k_gemv_down_head<LAYOUT, LPR, 1024, REC>), grid, dim3(1024), lds, st, a, wts, x, out, k,
                           wnext, part, E);
}
template <int LAYOUT, int LPR>
static void launch_down_head(bool rec, int nt, dim3 grid, size_t lds, hipStream_t st, const GemvArgs& a,
                             const float* wts, const float* x, float* out, int k, const float* wnext, float* part,
                             int E) {
    if (rec) launch_down_head_r<LAYOUT, LPR, true>(nt, grid, lds, st, a, wts, x, out, k, wnext, part, E);
    else launch_down_head_r<LAYOUT, LPR, false>(nt, grid, lds, st, a, wts, x, out, k, wnext, part, E);
}

// Test record of one layer of the launch-by-launch path (ft_hip_set_layer_record):
// where this layer's records go, or all null.
struct LayerRecPtrs {
    bool on;
    float* x;
    uint8_t* q8x;
    float* gu;
    uint8_t* act;
    int32_t* gu_dots;
    int32_t* dn_dots;
};

// Layer l's slice of the context's layer record for n_seqs seqs of top_k pairs.
static LayerRecPtrs layer_rec(const ft_hip_ctx* ctx, int64_t l, int64_t B, int64_t H, int64_t I, int64_t K) {
    const LayerRecord& r = ctx->lrec;
    LayerRecPtrs p{};
    p.on = r.on;
    if (!r.on) return p;
    const int64_t P = B * K;
    auto off = [&](auto* base, int64_t per) { return base ? base + l * per : nullptr; };
    p.x = off(r.x, B * H);
    p.q8x = off(r.q8x, B * (H / 32) * Q8_BLK);
    p.gu = off(r.gu, P * 2 * I);
    p.act = off(r.act, P * (I / 32) * Q8_BLK);
    p.gu_dots = off(r.gu_dots, P * 2 * I * (H / 32));
    p.dn_dots = off(r.dn_dots, P * H * (I / 32));
    return p;
}

// One layer of the launch-by-launch path. In a stack (head_fold_ok): part_in
// set = this layer's head comes from the partials the previous down launch
// left in part_in (no head launch; k_gemv_gu_act<HEAD>); wnext set = the down
// launch also writes the next layer's partials (router rows wnext) to
// part_out. Either way the bits are those of the plain layer.
static int moe_layer_impl(const char* nm, ft_hip_ctx* ctx, void* stream, const float* x, float* x_out,
                          int64_t n_seqs, int64_t hidden, int64_t inter, int64_t n_experts, int64_t top_k,
                          const float* router_w, const float* router_bias, const float* expert_scale,
                          const void* bank, uint64_t expert_bytes, int layout, int32_t* ids, float* wts,
                          void* workspace, size_t workspace_bytes, const float* part_in = nullptr,
                          const float* wnext = nullptr, float* part_out = nullptr,
                          const LayerRecPtrs& rec = LayerRecPtrs{}) {
    if (hidden <= 0 || hidden % 128) return fail(FT_HIP_E_SHAPE, "%s: hidden=%lld must be a positive multiple of 128", nm, (long long)hidden);
    if (inter <= 0 || inter % 32) return fail(FT_HIP_E_SHAPE, "%s: inter=%lld must be a positive multiple of 32", nm, (long long)inter);
    if (n_experts <= 0 || n_experts > 1024) return fail(FT_HIP_E_SHAPE, "%s: n_experts not in [1, 1024]", nm);
    if (top_k <= 0 || top_k > 32 || top_k > n_experts) return fail(FT_HIP_E_SHAPE, "%s: top_k not in [1, min(32, n_experts)]", nm);
    // by division: a product of a huge n_seqs could wrap
    if (n_seqs < 0 || n_seqs > 65535 / top_k) return fail(FT_HIP_E_SHAPE, "%s: n_seqs out of range", nm);
    if (int rc = check_layout(layout)) return rc;
    const int64_t gu_bytes = 2 * inter * row_bytes_of(layout, (int)hidden);
    const int64_t need = gu_bytes + hidden * row_bytes_of(layout, (int)inter);
    if ((int64_t)expert_bytes < need) return fail(FT_HIP_E_SHAPE, "%s: expert_bytes=%llu < %lld", nm, (unsigned long long)expert_bytes, (long long)need);
    const LayerWs w = layer_ws(workspace, n_seqs, hidden, inter, n_experts, top_k);
    if (workspace_bytes < w.bytes) return fail(FT_HIP_E_SHAPE, "%s: workspace_bytes=%zu < %zu", nm, workspace_bytes, w.bytes);
    if (!ctx || !x || !x_out || !router_w || !bank || !ids || !wts || !workspace) return fail(FT_HIP_E_INVALID, "%s: null argument", nm);
    if (hidden > 32 * 4096 || inter > 32 * 4096) return fail(FT_HIP_E_SHAPE, "%s: rows longer than 131072", nm);
    if (layout == FT_LAYOUT_Q4R && ((reinterpret_cast<uintptr_t>(bank) | expert_bytes | (uint64_t)gu_bytes) & 15))
        return fail(FT_HIP_E_SHAPE, "%s: q4r banks need 16-byte aligned base and expert_bytes", nm);
    if (n_seqs == 0) return FT_HIP_OK;
    int rc;
    hipStream_t st = S(stream);
    // test record: this layer's input as read, then (below) q8(x) and the activations
    if (rec.x && hipMemcpyAsync(rec.x, x, sizeof(float) * n_seqs * hidden, hipMemcpyDeviceToDevice, st) != hipSuccess)
        return launch_status("moe_layer/record");
    const float* inv = ctx->input_norm ? w.inv : nullptr;
    if ((part_in || wnext) && !head_fold_ok(hidden, inter, n_experts, top_k))
        return fail(FT_HIP_E_SHAPE, "%s: this shape cannot take the layer head from the down launch", nm);
    if (part_in) {
        // the head was computed by the previous layer's down launch
    } else if (n_experts * 16 >= hidden / 32) {  // logits, norm scale and q8(x) in one launch
        if ((rc = ft::launch_route_prep(stream, router_w, x, router_bias, ctx->input_norm, w.inv, w.q8x, w.logits,
                                        hidden, n_experts, n_seqs)))
            return rc;
    } else {
        if (inv && (rc = ft::launch_rms_inv(stream, x, w.inv, hidden, n_seqs))) return rc;
        if ((rc = ft::launch_router_logits(stream, router_w, x, router_bias, inv, w.logits, hidden, n_experts, n_seqs)))
            return rc;
        if ((rc = ft_hip_quantize_q8(ctx, stream, x, hidden, w.q8x, hidden, n_seqs))) return rc;
    }
    if (!part_in && rec.q8x &&
        hipMemcpyAsync(rec.q8x, w.q8x, (size_t)n_seqs * (hidden / 32) * Q8_BLK, hipMemcpyDeviceToDevice, st) !=
            hipSuccess)
        return launch_status("moe_layer/record");
    // top-k in the gate|up launch when the logits fit one thread each
    const bool topk_in = n_experts <= 256;
    if (!topk_in && (rc = ft_hip_topk_router(ctx, stream, w.logits, expert_scale, ids, wts, n_experts, top_k, n_seqs)))
        return rc;
    const int64_t n_pairs = n_seqs * top_k;
    GemvArgs a{};
    a.base = (const uint8_t*)bank;
    a.expert_bytes = expert_bytes;
    a.slots = ids;
    a.bank_off = 0;
    a.x_idx = nullptr;
    a.x_div = (int)top_k;  // pair p reads token p / top_k
    a.q8 = w.q8x;
    a.q8_stride_blocks = hidden / 32;
    // gate|up with GELU*up and q8 (one launch), then down with the combine
    // (one launch when the k activation rows of a seq fit in LDS together)
    a.n_rows = (int)(2 * inter);
    a.k = (int)hidden;
    const dim3 g_gu((unsigned)(inter / 32), (unsigned)n_pairs);
    const size_t l_gu = (size_t)(hidden / 32) * Q8_BLK;
    const int gbpl = gu_long_bpl(layout, hidden);
    a.sums = rec.gu;
    a.dots = rec.gu_dots;
    a.x8rec = rec.q8x;
    if (part_in) {
        const HeadArgs h{x, part_in, router_bias, ctx->input_norm};
        const size_t l_head = l_gu + (size_t)(hidden / 16) * (n_experts + 1) * 4;
        if (gbpl)
            launch_gu_long<true, true>(gbpl, g_gu, l_head, st, a, (int)inter, w.q8a, nullptr, (int)top_k, nullptr,
                                       expert_scale, ids, wts, (int)n_experts, h, rec.on);
        else
            launch_gu_act<true, true>(layout, rec.on, g_gu, l_head, st, a, (int)inter, w.q8a, nullptr, (int)top_k,
                                      nullptr, expert_scale, ids, wts, (int)n_experts, h);
    } else if (gbpl) {
        if (topk_in)
            launch_gu_long<true, false>(gbpl, g_gu, l_gu, st, a, (int)inter, w.q8a, inv, (int)top_k, w.logits,
                                        expert_scale, ids, wts, (int)n_experts, HeadArgs{}, rec.on);
        else
            launch_gu_long<false, false>(gbpl, g_gu, l_gu, st, a, (int)inter, w.q8a, inv, (int)top_k, w.logits,
                                         expert_scale, ids, wts, (int)n_experts, HeadArgs{}, rec.on);
    } else if (topk_in) {
        launch_gu_act<true, false>(layout, rec.on, g_gu, l_gu, st, a, (int)inter, w.q8a, inv, (int)top_k, w.logits,
                                   expert_scale, ids, wts, (int)n_experts, HeadArgs{});
    } else {
        launch_gu_act<false, false>(layout, rec.on, g_gu, l_gu, st, a, (int)inter, w.q8a, inv, (int)top_k, w.logits,
                                    expert_scale, ids, wts, (int)n_experts, HeadArgs{});
    }
    if ((rc = launch_status("moe_layer/gate_up_act"))) return rc;
    a.sums = nullptr;
    a.x8rec = nullptr;
    a.dots = rec.dn_dots;
    if (rec.act && hipMemcpyAsync(rec.act, w.q8a, (size_t)n_pairs * (inter / 32) * Q8_BLK, hipMemcpyDeviceToDevice,
                                  st) != hipSuccess)
        return launch_status("moe_layer/record");
    a.bank_off = (uint64_t)gu_bytes;
    a.x_div = 1;
    a.q8 = w.q8a;
    a.q8_stride_blocks = inter / 32;
    a.y = w.ydn;
    a.y_stride = hidden;
    const size_t l_dn = (size_t)top_k * (inter / 32) * Q8_BLK;
    if (wnext) {  // head_fold_ok: 16 rows of every pair per workgroup, then the next layer's partials
        a.n_rows = (int)hidden;
        a.k = (int)inter;
        const int lpr = down_lanes(inter, top_k), nt = (int)(16 * top_k * lpr);
        const dim3 g_dn((unsigned)(hidden / 16), (unsigned)n_seqs);
        auto launch = layout == FT_LAYOUT_Q4R
                          ? (lpr == 16 ? launch_down_head<FT_LAYOUT_Q4R, 16> : launch_down_head<FT_LAYOUT_Q4R, 8>)
                          : (lpr == 16 ? launch_down_head<FT_LAYOUT_Q4_0, 16> : launch_down_head<FT_LAYOUT_Q4_0, 8>);
        launch(rec.on, nt, g_dn, l_dn, st, a, wts, x, x_out, (int)top_k, wnext, part_out, (int)n_experts);
        return launch_status("moe_layer/down_head");
    }
    if (32 % top_k == 0 && l_dn <= 64 * 1024) {
        a.n_rows = (int)hidden;
        a.k = (int)inter;
        // 16 lanes per row for long rows (at least 256 blocks) when k divides 16
        const bool l16 = down_lanes(inter, top_k) == 16;
        const int R = (int)((l16 ? 16 : 32) / top_k);
        const dim3 g_dn((unsigned)((hidden + R - 1) / R), (unsigned)n_seqs);
        auto kern = layout == FT_LAYOUT_Q4R
                        ? (l16 ? (rec.on ? k_gemv_down_combine<FT_LAYOUT_Q4R, 16, true>
                                         : k_gemv_down_combine<FT_LAYOUT_Q4R, 16, false>)
                               : (rec.on ? k_gemv_down_combine<FT_LAYOUT_Q4R, 8, true>
                                         : k_gemv_down_combine<FT_LAYOUT_Q4R, 8, false>))
                        : (l16 ? (rec.on ? k_gemv_down_combine<FT_LAYOUT_Q4_0, 16, true>
                                         : k_gemv_down_combine<FT_LAYOUT_Q4_0, 16, false>)
                               : (rec.on ? k_gemv_down_combine<FT_LAYOUT_Q4_0, 8, true>
                                         : k_gemv_down_combine<FT_LAYOUT_Q4_0, 8, false>));
        hipLaunchKernelGGL(kern, g_dn, dim3(256), l_dn, st, a, (const float*)wts, x, x_out, (int)top_k);
        return launch_status("moe_layer/down_combine");
    }
    if (rec.dn_dots) {  // the record instantiation of the grouped GEMV, dots to the layer record
        a.n_rows = (int)hidden;
        a.k = (int)inter;
        const dim3 g_dn((unsigned)((hidden + 31) / 32), (unsigned)n_pairs);
        const size_t l_q8 = (size_t)(inter / 32) * Q8_BLK;
        hipLaunchKernelGGL((layout == FT_LAYOUT_Q4R ? k_gemv_q4_grouped<FT_LAYOUT_Q4R, true>
                                                    : k_gemv_q4_grouped<FT_LAYOUT_Q4_0, true>),
                           g_dn, dim3(256), l_q8, st, a);
        if ((rc = launch_status("moe_layer/down"))) return rc;
    } else {
        a.dots = nullptr;
        if ((rc = gemv_common(ctx, stream, a, n_pairs, hidden, inter, layout, false, "moe_layer/down"))) return rc;
    }
    hipLaunchKernelGGL(k_combine_residual, dim3((unsigned)((hidden + 255) / 256), (unsigned)n_seqs), dim3(256), 0,
                       S(stream), w.ydn, wts, x, x_out, (int)hidden, (int)top_k);
    return launch_status("moe_layer/combine");
}

extern "C" int ft_hip_moe_layer(ft_hip_ctx* ctx, void* stream, const float* x, float* x_out, int64_t n_seqs,
                                int64_t hidden, int64_t inter, int64_t n_experts, int64_t top_k,
                                const float* router_w, const float* router_bias, const float* expert_scale,
                                const void* bank, uint64_t expert_bytes, int layout, int32_t* ids, float* wts,
                                void* workspace, size_t workspace_bytes) {
    clear_error();
    // (shape errors are reported before a null context: the record is read only with one)
    return moe_layer_impl("moe_layer", ctx, stream, x, x_out, n_seqs, hidden, inter, n_experts, top_k, router_w,
                          router_bias, expert_scale, bank, expert_bytes, layout, ids, wts, workspace, workspace_bytes,
                          nullptr, nullptr, nullptr,
                          ctx ? layer_rec(ctx, 0, n_seqs, hidden, inter, top_k) : LayerRecPtrs{});
}

extern "C" int ft_hip_moe_layer_noalloc(ft_hip_ctx* ctx, void* stream, const float* x, float* x_out,
                                        int64_t n_seqs, int64_t hidden, int64_t inter, int64_t n_experts,
                                        int64_t top_k, const float* router_w, const float* router_bias,
                                        const float* expert_scale, const void* bank, uint64_t expert_bytes,
                                        int layout, int32_t* ids, float* wts) {
    clear_error();
    const char* nm = "moe_layer_noalloc";
    if (!ctx) return fail(FT_HIP_E_INVALID, "%s: null ctx", nm);
    if (!ctx->noalloc_scratch) return fail(FT_HIP_E_DEVICE, "%s: the context has no scratch address", nm);
    if (!layer_shape_in_range(n_seqs, hidden, inter, n_experts, top_k))
        return fail(FT_HIP_E_SHAPE, "%s: n_seqs=%lld hidden=%lld inter=%lld n_experts=%lld top_k=%lld out of range", nm,
                    (long long)n_seqs, (long long)hidden, (long long)inter, (long long)n_experts, (long long)top_k);
    const size_t need = ft_hip_moe_layer_workspace_bytes(n_seqs, hidden, inter, n_experts, top_k);
    if (need > (size_t)FT_HIP_NOALLOC_SCRATCH_BYTES)
        return fail(FT_HIP_E_SHAPE,
                    "%s: n_seqs=%lld hidden=%lld inter=%lld n_experts=%lld top_k=%lld needs %zu bytes of scratch; "
                    "this entry point holds %d (use ft_hip_moe_layer with a workspace)",
                    nm, (long long)n_seqs, (long long)hidden, (long long)inter, (long long)n_experts,
                    (long long)top_k, need, FT_HIP_NOALLOC_SCRATCH_BYTES);
    return moe_layer_impl(nm, ctx, stream, x, x_out, n_seqs, hidden, inter, n_experts, top_k, router_w, router_bias,
                          expert_scale, bank, expert_bytes, layout, ids, wts, ctx->noalloc_scratch,
                          (size_t)FT_HIP_NOALLOC_SCRATCH_BYTES, nullptr, nullptr, nullptr,
                          layer_rec(ctx, 0, n_seqs, hidden, inter, top_k));
}

// Workspace of ft_hip_moe_stack: a layer's, the two states between layers and
// the head partials [n_seqs][H/16][E+1].
struct StackLayerWs {
    size_t layer_bytes;
    float* state[2];
    float* part;
    size_t bytes;
};

static StackLayerWs stack_layer_ws(void* base, int64_t B, int64_t H, int64_t I, int64_t E, int64_t K) {
    auto up = [](size_t v) { return (v + 255) / 256 * 256; };
    StackLayerWs w{};
    uint8_t* p = (uint8_t*)base;
    size_t off = layer_ws(nullptr, B, H, I, E, K).bytes;
    w.layer_bytes = off;
    for (int i = 0; i < 2; ++i) {
        w.state[i] = (float*)(p + off);
        off += up(sizeof(float) * B * H);
    }
    w.part = (float*)(p + off);
    off += up(sizeof(float) * B * (H / 16) * (E + 1));
    w.bytes = off;
    return w;
}

extern "C" size_t ft_hip_moe_stack_workspace_bytes(int64_t n_seqs, int64_t hidden, int64_t inter, int64_t n_experts,
                                                   int64_t top_k) {
    if (!layer_shape_in_range(n_seqs, hidden, inter, n_experts, top_k) || hidden % 16) return 0;
    return stack_layer_ws(nullptr, n_seqs, hidden, inter, n_experts, top_k).bytes;
}

extern "C" int ft_hip_moe_stack(ft_hip_ctx* ctx, void* stream, const float* x_in, float* x_out, int64_t n_seqs,
                                int64_t hidden, int64_t inter, int64_t n_experts, int64_t top_k, int64_t n_layers,
                                const float* routers, const float* router_bias, const float* expert_scale,
                                const void* banks, uint64_t expert_bytes, int layout, int32_t* ids, float* wts,
                                void* workspace, size_t workspace_bytes) {
    clear_error();
    const char* nm = "moe_stack";
    if (n_layers <= 0) return fail(FT_HIP_E_SHAPE, "%s: n_layers must be positive", nm);
    if (!ctx || !x_in || !x_out || !routers || !banks || !ids || !wts || !workspace)
        return fail(FT_HIP_E_INVALID, "%s: null argument", nm);
    if (hidden <= 0 || hidden % 128 || n_experts <= 0 || top_k <= 0 || n_seqs < 0)
        return fail(FT_HIP_E_SHAPE, "%s: hidden=%lld n_experts=%lld top_k=%lld n_seqs=%lld", nm, (long long)hidden,
                    (long long)n_experts, (long long)top_k, (long long)n_seqs);
    const StackLayerWs sw = stack_layer_ws(workspace, n_seqs, hidden, inter, n_experts, top_k);
    if (workspace_bytes < sw.bytes)
        return fail(FT_HIP_E_SHAPE, "%s: workspace_bytes=%zu < %zu", nm, workspace_bytes, sw.bytes);
    if (n_seqs == 0) return FT_HIP_OK;
    const bool fold = head_fold_ok(hidden, inter, n_experts, top_k);
    const int64_t per = n_seqs * top_k;
    for (int64_t l = 0; l < n_layers; ++l) {
        const float* xl = l == 0 ? x_in : sw.state[(l - 1) & 1];
        float* out = l == n_layers - 1 ? x_out : sw.state[l & 1];
        const bool last = l == n_layers - 1;
        const uint8_t* bank = (const uint8_t*)banks + (uint64_t)l * n_experts * expert_bytes;
        if (int rc = moe_layer_impl(nm, ctx, stream, xl, out, n_seqs, hidden, inter, n_experts, top_k,
                                    routers + l * n_experts * hidden, router_bias ? router_bias + l * n_experts : nullptr,
                                    expert_scale ? expert_scale + l * n_experts : nullptr, bank, expert_bytes, layout,
                                    ids + l * per, wts + l * per, workspace, sw.layer_bytes,
                                    fold && l > 0 ? sw.part : nullptr,
                                    fold && !last ? routers + (l + 1) * n_experts * hidden : nullptr,
                                    fold && !last ? sw.part : nullptr, layer_rec(ctx, l, n_seqs, hidden, inter, top_k)))
            return rc;
    }
    return FT_HIP_OK;
}
