// ft_hip_fused.hip -- the whole MoE expert-FFN section of an L-layer stack for
// one decode token in ONE persistent, cooperatively launched kernel.
//
// Why one kernel: at batch 1 a Gemma-shaped layer streams only ~28 MB, i.e.
// ~4.6 us at the MI355X's achievable HBM rate, while every kernel boundary
// costs several us. The layer is therefore run as dataflow between resident
// workgroups. Its all-to-all dependencies (gate|up -> down; down -> router
// chunk partials -> logits -> top-k) are handed over through single-writer,
// epoch-tagged 64-bit words in device memory: bits 63..32 = epoch tag,
// bits 31..0 = payload. Producers write with device-coherent (agent-scope)
// relaxed stores; consumers read with device-coherent loads, keep the words
// that already carry the expected tag and re-read only the missing ones.
// Data and flag travel in the same word, so a hand-over costs one memory
// round trip once the producer is done, with no read-modify-write contention
// and no cache-maintenance fences (the alternatives measured 1.4-20 us per
// barrier on this part).
//
// Work of one layer (G shape: H 2816, I 704, top-8), 176 workgroups:
//   gate|up units : (routed expert p, 32 output columns jb) -> 64 rows (32
//                   gate, 32 up) x H/32 blocks streamed into registers by 8
//                   waves; GELU*up -> one q8 block published.
//   down units    : 16 output rows x the K routed experts, weights prefetched
//                   into LDS (global_load_lds); combine x_{l+1} = x_l + sum_p
//                   w_p y_p in pair order; router chunk partials of layer l+1
//                   over those 16 rows (R-order) and the 16 x values published.
//   logit units   : 16 experts each: R-order sums of all chunk partials (+bias)
//                   -> 16 final logits published.
//   every WG      : reads the logits, rank-based top-k and softmax; gate|up
//                   workgroups read x_{l+1} and quantize it while the logits
//                   are still being reduced.
// Weight layouts are lossless repacks of q4_0 with exactly q4_0's byte count.

#include "ft_device.hpp"
#include "ft_runtime.hpp"

using namespace ft;

namespace {

constexpr int FT_THREADS = 512;
constexpr int FT_WAVES = FT_THREADS / 64;
constexpr int GU_BPW_MAX = 16;  // gate|up blocks per wave held in flight (H <= 4096)
constexpr int MAX_K = 8;
constexpr int MAX_E = 512;
constexpr int DN_ROWS = 16;     // rows per down tile / router chunk
constexpr int WAIT_U = 8;       // tagged words per thread per wait (n <= 4096)
constexpr int POLL_SLEEP = 1;   // s_sleep units (64 clocks) between polls
constexpr int NREP = 8;         // replicas of each broadcast buffer: one per XCD, so each
                                // copy is polled by ~1/8 of the workgroups
constexpr int CTL_EPOCH = 0;    // control words (u32 indices)
constexpr int CTL_ABORT = 32;
constexpr int TRACE_SLOTS = 32; // stamps per workgroup per layer in the debug trace

struct FusedParams {
    const uint8_t* banks;       // [L][E][expert_bytes], fused layout
    const float* routers;       // [L][H/16][E][16]
    const float* bias;          // [L][E] or null
    const float* escale;        // [L][E] or null
    const float* x_in;          // [H]
    float* x_out;               // [H]
    int32_t* ids_out;           // [L][K] or null
    float* wts_out;             // [L][K] or null
    uint64_t* act_t;            // tagged [NREP][K][I/32][10]
    uint64_t* x_t;              // tagged [NREP][H]
    uint64_t* part_t;           // tagged [H/16][E]
    uint64_t* lg_t;             // tagged [NREP][E]
    int64_t rs_act, rs_x, rs_lg;  // replica strides (words)
    uint32_t* ctl;              // [CTL_EPOCH] epoch, [CTL_ABORT] abort epoch
    float* dbg_gu;              // [L][K][2I] or null
    uint8_t* dbg_act;           // [L][K][I/32][40] or null
    float* dbg_x;               // [L+1][H] or null
    uint64_t* trace;            // [grid][L+1][16] wall-clock stamps or null
    int64_t expert_bytes, gu_bytes;
    int H, I, E, K, L;
    int n_gu, n_dn, n_red;
    int spin_limit;
    int o_x, o_q8x, o_act8, o_wr, o_red, o_misc, lds_bytes;
};

struct Misc {
    float logits[MAX_E];
    float y[MAX_K][DN_ROWS];
    float xrow[DN_ROWS];
    float xnew[DN_ROWS];
    float gsum[64];
    float G[8 * 16];
    float act[32];
    uint32_t actblk[10];
    float sel_v[MAX_K];
    int sel_i[MAX_K];
    int ids[MAX_K];
    float wts[MAX_K];
    int abort_flag;
};

// Orders LDS accesses between lanes of ONE wave (LDS operations of a wave
// execute in issue order; this only stops the compiler from reordering them).
__device__ __forceinline__ void wave_lds_order() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    asm volatile("" ::: "memory");
}

__device__ __forceinline__ uint64_t ld_tag(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_tag(uint64_t* p, uint32_t tag, uint32_t v) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_ctl(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Block-wide wait until the n (<= 4096) tagged words src[idx(i)] all carry
// `tag`; payloads land in dst[i] (LDS). Each thread re-reads only its words
// still missing, so a consumer that arrives early costs little traffic.
// Bounded: after spin_limit polls (or when another workgroup has aborted) it
// records the abort and returns false.
template <typename Idx, typename DIdx>
__device__ bool wait_words(const FusedParams& P, Misc* m, uint32_t epoch, const uint64_t* src, int n, Idx idx,
                           uint32_t tag, uint32_t* dst, DIdx didx) {
    // An opaque copy of the thread index: keeps the compiler from hoisting the
    // per-call-site address arithmetic out of the layer loop, where it would
    // stay live (in registers) for the whole kernel.
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    uint32_t pending = 0;
#pragma unroll
    for (int u = 0; u < WAIT_U; ++u)
        if (u * FT_THREADS + tid < n) pending |= 1u << u;
    for (int it = 0;; ++it) {
        uint64_t v[WAIT_U];
#pragma unroll
        for (int u = 0; u < WAIT_U; ++u)
            v[u] = (pending >> u) & 1 ? ld_tag(src + idx(u * FT_THREADS + tid)) : 0;
#pragma unroll
        for (int u = 0; u < WAIT_U; ++u)
            if (((pending >> u) & 1) && (uint32_t)(v[u] >> 32) == tag) {
                dst[didx(u * FT_THREADS + tid)] = (uint32_t)v[u];
                pending &= ~(1u << u);
            }
        if (__syncthreads_and(pending == 0)) return true;
        if ((it & 63) == 63) {
            if (threadIdx.x == 0) {
                const bool ab = ld_ctl(P.ctl + CTL_ABORT) == epoch || it >= P.spin_limit;
                if (ab) __hip_atomic_store(P.ctl + CTL_ABORT, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                m->abort_flag = ab;
            }
            __syncthreads();
            if (m->abort_flag) return false;
        }
        __builtin_amdgcn_s_sleep(POLL_SLEEP);
    }
}

template <typename Idx>
__device__ __forceinline__ bool wait_words(const FusedParams& P, Misc* m, uint32_t epoch, const uint64_t* src, int n,
                                           Idx idx, uint32_t tag, uint32_t* dst) {
    return wait_words(P, m, epoch, src, n, idx, tag, dst, [](int i) { return i; });
}

__device__ __forceinline__ void stamp(const FusedParams& P, int l, int ev) {
    if (P.trace && threadIdx.x == 0)
        P.trace[((int64_t)blockIdx.x * (P.L + 1) + (l + 1)) * TRACE_SLOTS + ev] = wall_clock64();
}
// shader-clock stamp (slots 4 and 8): with the wall-clock slots it gives the
// effective core clock over a layer
__device__ __forceinline__ void stamp_clk(const FusedParams& P, int l, int ev) {
    if (P.trace && threadIdx.x == 0)
        P.trace[((int64_t)blockIdx.x * (P.L + 1) + (l + 1)) * TRACE_SLOTS + ev] = clock64();
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

// A lane quad quantizes one 32-value block to q8 {d, qsum, qs[32]}
// (ft-core/src/q4_0.rs:62-78; the same arithmetic as q8_quantize_half): lane
// part (0..3) owns values 8*part..8*part+7 and writes output words 2+2*part
// and 3+2*part; part 0 also writes d and qsum. All four lanes must be active.
__device__ __forceinline__ void quantize_block_quad(const float* v, int part, uint32_t* out) {
    const float4 a = reinterpret_cast<const float4*>(v)[2 * part];
    const float4 b = reinterpret_cast<const float4*>(v)[2 * part + 1];
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
        r = fminf(127.0f, fmaxf(-127.0f, r));
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

// q8-quantize x (H floats in LDS) into LDS blocks, one lane quad per block.
__device__ void quantize_x_lds(const FusedParams& P, const float* x, uint8_t* q8x) {
    const int nb = P.H >> 5;
    for (int base = 0; base < nb * 4; base += FT_THREADS) {
        const int i = base + threadIdx.x;
        const int b = min(i >> 2, nb - 1);  // surplus quads redo the last block (same values)
        quantize_block_quad(x + 32 * b, i & 3, reinterpret_cast<uint32_t*>(q8x + b * Q8_BLK));
    }
}

// Top-k by rank over logits in LDS (rank = number of logits that sort before:
// larger, or equal with a lower index, as the stable descending sort of
// ft-model/src/lib.rs:1491-1492; NaN sorts after every number, where the
// reference would panic), then softmax over the chosen
// (ft-model/src/lib.rs:1494-1503): exp(l - l_max), summed in rank order.
// Four threads share one logit's comparisons (E <= 512, E % 16 == 0). LDS
// reads are issued in batches of 8 float4 so that one wait covers them, and
// the softmax runs in wave 0 from registers.
__device__ __forceinline__ bool sorts_before(float u, int j, float v, int i, bool v_nan) {
    return (u > v) || (u == v && j < i) || (v_nan && (!(u == u) ? j < i : true));
}

__device__ void topk_rank(const FusedParams& P, Misc* m, int layer) {
    const int E = P.E, K = P.K, t = threadIdx.x;
    const int q = E >> 2;        // comparisons per thread, a multiple of 4
    for (int base = 0; base < E * 4; base += FT_THREADS) {
        const int k = base + t;
        const int i = k >> 2, part = k & 3;
        const bool live = i < E;
        const float v = m->logits[live ? i : 0];
        const bool v_nan = !(v == v);
        int rank = 0;
        for (int c0 = 0; c0 < q; c0 += 32) {
            const float4* l4 = reinterpret_cast<const float4*>(m->logits + part * q + c0);
            const int n4 = min(8, (q - c0) >> 2);
            float4 u[8];
#pragma unroll
            for (int j4 = 0; j4 < 8; ++j4) u[j4] = l4[min(j4, n4 - 1)];
#pragma unroll
            for (int j4 = 0; j4 < 8; ++j4) {
                if (j4 < n4) {
                    const int j = part * q + c0 + 4 * j4;
                    rank += sorts_before(u[j4].x, j, v, i, v_nan);
                    rank += sorts_before(u[j4].y, j + 1, v, i, v_nan);
                    rank += sorts_before(u[j4].z, j + 2, v, i, v_nan);
                    rank += sorts_before(u[j4].w, j + 3, v, i, v_nan);
                }
            }
        }
        rank += quad_xor1i(rank);
        rank += quad_xor2i(rank);
        if (live && part == 0 && rank < K) {  // ranks are distinct: each slot written once
            m->sel_i[rank] = i;
            m->sel_v[rank] = v;
        }
    }
    __syncthreads();
    if (t < 64) {  // wave 0: softmax from registers
        const float v0 = m->sel_v[0];
        const float vt = m->sel_v[min(t, K - 1)];
        const int it = m->sel_i[min(t, K - 1)];
        const float ex = expf_portable(vt - v0);
        float denom = 0.0f;
        for (int j = 0; j < K; ++j)  // in rank order, as the reference's iterator sum
            denom = denom + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ex), j));
        if (t < K) {
            float w = ex / denom;
            if (P.escale) w = w * P.escale[(int64_t)layer * E + it];
            m->ids[t] = it;
            m->wts[t] = w;
            if (blockIdx.x == 0) {
                if (P.ids_out) P.ids_out[layer * K + t] = it;
                if (P.wts_out) P.wts_out[layer * K + t] = w;
            }
        }
    }
    __syncthreads();
}

// Logit unit: final logits of experts [e0, e0+16) in the R-order: chunk
// partials summed in chunk order per group of C = H/128 chunks (from 0.0f),
// then the 8 group sums in order (from 0.0f), then + bias. C is a compile-time
// constant so that each thread's C partials are read from LDS in one batch.
template <int C>
__device__ bool logit_task(const FusedParams& P, Misc* m, uint32_t epoch, int task, int layer, uint32_t tag_in,
                           uint32_t tag_out, uint32_t* scratch) {
    const int E = P.E, NC = P.H / DN_ROWS;
    const int e0 = task * 16;  // E % 16 == 0: every task has 16 experts
    auto idx = [=](int i) { return (int64_t)(i >> 4) * E + e0 + (i & 15); };
    if (!wait_words(P, m, epoch, P.part_t, NC * 16, idx, tag_in, scratch)) return false;
    stamp(P, layer - 1, 16);
    float* G = m->G;  // [8][16] group sums
    const int t = threadIdx.x;
    if (t < 8 * 16) {
        const int g = t >> 4, el = t & 15;
        float pv[C];
#pragma unroll
        for (int c = 0; c < C; ++c) pv[c] = __uint_as_float(scratch[(g * C + c) * 16 + el]);
        float gs = 0.0f;
#pragma unroll
        for (int c = 0; c < C; ++c) gs = gs + pv[c];
        G[g * 16 + el] = gs;
    }
    __syncthreads();
    if (t < 16 * NREP) {
        const int el = t & 15;
        float gv[8];
#pragma unroll
        for (int g = 0; g < 8; ++g) gv[g] = G[g * 16 + el];
        float total = 0.0f;
#pragma unroll
        for (int g = 0; g < 8; ++g) total = total + gv[g];
        if (P.bias) total = total + P.bias[(int64_t)layer * E + e0 + el];
        st_tag(P.lg_t + (t >> 4) * P.rs_lg + e0 + el, tag_out, __float_as_uint(total));
    }
    stamp(P, layer - 1, 17);
    __syncthreads();
    return true;
}

// Router chunk partials of one 16-row chunk (R-order: fma chain over the rows
// in order, from 0.0f) and the chunk's x values, published with tag.
__device__ void publish_chunk(const FusedParams& P, const float* wr, const float* xv, int chunk, uint32_t tag) {
    const int E = P.E;
    for (int e = threadIdx.x; e < E; e += FT_THREADS) {
        const float4* w4 = reinterpret_cast<const float4*>(wr + e * DN_ROWS);
        float p = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 a = w4[q];
            p = fmaf(a.x, xv[4 * q + 0], p);
            p = fmaf(a.y, xv[4 * q + 1], p);
            p = fmaf(a.z, xv[4 * q + 2], p);
            p = fmaf(a.w, xv[4 * q + 3], p);
        }
        st_tag(P.part_t + (int64_t)chunk * E + e, tag, __float_as_uint(p));
    }
    if (threadIdx.x < DN_ROWS * NREP) {
        const int r = threadIdx.x & (DN_ROWS - 1), rep = threadIdx.x / DN_ROWS;
        st_tag(P.x_t + rep * P.rs_x + chunk * DN_ROWS + r, tag, __float_as_uint(xv[r]));
    }
}

// Copy `bytes` (multiple of 16) from global to LDS with global_load_lds: each
// wave moves 1 KB per instruction, lanes past the end are masked off.
__device__ __forceinline__ void prefetch_lds(const uint8_t* src, uint8_t* dst, int bytes) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int off = wave * 1024; off < bytes; off += FT_WAVES * 1024) {
        const int o = off + lane * 16;
        if (o < bytes)
            __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(src + o),
                                             reinterpret_cast<void*>(dst + off), 16, 0, 0);
    }
}

// BPW: gate|up blocks per wave, exactly H/32/8; DB: down blocks per thread,
// ceil(I/32/4) rounded up (the loads are unconditional so they issue back to
// back; surplus down blocks re-read a valid one and are masked).
template <int BPW, int DB>
__global__ __launch_bounds__(FT_THREADS, 1) void k_moe_stack_fused(FusedParams P) {
    extern __shared__ __align__(16) uint8_t lds[];
    float* x_l = reinterpret_cast<float*>(lds + P.o_x);
    uint8_t* q8x = lds + P.o_q8x;
    uint8_t* act8 = lds + P.o_act8;
    float* wr = reinterpret_cast<float*>(lds + P.o_wr);
    float* red = reinterpret_cast<float*>(lds + P.o_red);
    Misc* m = reinterpret_cast<Misc*>(lds + P.o_misc);

    const int w = blockIdx.x, t = threadIdx.x;
    const int H = P.H, I = P.I, E = P.E, K = P.K, L = P.L;
    const int nb = H >> 5, nbj = I >> 5;
    const int dn_tile = nbj * 288;  // bytes of one 16-row down tile
    const bool is_gu = w < P.n_gu, is_dn = w < P.n_dn, is_red = w < P.n_red;
    if (t == 0) m->abort_flag = 0;
    const uint32_t epoch = ld_ctl(P.ctl + CTL_EPOCH);
    auto tag_x = [&](int l) { return epoch + 4u * l + 1u; };
    auto tag_g = [&](int l) { return epoch + 4u * l + 2u; };
    auto tag_a = [&](int l) { return epoch + 4u * l + 3u; };
    auto ident = [](int i) { return (int64_t)i; };

    // ---- prologue: router of layer 0 on x_in ----
    stamp(P, -1, 0);
    if (is_dn) {
        if (t < DN_ROWS) m->xrow[t] = P.x_in[w * DN_ROWS + t];
        prefetch_lds(reinterpret_cast<const uint8_t*>(P.routers + (int64_t)w * E * DN_ROWS),
                     reinterpret_cast<uint8_t*>(wr), E * DN_ROWS * 4);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        publish_chunk(P, wr, m->xrow, w, tag_x(0));
        if (P.dbg_x && t < DN_ROWS) P.dbg_x[w * DN_ROWS + t] = m->xrow[t];
        stamp(P, -1, 7);
    }
    if (is_red && !logit_task<2 * BPW>(P, m, epoch, w, 0, tag_x(0), tag_g(0), reinterpret_cast<uint32_t*>(red)))
        return;
    stamp(P, -1, 9);
    if (is_gu) {
        for (int i = t; i < H; i += FT_THREADS) x_l[i] = P.x_in[i];
        __syncthreads();
        quantize_x_lds(P, x_l, q8x);
    }
    const int rep = w % NREP;  // this workgroup's XCD (workgroups are dealt to the 8 XCDs round-robin)
    if (!wait_words(P, m, epoch, P.lg_t + rep * P.rs_lg, E, ident, tag_g(0), reinterpret_cast<uint32_t*>(m->logits)))
        return;
    topk_rank(P, m, 0);
    stamp(P, -1, 15);

    for (int l = 0; l < L; ++l) {
        stamp(P, l, 0);
        stamp_clk(P, l, 4);
        const uint8_t* layer_banks = P.banks + (int64_t)l * E * P.expert_bytes;
        // ---- gate|up unit: issue its whole tile into registers ----
        const int wave = t >> 6, r = t & 63;
        // The gate|up loads and the down/router loads below are issued without
        // any branch between them (workgroups without a unit re-read a valid
        // tile), so the compiler issues them back to back and the gate|up
        // compute waits only for its own loads.
        const int p = min(w / nbj, K - 1), jb = w % nbj;
        const int b0 = wave * BPW;
        uint32_t sc[BPW];  // 32-bit: 16-bit elements would be packed in pairs, forcing a wait per load
        uint4 qv[BPW];
        {
            const uint8_t* T = layer_banks + (int64_t)m->ids[p] * P.expert_bytes + (int64_t)jb * nb * 1152;
            const uint8_t* Ts = T + b0 * 128 + r * 2;
            const uint8_t* Tq = T + nb * 128 + b0 * 1024 + r * 16;
            // all 16-byte loads first, then the 2-byte scales: interleaving
            // them (35 loads a wave in flight) more than doubled the time to
            // stream a layer in a standalone probe
#pragma unroll
            for (int i = 0; i < BPW; ++i) qv[i] = *reinterpret_cast<const uint4*>(Tq + i * 1024);
#pragma unroll
            for (int i = 0; i < BPW; ++i) sc[i] = *reinterpret_cast<const uint16_t*>(Ts + i * 128);
        }
        // ---- down unit: its K tiles go straight into the registers of the
        // threads that use them (thread (pp, rr, s) holds row rr of expert pp,
        // blocks s, s+4, ...), and the next router chunk (one uint4 per
        // thread), right behind the gate|up loads ----
        const int s4 = t & 3, rr = (t >> 2) & 15, pp = t >> 6;
        uint32_t dsc[DB];
        uint4 dq[DB];
        uint4 rv = make_uint4(0, 0, 0, 0);
        {
            const int wd = min(w, P.n_dn - 1);
            const uint8_t* D = layer_banks + (int64_t)m->ids[min(pp, K - 1)] * P.expert_bytes + P.gu_bytes +
                               (int64_t)wd * dn_tile;
#pragma unroll
            for (int k = 0; k < DB; ++k) {
                const int b = min(s4 + 4 * k, nbj - 1);
                dq[k] = *reinterpret_cast<const uint4*>(D + nbj * 32 + b * 256 + rr * 16);
            }
            asm volatile("" ::: "memory");  // keep the scale loads behind the 16-byte loads
#pragma unroll
            for (int k = 0; k < DB; ++k) {
                const int b = min(s4 + 4 * k, nbj - 1);
                dsc[k] = *reinterpret_cast<const uint16_t*>(D + b * 32 + rr * 2);
            }
            const uint4* rsrc = reinterpret_cast<const uint4*>(
                P.routers + ((int64_t)(l + 1 < L ? l + 1 : l) * (H / DN_ROWS) + wd) * E * DN_ROWS);
            rv = rsrc[min(t, 4 * E - 1)];
        }
        stamp(P, l, 1);
        // ---- gate|up compute -> GELU*up -> q8 block, published ----
        if (is_gu) {
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < BPW; ++i) {
                const int* xb = reinterpret_cast<const int*>(q8x + (b0 + i) * Q8_BLK);
                const int diff = block_dot(qv[i], xb + 2, xb[1]);
                acc = fmaf((float)diff, h2f((uint16_t)sc[i]) * __int_as_float(xb[0]), acc);
            }
            red[wave * 64 + r] = acc;
            __syncthreads();
            if (t < 64) {  // wave 0 finishes the unit: only wave-local ordering from here
                float rv[FT_WAVES];
#pragma unroll
                for (int v = 0; v < FT_WAVES; ++v) rv[v] = red[v * 64 + t];
                float s = 0.0f;
#pragma unroll
                for (int v = 0; v < FT_WAVES; ++v) s = s + rv[v];
                if (P.dbg_gu) {
                    const int row = t < 32 ? jb * 32 + t : I + jb * 32 + (t - 32);
                    P.dbg_gu[((int64_t)l * K + p) * 2 * I + row] = s;
                }
                m->gsum[t] = s;
                wave_lds_order();
                if (t < 32) m->act[t] = gelu_tanh(s) * m->gsum[t + 32];
                wave_lds_order();
                if (t < 4) quantize_block_quad(m->act, t, m->actblk);
                wave_lds_order();
                for (int i = t; i < 10 * NREP; i += 64) {  // 80 contiguous bytes per replica
                    const int k = i % 10, rep = i / 10;
                    st_tag(P.act_t + rep * P.rs_act + ((int64_t)p * nbj + jb) * 10 + k, tag_a(l), m->actblk[k]);
                    if (P.dbg_act && rep == 0)
                        reinterpret_cast<uint32_t*>(P.dbg_act + (((int64_t)l * K + p) * nbj + jb) * Q8_BLK)[k] =
                            m->actblk[k];
                }
            }
            stamp(P, l, 19);
        }
        stamp(P, l, 2);
        // ---- land the router chunk in LDS (after the gate|up compute, which
        // waited only for its own, earlier loads) ----
        if (is_dn && l + 1 < L && t < 4 * E) reinterpret_cast<uint4*>(wr)[t] = rv;
        stamp(P, l, 3);
        // ---- down unit: wait for all act blocks, combine, router partials ----
        if (is_dn) {
            // act8 in LDS: [K*nbj blocks x 32 B qs][K*nbj f32 d][K*nbj i32 qsum] (16-B aligned qs)
            const int nblk = K * nbj;
            auto act_dst = [=](int i) {
                const int bi = i / 10, k = i - bi * 10;
                return k >= 2 ? bi * 8 + (k - 2) : nblk * 8 + (k == 0 ? bi : nblk + bi);
            };
            if (!wait_words(P, m, epoch, P.act_t + rep * P.rs_act, nblk * 10, ident, tag_a(l),
                            reinterpret_cast<uint32_t*>(act8), act_dst))
                return;
            stamp(P, l, 5);
            __syncthreads();
            float acc = 0.0f;
            {
                const int* aqs = reinterpret_cast<const int*>(act8);
                const float* ad = reinterpret_cast<const float*>(act8) + nblk * 8;
                const int* asum = reinterpret_cast<const int*>(act8) + nblk * 9;
                const int pc = min(pp, K - 1);
#pragma unroll
                for (int k = 0; k < DB; ++k) {
                    const int b = s4 + 4 * k;
                    const int bi = pc * nbj + min(b, nbj - 1);
                    const float v = (float)block_dot(dq[k], aqs + bi * 8, asum[bi]) * (h2f((uint16_t)dsc[k]) * ad[bi]);
                    acc = b < nbj ? acc + v : acc;
                }
            }
            acc += quad_xor1(acc);
            acc += quad_xor2(acc);
            if (s4 == 0 && pp < K) m->y[pp][rr] = acc;
            stamp(P, l, 20);
            __syncthreads();
            if (t < DN_ROWS) {
                float yv[MAX_K], wv[MAX_K];
#pragma unroll
                for (int q = 0; q < MAX_K; ++q) {
                    yv[q] = m->y[q][t];
                    wv[q] = m->wts[q];
                }
                float h = 0.0f;
#pragma unroll
                for (int q = 0; q < MAX_K; ++q) {
                    const float part = yv[q] * wv[q];
                    h = q < K ? h + part : h;
                }
                const float xn = m->xrow[t] + h;
                m->xnew[t] = xn;
                m->xrow[t] = xn;
                if (l == L - 1) P.x_out[w * DN_ROWS + t] = xn;
                if (P.dbg_x) P.dbg_x[(int64_t)(l + 1) * H + w * DN_ROWS + t] = xn;
            }
            __syncthreads();
            stamp(P, l, 6);
            if (l + 1 < L) publish_chunk(P, wr, m->xnew, w, tag_x(l + 1));
            stamp(P, l, 7);
        }
        if (l + 1 == L) break;
        // ---- logits of layer l+1; meanwhile gate|up units take x_{l+1} ----
        if (is_red &&
            !logit_task<2 * BPW>(P, m, epoch, w, l + 1, tag_x(l + 1), tag_g(l + 1), reinterpret_cast<uint32_t*>(red)))
            return;
        stamp(P, l, 9);
        if (is_gu) {
            if (!wait_words(P, m, epoch, P.x_t + rep * P.rs_x, H, ident, tag_x(l + 1), reinterpret_cast<uint32_t*>(x_l)))
                return;
            stamp(P, l, 10);
            quantize_x_lds(P, x_l, q8x);
            stamp(P, l, 11);
        }
        if (!wait_words(P, m, epoch, P.lg_t + rep * P.rs_lg, E, ident, tag_g(l + 1), reinterpret_cast<uint32_t*>(m->logits)))
            return;
        stamp(P, l, 12);
        topk_rank(P, m, l + 1);
        stamp(P, l, 15);
        stamp_clk(P, l, 8);
    }
    if (w == 0 && t == 0)
        __hip_atomic_store(P.ctl + CTL_EPOCH, epoch + 4u * (L + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Layout packing (setup). Source: an expert bank in q4_0 or q4r rows (gate
// rows, up rows, then down rows). Destination: the fused layout (same bytes).
// ---------------------------------------------------------------------------
__device__ __forceinline__ void src_block(const uint8_t* row, int layout, int nb, int b, uint16_t& d, uint4& q) {
    if (layout == FT_LAYOUT_Q4R) {
        const int qs_off = (nb * 2 + 15) / 16 * 16;
        d = reinterpret_cast<const uint16_t*>(row)[b];
        q = *reinterpret_cast<const uint4*>(row + qs_off + 16 * b);
    } else {
        const uint16_t* p = reinterpret_cast<const uint16_t*>(row + 18 * b);
        d = p[0];
        q.x = (uint32_t)p[1] | ((uint32_t)p[2] << 16);
        q.y = (uint32_t)p[3] | ((uint32_t)p[4] << 16);
        q.z = (uint32_t)p[5] | ((uint32_t)p[6] << 16);
        q.w = (uint32_t)p[7] | ((uint32_t)p[8] << 16);
    }
}

__host__ __device__ __forceinline__ int64_t rowb(int layout, int k) {
    const int nb = k / 32;
    return layout == FT_LAYOUT_Q4R ? (int64_t)((nb * 2 + 15) / 16 * 16) + (int64_t)nb * 16 : (int64_t)nb * 18;
}

// one thread per (expert, gate|up tile jb, block b, lane r)
__global__ __launch_bounds__(256) void k_pack_gu(const uint8_t* src, int layout, int64_t src_eb, uint8_t* dst,
                                                 int64_t dst_eb, int H, int I, int64_t n_experts) {
    const int nb = H >> 5, nbj = I >> 5;
    const int64_t per_e = (int64_t)nbj * nb * 64;
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n_experts * per_e) return;
    const int64_t e = g / per_e;
    int64_t rem = g % per_e;
    const int jb = (int)(rem / (nb * 64));
    rem %= nb * 64;
    const int b = (int)(rem / 64), r = (int)(rem % 64);
    const int row = r < 32 ? jb * 32 + r : I + jb * 32 + (r - 32);
    uint16_t d;
    uint4 q;
    src_block(src + e * src_eb + row * rowb(layout, H), layout, nb, b, d, q);
    uint8_t* T = dst + e * dst_eb + (int64_t)jb * nb * 1152;
    *reinterpret_cast<uint16_t*>(T + b * 128 + r * 2) = d;
    *reinterpret_cast<uint4*>(T + nb * 128 + b * 1024 + r * 16) = q;
}

// one thread per (expert, down tile jt, block b, row r)
__global__ __launch_bounds__(256) void k_pack_dn(const uint8_t* src, int layout, int64_t src_eb, uint8_t* dst,
                                                 int64_t dst_eb, int H, int I, int64_t n_experts) {
    const int nbj = I >> 5, nt = H / DN_ROWS;
    const int64_t per_e = (int64_t)nt * nbj * DN_ROWS;
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n_experts * per_e) return;
    const int64_t e = g / per_e;
    int64_t rem = g % per_e;
    const int jt = (int)(rem / (nbj * DN_ROWS));
    rem %= nbj * DN_ROWS;
    const int b = (int)(rem / DN_ROWS), r = (int)(rem % DN_ROWS);
    const int64_t src_gu = 2LL * I * rowb(layout, H);
    const int64_t dst_gu = 2LL * I * (H / 32) * 18;
    uint16_t d;
    uint4 q;
    src_block(src + e * src_eb + src_gu + (int64_t)(jt * DN_ROWS + r) * rowb(layout, I), layout, nbj, b, d, q);
    uint8_t* T = dst + e * dst_eb + dst_gu + (int64_t)jt * nbj * 288;
    *reinterpret_cast<uint16_t*>(T + b * 32 + r * 2) = d;
    *reinterpret_cast<uint4*>(T + nbj * 32 + b * 256 + r * 16) = q;
}

__global__ __launch_bounds__(256) void k_pack_router(const float* src, float* dst, int64_t n_layers, int E, int H) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t per_l = (int64_t)E * H;
    if (g >= n_layers * per_l) return;
    const int64_t l = g / per_l;
    const int64_t rem = g % per_l;
    const int c = (int)(rem / ((int64_t)E * DN_ROWS));
    const int e = (int)(rem / DN_ROWS % E);
    const int i = (int)(rem % DN_ROWS);
    dst[g] = src[l * per_l + (int64_t)e * H + c * DN_ROWS + i];
}

__global__ void k_fill_u32(uint32_t* p, int64_t n, uint32_t v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
struct WsLayout {
    int64_t act, x, part, lg, ctl, total;
};

WsLayout ws_layout(int64_t H, int64_t I, int64_t E, int64_t K) {
    auto up = [](int64_t v) { return (v + 255) / 256 * 256; };
    WsLayout w{};
    int64_t off = 0;
    w.ctl = off; off += 256;
    w.act = off; off += NREP * up(K * (I / 32) * 10 * 8);
    w.x = off; off += NREP * up(H * 8);
    w.part = off; off += up((H / DN_ROWS) * E * 8);
    w.lg = off; off += NREP * up(E * 8);
    w.total = off;
    return w;
}

int check_fused_shape(const char* nm, int64_t H, int64_t I, int64_t E, int64_t K, int64_t L) {
    if (H <= 0 || H % 256) return fail(FT_HIP_E_SHAPE, "%s: hidden=%lld must be a positive multiple of 256", nm, (long long)H);
    if (H != 2816 && H != 4096)
        return fail(FT_HIP_E_SHAPE, "%s: hidden=%lld: the fused kernel is built for hidden 2816 and 4096", nm, (long long)H);
    if (I <= 0 || I % 32) return fail(FT_HIP_E_SHAPE, "%s: inter=%lld must be a positive multiple of 32", nm, (long long)I);
    if (E <= 0 || E > MAX_E) return fail(FT_HIP_E_SHAPE, "%s: n_experts=%lld not in [1, %d]", nm, (long long)E, MAX_E);
    if (K <= 0 || K > MAX_K || K > E) return fail(FT_HIP_E_SHAPE, "%s: top_k=%lld not in [1, min(%d, n_experts)]", nm, (long long)K, MAX_K);
    if (L <= 0) return fail(FT_HIP_E_SHAPE, "%s: n_layers must be positive", nm);
    if (E % 16) return fail(FT_HIP_E_SHAPE, "%s: n_experts=%lld must be a multiple of 16", nm, (long long)E);
    if (K * DN_ROWS * 4 > FT_THREADS || I / 32 > 4 * 8 || 4 * E > FT_THREADS)
        return fail(FT_HIP_E_SHAPE, "%s: needs top_k <= 8, inter <= 1024 and n_experts <= 128; use ft_hip_moe_layer", nm);
    return FT_HIP_OK;
}

}  // namespace

extern "C" int64_t ft_hip_fused_expert_bytes(int64_t hidden, int64_t inter) {
    if (hidden <= 0 || hidden % 32 || inter <= 0 || inter % 32) return -1;
    return 3 * hidden * inter / 32 * 18;
}

extern "C" size_t ft_hip_fused_workspace_bytes(int64_t hidden, int64_t inter, int64_t n_experts, int64_t top_k) {
    if (hidden <= 0 || hidden % 256 || inter <= 0 || inter % 32 || n_experts <= 0 || top_k <= 0) return 0;
    return (size_t)ws_layout(hidden, inter, n_experts, top_k).total;
}

extern "C" int ft_hip_fused_workspace_init(ft_hip_ctx* ctx, void* stream, void* workspace, size_t workspace_bytes) {
    clear_error();
    if (!ctx || !workspace) return fail(FT_HIP_E_INVALID, "fused_workspace_init: null argument");
    if (workspace_bytes % 4) return fail(FT_HIP_E_SHAPE, "fused_workspace_init: size not a multiple of 4");
    const int64_t n = (int64_t)(workspace_bytes / 4);
    hipLaunchKernelGGL(k_fill_u32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       (uint32_t*)workspace, n, 0u);
    if (int rc = launch_status("fused_workspace_init")) return rc;
    // epoch 1: tags of zero-filled words never match
    hipLaunchKernelGGL(k_fill_u32, dim3(1), dim3(1), 0, reinterpret_cast<hipStream_t>(stream),
                       (uint32_t*)workspace + CTL_EPOCH, (int64_t)1, 1u);
    return launch_status("fused_workspace_init");
}

extern "C" int ft_hip_pack_experts_fused(ft_hip_ctx* ctx, void* stream, const void* src, int src_layout,
                                         uint64_t src_expert_bytes, void* dst, int64_t n_experts, int64_t hidden,
                                         int64_t inter) {
    clear_error();
    const char* nm = "pack_experts_fused";
    if (hidden <= 0 || hidden % 32 || inter <= 0 || inter % 32)
        return fail(FT_HIP_E_SHAPE, "%s: hidden and inter must be positive multiples of 32", nm);
    if (src_layout != FT_LAYOUT_Q4_0 && src_layout != FT_LAYOUT_Q4R) return fail(FT_HIP_E_INVALID, "%s: bad layout", nm);
    if (n_experts < 0) return fail(FT_HIP_E_SHAPE, "%s: negative n_experts", nm);
    const int64_t need = 2 * inter * rowb(src_layout, (int)hidden) + hidden * rowb(src_layout, (int)inter);
    if ((int64_t)src_expert_bytes < need) return fail(FT_HIP_E_SHAPE, "%s: src_expert_bytes < %lld", nm, (long long)need);
    if (src_layout == FT_LAYOUT_Q4R && ((reinterpret_cast<uintptr_t>(src) | src_expert_bytes) & 15))
        return fail(FT_HIP_E_SHAPE, "%s: q4r source must be 16-byte aligned", nm);
    if (!ctx || !src || !dst) return fail(FT_HIP_E_INVALID, "%s: null argument", nm);
    if (reinterpret_cast<uintptr_t>(dst) & 15) return fail(FT_HIP_E_SHAPE, "%s: dst must be 16-byte aligned", nm);
    if (n_experts == 0) return FT_HIP_OK;
    const int64_t eb = ft_hip_fused_expert_bytes(hidden, inter);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int64_t n1 = n_experts * (inter / 32) * (hidden / 32) * 64;
    hipLaunchKernelGGL(k_pack_gu, dim3((unsigned)((n1 + 255) / 256)), dim3(256), 0, s, (const uint8_t*)src, src_layout,
                       (int64_t)src_expert_bytes, (uint8_t*)dst, eb, (int)hidden, (int)inter, n_experts);
    if (int rc = launch_status(nm)) return rc;
    const int64_t n2 = n_experts * (hidden / DN_ROWS) * (inter / 32) * DN_ROWS;
    hipLaunchKernelGGL(k_pack_dn, dim3((unsigned)((n2 + 255) / 256)), dim3(256), 0, s, (const uint8_t*)src, src_layout,
                       (int64_t)src_expert_bytes, (uint8_t*)dst, eb, (int)hidden, (int)inter, n_experts);
    return launch_status(nm);
}

extern "C" int ft_hip_pack_router_fused(ft_hip_ctx* ctx, void* stream, const float* src, float* dst, int64_t n_layers,
                                        int64_t n_experts, int64_t hidden) {
    clear_error();
    const char* nm = "pack_router_fused";
    if (hidden <= 0 || hidden % 256 || n_experts <= 0 || n_experts > MAX_E || n_layers < 0)
        return fail(FT_HIP_E_SHAPE, "%s: bad shape", nm);
    if (!ctx || !src || !dst) return fail(FT_HIP_E_INVALID, "%s: null argument", nm);
    const int64_t n = n_layers * n_experts * hidden;
    if (n == 0) return FT_HIP_OK;
    hipLaunchKernelGGL(k_pack_router, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream), src, dst, n_layers, (int)n_experts, (int)hidden);
    return launch_status(nm);
}

extern "C" int ft_hip_moe_stack_fused(ft_hip_ctx* ctx, void* stream, const float* x_in, float* x_out, int64_t hidden,
                                      int64_t inter, int64_t n_experts, int64_t top_k, int64_t n_layers,
                                      const void* banks, const float* routers, const float* bias,
                                      const float* expert_scale, int32_t* ids, float* wts, void* workspace,
                                      size_t workspace_bytes, float* dbg_gu, void* dbg_act, float* dbg_x,
                                      uint64_t* dbg_trace) {
    clear_error();
    const char* nm = "moe_stack_fused";
    if (int rc = check_fused_shape(nm, hidden, inter, n_experts, top_k, n_layers)) return rc;
    const WsLayout wl = ws_layout(hidden, inter, n_experts, top_k);
    if ((int64_t)workspace_bytes < wl.total)
        return fail(FT_HIP_E_SHAPE, "%s: workspace_bytes=%zu < %lld", nm, workspace_bytes, (long long)wl.total);
    FusedParams P{};
    P.H = (int)hidden;
    P.I = (int)inter;
    P.E = (int)n_experts;
    P.K = (int)top_k;
    P.L = (int)n_layers;
    P.n_gu = (int)(top_k * (inter / 32));
    P.n_dn = (int)(hidden / DN_ROWS);
    P.n_red = (int)((n_experts + 15) / 16);
    const int nw = std::max(P.n_gu, std::max(P.n_dn, P.n_red));
    // LDS plan
    auto up16 = [](int v) { return (v + 15) / 16 * 16; };
    int off = 0;
    P.o_x = off; off += up16((int)hidden * 4);
    P.o_q8x = off; off += up16((int)(hidden / 32) * Q8_BLK);
    P.o_act8 = off; off += up16((int)(top_k * (inter / 32)) * Q8_BLK);
    P.o_wr = off; off += up16((int)n_experts * DN_ROWS * 4);
    const int red_bytes = std::max(FT_WAVES * 64 * 4, (int)(hidden / DN_ROWS) * 16 * 4);
    P.o_red = off; off += up16(red_bytes);
    P.o_misc = off; off += up16((int)sizeof(Misc));
    P.lds_bytes = off;
    if (off > 160 * 1024)
        return fail(FT_HIP_E_SHAPE, "%s: this shape needs %d B of LDS per workgroup (> 160 KB); use ft_hip_moe_layer", nm, off);
    if (!ctx || !x_in || !x_out || !banks || !routers || !workspace) return fail(FT_HIP_E_INVALID, "%s: null argument", nm);
    if (nw > ctx->num_cus)
        return fail(FT_HIP_E_SHAPE, "%s: needs %d co-resident workgroups, device has %d CUs", nm, nw, ctx->num_cus);
    if ((reinterpret_cast<uintptr_t>(banks) | reinterpret_cast<uintptr_t>(routers)) & 15)
        return fail(FT_HIP_E_SHAPE, "%s: banks and routers must be 16-byte aligned", nm);
    uint8_t* ws = (uint8_t*)workspace;
    P.banks = (const uint8_t*)banks;
    P.routers = routers;
    P.bias = bias;
    P.escale = expert_scale;
    P.x_in = x_in;
    P.x_out = x_out;
    P.ids_out = ids;
    P.wts_out = wts;
    auto up256 = [](int64_t v) { return (v + 255) / 256 * 256; };
    P.act_t = (uint64_t*)(ws + wl.act);
    P.x_t = (uint64_t*)(ws + wl.x);
    P.rs_act = up256(top_k * (inter / 32) * 10 * 8) / 8;
    P.rs_x = up256(hidden * 8) / 8;
    P.rs_lg = up256(n_experts * 8) / 8;
    P.part_t = (uint64_t*)(ws + wl.part);
    P.lg_t = (uint64_t*)(ws + wl.lg);
    P.ctl = (uint32_t*)(ws + wl.ctl);
    P.dbg_gu = dbg_gu;
    P.dbg_act = (uint8_t*)dbg_act;
    P.dbg_x = dbg_x;
    P.trace = dbg_trace;
    P.expert_bytes = ft_hip_fused_expert_bytes(hidden, inter);
    P.gu_bytes = 2 * inter * (hidden / 32) * 18;
    P.spin_limit = 1 << 21;
    void* args[] = {&P};
    // blocks per wave of a gate|up tile: the kernel keeps exactly that many in flight
    const bool db6 = inter / 32 <= 24;
    const void* kern = hidden == 2816 ? (db6 ? reinterpret_cast<const void*>(k_moe_stack_fused<11, 6>)
                                             : reinterpret_cast<const void*>(k_moe_stack_fused<11, 8>))
                                      : (db6 ? reinterpret_cast<const void*>(k_moe_stack_fused<GU_BPW_MAX, 6>)
                                             : reinterpret_cast<const void*>(k_moe_stack_fused<GU_BPW_MAX, 8>));
    hipError_t e = hipLaunchCooperativeKernel(kern, dim3((unsigned)nw),
                                              dim3(FT_THREADS), args, (unsigned)P.lds_bytes,
                                              reinterpret_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(FT_HIP_E_LAUNCH, "%s: cooperative launch failed: %s", nm, hipGetErrorString(e));
    return FT_HIP_OK;
}

extern "C" int ft_hip_fused_status(ft_hip_ctx* ctx, void* workspace, int* aborted) {
    clear_error();
    if (!ctx || !workspace || !aborted) return fail(FT_HIP_E_INVALID, "fused_status: null argument");
    uint32_t ctl[64];
    hipError_t e = hipMemcpy(ctl, workspace, sizeof ctl, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return fail(FT_HIP_E_LAUNCH, "fused_status: %s", hipGetErrorString(e));
    *aborted = ctl[CTL_ABORT] != 0;
    if (*aborted) return fail(FT_HIP_E_TIMEOUT, "fused kernel aborted a bounded wait (epoch %u)", ctl[CTL_ABORT]);
    return FT_HIP_OK;
}
