// ft_hip_grouped.hip -- one MoE layer for a batch of decode tokens with the
// (token, expert) pairs grouped by expert, so each routed expert's weights
// stream from HBM once for all of its tokens.
//
// The reference runs batched decode as one GEMV per pair over the pair list
// (ft-model/src/lib.rs:1507-1606: gemv_q4r_ptr per pair, gelu_mul_q8,
// gemv_q4r_ptr, reduce_pairs_weighted), re-reading an expert's weights for
// every token routed to it. Here:
//   router logits + top-k + q8(x)         (the launch-by-launch kernels)
//   k_group_pairs     one workgroup: pairs per expert, active-expert list
//   k_grouped_gu      per (active expert, gate|up tile j): the tile's 64 rows
//                     in registers, dots against every token of the expert,
//                     GELU*up, q8 of the act block -> act[pair][j]
//   k_grouped_down    per (active expert, 128-row unit): y[pair][rows]
//   k_grouped_combine x_out[t] = x[t] + sum_k y[t*K+k] * w[t*K+k] in slot order
// Weights are in the fused layout (ft_hip_pack_experts_fused), so one packed
// bank serves this path and the batch-1 fused kernel.

#include "ft_device.hpp"
#include "ft_runtime.hpp"

#include <algorithm>

using namespace ft;

namespace {

constexpr int GT = 512;       // threads per workgroup
constexpr int GW = GT / 64;   // waves
constexpr int NT = 8;         // tokens per chunk of the gate|up kernel (LDS stays under 64 KB)
constexpr int NTD = 16;       // tokens per chunk of the down kernel
constexpr int DU = 16 * GW;   // rows per down unit (one 16-row tile per wave)
constexpr int MAX_PAIRS = 4096;

struct GroupWs {
    float* logits;      // [B][E]
    uint8_t* q8x;       // [B][H/32][40]
    int32_t* meta;      // [0] active experts; [1..] gexp[E], gstart[E], gcount[E]
    int32_t* plist;     // [P] pairs grouped by expert
    int32_t* ppos;      // [P] scratch
    uint8_t* q8a;       // [P][I/32][40]
    float* ydn;         // [P][H]
    float* inv;         // [B] input RMS norm scales
    size_t bytes;
};

GroupWs group_ws(void* base, int64_t B, int64_t H, int64_t I, int64_t E, int64_t K) {
    auto up = [](size_t v) { return (v + 255) / 256 * 256; };
    const int64_t P = B * K;
    size_t off = 0;
    GroupWs w{};
    uint8_t* p = (uint8_t*)base;
    w.logits = (float*)(p + off); off += up(sizeof(float) * B * E);
    w.q8x = p + off; off += up((size_t)B * (H / 32) * Q8_BLK);
    w.meta = (int32_t*)(p + off); off += up(sizeof(int32_t) * (1 + 3 * E));
    w.plist = (int32_t*)(p + off); off += up(sizeof(int32_t) * P);
    w.ppos = (int32_t*)(p + off); off += up(sizeof(int32_t) * P);
    w.q8a = p + off; off += up((size_t)P * (I / 32) * Q8_BLK);
    w.ydn = (float*)(p + off); off += up(sizeof(float) * P * H);
    w.inv = (float*)(p + off); off += up(sizeof(float) * B);
    w.bytes = off;
    return w;
}

// Pairs p = t*K + k grouped by expert ids[p]. The order inside a group does
// not matter: every (row, token) dot is independent and outputs are written
// to the pair's own slot, so results are the same for any order.
__global__ __launch_bounds__(1024) void k_group_pairs(const int32_t* ids, int P, int E, int32_t* meta, int32_t* plist,
                                                      int32_t* ppos) {
    __shared__ int cnt[1024];
    __shared__ int scan[1024];
    __shared__ int act[1024];
    const int t = threadIdx.x;
    for (int e = t; e < E; e += 1024) cnt[e] = 0;
    __syncthreads();
    for (int p = t; p < P; p += 1024) {
        const int e = min(max(ids[p], 0), E - 1);
        ppos[p] = atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    // exclusive prefix sums of counts and of "active" flags (E <= 1024)
    const int c = t < E ? cnt[t] : 0;
    scan[t] = c;
    act[t] = c > 0;
    __syncthreads();
    for (int d = 1; d < 1024; d <<= 1) {
        const int a = t >= d ? scan[t - d] : 0;
        const int b = t >= d ? act[t - d] : 0;
        __syncthreads();
        scan[t] += a;
        act[t] += b;
        __syncthreads();
    }
    if (t < E && c > 0) {
        const int g = act[t] - 1;
        meta[1 + g] = t;                 // gexp
        meta[1 + E + g] = scan[t] - c;   // gstart
        meta[1 + 2 * E + g] = c;         // gcount
    }
    if (t == 0) meta[0] = act[1023];
    __syncthreads();
    for (int p = t; p < P; p += 1024) {
        const int e = min(max(ids[p], 0), E - 1);
        plist[scan[e] - cnt[e] + ppos[p]] = p;
    }
}

// Gate|up tile j of active expert g for all of its tokens, then GELU*up and
// the q8 of act block j per token. BPW = H/32/8 blocks per wave. in_scale
// (input RMS norm, or null): a token's gate|up sums are first multiplied by
// in_scale[token].
template <int BPW>
__global__ __launch_bounds__(GT, 1) void k_grouped_gu(const uint8_t* bank, int64_t expert_bytes, const int32_t* meta,
                                                      const int32_t* plist, const uint8_t* q8x, uint8_t* q8a,
                                                      float* dbg_gu, const float* in_scale, int H, int I, int E,
                                                      int K) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int nb = H >> 5, nbj = I >> 5;
    const int j = blockIdx.x, g = blockIdx.y;
    if (g >= meta[0]) return;
    const int e = meta[1 + g], s0 = meta[1 + E + g], n = meta[1 + 2 * E + g];
    // LDS: x q8 of NT tokens as [NT][nb][8 words] qs + [NT][nb] (d, qsum) pairs;
    // wave partial sums [GW][NT][64]; row sums [NT][64]; act [NT][32]
    uint4* xq = reinterpret_cast<uint4*>(lds);
    int2* xp = reinterpret_cast<int2*>(lds + NT * nb * 32);
    float* red = reinterpret_cast<float*>(lds + NT * nb * 40);
    float* rows = red + GW * NT * 64;
    float* actv = rows + NT * 64;
    uint32_t* ablk = reinterpret_cast<uint32_t*>(actv + NT * 32);
    const int t = threadIdx.x, wave = t >> 6, r = t & 63, b0 = wave * BPW;
    uint4 qv[BPW];
    uint32_t sc[BPW];
    {
        const uint8_t* T = bank + (int64_t)e * expert_bytes + (int64_t)j * nb * 1152;
#pragma unroll
        for (int i = 0; i < BPW; ++i) qv[i] = *reinterpret_cast<const uint4*>(T + nb * 128 + (b0 + i) * 1024 + r * 16);
#pragma unroll
        for (int i = 0; i < BPW; ++i) sc[i] = *reinterpret_cast<const uint16_t*>(T + (b0 + i) * 128 + r * 2);
    }
    for (int c0 = 0; c0 < n; c0 += NT) {
        const int nt = min(NT, n - c0);
        __syncthreads();  // the previous chunk's LDS is consumed
        for (int i = t; i < nt * nb * 10; i += GT) {  // stage x q8 of this chunk's tokens
            const int tt = i / (nb * 10), rem = i - tt * nb * 10, b = rem / 10, wd = rem - b * 10;
            const int tok = plist[s0 + c0 + tt] / K;
            const uint32_t v = reinterpret_cast<const uint32_t*>(q8x + ((int64_t)tok * nb + b) * Q8_BLK)[wd];
            if (wd >= 2) reinterpret_cast<uint32_t*>(xq)[(tt * nb + b) * 8 + (wd - 2)] = v;
            else reinterpret_cast<uint32_t*>(xp)[(tt * nb + b) * 2 + wd] = v;
        }
        __syncthreads();
        for (int tt = 0; tt < nt; ++tt) {  // one token at a time: its BPW blocks' LDS reads in one batch
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < BPW; ++i) {
                const int xb = tt * nb + b0 + i;
                const int2 dq = xp[xb];
                const int dot = block_dot_v(qv[i], xq[xb * 2], xq[xb * 2 + 1], dq.y);
                acc = fmaf((float)dot, h2f((uint16_t)sc[i]) * __int_as_float(dq.x), acc);
            }
            red[(wave * NT + tt) * 64 + r] = acc;
        }
        __syncthreads();
        for (int i = t; i < nt * 64; i += GT) {  // (token, row) sums over the waves, in wave order
            const int tt = i >> 6, rr = i & 63;
            float sv = 0.0f;
#pragma unroll
            for (int v = 0; v < GW; ++v) sv = sv + red[(v * NT + tt) * 64 + rr];
            if (in_scale) sv = sv * in_scale[plist[s0 + c0 + tt] / K];
            rows[tt * 64 + rr] = sv;
            if (dbg_gu) {
                const int p = plist[s0 + c0 + tt];
                const int row = rr < 32 ? j * 32 + rr : I + j * 32 + (rr - 32);
                dbg_gu[(int64_t)p * 2 * I + row] = sv;
            }
        }
        __syncthreads();
        for (int i = t; i < nt * 32; i += GT) {
            const int tt = i >> 5, cc = i & 31;
            actv[tt * 32 + cc] = gelu_tanh(rows[tt * 64 + cc]) * rows[tt * 64 + 32 + cc];
        }
        __syncthreads();
        if (t < 4 * nt) quantize_block_quad(actv + (t >> 2) * 32, t & 3, ablk + (t >> 2) * 10);
        __syncthreads();
        for (int i = t; i < nt * 10; i += GT) {
            const int tt = i / 10, wd = i - tt * 10;
            const int p = plist[s0 + c0 + tt];
            reinterpret_cast<uint32_t*>(q8a + ((int64_t)p * nbj + j) * Q8_BLK)[wd] = ablk[tt * 10 + wd];
        }
    }
}

// Down rows 128u..128u+127 of active expert g (one 16-row tile per wave;
// thread (rr, s4) holds row rr's blocks s4, s4+4, ...) for all of its tokens.
template <int DB>
__global__ __launch_bounds__(GT, 1) void k_grouped_down(const uint8_t* bank, int64_t expert_bytes, int64_t gu_bytes,
                                                        const int32_t* meta, const int32_t* plist, const uint8_t* q8a,
                                                        float* ydn, int H, int I, int E) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int nbj = I >> 5;
    const int u = blockIdx.x, g = blockIdx.y;
    if (g >= meta[0]) return;
    const int e = meta[1 + g], s0 = meta[1 + E + g], n = meta[1 + 2 * E + g];
    uint4* aq = reinterpret_cast<uint4*>(lds);                  // [NTD][nbj][2 uint4]
    int2* ap = reinterpret_cast<int2*>(lds + NTD * nbj * 32);   // [NTD][nbj]
    const int t = threadIdx.x, wave = t >> 6, s4 = t & 3, rr = (t >> 2) & 15;
    const int dn_tile = nbj * 288;
    uint4 dq[DB];
    uint32_t dsc[DB];
    {
        const uint8_t* D = bank + (int64_t)e * expert_bytes + gu_bytes + (int64_t)(u * GW + wave) * dn_tile;
#pragma unroll
        for (int k = 0; k < DB; ++k) {
            const int b = min(s4 + 4 * k, nbj - 1);
            dq[k] = *reinterpret_cast<const uint4*>(D + nbj * 32 + b * 256 + rr * 16);
        }
#pragma unroll
        for (int k = 0; k < DB; ++k) {
            const int b = min(s4 + 4 * k, nbj - 1);
            dsc[k] = *reinterpret_cast<const uint16_t*>(D + b * 32 + rr * 2);
        }
    }
    for (int c0 = 0; c0 < n; c0 += NTD) {
        const int nt = min(NTD, n - c0);
        __syncthreads();
        for (int i = t; i < nt * nbj * 10; i += GT) {
            const int tt = i / (nbj * 10), rem = i - tt * nbj * 10, b = rem / 10, wd = rem - b * 10;
            const int p = plist[s0 + c0 + tt];
            const uint32_t v = reinterpret_cast<const uint32_t*>(q8a + ((int64_t)p * nbj + b) * Q8_BLK)[wd];
            if (wd >= 2) reinterpret_cast<uint32_t*>(aq)[(tt * nbj + b) * 8 + (wd - 2)] = v;
            else reinterpret_cast<uint32_t*>(ap)[(tt * nbj + b) * 2 + wd] = v;
        }
        __syncthreads();
        for (int tt = 0; tt < nt; ++tt) {
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < DB; ++k) {
                const int b = s4 + 4 * k;
                const int xb = tt * nbj + min(b, nbj - 1);
                const int2 pq = ap[xb];
                const float v = (float)block_dot_v(dq[k], aq[xb * 2], aq[xb * 2 + 1], pq.y) *
                                (h2f((uint16_t)dsc[k]) * __int_as_float(pq.x));
                acc = b < nbj ? acc + v : acc;
            }
            acc += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(acc), 0xB1, 0xF, 0xF, false));
            acc += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(acc), 0x4E, 0xF, 0xF, false));
            if (s4 == 0) {
                const int p = plist[s0 + c0 + tt];
                ydn[(int64_t)p * H + u * DU + wave * 16 + rr] = acc;
            }
        }
    }
}

// x_out[t] = x[t] + sum_k (y[t*K+k] * w[t*K+k]), slots in order
// (ft-model/src/lib.rs:1634-1646).
__global__ __launch_bounds__(256) void k_grouped_combine(const float* y, const float* wts, const float* x, float* out,
                                                         int H, int K) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x, s = blockIdx.y;
    if (i >= H) return;
    float h = 0.0f;
    for (int k = 0; k < K; ++k) {
        const float part = y[((int64_t)s * K + k) * H + i] * wts[s * K + k];
        h = h + part;
    }
    out[(int64_t)s * H + i] = x[(int64_t)s * H + i] + h;
}

int check_grouped_shape(const char* nm, int64_t B, int64_t H, int64_t I, int64_t E, int64_t K) {
    if (H != 2816 && H != 4096)
        return fail(FT_HIP_E_SHAPE, "%s: hidden=%lld: built for hidden 2816 and 4096", nm, (long long)H);
    if (I <= 0 || I % 32 || I / 32 > 32)
        return fail(FT_HIP_E_SHAPE, "%s: inter=%lld must be a multiple of 32 in [32, 1024]", nm, (long long)I);
    if (E <= 0 || E > 1024) return fail(FT_HIP_E_SHAPE, "%s: n_experts not in [1, 1024]", nm);
    if (K <= 0 || K > 32 || K > E) return fail(FT_HIP_E_SHAPE, "%s: top_k not in [1, min(32, n_experts)]", nm);
    if (B < 0 || B * K > MAX_PAIRS) return fail(FT_HIP_E_SHAPE, "%s: n_seqs*top_k must be <= %d", nm, MAX_PAIRS);
    return FT_HIP_OK;
}

}  // namespace

extern "C" size_t ft_hip_moe_layer_grouped_workspace_bytes(int64_t n_seqs, int64_t hidden, int64_t inter,
                                                           int64_t n_experts, int64_t top_k) {
    if (n_seqs < 0 || hidden <= 0 || inter <= 0 || n_experts <= 0 || top_k <= 0) return 0;
    return group_ws(nullptr, n_seqs, hidden, inter, n_experts, top_k).bytes;
}

extern "C" int ft_hip_moe_layer_grouped(ft_hip_ctx* ctx, void* stream, const float* x, float* x_out, int64_t n_seqs,
                                        int64_t hidden, int64_t inter, int64_t n_experts, int64_t top_k,
                                        const float* router_w, const float* router_bias, const float* expert_scale,
                                        const void* bank, int32_t* ids, float* wts, void* workspace,
                                        size_t workspace_bytes, float* dbg_gu, void* dbg_act) {
    clear_error();
    const char* nm = "moe_layer_grouped";
    if (int rc = check_grouped_shape(nm, n_seqs, hidden, inter, n_experts, top_k)) return rc;
    const GroupWs w = group_ws(workspace, n_seqs, hidden, inter, n_experts, top_k);
    if (workspace_bytes < w.bytes) return fail(FT_HIP_E_SHAPE, "%s: workspace_bytes=%zu < %zu", nm, workspace_bytes, w.bytes);
    if (!ctx || !x || !x_out || !router_w || !bank || !ids || !wts || !workspace)
        return fail(FT_HIP_E_INVALID, "%s: null argument", nm);
    if (reinterpret_cast<uintptr_t>(bank) & 15) return fail(FT_HIP_E_SHAPE, "%s: bank must be 16-byte aligned", nm);
    if (n_seqs == 0) return FT_HIP_OK;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int H = (int)hidden, I = (int)inter, E = (int)n_experts, K = (int)top_k;
    const int P = (int)(n_seqs * top_k), nb = H / 32, nbj = I / 32;
    const int64_t eb = ft_hip_fused_expert_bytes(hidden, inter);
    const int64_t gu_bytes = 2LL * I * nb * 18;
    int rc;
    const float* inv = ctx->input_norm ? w.inv : nullptr;
    if (inv && (rc = ft::launch_rms_inv(stream, x, w.inv, hidden, n_seqs))) return rc;
    if ((rc = ft::launch_router_logits(stream, router_w, x, router_bias, inv, w.logits, hidden, n_experts, n_seqs)))
        return rc;
    if ((rc = ft_hip_topk_router(ctx, stream, w.logits, expert_scale, ids, wts, n_experts, top_k, n_seqs))) return rc;
    if ((rc = ft_hip_quantize_q8(ctx, stream, x, hidden, w.q8x, hidden, n_seqs))) return rc;
    hipLaunchKernelGGL(k_group_pairs, dim3(1), dim3(1024), 0, s, (const int32_t*)ids, P, E, w.meta, w.plist, w.ppos);
    if ((rc = launch_status("moe_layer_grouped/group"))) return rc;
    const int gmax = std::min(E, P);
    const size_t lds_gu = (size_t)NT * nb * 40 + sizeof(float) * (GW * NT * 64 + NT * 64 + NT * 32) + 4 * NT * 10;
    if (H == 2816)
        hipLaunchKernelGGL(k_grouped_gu<11>, dim3(nbj, gmax), dim3(GT), lds_gu, s, (const uint8_t*)bank, eb,
                           (const int32_t*)w.meta, (const int32_t*)w.plist, (const uint8_t*)w.q8x, w.q8a, dbg_gu, inv, H, I, E, K);
    else
        hipLaunchKernelGGL(k_grouped_gu<16>, dim3(nbj, gmax), dim3(GT), lds_gu, s, (const uint8_t*)bank, eb,
                           (const int32_t*)w.meta, (const int32_t*)w.plist, (const uint8_t*)w.q8x, w.q8a, dbg_gu, inv, H, I, E, K);
    if ((rc = launch_status("moe_layer_grouped/gate_up"))) return rc;
    if (dbg_act && hipMemcpyAsync(dbg_act, w.q8a, (size_t)P * nbj * Q8_BLK, hipMemcpyDeviceToDevice, s) != hipSuccess)
        return fail(FT_HIP_E_LAUNCH, "%s: debug copy failed", nm);
    const size_t lds_dn = (size_t)NTD * nbj * 40;
    if (nbj <= 24)
        hipLaunchKernelGGL(k_grouped_down<6>, dim3(H / DU, gmax), dim3(GT), lds_dn, s, (const uint8_t*)bank, eb, gu_bytes,
                           (const int32_t*)w.meta, (const int32_t*)w.plist, (const uint8_t*)w.q8a, w.ydn, H, I, E);
    else
        hipLaunchKernelGGL(k_grouped_down<8>, dim3(H / DU, gmax), dim3(GT), lds_dn, s, (const uint8_t*)bank, eb, gu_bytes,
                           (const int32_t*)w.meta, (const int32_t*)w.plist, (const uint8_t*)w.q8a, w.ydn, H, I, E);
    if ((rc = launch_status("moe_layer_grouped/down"))) return rc;
    hipLaunchKernelGGL(k_grouped_combine, dim3((H + 255) / 256, (unsigned)n_seqs), dim3(256), 0, s, (const float*)w.ydn,
                       (const float*)wts, x, x_out, H, K);
    return launch_status("moe_layer_grouped/combine");
}
