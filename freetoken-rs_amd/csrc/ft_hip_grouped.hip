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
#include <type_traits>
#include <limits>

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
    int32_t* meta;      // [0] active experts; [1..] gexp[E], gstart[E], gcount[E]; [1+3E] MFMA groups
    int32_t* plist;     // [P] pairs grouped by expert
    int32_t* ppos;      // [P] scratch
    uint8_t* q8a;       // [P][I/32][40]
    uint8_t* q8m;       // the MFMA groups' act quants by group position q: [I/32][4][P] (qs words g, g+4), then [I/32][P] (d, qsum)
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
    w.meta = (int32_t*)(p + off); off += up(sizeof(int32_t) * (2 + 3 * E));
    w.plist = (int32_t*)(p + off); off += up(sizeof(int32_t) * P);
    w.ppos = (int32_t*)(p + off); off += up(sizeof(int32_t) * P);
    w.q8a = p + off; off += up((size_t)P * (I / 32) * Q8_BLK);
    w.q8m = p + off; off += up((size_t)P * (I / 32) * Q8_BLK);
    w.ydn = (float*)(p + off); off += up(sizeof(float) * P * H);
    w.inv = (float*)(p + off); off += up(sizeof(float) * B);
    w.bytes = off;
    return w;
}

// Global -> LDS copy of n 32-bit items: item i is ld(i), stored by st(i, v).
// Each thread issues up to R loads before its first store, so the copy
// costs ceil(n / (R * GT)) load latencies rather than ceil(n / GT).
template <int R, typename Ld, typename St>
__device__ __forceinline__ void stage(int n, Ld ld, St st) {
    const int t = threadIdx.x;
    for (int base = 0; base < n; base += R * GT) {
        uint32_t v[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int i = base + r * GT + t;
            v[r] = i < n ? ld(i) : 0u;
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int i = base + r * GT + t;
            if (i < n) st(i, v[r]);
        }
    }
}

// Pairs p = t*K + k grouped by expert ids[p]. The order inside a group does
// not matter: every (row, token) dot is independent and outputs are written
// to the pair's own slot, so results are the same for any order.
// Groups are numbered with the experts of >= n_mfma tokens first (meta[1 +
// 3E] of them, for the MFMA kernels), then the others (for the dot4
// kernels), each in expert order.
//
// TOPK (E <= 32 as launched): the routing itself first, from the logits (the
// arithmetic of k_topk_router, so the same ids and weights): 1024/E tokens
// per round, one thread per logit ranking it by rank_key among its token's
// E, then the softmax over each token's K in rank order; ids/wts written to
// ids_out/wts_out and kept in LDS for the grouping.
template <bool TOPK>
__global__ __launch_bounds__(1024) void k_group_pairs(const int32_t* ids, int P, int E, int n_mfma, int32_t* meta,
                                                      int32_t* plist, int32_t* ppos, const float* logits,
                                                      const float* escale, int32_t* ids_out, float* wts_out, int K) {
    __shared__ int cnt[1024];
    __shared__ int scan[1024];
    __shared__ int act[1024];
    __shared__ int big[1024];
    __shared__ int sid[TOPK ? MAX_PAIRS : 1];
    __shared__ uint64_t key[TOPK ? 1024 : 1];
    __shared__ float sv[TOPK ? 1024 : 1], selv[TOPK ? 1024 : 1], exv[TOPK ? 1024 : 1];
    __shared__ int seli[TOPK ? 1024 : 1];
    const int t = threadIdx.x;
    if constexpr (TOPK) {
        const int B = P / K, TPR = 1024 / E;  // tokens per round
        const int slot = t / E, e = t - slot * E;
        const int ss = t / K, rr = t - ss * K;  // softmax: token slot ss, rank rr
        for (int r0 = 0; r0 < B; r0 += TPR) {
            const bool on = slot < TPR && r0 + slot < B;
            if (on) {
                const float v = logits[(int64_t)(r0 + slot) * E + e];
                sv[t] = v;
                key[t] = rank_key(v, e);
            }
            __syncthreads();
            if (on) {
                const uint64_t kt = key[t];
                const uint64_t* kr = key + slot * E;
                int rank = 0;
                for (int i0 = 0; i0 < E; i0 += 16) {  // 16 keys per step, their LDS reads issued together
                    uint64_t c[16];
#pragma unroll
                    for (int q = 0; q < 16; ++q) c[q] = kr[min(i0 + q, E - 1)];
#pragma unroll
                    for (int q = 0; q < 16; ++q) rank += (i0 + q < E && c[q] > kt) ? 1 : 0;
                }
                if (rank < K) {
                    selv[slot * K + rank] = sv[t];
                    seli[slot * K + rank] = e;
                }
            }
            __syncthreads();
            const bool on2 = ss < TPR && r0 + ss < B;
            if (on2) exv[t] = expf_libm(selv[t] - selv[ss * K]);
            __syncthreads();
            if (on2) {
                float denom = 0.0f;
                for (int j = 0; j < K; ++j) denom = denom + exv[ss * K + j];
                float w = exv[t] / denom;
                const int id = seli[t];
                if (escale) w = w * escale[id];
                const int p = (r0 + ss) * K + rr;
                ids_out[p] = id;
                wts_out[p] = w;
                sid[p] = id;
            }
            __syncthreads();
        }
    }
    auto pid = [&](int p) { return TOPK ? sid[p] : ids[p]; };
    for (int e = t; e < E; e += 1024) cnt[e] = 0;
    __syncthreads();
    for (int p = t; p < P; p += 1024) {
        const int e = min(max(pid(p), 0), E - 1);
        ppos[p] = atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    // inclusive prefix sums of counts and of "active" / "big" flags (E <=
    // 1024): within each wavefront by shuffles, then each thread adds the
    // totals of the wavefronts before its own (integer sums: exact in any order)
    const int c = t < E ? cnt[t] : 0;
    int vc = c, va = c > 0, vf = c > 0 && c >= n_mfma;
    const int lane = t & 63, wv = t >> 6;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int nc = __shfl_up(vc, d), na = __shfl_up(va, d), nf = __shfl_up(vf, d);
        if (lane >= d) {
            vc += nc;
            va += na;
            vf += nf;
        }
    }
    __shared__ int wtot[3][16];
    if (lane == 63) {
        wtot[0][wv] = vc;
        wtot[1][wv] = va;
        wtot[2][wv] = vf;
    }
    __syncthreads();
    for (int q = 0; q < wv; ++q) {
        vc += wtot[0][q];
        va += wtot[1][q];
        vf += wtot[2][q];
    }
    scan[t] = vc;
    act[t] = va;
    big[t] = vf;
    __syncthreads();
    if (t < E && c > 0) {
        const int g = c >= n_mfma ? big[t] - 1 : big[1023] + (act[t] - big[t]) - 1;
        meta[1 + g] = t;                 // gexp
        meta[1 + E + g] = scan[t] - c;   // gstart
        meta[1 + 2 * E + g] = c;         // gcount
    }
    if (t == 0) {
        meta[0] = act[1023];
        meta[1 + 3 * E] = big[1023];
    }
    __syncthreads();
    for (int p = t; p < P; p += 1024) {
        const int e = min(max(pid(p), 0), E - 1);
        plist[scan[e] - cnt[e] + ppos[p]] = p;
    }
}

// The pairs p < P routed to expert e (ids[p] == e), ascending, into lst
// (LDS, at most SCAN_MAX); returns their count (the same in every thread).
// Lets a layer whose experts all take the dot4 kernels skip the grouping
// launch: each (tile, expert) workgroup finds its expert's pairs itself.
constexpr int SCAN_MAX = 1024;
__device__ __forceinline__ int scan_pairs(const int32_t* ids, int P, int e, int* lst, int* wcnt) {
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
    int total = 0;
    for (int base = 0; base < P; base += GT) {
        const int p = base + t;
        const bool m = p < P && ids[p] == e;
        const uint64_t bal = __ballot(m);
        if (lane == 0) wcnt[wv] = __popcll(bal);
        __syncthreads();
        int off = total, sum = 0;
#pragma unroll
        for (int q = 0; q < GW; ++q) {
            off += q < wv ? wcnt[q] : 0;
            sum += wcnt[q];
        }
        if (m) lst[off + __popcll(bal & ((1ull << lane) - 1))] = p;
        total += sum;
        __syncthreads();  // wcnt is rewritten in the next round
    }
    return total;
}

// Gate|up tile j of active expert g for all of its tokens, then GELU*up and
// the q8 of act block j per token. BPW = H/32/8 blocks per wave. in_scale
// (input RMS norm, or null): a token's gate|up sums are first multiplied by
// in_scale[token]. SCAN: the grid's y is the expert, whose pairs the
// workgroup finds in ids[0..P) (scan_pairs) instead of the group list.
template <int BPW, bool REC, bool SCAN>
__global__ __launch_bounds__(GT, 2) void k_grouped_gu(const uint8_t* bank, int64_t expert_bytes, const int32_t* meta,
                                                      const int32_t* plist, const uint8_t* q8x, uint8_t* q8a,
                                                      float* dbg_gu, const float* in_scale, int H, int I, int E,
                                                      int K, int n_mfma, int32_t* rec, const int32_t* ids, int P) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ int slst[SCAN ? SCAN_MAX : 1];
    __shared__ int wcnt[GW];
    const int nb = H >> 5, nbj = I >> 5;
    const int j = blockIdx.x;
    int e, n;
    const int32_t* lst;
    if constexpr (SCAN) {
        e = blockIdx.y;
        n = scan_pairs(ids, P, e, slst, wcnt);
        if (n == 0) return;
        lst = slst;
    } else {
        const int g = blockIdx.y + meta[1 + 3 * E];  // after the MFMA kernels' groups
        if (g >= meta[0]) return;
        e = meta[1 + g];
        n = meta[1 + 2 * E + g];
        if (n >= n_mfma) return;
        lst = plist + meta[1 + E + g];
    }
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
    __shared__ int ctok[NT];
    __shared__ float cscl[NT];  // the tokens' input-norm scales, loaded with the chunk's staging
    for (int c0 = 0; c0 < n; c0 += NT) {
        const int nt = min(NT, n - c0);
        __syncthreads();  // the previous chunk's LDS is consumed
        if (t < nt) ctok[t] = lst[c0 + t] / K;
        __syncthreads();
        {  // x q8 of this chunk's tokens: every load issued before the first store
            constexpr int W = 80 * BPW;  // q8 words per token (nb = 8 * BPW blocks of 10)
            constexpr int MW = (W + GT - 1) / GT;
            // an opaque thread index: the LDS offsets below are not hoisted
            // out of the chunk loop (they would stay live through the dots)
            int tq = t;
            asm volatile("" : "+v"(tq));
            uint32_t v[NT][MW];
#pragma unroll
            for (int tt = 0; tt < NT; ++tt) {
                const uint32_t* src =
                    reinterpret_cast<const uint32_t*>(q8x + (int64_t)ctok[min(tt, nt - 1)] * nb * Q8_BLK);
#pragma unroll
                for (int m = 0; m < MW; ++m) {
                    const int wi = tq + m * GT;
                    v[tt][m] = (tt < nt && wi < W) ? src[wi] : 0u;
                }
            }
            const float sct = in_scale && t < nt ? in_scale[ctok[t]] : 1.0f;  // with the row loads
            if (t < NT) cscl[t] = sct;
#pragma unroll
            for (int tt = 0; tt < NT; ++tt) {
#pragma unroll
                for (int m = 0; m < MW; ++m) {
                    const int wi = tq + m * GT, b = wi / 10, wd = wi - b * 10;
                    if (tt < nt && wi < W) {
                        if (wd >= 2) reinterpret_cast<uint32_t*>(xq)[(tt * nb + b) * 8 + (wd - 2)] = v[tt][m];
                        else reinterpret_cast<uint32_t*>(xp)[(tt * nb + b) * 2 + wd] = v[tt][m];
                    }
                }
            }
        }
        __syncthreads();
#pragma unroll 1
        for (int tt = 0; tt < nt; ++tt) {
            // one token at a time (not unrolled), its blocks' LDS reads in
            // batches of four blocks. The weights pass through an opaque move per token:
            // their nibble masks and f32 scales are not hoisted out of the
            // token loop, where they would take ~100 more registers.
            float acc = 0.0f;
#pragma unroll
            for (int i = 0; i < BPW; ++i)
                asm volatile("" : "+v"(qv[i].x), "+v"(qv[i].y), "+v"(qv[i].z), "+v"(qv[i].w), "+v"(sc[i]));
#pragma unroll
            for (int i = 0; i < BPW; ++i) {
                if (i % 4 == 0 && i > 0) __builtin_amdgcn_sched_barrier(0);
                const int xb = tt * nb + b0 + i;
                const int2 dq = xp[xb];
                const int dot = block_dot_v(qv[i], xq[xb * 2], xq[xb * 2 + 1], dq.y);
                acc = fmaf((float)dot, h2f((uint16_t)sc[i]) * __int_as_float(dq.x), acc);
                if constexpr (REC) {  // test record: the block's int32 dot
                    const int row = r < 32 ? j * 32 + r : I + j * 32 + (r - 32);
                    rec[((int64_t)lst[c0 + tt] * 2 * I + row) * nb + b0 + i] = dot;
                }
            }
            red[(wave * NT + tt) * 64 + r] = acc;
        }
        __syncthreads();
        for (int i = t; i < nt * 64; i += GT) {  // (token, row) sums over the waves, in wave order
            const int tt = i >> 6, rr = i & 63;
            float sv = 0.0f;
#pragma unroll
            for (int v = 0; v < GW; ++v) sv = sv + red[(v * NT + tt) * 64 + rr];
            if (in_scale) sv = sv * cscl[tt];
            rows[tt * 64 + rr] = sv;
            if (dbg_gu) {
                const int p = lst[c0 + tt];
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
            const int p = lst[c0 + tt];
            reinterpret_cast<uint32_t*>(q8a + ((int64_t)p * nbj + j) * Q8_BLK)[wd] = ablk[tt * 10 + wd];
        }
    }
}

// Down rows 128u..128u+127 of active expert g (one 16-row tile per wave;
// thread (rr, s4) holds row rr's blocks s4, s4+4, ...) for all of its tokens.
// SCAN: as k_grouped_gu's.
template <int DB, bool REC, bool SCAN>
__global__ __launch_bounds__(GT, 1) void k_grouped_down(const uint8_t* bank, int64_t expert_bytes, int64_t gu_bytes,
                                                        const int32_t* meta, const int32_t* plist, const uint8_t* q8a,
                                                        float* ydn, int H, int I, int E, int n_mfma, int32_t* rec,
                                                        const int32_t* ids, int P) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ int slst[SCAN ? SCAN_MAX : 1];
    __shared__ int wcnt[GW];
    const int nbj = I >> 5;
    const int u = blockIdx.x;
    int e, n;
    const int32_t* lst;
    if constexpr (SCAN) {
        e = blockIdx.y;
        n = scan_pairs(ids, P, e, slst, wcnt);
        if (n == 0) return;
        lst = slst;
    } else {
        const int g = blockIdx.y + meta[1 + 3 * E];  // after the MFMA kernels' groups
        if (g >= meta[0]) return;
        e = meta[1 + g];
        n = meta[1 + 2 * E + g];
        if (n >= n_mfma) return;
        lst = plist + meta[1 + E + g];
    }
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
        stage<8>(  // act q8 of this chunk's pairs
            nt * nbj * 10,
            [&](int i) {
                const int tt = i / (nbj * 10), rem = i - tt * nbj * 10;
                const int p = lst[c0 + tt];
                return reinterpret_cast<const uint32_t*>(q8a + (int64_t)p * nbj * Q8_BLK)[rem];
            },
            [&](int i, uint32_t v) {
                const int tt = i / (nbj * 10), rem = i - tt * nbj * 10, b = rem / 10, wd = rem - b * 10;
                if (wd >= 2) reinterpret_cast<uint32_t*>(aq)[(tt * nbj + b) * 8 + (wd - 2)] = v;
                else reinterpret_cast<uint32_t*>(ap)[(tt * nbj + b) * 2 + wd] = v;
            });
        __syncthreads();
        for (int tt = 0; tt < nt; ++tt) {
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < DB; ++k) {
                const int b = s4 + 4 * k;
                const int xb = tt * nbj + min(b, nbj - 1);
                const int2 pq = ap[xb];
                const int dot = block_dot_v(dq[k], aq[xb * 2], aq[xb * 2 + 1], pq.y);
                const float v = (float)dot * (h2f((uint16_t)dsc[k]) * __int_as_float(pq.x));
                acc = b < nbj ? acc + v : acc;
                if constexpr (REC) {  // test record: the block's int32 dot
                    if (b < nbj)
                        rec[((int64_t)lst[c0 + tt] * H + u * DU + wave * 16 + rr) * nbj + b] = dot;
                }
            }
            acc += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(acc), 0xB1, 0xF, 0xF, false));
            acc += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(acc), 0x4E, 0xF, 0xF, false));
            if (s4 == 0) {
                const int p = lst[c0 + tt];
                ydn[(int64_t)p * H + u * DU + wave * 16 + rr] = acc;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// int8 MFMA tile path, for groups of at least n_min tokens.
//
// v_mfma_i32_16x16x32_i8: D[16 rows][16 tokens] += A[16 rows][32] *
// B[32][16 tokens]; lane l holds A row l%16 and B column l%16 at k =
// 8*(l/16)..+7, and D rows 4*(l/16)..+3 of column l%16. One MFMA is one q4_0
// block (32 weights) of 16 rows against the q8 blocks of 16 tokens. The 32 k
// of a block are ordered so that lane group g = l/16 takes elements
// 4g..4g+3 and 16+4g..16+4g+3: for the weights the low and the high nibbles
// of qs word g (one dword, two masks), for the activations q8 words g and
// 4+g. The nibbles enter unsigned (0..15) and the accumulator starts at
// -8 * qsum of the token's block, so D is exactly the block's int32 dot
// sum (q-8)*q8 (ft-core/src/q4_0.rs:105-118). Per (row, token) the blocks
// then accumulate as acc = fma(float(D), d4 * d8, acc), in block order.
// ---------------------------------------------------------------------------
typedef int v4i __attribute__((ext_vector_type(4)));
constexpr int MT = 16;  // tokens per MFMA tile
// token stride of the gate|up wave partials in LDS: one more than MT, so the
// wave-order sums (consecutive lanes: consecutive rows) read distinct banks
constexpr int MTP = MT + 1;
static_assert(MT * 10 <= GT, "k_mfma_gu stores a chunk's q8 words with one thread each");

struct ActOp {
    long b;    // B operand: q8 words g and 4+g
    float d;   // the block's d
    int qsum;  // the block's sum of q
};

// Raw buffer loads: a per-lane 32-bit offset plus a uniform one (scalar
// register or immediate), so per-block addresses cost no vector registers;
// an offset past num_records reads 0.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint32_t buf_ld(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}

// A token's q8 block as the B operand of lane group g, from the q8m layout
// (GroupWs::q8m): q8 words (g, g+4) at vq + sq, {d, qsum} at vd + sd, one
// 8-byte load each. A lane without a token passes offsets past the buffer's
// end (NO_TOKEN; the buffer is smaller) and gets zeros.
constexpr uint32_t NO_TOKEN = 0x80000000u;
__device__ __forceinline__ ActOp act_op_m(__amdgpu_buffer_rsrc_t r, uint32_t vq, uint32_t vd, uint32_t sq,
                                          uint32_t sd) {
    const u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(r, vq, sq, 0);
    const u32x2 dq = __builtin_amdgcn_raw_buffer_load_b64(r, vd, sd, 0);
    ActOp a;
    a.b = (long)(((uint64_t)w.y << 32) | w.x);
    a.d = __uint_as_float(dq.x);
    a.qsum = (int)dq.y;
    return a;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 4x4 transpose across the 16-lane rows of a wavefront: on entry lane row g
// holds M[g][0..3] in (a0..a3), on exit T[g][j] = M[j][g]. Two 32-lane swaps
// exchange the off-diagonal 2x2 blocks, two 16-lane swaps the off-diagonal
// elements inside each block.
__device__ __forceinline__ void quad_transpose(uint32_t& a0, uint32_t& a1, uint32_t& a2, uint32_t& a3) {
    const auto s0 = __builtin_amdgcn_permlane32_swap(a0, a2, false, false);
    const auto s1 = __builtin_amdgcn_permlane32_swap(a1, a3, false, false);
    const auto s2 = __builtin_amdgcn_permlane16_swap(s0[0], s1[0], false, false);
    const auto s3 = __builtin_amdgcn_permlane16_swap(s0[1], s1[1], false, false);
    a0 = s2[0];
    a1 = s2[1];
    a2 = s3[0];
    a3 = s3[1];
}

// A operand from qs word g of a row's block: low nibbles, then high nibbles.
__device__ __forceinline__ long nib_op(uint32_t w) {
    return (long)(((uint64_t)((w >> 4) & 0x0F0F0F0Fu) << 32) | (w & 0x0F0F0F0Fu));
}

__device__ __forceinline__ v4i c_init(int qsum) {
    const int c = -8 * qsum;
    const v4i v = {c, c, c, c};
    return v;
}

// Four f16 scales (8 bytes) at p, widened.
__device__ __forceinline__ void scales4(const uint16_t* p, float (&sc)[4]) {
    const uint2 s2 = *reinterpret_cast<const uint2*>(p);
    sc[0] = h2f((uint16_t)(s2.x & 0xFFFF));
    sc[1] = h2f((uint16_t)(s2.x >> 16));
    sc[2] = h2f((uint16_t)(s2.y & 0xFFFF));
    sc[3] = h2f((uint16_t)(s2.y >> 16));
}

// Gate|up tiles of the MFMA groups (tile j: 64 rows, gate rows 32j.. and up
// rows I+32j..), each for its expert's tokens 16 at a time, then GELU*up and
// the q8 of act block j per token. Persistent: one workgroup per CU walks a
// contiguous range of (expert group, tile j) items, each in chunks of 16
// tokens (units). Wave w takes blocks [w*BPW, (w+1)*BPW) of the 64 rows as
// four 16-row MFMA tiles; the 8 wave partials of a (row, token) are summed
// in wave order. The tokens' q8 rows of the current chunk sit in LDS
// (staged when the group or chunk changes, which a contiguous range makes
// rare), so the MFMA B operands are LDS reads, read one block ahead. The
// weights stream through registers: a wave holds its BPW blocks' qs dwords
// of a unit, and consuming block b refills that slot with block b of the
// NEXT unit, so the next tile streams during this unit's MFMAs and its
// epilogue (wave sums, GELU*up, q8). A tile's f16 scales go through one LDS
// buffer as f32 (widened once there, not by each of the 16 lanes of a lane
// group per block): the next unit's are loaded into registers (16 bytes per
// thread and round) once every wave is past this unit's MFMAs, and stored to
// LDS at the end of this unit's epilogue. Per (row, token): acc = fma(float(D_b), d4_b *
// d8_b, acc) over the wave's blocks in block order, then the wave partials in
// wave order.
//
// The scales once went to LDS by direct global-to-LDS loads two units ahead.
// A load into LDS completes in order behind the ring's weight loads, and the
// compiler cannot tell it apart from the epilogue's LDS traffic: the fence of
// the next barrier and the next LDS read each waited for it with s_waitcnt
// vmcnt(0), which drained the next unit's weight loads at the start of every
// epilogue. Loaded into registers, the only wait is the one before their LDS
// store at the end of the epilogue.

struct MfUnit {
    const uint8_t* T;  // the tile: [nb][64] f16 scales, then [nb][64][16 B] qs
    int g, s0, n, j, c0, nt, item;
    bool live;
};

template <int BPW, bool REC>
__global__ __launch_bounds__(GT, 1) void k_mfma_gu(const uint8_t* __restrict__ bank, int64_t expert_bytes,
                                                     const int32_t* __restrict__ meta,
                                                     const int32_t* __restrict__ plist,
                                                     const uint8_t* __restrict__ q8x, uint8_t* q8m, float* dbg_gu,
                                                     const float* __restrict__ in_scale, int H, int I, int E, int K,
                                                     int P, int32_t* rec) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int SPT = (128 * 128 + GT * 16 - 1) / (GT * 16);  // scale rounds, up to nb = 128 (H 4096)
    const int nb = H >> 5, nbj = I >> 5;
    const int n_items = meta[1 + 3 * E] * nbj;  // (group, tile) pairs of the MFMA groups (first in the list)
    const int per = (n_items + (int)gridDim.x - 1) / (int)gridDim.x;
    const int it0 = (int)blockIdx.x * per, it1 = min(n_items, it0 + per);
    if (it0 >= it1) return;
    // LDS: scales [nb][64] f32 | wave partials [GW][64][MTP] | sums [MT][64] |
    // act [MT][32] | act q8 [MT][10] | the chunk's tokens (pair, norm scale)
    // [MT] x2 | the chunk's q8 rows [MT][nb*10 + 1] u32
    float* scl = reinterpret_cast<float*>(lds);
    float* red = reinterpret_cast<float*>(lds + nb * 256);
    float* rows = red + GW * 64 * MTP;
    float* actv = rows + MT * 64;
    uint32_t* ablk = reinterpret_cast<uint32_t*>(actv + MT * 32);
    int* tok_p = reinterpret_cast<int*>(ablk + MT * 10);
    float* tok_s = reinterpret_cast<float*>(tok_p + MT);
    uint32_t* xq = reinterpret_cast<uint32_t*>(tok_s + MT);
    const int xs = nb * 10 + 1;  // token stride (dwords), odd: the 16 tokens' rows start in different banks
    const int t = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(t >> 6), li = t & 15, lg = (t >> 4) & 3;
    const int b0 = wave * BPW;
    const uint32_t vw16 = lg * 256 + li * 16;
    auto bind = [&](int it, int c, bool live) __attribute__((always_inline)) {
        MfUnit u;
        u.live = live;
        u.item = it;
        it = live ? it : it0;  // a dead unit is bound to a valid item and never computed
        u.g = it / nbj;
        u.j = it - u.g * nbj;
        const int e = meta[1 + u.g];
        u.s0 = meta[1 + E + u.g];
        u.n = meta[1 + 2 * E + u.g];
        u.c0 = live ? c : 0;
        u.nt = min(MT, u.n - u.c0);
        u.T = bank + (int64_t)e * expert_bytes + (int64_t)u.j * nb * 1152;
        return u;
    };
    auto after = [&](const MfUnit& u) __attribute__((always_inline)) {  // the unit after u in this range
        if (!u.live) return u;
        if (u.c0 + MT < u.n) return bind(u.item, u.c0 + MT, true);
        return bind(u.item + 1, 0, u.item + 1 < it1);
    };
    auto same_tile = [](const MfUnit& a, const MfUnit& c) { return a.g == c.g && a.j == c.j; };
    uint32_t aw[BPW][4];
    // slot b <- block b of unit u (dead: a descriptor of 0 bytes returns zeros and reads nothing)
    auto issue_block = [&](int b, const MfUnit& u) __attribute__((always_inline)) {
        // one 16-byte load: lane group g takes the four qs words of row
        // 16g + li (1 KB contiguous per wave); quad_transpose turns them into
        // word g of rows li, 16 + li, 32 + li, 48 + li when the block is used
        const __amdgpu_buffer_rsrc_t rw = buf_rsrc(u.T + nb * 128, u.live ? (uint32_t)nb * 1024 : 0u);
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rw, vw16, (b0 + b) * 1024, 0);
        aw[b][0] = v.x;
        aw[b][1] = v.y;
        aw[b][2] = v.z;
        aw[b][3] = v.w;
    };
    // unit u's tile scales (nb * 128 bytes of f16) into registers, 16 bytes
    // per thread and round (dead or past the end: zeros, nothing read), and
    // from there, widened, into scl once no wave reads the previous tile's
    u32x4 sst[SPT];
    auto load_scales = [&](const MfUnit& u) __attribute__((always_inline)) {
        const __amdgpu_buffer_rsrc_t rs = buf_rsrc(u.T, u.live ? (uint32_t)nb * 128 : 0u);
#pragma unroll
        for (int r = 0; r < SPT; ++r)  // the offset in the per-lane part: that is the part the range check sees
            sst[r] = __builtin_amdgcn_raw_buffer_load_b128(rs, (r * GT + t) * 16, 0, 0);
    };
    auto store_scales = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < SPT; ++r) {
            const int i = (r * GT + t) * 8;  // the first of this thread's 8 scales
            if (i < nb * 64) {
                const u32x4 h = sst[r];
                float4* d = reinterpret_cast<float4*>(scl + i);
                d[0] = make_float4(h2f((uint16_t)(h.x & 0xFFFF)), h2f((uint16_t)(h.x >> 16)),
                                   h2f((uint16_t)(h.y & 0xFFFF)), h2f((uint16_t)(h.y >> 16)));
                d[1] = make_float4(h2f((uint16_t)(h.z & 0xFFFF)), h2f((uint16_t)(h.z >> 16)),
                                   h2f((uint16_t)(h.w & 0xFFFF)), h2f((uint16_t)(h.w >> 16)));
            }
        }
    };
    // unit u's tokens (pair, norm scale) into tok_p/tok_s and their q8 rows
    // into xq (token slots >= nt: the last token again; their MFMA columns
    // are never read). Only between units; the caller syncs afterwards.
    auto stage_act = [&](const MfUnit& u) __attribute__((always_inline)) {
        if (t < MT) {
            const int pp = plist[u.s0 + u.c0 + min(t, u.nt - 1)];
            tok_p[t] = pp;
            tok_s[t] = in_scale ? in_scale[pp / K] : 1.0f;
        }
        __syncthreads();
        const int per_tok = nb * 10;
        for (int i = t; i < MT * per_tok; i += GT) {
            const int tt = i / per_tok, w = i - tt * per_tok;
            xq[tt * xs + w] = reinterpret_cast<const uint32_t*>(q8x + (int64_t)(tok_p[tt] / K) * nb * Q8_BLK)[w];
        }
    };
    // a block's LDS operands: this lane's token words, its d and qsum, and
    // the scales of rows 16m + 4lg .. +3 for the 4 tiles m
    struct Ops {
        uint32_t lo, hi, d, qsum;
        float4 sc[4];
    };
    MfUnit cur = bind(it0, 0, true);
    MfUnit nxt = after(cur);
    load_scales(cur);
#pragma unroll
    for (int b = 0; b < BPW; ++b) issue_block(b, cur);
    store_scales();
    stage_act(cur);
    int act_g = cur.g, act_c0 = cur.c0;  // the chunk whose q8 rows are in xq
    __syncthreads();
    auto step = [&]() __attribute__((always_inline)) {
        const MfUnit n2 = after(nxt);
        const bool nxt_scales = nxt.live && !same_tile(nxt, cur);  // a new tile (else scl already holds them)
        const int pme = tok_p[li];  // this lane's token pair (REC)
        const uint32_t* xl = xq + li * xs;  // this lane's token row
        auto ops = [&](int blk) __attribute__((always_inline)) {
            Ops o;
            o.lo = xl[blk * 10 + 2 + lg];
            o.hi = xl[blk * 10 + 6 + lg];
            o.d = xl[blk * 10];
            o.qsum = xl[blk * 10 + 1];
#pragma unroll
            for (int m = 0; m < 4; ++m) o.sc[m] = *reinterpret_cast<const float4*>(scl + blk * 64 + 16 * m + 4 * lg);
            return o;
        };
        float acc[4][4];
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[m][v] = 0.0f;
        Ops o = ops(b0);
#pragma unroll
        for (int b = 0; b < BPW; ++b) {
            const int blk = b0 + b;
            const Ops cu = o;
            if (b + 1 < BPW) o = ops(blk + 1);  // the next block's LDS operands, in flight during these MFMAs
            const v4i c = c_init((int)cu.qsum);
            const long bop = (long)(((uint64_t)cu.hi << 32) | cu.lo);
            v4i d[4];
            quad_transpose(aw[b][0], aw[b][1], aw[b][2], aw[b][3]);
#pragma unroll
            for (int m = 0; m < 4; ++m) d[m] = __builtin_amdgcn_mfma_i32_16x16x32_i8(nib_op(aw[b][m]), bop, c, 0, 0, 0);
            issue_block(b, nxt);
            const float ad = __uint_as_float(cu.d);
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                if constexpr (REC) {  // test record: D = the (row, token) blocks' int32 dots
                    if (li < cur.nt)
#pragma unroll
                        for (int v = 0; v < 4; ++v) {
                            const int rr = 16 * m + 4 * lg + v;
                            const int row = rr < 32 ? cur.j * 32 + rr : I + cur.j * 32 + (rr - 32);
                            rec[((int64_t)pme * 2 * I + row) * nb + blk] = d[m][v];
                        }
                }
                const float sc[4] = {cu.sc[m].x, cu.sc[m].y, cu.sc[m].z, cu.sc[m].w};
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[m][v] = fmaf((float)d[m][v], sc[v] * ad, acc[m][v]);
            }
            __builtin_amdgcn_sched_barrier(0);  // one block's MFMA results live at a time
        }
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int v = 0; v < 4; ++v) red[(wave * 64 + 16 * m + 4 * lg + v) * MTP + li] = acc[m][v];
        __syncthreads();  // every wave is past its MFMAs: act rows and scl may change below
        if (nxt_scales) load_scales(nxt);
        for (int i = t; i < cur.nt * 64; i += GT) {  // (token, row) sums over the waves, in wave order
            const int tt = i >> 6, rr = i & 63;
            float sv = 0.0f;
#pragma unroll
            for (int v = 0; v < GW; ++v) sv = sv + red[(v * 64 + rr) * MTP + tt];
            const int pp = tok_p[tt];
            if (in_scale) sv = sv * tok_s[tt];
            rows[tt * 64 + rr] = sv;
            if (dbg_gu) dbg_gu[(int64_t)pp * 2 * I + (rr < 32 ? cur.j * 32 + rr : I + cur.j * 32 + (rr - 32))] = sv;
        }
        __syncthreads();
        for (int i = t; i < cur.nt * 32; i += GT) {
            const int tt = i >> 5, cc = i & 31;
            actv[tt * 32 + cc] = gelu_tanh(rows[tt * 64 + cc]) * rows[tt * 64 + 32 + cc];
        }
        __syncthreads();
        if (t < 4 * cur.nt) quantize_block_quad(actv + (t >> 2) * 32, t & 3, ablk + (t >> 2) * 10);
        __syncthreads();
        if (t < cur.nt * 10) {  // q8m at group position q (MT * 10 <= GT)
            const int tt = t / 10, wd = t - tt * 10, q = cur.s0 + cur.c0 + tt, wq = wd - 2;
            const uint32_t o = wd < 2 ? (uint32_t)((P * nbj * 4 + cur.j * P + q) * 2 + wd)
                                      : (uint32_t)(((cur.j * 4 + (wq & 3)) * P + q) * 2 + (wq >> 2));
            reinterpret_cast<uint32_t*>(q8m)[o] = ablk[t];
        }
        if (!nxt.live) return false;
        if (nxt_scales) store_scales();
        if (nxt.g != act_g || nxt.c0 != act_c0) {
            stage_act(nxt);
            act_g = nxt.g;
            act_c0 = nxt.c0;
        }
        __syncthreads();
        cur = nxt;
        nxt = n2;
        return true;
    };
    while (step()) {
    }
}

// Down rows of active expert g for its tokens, 16 at a time. The workgroup
// takes GW/KS groups of RT consecutive 16-row down tiles; wave w works on the
// RT tiles of group w/KS (they share each block's activation operand), K
// slice w%KS (blocks [s*BW, s*BW+BW) below nbj); the KS slice partials of a
// (row, token) are summed in slice order into y[pair][row]. With KS > 1 the
// partials overlay the tiles' scales in LDS (restaged for each 16 tokens),
// so two workgroups fit a CU. Blocks go in NBB-block batches, NBUF batches in
// flight (register buffers).
template <int KS, int BW, int RT, int NBB, int NBUF, bool REC>
__global__ __launch_bounds__(GT, 4) void k_mfma_down(const uint8_t* bank, int64_t expert_bytes, int64_t gu_bytes,
                                                     const int32_t* meta, const int32_t* plist, const uint8_t* q8m,
                                                     int P, float* ydn, int H, int I, int E, int n_min,
                                                     int32_t* rec) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int TPW = GW / KS;   // tile groups per workgroup
    constexpr int TW = TPW * RT;   // tiles per workgroup
    const int nbj = I >> 5, dn_tile = nbj * 288;
    const int u = blockIdx.x, g = blockIdx.y;
    if (g >= meta[1 + 3 * E]) return;  // groups of >= n_min tokens come first
    const int e = meta[1 + g], s0 = meta[1 + E + g], n = meta[1 + 2 * E + g];
    if (n < n_min) return;
    // LDS: the tiles' scales [TW][nbj][16] f16; slice partials [GW][RT][16][MT]
    // in the same bytes once the K loop is done
    uint16_t* scl = reinterpret_cast<uint16_t*>(lds);
    float* red = reinterpret_cast<float*>(lds);
    const int t = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(t >> 6), li = t & 15, lg = (t >> 4) & 3;
    const int tl = wave / KS, sl = wave % KS, bs = sl * BW;
    const int tile0 = (u * TPW + tl) * RT;  // this wave's first tile
    const uint8_t* D0 = bank + (int64_t)e * expert_bytes + gu_bytes;  // the expert's down tiles
    const uint16_t* st = scl + tl * RT * nbj * 16;
    // the wave's RT tiles: qs of tile tile0+m at m*dn_tile + nbj*32 from D0 + tile0*dn_tile
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(D0 + (int64_t)tile0 * dn_tile, (uint32_t)(RT * dn_tile));
    const __amdgpu_buffer_rsrc_t ra = buf_rsrc(q8m, (uint32_t)P * nbj * Q8_BLK);  // < NO_TOKEN bytes
    const uint32_t vw = nbj * 32 + li * 16 + 4 * lg, vw4 = nbj * 32 + lg * 256 + li * 16;
    for (int c0 = 0; c0 < n; c0 += MT) {
        const int nt = min(MT, n - c0);
        const int q = s0 + c0 + min(li, nt - 1), p = plist[q];
        // this lane's operand words of block bb: 8 bytes at bb * 32P + vq (the
        // 16 tokens' words of a lane group in 128 contiguous bytes), d and
        // qsum at P * nbj * 32 + bb * 8P + vd
        const bool ok = li < nt;
        const uint32_t vq = ok ? (uint32_t)(lg * P + q) * 8 : NO_TOKEN;
        const uint32_t vd = ok ? (uint32_t)P * nbj * 32 + (uint32_t)q * 8 : NO_TOKEN;
        // blocks in NBB-block batches, the loads of the batch NBUF - 1 ahead
        // issued before the current batch's MFMAs (NBUF register buffers)
        constexpr int NBATCH = BW / NBB;
        uint32_t aw[NBUF][NBB][RT];
        ActOp av[NBUF][NBB];
        // NBB == 4: one 16-byte load per tile for the batch's four blocks,
        // lane group g taking all four qs words of its row in block 4k+g (1 KB
        // contiguous per wave), turned into word g of each block by
        // quad_transpose when the batch is consumed (blocks past the row are
        // read, never used: the descriptor bounds the reads)
        auto load = [&](int k, int buf) __attribute__((always_inline)) {
            if constexpr (NBB == 4) {
#pragma unroll
                for (int m = 0; m < RT; ++m) {
                    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rw, vw4, m * dn_tile + (bs + k * 4) * 256, 0);
                    aw[buf][0][m] = v.x;
                    aw[buf][1][m] = v.y;
                    aw[buf][2][m] = v.z;
                    aw[buf][3][m] = v.w;
                }
            }
#pragma unroll
            for (int b = 0; b < NBB; ++b) {
                const int bb = min(bs + k * NBB + b, nbj - 1);
                if constexpr (NBB != 4) {
#pragma unroll
                    for (int m = 0; m < RT; ++m) aw[buf][b][m] = buf_ld(rw, vw, m * dn_tile + bb * 256);
                }
                av[buf][b] = act_op_m(ra, vq, vd, bb * 32 * P, bb * 8 * P);
            }
        };
        float acc[RT][4];
#pragma unroll
        for (int m = 0; m < RT; ++m)
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[m][v] = 0.0f;
        // this slice's batches (uniform; none when the slice starts past nbj)
        const int nbat = max(0, min(NBATCH, (nbj - bs + NBB - 1) / NBB));
#pragma unroll
        for (int k = 0; k < NBUF - 1; ++k)
            if (k < nbat) load(k, k);
        if (c0 == 0 || KS > 1) {  // the tiles' scales to LDS, with the first batches in flight
            stage<8>(
                TW * nbj * 8,
                [&](int i) {
                    const int k = i / (nbj * 8), r = i - k * nbj * 8;
                    return reinterpret_cast<const uint32_t*>(D0 + (int64_t)(u * TW + k) * dn_tile)[r];
                },
                [&](int i, uint32_t v) { reinterpret_cast<uint32_t*>(scl)[i] = v; });
            __syncthreads();
        }
        // rounds of NBUF batches, register buffer j holding batch kb + j; the
        // rounds are a loop (not unrolled), so a block's offsets are scalar
        // adds rather than registers held across the slice
#pragma unroll 1
        for (int kb = 0; kb < nbat; kb += NBUF) {
#pragma unroll
          for (int j = 0; j < NBUF; ++j) {
            const int k = kb + j;
            if (k >= nbat) break;  // uniform
            // unconditional (past the slice: the last block again), so the
            // wait below counts only this batch's loads, not the prefetch's
            load(k + NBUF - 1, (j + NBUF - 1) % NBUF);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (NBB == 4) {
#pragma unroll
                for (int m = 0; m < RT; ++m) quad_transpose(aw[j][0][m], aw[j][1][m], aw[j][2][m], aw[j][3][m]);
            }
#pragma unroll
            for (int b = 0; b < NBB; ++b) {
                if (bs + k * NBB + b < nbj) {  // uniform
                    const ActOp a = av[j][b];
                    const v4i c = c_init(a.qsum);
#pragma unroll
                    for (int m = 0; m < RT; ++m) {
                        const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(nib_op(aw[j][b][m]), a.b, c, 0, 0, 0);
                        if constexpr (REC) {  // test record: D = the (row, token) blocks' int32 dots
                            if (li < nt)
#pragma unroll
                                for (int v = 0; v < 4; ++v)
                                    rec[((int64_t)p * H + (tile0 + m) * 16 + 4 * lg + v) * nbj + bs + k * NBB + b] = d[v];
                        }
                        float sc[4];
                        scales4(st + (m * nbj + bs + k * NBB + b) * 16 + 4 * lg, sc);
#pragma unroll
                        for (int v = 0; v < 4; ++v) acc[m][v] = fmaf((float)d[v], sc[v] * a.d, acc[m][v]);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);  // one block's MFMA results live at a time
            }
          }
        }
        if (KS == 1) {
            if (li < nt) {
#pragma unroll
                for (int m = 0; m < RT; ++m)
#pragma unroll
                    for (int v = 0; v < 4; ++v) ydn[(int64_t)p * H + (tile0 + m) * 16 + 4 * lg + v] = acc[m][v];
            }
        } else {
            __syncthreads();  // every wave is done with the scales
#pragma unroll
            for (int m = 0; m < RT; ++m)
#pragma unroll
                for (int v = 0; v < 4; ++v) red[((wave * RT + m) * 16 + 4 * lg + v) * MT + li] = acc[m][v];
            __syncthreads();
            for (int i = t; i < TW * 16 * nt; i += GT) {  // (tile, row, token) sums over the slices in order
                const int k = i / (16 * nt), r = (i / nt) % 16, tt = i % nt;
                const int kg = k / RT, m = k % RT;
                float sv = 0.0f;
#pragma unroll
                for (int q = 0; q < KS; ++q) sv = sv + red[(((kg * KS + q) * RT + m) * 16 + r) * MT + tt];
                ydn[(int64_t)plist[s0 + c0 + tt] * H + (u * TW + k) * 16 + r] = sv;
            }
            __syncthreads();
        }
    }
}

// The MFMA groups' act quants from q8m back into the pairs' rows of q8a
// ([P][nbj][40]), for the debug copy: MFMA group blockIdx.y, one thread per
// (position, block, word) of the group.
__global__ __launch_bounds__(256) void k_q8m_rows(const uint32_t* q8m, const int32_t* meta, const int32_t* plist,
                                                  uint8_t* q8a, int P, int nbj, int E) {
    const int g = blockIdx.y;
    if (g >= meta[1 + 3 * E]) return;  // not an MFMA group
    const int s0 = meta[1 + E + g], n = meta[1 + 2 * E + g];
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n * nbj * 10; i += gridDim.x * 256) {
        const int wd = i % 10, j = i / 10 % nbj, q = s0 + i / (10 * nbj), wq = wd - 2;
        const int64_t o = wd < 2 ? ((int64_t)P * nbj * 4 + (int64_t)j * P + q) * 2 + wd
                                 : (((int64_t)j * 4 + (wq & 3)) * P + q) * 2 + (wq >> 2);
        reinterpret_cast<uint32_t*>(q8a + ((int64_t)plist[q] * nbj + j) * Q8_BLK)[wd] = q8m[o];
    }
}

// x_out[t] = x[t] + sum_k (y[t*K+k] * w[t*K+k]), slots in order
// (ft-model/src/lib.rs:1634-1646).
__global__ __launch_bounds__(256) void k_grouped_combine(const float* y, const float* wts, const float* x, float* out,
                                                         int H, int K) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x, s = blockIdx.y;
    if (i >= H) return;
    const float xv = x[(int64_t)s * H + i];
    float h = 0.0f;
    for (int k0 = 0; k0 < K; k0 += 8) {  // the loads of 8 slots issued together, then the sum in slot order
        float yv[8], wv[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int k = min(k0 + q, K - 1);
            yv[q] = y[((int64_t)s * K + k) * H + i];
            wv[q] = wts[s * K + k];
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float part = yv[q] * wv[q];
            h = k0 + q < K ? h + part : h;
        }
    }
    out[(int64_t)s * H + i] = xv + h;
}

int check_grouped_shape(const char* nm, int64_t B, int64_t H, int64_t I, int64_t E, int64_t K) {
    if (H != 2816 && H != 4096)
        return fail(FT_HIP_E_SHAPE, "%s: hidden=%lld: built for hidden 2816 and 4096", nm, (long long)H);
    if (I <= 0 || I % 32 || I / 32 > 512)
        return fail(FT_HIP_E_SHAPE, "%s: inter=%lld must be a multiple of 32 in [32, 16384]", nm, (long long)I);
    if (E <= 0 || E > 1024) return fail(FT_HIP_E_SHAPE, "%s: n_experts not in [1, 1024]", nm);
    if (K <= 0 || K > 32 || K > E) return fail(FT_HIP_E_SHAPE, "%s: top_k not in [1, min(32, n_experts)]", nm);
    if (B < 0 || B * K > MAX_PAIRS) return fail(FT_HIP_E_SHAPE, "%s: n_seqs*top_k must be <= %d", nm, MAX_PAIRS);
    return FT_HIP_OK;
}

}  // namespace

extern "C" size_t ft_hip_moe_layer_grouped_workspace_bytes(int64_t n_seqs, int64_t hidden, int64_t inter,
                                                           int64_t n_experts, int64_t top_k) {
    // by division, so that no product below can wrap
    if (n_seqs < 0 || top_k <= 0 || top_k > 1024 || n_seqs > 65535 / top_k || hidden <= 0 || hidden > 32 * 4096 ||
        inter <= 0 || inter > 32 * 4096 || n_experts <= 0 || n_experts > 65535)
        return 0;
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
    if (n_experts * 16 >= hidden / 32) {  // logits, norm scale and q8(x) in one launch
        if ((rc = ft::launch_route_prep(stream, router_w, x, router_bias, ctx->input_norm, w.inv, w.q8x, w.logits,
                                        hidden, n_experts, n_seqs)))
            return rc;
    } else {
        if (inv && (rc = ft::launch_rms_inv(stream, x, w.inv, hidden, n_seqs))) return rc;
        if ((rc = ft::launch_router_logits(stream, router_w, x, router_bias, inv, w.logits, hidden, n_experts, n_seqs)))
            return rc;
        if ((rc = ft_hip_quantize_q8(ctx, stream, x, hidden, w.q8x, hidden, n_seqs))) return rc;
    }
    // the routing inside the grouping launch for few experts (up to 32, in up
    // to 4 rounds of 1024/E tokens), else its own launch: one workgroup
    // ranking 128 logits per token is LDS-bound (batch 16 of the Gemma
    // shape: 188.4 vs 172.6 us/token); at 8 experts it saves the launch
    const bool topk_in = E <= 32 && n_seqs <= 4 * (1024 / E);
    if (!topk_in && (rc = ft_hip_topk_router(ctx, stream, w.logits, expert_scale, ids, wts, n_experts, top_k, n_seqs)))
        return rc;
    // groups of >= n_mfma tokens take the MFMA tile kernels, the others the
    // dot4 kernels; rows longer than 32 blocks (I > 1024) only the former.
    // Automatic (0): every group on one family, MFMA from 4 pairs per expert
    // on (measured on the Gemma shape: dot4 faster at 1 pair per expert,
    // 168.9 vs 217.5 us/token at batch 16; MFMA at 4, 73.5 vs 76.7 at batch
    // 64, and above; one family's launches beat a split of both)
    int n_mfma = ctx->grouped_mfma_min;
    if (n_mfma <= 0) n_mfma = (int64_t)P >= 4 * n_experts ? 1 : std::numeric_limits<int>::max();
    if (nbj > 32) n_mfma = 1;
    // every expert on the dot4 kernels, routing already in ids: the dot4
    // workgroups find their expert's pairs themselves (no grouping launch)
    const bool scan = !topk_in && n_mfma > P && P <= SCAN_MAX;
    if (!scan) {
        hipLaunchKernelGGL(topk_in ? k_group_pairs<true> : k_group_pairs<false>, dim3(1), dim3(1024), 0, s,
                           (const int32_t*)ids, P, E, n_mfma, w.meta, w.plist, w.ppos, (const float*)w.logits,
                           expert_scale, ids, wts, K);
        if ((rc = launch_status("moe_layer_grouped/group"))) return rc;
    }
    const int gmax = std::min(E, P);
    const int gbig = std::min(gmax, n_mfma > P ? 0 : P / n_mfma);  // at most this many groups of >= n_mfma tokens
    const bool dot4 = n_mfma > 1, mfma = n_seqs >= n_mfma;
    if (mfma && (int64_t)P * nbj * Q8_BLK >= (int64_t)NO_TOKEN)
        return fail(FT_HIP_E_SHAPE, "%s: %d pairs x %d act blocks: the MFMA path's activation buffer must stay under 2 GiB",
                    nm, P, nbj);
    // a block-dot record (ft_hip_set_block_dot_record, tests only) selects
    // the instantiations that store every int32 block dot
    int32_t* rgu = ctx->rec_gu;
    int32_t* rdn = ctx->rec_dn;
    const bool rec = rgu && rdn;
    if (dot4) {
        const size_t lds_gu = (size_t)NT * nb * 40 + sizeof(float) * (GW * NT * 64 + NT * 64 + NT * 32) + 4 * NT * 10;
        auto kern = scan ? (H == 2816 ? (rec ? k_grouped_gu<11, true, true> : k_grouped_gu<11, false, true>)
                                      : (rec ? k_grouped_gu<16, true, true> : k_grouped_gu<16, false, true>))
                         : (H == 2816 ? (rec ? k_grouped_gu<11, true, false> : k_grouped_gu<11, false, false>)
                                      : (rec ? k_grouped_gu<16, true, false> : k_grouped_gu<16, false, false>));
        hipLaunchKernelGGL(kern, dim3(nbj, scan ? E : gmax), dim3(GT), lds_gu, s, (const uint8_t*)bank, eb,
                           (const int32_t*)w.meta, (const int32_t*)w.plist, (const uint8_t*)w.q8x, w.q8a, dbg_gu, inv, H,
                           I, E, K, n_mfma, rgu, (const int32_t*)ids, P);
        if ((rc = launch_status("moe_layer_grouped/gate_up"))) return rc;
    }
    if (mfma) {
        const size_t lds_mg = (size_t)nb * 256 + sizeof(float) * (GW * 64 * MTP + MT * 64 + MT * 32) + 4 * MT * 10 +
                              8 * MT + 4 * (size_t)MT * (nb * 10 + 1);
        auto kern = H == 2816 ? (rec ? k_mfma_gu<11, true> : k_mfma_gu<11, false>)
                              : (rec ? k_mfma_gu<16, true> : k_mfma_gu<16, false>);
        const int grid = std::min(ctx->num_cus, nbj * gbig);  // persistent: one workgroup per CU
        hipLaunchKernelGGL(kern, dim3(grid), dim3(GT), lds_mg, s, (const uint8_t*)bank, eb, (const int32_t*)w.meta,
                           (const int32_t*)w.plist, (const uint8_t*)w.q8x, w.q8m, dbg_gu, inv, H, I, E, K, P, rgu);
        if ((rc = launch_status("moe_layer_grouped/gate_up_mfma"))) return rc;
        if (dbg_act) {  // the debug copy below reads q8a's pair rows
            hipLaunchKernelGGL(k_q8m_rows, dim3(64, (unsigned)gbig), dim3(256), 0, s,
                               (const uint32_t*)w.q8m, (const int32_t*)w.meta, (const int32_t*)w.plist, w.q8a, P, nbj,
                               E);
            if ((rc = launch_status("moe_layer_grouped/q8m_rows"))) return rc;
        }
    }
    if (dbg_act && hipMemcpyAsync(dbg_act, w.q8a, (size_t)P * nbj * Q8_BLK, hipMemcpyDeviceToDevice, s) != hipSuccess)
        return fail(FT_HIP_E_LAUNCH, "%s: debug copy failed", nm);
    if (dot4) {
        const size_t lds_dn = (size_t)NTD * nbj * 40;
        auto kern = scan ? (nbj <= 24 ? (rec ? k_grouped_down<6, true, true> : k_grouped_down<6, false, true>)
                                      : (rec ? k_grouped_down<8, true, true> : k_grouped_down<8, false, true>))
                         : (nbj <= 24 ? (rec ? k_grouped_down<6, true, false> : k_grouped_down<6, false, false>)
                                      : (rec ? k_grouped_down<8, true, false> : k_grouped_down<8, false, false>));
        hipLaunchKernelGGL(kern, dim3(H / DU, scan ? E : gmax), dim3(GT), lds_dn, s, (const uint8_t*)bank, eb, gu_bytes,
                           (const int32_t*)w.meta, (const int32_t*)w.plist, (const uint8_t*)w.q8a, w.ydn, H, I, E,
                           n_mfma, rdn, (const int32_t*)ids, P);
        if ((rc = launch_status("moe_layer_grouped/down"))) return rc;
    }
    if (mfma) {
        if (nbj <= 32) {  // one K slice: 8 waves x 2 tiles of 16 rows per workgroup
            const size_t lds_md = (size_t)GW * 2 * nbj * 32 + sizeof(float) * GW * 2 * 16 * MT;
            auto kern = rec ? k_mfma_down<1, 32, 2, 4, 2, true> : k_mfma_down<1, 32, 2, 4, 2, false>;
            hipLaunchKernelGGL(kern, dim3(H / (16 * GW * 2), gbig), dim3(GT), lds_md, s, (const uint8_t*)bank, eb,
                               gu_bytes, (const int32_t*)w.meta, (const int32_t*)w.plist, (const uint8_t*)w.q8m, P,
                               w.ydn, H, I, E, n_mfma, rdn);
        } else {  // long rows: DRT tiles per workgroup, 8 K slices of 56 (rows up to 448 blocks) or 64 blocks
            constexpr int DRT = 4;
            const size_t lds_md = std::max((size_t)DRT * nbj * 32, sizeof(float) * GW * DRT * 16 * MT);
            auto kern = nbj <= 8 * 56 ? (rec ? k_mfma_down<GW, 56, DRT, 4, 2, true> : k_mfma_down<GW, 56, DRT, 4, 2, false>)
                                      : (rec ? k_mfma_down<GW, 64, DRT, 4, 2, true> : k_mfma_down<GW, 64, DRT, 4, 2, false>);
            hipLaunchKernelGGL(kern, dim3(H / (16 * DRT), gbig), dim3(GT), lds_md, s, (const uint8_t*)bank, eb,
                               gu_bytes, (const int32_t*)w.meta, (const int32_t*)w.plist, (const uint8_t*)w.q8m, P,
                               w.ydn, H, I, E, n_mfma, rdn);
        }
        if ((rc = launch_status("moe_layer_grouped/down_mfma"))) return rc;
    }
    hipLaunchKernelGGL(k_grouped_combine, dim3((H + 255) / 256, (unsigned)n_seqs), dim3(256), 0, s, (const float*)w.ydn,
                       (const float*)wts, x, x_out, H, K);
    return launch_status("moe_layer_grouped/combine");
}

// ---------------------------------------------------------------------------
// The L-layer stack for a batch (forward_batch's expert section for every
// layer, ft-model/src/lib.rs:1507-1606, called per layer from :1151-1154).
// Workspace: the layer workspace for max_seqs, then two [max_seqs][H] f32
// states and [L][max_seqs*K] ids/wts for callers that pass no record.
// ---------------------------------------------------------------------------
namespace {
struct StackWs {
    void* layer;
    size_t layer_bytes;
    float* state[2];
    int32_t* ids;
    float* wts;
    size_t bytes;
};

StackWs stack_ws(void* base, int64_t max_seqs, int64_t H, int64_t I, int64_t E, int64_t K, int64_t L) {
    auto up = [](size_t v) { return (v + 255) / 256 * 256; };
    StackWs w{};
    uint8_t* p = (uint8_t*)base;
    size_t off = 0;
    w.layer = p;
    w.layer_bytes = group_ws(nullptr, max_seqs, H, I, E, K).bytes;
    off += up(w.layer_bytes);
    for (int i = 0; i < 2; ++i) {
        w.state[i] = (float*)(p + off);
        off += up(sizeof(float) * max_seqs * H);
    }
    w.ids = (int32_t*)(p + off);
    off += up(sizeof(int32_t) * L * max_seqs * K);
    w.wts = (float*)(p + off);
    off += up(sizeof(float) * L * max_seqs * K);
    w.bytes = off;
    return w;
}
}  // namespace

extern "C" size_t ft_hip_moe_stack_grouped_workspace_bytes(int64_t max_seqs, int64_t hidden, int64_t inter,
                                                           int64_t n_experts, int64_t top_k, int64_t n_layers) {
    if (max_seqs < 0 || hidden <= 0 || inter <= 0 || n_experts <= 0 || top_k <= 0 || n_layers <= 0) return 0;
    return stack_ws(nullptr, max_seqs, hidden, inter, n_experts, top_k, n_layers).bytes;
}

extern "C" int ft_hip_moe_stack_grouped(ft_hip_ctx* ctx, void* stream, const float* x_in, float* x_out,
                                        int64_t n_seqs, int64_t max_seqs, int64_t hidden, int64_t inter,
                                        int64_t n_experts, int64_t top_k, int64_t n_layers, const void* banks,
                                        const float* routers, const float* router_bias, const float* expert_scale,
                                        int32_t* ids, float* wts, void* workspace, size_t workspace_bytes) {
    clear_error();
    const char* nm = "moe_stack_grouped";
    if (int rc = check_grouped_shape(nm, max_seqs, hidden, inter, n_experts, top_k)) return rc;
    if (n_seqs < 0 || n_seqs > max_seqs)
        return fail(FT_HIP_E_SHAPE, "%s: n_seqs=%lld not in [0, max_seqs=%lld]", nm, (long long)n_seqs, (long long)max_seqs);
    if (n_layers <= 0) return fail(FT_HIP_E_SHAPE, "%s: n_layers=%lld must be positive", nm, (long long)n_layers);
    if (!ctx || !x_in || !x_out || !banks || !routers || !workspace) return fail(FT_HIP_E_INVALID, "%s: null argument", nm);
    if ((ids == nullptr) != (wts == nullptr)) return fail(FT_HIP_E_INVALID, "%s: give ids and wts or neither", nm);
    const StackWs w = stack_ws(workspace, max_seqs, hidden, inter, n_experts, top_k, n_layers);
    if (workspace_bytes < w.bytes)
        return fail(FT_HIP_E_SHAPE, "%s: workspace_bytes=%zu < %zu (for max_seqs %lld)", nm, workspace_bytes, w.bytes,
                    (long long)max_seqs);
    if (n_seqs == 0) return FT_HIP_OK;
    const int64_t eb = ft_hip_fused_expert_bytes(hidden, inter);
    const int64_t P = n_seqs * top_k;
    const size_t lbytes = group_ws(nullptr, n_seqs, hidden, inter, n_experts, top_k).bytes;
    const float* src = x_in;
    for (int64_t l = 0; l < n_layers; ++l) {
        // the last layer writes x_out, unless it would overwrite its own input
        // in a one-layer in-place call
        const bool last = l == n_layers - 1;
        float* dst = last && !(n_layers == 1 && x_out == x_in) ? x_out : w.state[l & 1];
        int32_t* il = ids ? ids + l * P : w.ids + l * P;
        float* wl = wts ? wts + l * P : w.wts + l * P;
        const uint8_t* bank = static_cast<const uint8_t*>(banks) + l * n_experts * eb;
        if (int rc = ft_hip_moe_layer_grouped(ctx, stream, src, dst, n_seqs, hidden, inter, n_experts, top_k,
                                              routers + l * n_experts * hidden,
                                              router_bias ? router_bias + l * n_experts : nullptr,
                                              expert_scale ? expert_scale + l * n_experts : nullptr, bank, il, wl,
                                              w.layer, lbytes, nullptr, nullptr))
            return rc;
        src = dst;
    }
    if (src != x_out) {
        hipError_t e = hipMemcpyAsync(x_out, src, sizeof(float) * n_seqs * hidden, hipMemcpyDeviceToDevice,
                                      reinterpret_cast<hipStream_t>(stream));
        if (e != hipSuccess) return fail(FT_HIP_E_LAUNCH, "%s: copy of the result: %s", nm, hipGetErrorString(e));
    }
    return FT_HIP_OK;
}
