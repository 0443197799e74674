// ft_hip_fused.hip -- the whole MoE expert-FFN section of an L-layer stack for
// one decode token in ONE persistent kernel.
//
// Why one kernel: at batch 1 a Gemma-shaped layer streams only ~28 MB, i.e.
// ~4.6 us at the MI355X's achievable HBM rate, while every kernel boundary
// costs several us. The layer is therefore run as dataflow between resident
// workgroups, handing over through single-writer, epoch-tagged 64-bit words
// in device memory: bits 63..32 = epoch tag, bits 31..0 = payload.
// Producers write with device-coherent relaxed stores; consumers read with
// device-coherent loads, keep the words that already carry the expected tag
// and re-read only the missing ones. Data and flag travel in the same word,
// so there is no read-modify-write contention and no cache-maintenance fence
// (the alternatives measured 1.4-20 us per barrier on this part).
//
// Why prefetch: a layer's hand-over chain (act -> y -> routing) is several
// us during which HBM would sit idle. Every unit group streams the tiles of
// its PREDICTED expert of layer l+1 into registers as soon as it has
// finished layer l's dots, overlapping the stream with the chain. When the
// true routing arrives, predicted experts that were routed stay with the
// unit group that holds them; only the remaining unit groups load the
// experts nobody predicted (a miss). The prediction: the router of layer
// l+1 applied to x_l ("early routing", ~88 % of experts), refined, when a
// table M_{l,e} = R_{l+1} D_{l,e} is set, by the layer's own act blocks:
// R_{l+1} x_{l+1} = R_{l+1} x_l + sum_p w_p M_p a_p (~99 %).
//
// Workgroups (G shape: H 2816, I 704, E 128, top-8): 208.
//   expert unit (u, j), 176 of them, unit group u = w % K, j = w / K:
//     gate|up : 64 rows (32 gate, 32 up) of its expert for act block j
//               (32 columns), H/32 blocks held in registers by 8 waves;
//               GELU*up -> one q8 block, published (hop A).
//     down    : rows 128j..128j+127 of its expert (one 16-row tile per
//               wave), held in registers with the gate|up tile; waits for
//               the act blocks of ITS unit group only (hop A), publishes y
//               for its 128 rows (hop B), then prefetches layer l+1.
//     All units of group u run on XCD u (workgroups are dealt to XCDs
//     round-robin; each checks this at start through the XCD id register),
//     so hop A stays in that XCD's L2: plain stores, agent-scope polls.
//     If the placement check fails, hop A stores write through instead.
//   group units (g, s), GSPLIT = 2 per R-order group of H/8 rows (16 of
//     them, both of group g on XCD g): each waits for y of the group's rows
//     from every routed slot (hop B); x_{l+1} = x_l + sum_p w_p y_p in
//     routing order; router chunk partials of the group's H/128 chunks and
//     their group sum for half of the experts, s*E/2.. (layer l+1's router
//     weights were streamed into registers meanwhile); split 0 also the q8
//     of the rows and their sum of squares; publishes them (hop C),
//     double-buffered by parity.
//   pred unit g, 8 of them: the same combine of group g's rows, then the
//     group sums of layer l+2's router over x_{l+1} (pp), published.
//   refiner unit r, 8 of them (XCD r): per layer l, the early logits of
//     l+1 from every pred unit's sums; without a table their top-k is the
//     prediction of l+1; with one, their 16 best are candidates, and once
//     unit group r has published its act blocks of layer l the refiner
//     publishes its share w M a of the candidates' logits. Expert units
//     form the prediction from the candidates and the 8 shares themselves;
//     the refiner publishes it for the group and pred units of its XCD.
//   every expert and group unit: reads the 8 group sums of every expert
//     (and, expert units, the 88 q8 blocks of x_{l+1}) (hop C), logits =
//     sum over groups in order + bias, top-k (and, group units, softmax),
//     then the assignment of routed slots to unit groups.
// Weight layouts are lossless repacks of q4_0 with its byte count.

#include <type_traits>

#include "ft_device.hpp"
#include "ft_runtime.hpp"

using namespace ft;

namespace {

constexpr int FT_THREADS = 512;
constexpr int FT_WAVES = FT_THREADS / 64;
constexpr int MAX_K = 8;
constexpr int MAX_E = 128;      // group partials use four threads per expert
constexpr int NGROUP = 8;       // R-order groups
constexpr int GSPLIT = 2;       // group units per R-order group, each with E / GSPLIT experts' router sums
constexpr int DN_ROWS = 16;     // rows per router chunk and per down tile
constexpr int DN_UNIT = DN_ROWS * FT_WAVES;  // rows per down unit: one tile per wave
constexpr int POLL_SLEEP = 1;   // s_sleep units (64 clocks) between polls
constexpr int NREP = 1;         // replicas of the group broadcast
constexpr int CTL_EPOCH = 0;    // control words (u32 indices)
constexpr int CTL_ABORT = 32;
// CTL_ABORT value of a launch refused because its tags would pass 2^32
constexpr uint32_t ABORT_EPOCH_WRAP = 0xFFFFFFFFu;
constexpr int TRACE_SLOTS = 32; // stamps per workgroup per layer in the debug trace
constexpr int PID_STRIDE = 16;  // words per copy of the predicted experts
template <int N> using IC = std::integral_constant<int, N>;
constexpr int NCAND = 16;       // candidates of the refined prediction: the early routing's 16 best experts
constexpr int CW = 3 * NCAND + 1;  // candidate words: ids, sums of R_{l+1} x_l, biases, the norm scale of x_l
constexpr int CD_STRIDE = 64;   // words per refiner's copy of the candidate words
constexpr int CP_WORDS = NGROUP * CD_STRIDE + NGROUP * NCAND;  // per layer parity: candidate copies, then shares

struct FusedParams {
    const uint8_t* banks;       // [L][E][expert_bytes], fused layout
    const float* routers;       // [L][H/16][E][16]
    const float* bias;          // [L][E] or null
    const float* escale;        // [L][E] or null
    const float* x_in;          // [H]
    float* x_out;               // [H]
    int32_t* ids_out;           // [L][K] or null
    float* wts_out;             // [L][K] or null
    uint64_t* act_t;            // tagged [K][I/32][10]
    uint64_t* hp_t;             // tagged [K][I/32][8 wave slices][64 rows]: gate|up partials of missed tiles
    uint64_t* y_t;              // tagged [2][K][H], by layer parity
    uint64_t* gq_t;             // tagged [3][NREP][NGROUP][gq_stride] (by layer mod 3): E group sums, the
                                // group's sum of squares of x, then qw q8 words
    uint64_t* pp_t;             // tagged [2][NGROUP][E+1]: group sums of the predicting router, then the
                                // group's sum of squares of x
    uint64_t* pid_t;            // tagged [2][NGROUP][PID_STRIDE]: predicted experts, one copy per refiner
    uint64_t* pl_t;             // tagged [grid]: the XCD each workgroup runs on
    uint64_t* cp_t;             // tagged [2][CP_WORDS], by layer parity: each refiner's copy of the candidate
                                // words of layer l+1 (CD_STRIDE apart), then the refiners' shares [NGROUP][NCAND]
    const uint8_t* pred_tab;    // [L-1][E] refined-prediction records (E*(I/32)*36 bytes each), or null
    int64_t rs_gq;              // replica stride (words); the parity stride is NREP * rs_gq
    uint32_t* ctl;              // [CTL_EPOCH] epoch, [CTL_ABORT] abort epoch
    float* dbg_gu;              // [L][K][2I] or null
    uint8_t* dbg_act;           // [L][K][I/32][40] or null
    float* dbg_x;               // [L+1][H] or null
    uint64_t* trace;            // [grid][L+1][TRACE_SLOTS] wall-clock stamps or null
    int32_t* rec_gu;            // [L][K][2I][H/32] gate|up block dots (debug build, tests) or null
    int32_t* rec_dn;            // [L][K][H][I/32] down block dots (debug build, tests) or null
    int64_t expert_bytes, gu_bytes;
    int H, I, E, K, L;
    int n_gu, n_dn, n_unit;     // K*I/32 gate|up units, K*H/128 down units, max of the two
    int prefetch;               // 0: every layer loads its routed experts (no prediction)
    int input_norm;             // 1: each layer runs on rmsnorm(x) (logits and gate|up sums times inv_r)
    int gq_stride, qw;          // words per group in the broadcast; q8 words per group ((H/8)/32*10)
    int spin_limit;
    int o_q8x, o_act8, o_red, o_gq, o_gx, o_gy, o_gp, o_misc, lds_bytes;
};

struct alignas(16) Misc {       // placed 16-byte aligned
    uint64_t keys[MAX_E + 8];   // rank keys of the logits, four padded rows (16-byte aligned)
    float logits[MAX_E];
    float sel_v[MAX_K];         // the chosen logits, in rank order
    int sel_i[MAX_K];           // the chosen experts, in rank order
    int ids[MAX_K];             // routed experts of the current layer, in routing order
    float wts[MAX_K];
    alignas(16) int pid[2][MAX_K];  // by layer parity: the expert unit group u holds (predicted)
    int uslot[MAX_K];           // slot of unit group u's held expert, -1: not routed
    int pown[MAX_K];            // unit group that runs routed slot p
    int mlist[MAX_K];           // unit groups whose held expert was not routed (misses), ascending
    int mexp[MAX_K];            // the expert each of them runs instead
    int mslot[MAX_K];           // and its routed slot
    int mcount;
    int abort_flag;
    float inv_r;                // the input RMS norm's scale of the current layer (1 without the norm)
    uint64_t exp2[32];          // libm::exp2_table() for the routing weights' expf
    // expert units' routing (route_units)
    alignas(16) uint64_t cand[64];  // rank keys of the 8 best logits of each 16
    int slotheld[MAX_K];        // 1: routed slot s runs on the unit group holding its expert
    int freeslot[MAX_K];        // the routed slots no unit group holds, ascending
    int ufor[MAX_K];            // the slot unit group u runs
};

// The expf table read from the copy in LDS.
struct Exp2Lds {
    const uint64_t* t;
    __device__ __forceinline__ uint64_t operator[](uint64_t i) const { return t[i]; }
};

// Tagged words use system-scope (sc0 sc1) relaxed accesses: in a probe a
// one-way hand-over took ~0.40 us this way whether or not the two workgroups
// shared an XCD, against 0.85 us between workgroups of one XCD with
// agent-scope (sc1) accesses.
__device__ __forceinline__ uint64_t ld_tag(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void st_tag(uint64_t* p, uint32_t tag, uint32_t v) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
// Agent-scope (sc1) load: also sees a plain store made by a workgroup of the
// same XCD (the line is dirty in the shared L2), which is the fastest
// hand-over on this part (~0.27 us one-way even with HBM saturated).
__device__ __forceinline__ uint64_t ld_tag_agent(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Store that stays in this XCD's L2: only for consumers on the same XCD. A
// relaxed atomic store (one 64-bit store, never torn) with no cache-policy
// bits, which is what wavefront scope emits on gfx950 (workgroup scope adds
// sc0); the L1 writes through, so the line lands in the L2 that the
// consumer's agent-scope load reads. The scope is narrower than the
// consumer's: this relies on the two workgroups sharing the XCD's L2, which
// every unit checks at start (the placement words) before using this form.
__device__ __forceinline__ void st_tag_local(uint64_t* p, uint32_t tag, uint32_t v) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
}
__device__ __forceinline__ uint32_t xcc_id() {
    return __builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20);  // HW_REG_XCC_ID bits 3:0
}
__device__ __forceinline__ uint32_t ld_ctl(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// threadIdx.x behind an opaque move: comparisons against it are recomputed
// where they are used instead of being hoisted out of the layer loop as lane
// masks, which would be spilled and reloaded (scalar register pressure).
__device__ __forceinline__ int tid_here() {
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

template <bool DBG>
__device__ __forceinline__ void trace_value(const FusedParams& P, int l, int ev, uint64_t v) {
    if (DBG && P.trace && threadIdx.x == 0)
        P.trace[((int64_t)blockIdx.x * (P.L + 1) + (l + 1)) * TRACE_SLOTS + ev] = v;
}

// Block-wide wait until the n (<= U * FT_THREADS) tagged words src[idx(i)]
// all carry `tag`; payloads land in dst[didx(i)] (LDS). Each lane owns words
// tid, tid + FT_THREADS, ... and each wave spins on its own words without
// synchronising; one barrier ends the wait.
// Two poll rounds are kept in flight: a round is issued before the previous
// one is checked, so a word is seen about half a memory round trip after it
// lands instead of up to a whole one. Every round issues exactly U loads per
// polling lane (a lane's finished or surplus words re-read one of its own),
// so the compiler waits for the older round only.
// Bounded: after spin_limit rounds (or when another workgroup has aborted)
// the lane records the abort and the wait returns false in every thread.
template <bool DBG, int U, bool AGENT = false, int NPOLL = FT_THREADS, typename Idx, typename DIdx>
__device__ __forceinline__ bool wait_words(const FusedParams& P, Misc* m, uint32_t epoch, const uint64_t* src, int n,
                                           Idx idx, uint32_t tag, uint32_t* dst, DIdx didx, int tl = -2, int ts = 0) {
    // An opaque copy of the thread index: keeps the compiler from hoisting the
    // per-call-site address arithmetic out of the layer loop, where it would
    // stay live (in registers) for the whole kernel.
    const int tid = tid_here();
    uint32_t pending = 0;
#pragma unroll
    for (int u = 0; u < U; ++u)
        if (tid < NPOLL && u * NPOLL + tid < n) pending |= 1u << u;
    auto issue = [&](uint64_t (&v)[U]) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            // a slot beyond n re-reads the lane's first word (spread over the
            // payload: many lanes re-reading one word would make it a hot spot)
            const int64_t a = idx(u * NPOLL + tid < n ? u * NPOLL + tid : min(tid, n - 1));
            v[u] = AGENT ? ld_tag_agent(src + a) : ld_tag(src + a);
        }
    };
    auto check = [&](const uint64_t (&v)[U]) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (((pending >> u) & 1) && (uint32_t)(v[u] >> 32) == tag) {
                dst[didx(u * NPOLL + tid)] = (uint32_t)v[u];
                pending &= ~(1u << u);
            }
    };
    int it = 0;
    bool give_up = false;
    auto bounded = [&]() __attribute__((always_inline)) {
        ++it;
        if (it >= P.spin_limit || ((it & 63) == 0 && ld_ctl(P.ctl + CTL_ABORT) == epoch)) {
            // published at once: the other lanes, waves and workgroups see it
            // at their next check (every 64 rounds) and give up too
            __hip_atomic_store(P.ctl + CTL_ABORT, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            give_up = true;
        }
        return give_up;
    };
    uint64_t va[U], vb[U];
    if (pending) issue(va);
    while (pending) {
        __builtin_amdgcn_s_sleep(POLL_SLEEP);
        issue(vb);
        check(va);
        if (!pending || bounded()) break;
        __builtin_amdgcn_s_sleep(POLL_SLEEP);
        issue(va);
        check(vb);
        if (!pending || bounded()) break;
    }
    if (give_up) m->abort_flag = 1;
    if (tl > -2) trace_value<DBG>(P, tl, ts, (uint64_t)(it + 1));  // rounds this wait took (thread 0)
    __syncthreads();
    return m->abort_flag == 0;
}

template <bool DBG, int U, typename Idx>
__device__ __forceinline__ bool wait_words(const FusedParams& P, Misc* m, uint32_t epoch, const uint64_t* src, int n,
                                           Idx idx, uint32_t tag, uint32_t* dst, int tl = -2, int ts = 0) {
    return wait_words<DBG, U>(P, m, epoch, src, n, idx, tag, dst, [](int i) { return i; }, tl, ts);
}

// Trace slots (per workgroup and layer; layer -1 = prologue), wall-clock
// stamps unless noted: 0 layer start (routing known), 1 loads issued,
// 2 gate|up dots done, 3 act published, 4 act read, 5 down dots, 6 y
// published, 8 group: y read, 9 group: x combined, 11 group: published,
// 12 broadcast read, 13 logits, 14 top-k done, 15 top-k ranked, 16 softmax,
// 17-19 gate|up tail (wave sums, GELU, q8), 20-22 group (partials, sync,
// sums); 24-26 poll count of the broadcast / act / y waits and 28-30 the
// return of each one's first poll; 7 prefetch issued, 10 miss (1/0), 23
// shader clock at layer start, 27 poll count of the prediction wait;
// prologue row: 27 act hand-over local (1/0), 28 XCD id.
template <bool DBG>
__device__ __forceinline__ void stamp(const FusedParams& P, int l, int ev) {
    if (DBG && P.trace && threadIdx.x == 0)
        P.trace[((int64_t)blockIdx.x * (P.L + 1) + (l + 1)) * TRACE_SLOTS + ev] = wall_clock64();
}

// Top-k by rank (rank = number of logits that sort before: larger, or equal
// with a lower index, as the stable descending sort of
// ft-model/src/lib.rs:1491-1492; NaN after every number, where the reference
// would panic), then softmax over the chosen (ft-model/src/lib.rs:1494-1503):
// exp(l - l_max), summed in rank order. Each logit carries a 64-bit key
// (monotone float bits, then the complemented index) so that "sorts before"
// is one unsigned compare; four threads share one logit's E comparisons.
// (rank_key: ft_device.hpp)

// Scale of the input RMS norm from the 8 groups' sums of squares (R-order,
// like a router row with W = x): ss = the group sums in order from 0.0f,
// inv_r = 1 / sqrt(ss / H + 1e-6), each op rounded once. Whole wavefronts:
// lane g < 8 reads group g's sum and the sum runs over lane reads, which
// keeps one register live instead of eight.
__device__ __forceinline__ float rms_inv_groups(const float* gss, int H) {
    asm volatile("" : "+s"(H));  // (float)H formed here, not hoisted to the kernel's start and spilled
    const float p = gss[__lane_id() & (NGROUP - 1)];
    float ss = 0.0f;
#pragma unroll
    for (int g = 0; g < NGROUP; ++g) ss = ss + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), g));
    return 1.0f / sqrtf(ss / (float)H + 1e-6f);  // correctly rounded (HIP default)
}

// Rank keys sit in four rows of 32 (one row per comparing thread of a
// logit), padded by 16 bytes so the rows start in different LDS banks; keys
// of indices >= E are 0, below every real key, so every thread compares a
// full row without masks.
constexpr int KEY_ROW = MAX_E / 4;
__device__ __forceinline__ int key_slot(int i) { return (i / KEY_ROW) * (KEY_ROW + 2) + i % KEY_ROW; }

// Routing of `layer` from the NGROUP group sums gs[E][NGROUP] in LDS.
//   Logits: R-order, the group sums of expert e in group order from 0.0f,
//   times inv_r of the input RMS norm (routing, with the norm on: inv_r from
//   the groups' sums of squares in row E of gs; else 1), then + bias (bias_t:
//   this thread's expert's bias, read ahead by the caller). inv_r goes to
//   m->inv_r (routing only). Then each logit's rank, and the top K in rank order:
//   pred >= 0 (prediction): ids alone into m->pid[pred] (or, with sel_out,
//   the nsel best ids into sel_out);
//   otherwise ids into m->sel_i, logits into m->sel_v and, for every unit
//   group u whose held expert `held[u]` was routed, its slot into
//   m->uslot[u] (-1: not routed). Two barriers; the caller reads after the
//   second.
__device__ __forceinline__ void route_rank(const FusedParams& P, Misc* m, const float* gs, float bias_t, int pred,
                                           const int* held, int* sel_out = nullptr, int nsel = 0) {
    static_assert(NGROUP == 8 && MAX_E == 128, "the logit and key layouts below assume these");
    const int E = P.E, K = P.K, t = tid_here();
    if (t < MAX_E) {  // whole wavefronts (MAX_E is a multiple of 64)
        float ir = 1.0f;
        if (pred < 0 && P.input_norm) ir = rms_inv_groups(gs + E * NGROUP, P.H);
        // done before the group sums are read (its temporaries and those sums
        // are never live together) and kept in a scalar register (uniform)
        ir = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(ir)));
        asm volatile("" : "+s"(ir)::"memory");
        uint64_t key = 0;
        if (t < E) {
            const float4 a = reinterpret_cast<const float4*>(gs + t * NGROUP)[0];
            const float4 b = reinterpret_cast<const float4*>(gs + t * NGROUP)[1];
            const float gv[NGROUP] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            float total = 0.0f;
#pragma unroll
            for (int g = 0; g < NGROUP; ++g) total = total + gv[g];
            total = total * ir;
            if (P.bias) total = total + bias_t;
            m->logits[t] = total;
            if (t == 0 && pred < 0) m->inv_r = ir;
            key = rank_key(total, t);
        }
        m->keys[key_slot(t)] = key;
    }
    if (t < MAX_K) m->uslot[t] = -1;
    __syncthreads();
    const int i = min(t >> 2, E - 1), part = t & 3;
    const uint64_t ki = m->keys[key_slot(i)];
    const uint4* kk = reinterpret_cast<const uint4*>(m->keys + part * (KEY_ROW + 2));  // two keys per uint4
    int rank = 0;
#pragma unroll
    for (int j0 = 0; j0 < KEY_ROW / 2; j0 += 8) {  // two batches of LDS reads: fewer registers live
        uint4 kv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) kv[j] = kk[j0 + j];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint64_t k0 = ((uint64_t)kv[j].y << 32) | kv[j].x;
            const uint64_t k1 = ((uint64_t)kv[j].w << 32) | kv[j].z;
            rank += (int)(k0 > ki) + (int)(k1 > ki);
        }
    }
    rank += quad_xor1i(rank);
    rank += quad_xor2i(rank);
    // the held experts, two 16-byte LDS reads issued with the rank's (MAX_K == 8)
    int4 h0 = make_int4(-1, -1, -1, -1), h1 = h0;
    if (held) {
        h0 = reinterpret_cast<const int4*>(held)[0];
        h1 = reinterpret_cast<const int4*>(held)[1];
    }
    const float li = m->logits[i];
    if (sel_out) {  // (pred >= 0) the nsel best, in rank order
        if ((t >> 2) < E && part == 0 && rank < nsel) sel_out[rank] = i;
    } else if ((t >> 2) < E && part == 0 && rank < K) {  // ranks are distinct: each slot written once
        if (pred >= 0) {
            m->pid[pred][rank] = i;
        } else {
            m->sel_i[rank] = i;
            m->sel_v[rank] = li;
            const int hv[MAX_K] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
#pragma unroll
            for (int u = 0; u < MAX_K; ++u)
                if (u < K && hv[u] == i) m->uslot[u] = rank;
        }
    }
    __syncthreads();
}

// The refined prediction of layer l+1 from the candidate words cw (the
// early routing's NCAND best experts of l+1: ids, then their sums of
// R_{l+1} x_l, then their biases, then the input norm's scale of x_l, or 1)
// and the refiners' shares sh [NGROUP][NCAND] (w_p M_p a_p of the slot each
// unit group ran in layer l): logit_c = (base_c + sh[0][c] + ... +
// sh[7][c]) * ir + bias_c, each op rounded once; the K best candidates in
// rank order into pid. Wavefront 0 (its lanes' LDS accesses complete in
// program order); the caller synchronises before other waves read pid. Every
// workgroup that needs the prediction runs this on the same words, so all
// hold the same one.
__device__ __forceinline__ void cand_pid(const uint32_t* cw, const uint32_t* sh, uint64_t* keys, int* pid, int K) {
    const int c = tid_here();
    uint64_t key = 0;
    if (c < NCAND) {
        float s = __uint_as_float(cw[NCAND + c]);
#pragma unroll
        for (int p = 0; p < NGROUP; ++p) s = s + __uint_as_float(sh[p * NCAND + c]);
        key = rank_key(s * __uint_as_float(cw[3 * NCAND]) + __uint_as_float(cw[2 * NCAND + c]), (int)cw[c]);
        keys[c] = key;
    }
    if (c < NCAND) {
        int rank = 0;
#pragma unroll
        for (int q = 0; q < NCAND; ++q) rank += keys[q] > key ? 1 : 0;
        if (rank < K) pid[rank] = (int)cw[c];
    }
}

// Slot that unit group u runs (after route_rank with `held`): the slot of
// its held expert if that was routed; otherwise the r-th routed slot that no
// unit group holds, r = u's rank among the unit groups whose held expert was
// not routed. first (nothing held): slot u. Every workgroup computes the same
// assignment from the same routing and prediction.
__device__ __forceinline__ int unit_slot(const Misc* m, int K, int u, bool first) {
    if (first) return u;
    int us[MAX_K];
#pragma unroll
    for (int q = 0; q < MAX_K; ++q) us[q] = m->uslot[q];
    uint32_t held = 0, hit = 0;
    int mine = -1;
#pragma unroll
    for (int q = 0; q < MAX_K; ++q) {
        if (q < K && us[q] >= 0) {
            held |= 1u << us[q];
            hit |= 1u << q;
        }
        mine = q == u ? us[q] : mine;
    }
    if (mine >= 0) return mine;
    const int r = __popc(~hit & ((1u << u) - 1));
    uint32_t fr = ~held & ((1u << K) - 1);
#pragma unroll
    for (int k = 0; k < MAX_K; ++k)
        if (k < r) fr &= fr - 1;
    return fr ? (int)__builtin_ctz(fr) : 0;
}

// Routing of the expert units (the top-K ids, the slot of every unit group
// and the missed unit groups; no logits or weights, which only the group
// units need), with the same results as route_rank and unit_slot's rule:
//   logits as route_rank's (R-order group sums from 0.0f, times inv_r, +
//   bias_t), one rank key each (threads < 128);
//   top-K by a two-stage tournament on the keys (distinct: the index is in
//   the low word): each wavefront ranks 16 keys among themselves (four lanes
//   per key) and keeps its 8 best as candidates; every global top-8 key is a
//   candidate, and its rank among the 64 candidates is its global rank
//   (eight lanes per candidate). A routed expert held by unit group u gives
//   uslot[u] and marks its slot held;
//   wavefront 0, lane u < K: a unit group whose held expert was not routed
//   (a miss; every group when held is null) takes the r-th routed slot no
//   group holds, r = its rank among the missed groups, ascending: ufor[u],
//   mlist/mexp/mslot/mcount. Ends with a barrier.
__device__ __forceinline__ void route_units(const FusedParams& P, Misc* m, const float* gs, float bias_t,
                                            const int* held) {
    static_assert(NGROUP == 8 && MAX_E == 128 && MAX_K == 8 && FT_THREADS == 512, "the layouts below assume these");
    const int E = P.E, K = P.K, t = tid_here();
    if (t < MAX_E) {  // whole wavefronts
        float ir = 1.0f;
        if (P.input_norm) {
            const float4 a = reinterpret_cast<const float4*>(gs + E * NGROUP)[0];
            const float4 b = reinterpret_cast<const float4*>(gs + E * NGROUP)[1];
            const float gv[NGROUP] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            float ss = 0.0f;
#pragma unroll
            for (int g = 0; g < NGROUP; ++g) ss = ss + gv[g];
            int Hs = P.H;
            asm volatile("" : "+s"(Hs));  // (float)H formed here: hoisted, it was spilled and reloaded
            ir = 1.0f / sqrtf(ss / (float)Hs + 1e-6f);  // correctly rounded (HIP default)
        }
        uint64_t key = 0xFFFFFFFFu - (uint32_t)t;  // indices >= E: distinct, below every real key
        if (t < E) {
            const float4 a = reinterpret_cast<const float4*>(gs + t * NGROUP)[0];
            const float4 b = reinterpret_cast<const float4*>(gs + t * NGROUP)[1];
            const float gv[NGROUP] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            float total = 0.0f;
#pragma unroll
            for (int g = 0; g < NGROUP; ++g) total = total + gv[g];
            total = total * ir;
            if (P.bias) total = total + bias_t;
            key = rank_key(total, t);
        }
        m->keys[t] = key;
        if (t == 0) m->inv_r = ir;
    }
    if (t < MAX_K) {
        m->uslot[t] = -1;
        m->slotheld[t] = 0;
    }
    __syncthreads();
    {  // stage 1: wavefront w, keys 16w..16w+15; lane (i, part) against keys 16w+4part..+3
        const int w = t >> 6, l = t & 63, part = l & 3;
        const int i = 16 * w + (l >> 2);
        const uint64_t ki = m->keys[i];
        const uint4* kk = reinterpret_cast<const uint4*>(m->keys + 16 * w + 4 * part);
        const uint4 a = kk[0], b = kk[1];
        int lr = (int)((((uint64_t)a.y << 32) | a.x) > ki) + (int)((((uint64_t)a.w << 32) | a.z) > ki) +
                 (int)((((uint64_t)b.y << 32) | b.x) > ki) + (int)((((uint64_t)b.w << 32) | b.z) > ki);
        lr += quad_xor1i(lr);
        lr += quad_xor2i(lr);
        if (part == 0 && lr < 8) m->cand[8 * w + lr] = ki;
    }
    __syncthreads();
    {  // stage 2: candidate c = t/8 against candidates 8p..8p+7 (p = t%8)
        const int c = t >> 3, pp = t & 7;
        const uint64_t kc = m->cand[c];
        const uint4* kk = reinterpret_cast<const uint4*>(m->cand + 8 * pp);
        int4 h0 = make_int4(-1, -1, -1, -1), h1 = h0;
        if (held) {  // issued with the candidate reads
            h0 = reinterpret_cast<const int4*>(held)[0];
            h1 = reinterpret_cast<const int4*>(held)[1];
        }
        int rk = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint4 v = kk[j];
            rk += (int)((((uint64_t)v.y << 32) | v.x) > kc) + (int)((((uint64_t)v.w << 32) | v.z) > kc);
        }
        rk += quad_xor1i(rk);
        rk += quad_xor2i(rk);
        rk += swz_xor4_i(rk);  // no lane-address register (a shuffle's was spilled and reloaded)
        if (pp == 0 && rk < K) {  // ranks are distinct: each slot written once
            const int i = (int)(0xFFFFFFFFu - (uint32_t)kc);
            m->sel_i[rk] = i;
            const int hv[MAX_K] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
#pragma unroll
            for (int u = 0; u < MAX_K; ++u)
                if (u < K && hv[u] == i) {  // held experts are distinct
                    m->uslot[u] = rk;
                    m->slotheld[rk] = 1;
                }
        }
    }
    __syncthreads();
    if (t < 64) {  // wavefront 0: lane u is unit group u and also routed slot u
        const bool v8 = t < K;
        const int us = v8 ? m->uslot[t] : 0;
        const int hs = v8 ? m->slotheld[t] : 1;
        const uint64_t missm = __ballot(v8 && us < 0);
        const uint64_t freem = __ballot(v8 && hs == 0);
        if (v8 && hs == 0) m->freeslot[__builtin_amdgcn_mbcnt_lo((uint32_t)freem, 0)] = t;
        // (lanes of one wavefront: its LDS accesses complete in program order)
        int slot = us;
        if (v8 && us < 0) {
            const int r = __builtin_amdgcn_mbcnt_lo((uint32_t)missm, 0);  // missed groups below u
            slot = m->freeslot[r];
            m->mlist[r] = t;
            m->mslot[r] = slot;
            m->mexp[r] = m->sel_i[slot];
        }
        if (v8) m->ufor[t] = slot;
        if (t == 0) m->mcount = __popcll(missm);
    }
    __syncthreads();
}

// Group and pred units, wave 0, after route_rank: softmax over the chosen in
// rank order (weights into m->wts, ids into m->ids; the routing record when
// `record`), and pown[p] = the unit group running slot p. The caller
// synchronizes before other waves read them.
__device__ __forceinline__ void route_weights(const FusedParams& P, Misc* m, int layer, bool first, bool record) {
    const int E = P.E, K = P.K, t = tid_here();
    if (t >= 64) return;
    const float v0 = m->sel_v[0];
    const float vt = m->sel_v[min(t, K - 1)];
    const int it = m->sel_i[min(t, K - 1)];
    const float ex = expf_libm_t(vt - v0, Exp2Lds{m->exp2});
    float denom = 0.0f;
#pragma unroll
    for (int j = 0; j < MAX_K; ++j)  // in rank order, as the reference's iterator sum
        denom = j < K ? denom + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ex), j)) : denom;
    if (t < K) {
        float w = ex / denom;
        if (P.escale) w = w * P.escale[(int64_t)layer * E + min(max(it, 0), E - 1)];
        m->ids[t] = it;
        m->wts[t] = w;
        if (record) {
            if (P.ids_out) P.ids_out[layer * K + t] = it;
            if (P.wts_out) P.wts_out[layer * K + t] = w;
        }
        m->pown[unit_slot(m, K, t, first)] = t;
    }
}

// Router weights of `layer` for group g into registers, experts e0.. (LPE
// threads per expert, FT_THREADS / LPE experts): thread (e = e0 + t/LPE,
// q = t%LPE) holds chunks q, q+LPE, ... of the group (16 rows each).
template <int CPT, int C, int LPE>
__device__ __forceinline__ void group_load_router(const FusedParams& P, int layer, int g, int e0,
                                                  float4 (&wv)[CPT][4]) {
    static_assert(CPT * LPE >= C, "every chunk has a thread");
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));  // keeps the per-thread offsets inside the layer loop
    const int E = P.E;
    const int e = min(e0 + t / LPE, E - 1), q = t % LPE;
    const float* base = P.routers + (int64_t)layer * (P.H / DN_ROWS) * E * DN_ROWS;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        const int c = min(q + LPE * i, C - 1);
        const float4* s = reinterpret_cast<const float4*>(base + ((int64_t)(g * C + c) * E + e) * DN_ROWS);
#pragma unroll
        for (int k = 0; k < 4; ++k) wv[i][k] = s[k];
    }
}

// Group g's share of the router for its x rows gx (H/8 floats in LDS), in
// the R-order: chunk partials (fma chain over the chunk's 16 rows, from
// 0.0f), summed over the group's C chunks in order (from 0.0f); and the q8
// blocks of the rows; and the sum of squares of the rows in the same order
// (chunk fma chains of x*x). The sums are those of experts e0..e0 +
// FT_THREADS/LPE - 1 (the router weights group_load_router<CPT, C, LPE>
// gave); the q8 blocks and the sum of squares only when `primary`.
// Publishes, tagged, the unit's words of [E sums][sum of squares][qw q8
// words] into group g's slot of each replica; pred (all E experts):
// [E sums][sum of squares] to dst[g * (E + 1) + k] (no q8, one copy).
template <int CPT, int C, int LPE, bool DBG>
__device__ __forceinline__ void group_publish(const FusedParams& P, int g, int e0, const float4 (&wv)[CPT][4],
                                              const float* gx, float* gp, uint32_t* q8w, uint64_t* dst, uint32_t tag,
                                              int sl, bool pred, bool primary) {
    constexpr int NE = FT_THREADS / LPE;  // experts of this unit
    // E behind an opaque move: the C chunk offsets c*E are formed here, not
    // hoisted to the kernel's start and kept (spilled) for its lifetime
    int E = P.E;
    asm volatile("" : "+s"(E));
    const int t = tid_here();
    const int e = e0 + t / LPE, q = t % LPE;
    if (e < E) {
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = q + LPE * i;
            if (c < C) {
                const float4* x4 = reinterpret_cast<const float4*>(gx + c * DN_ROWS);
                float s = 0.0f;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float4 xv = x4[k];
                    s = fmaf(wv[i][k].x, xv.x, s);
                    s = fmaf(wv[i][k].y, xv.y, s);
                    s = fmaf(wv[i][k].z, xv.z, s);
                    s = fmaf(wv[i][k].w, xv.w, s);
                }
                gp[c * E + e] = s;
            }
        }
    }
    const int nbq = (P.H / NGROUP) >> 5;  // q8 blocks per group; one lane quad each
    float* sq = reinterpret_cast<float*>(q8w + P.qw);  // [C] chunk partials of x*x, then their sum
    if (!pred && primary && t < 4 * nbq) quantize_block_quad(gx + 32 * (t >> 2), t & 3, q8w + (t >> 2) * 10);
    // sum of squares: chunk c on thread SQ0 + c, in the last wavefront (the
    // q8 quads are in the first)
    constexpr int SQ0 = FT_THREADS - 64;
    static_assert(C <= 64, "one thread per chunk");
    if (primary && t >= SQ0 && t < SQ0 + C) {
        const int c = t - SQ0;
        const float4* x4 = reinterpret_cast<const float4*>(gx + c * DN_ROWS);
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float4 xv = x4[k];
            s = fmaf(xv.x, xv.x, s);
            s = fmaf(xv.y, xv.y, s);
            s = fmaf(xv.z, xv.z, s);
            s = fmaf(xv.w, xv.w, s);
        }
        sq[c] = s;
    }
    stamp<DBG>(P, sl, 20);
    __syncthreads();
    stamp<DBG>(P, sl, 21);
    if (t < NE && e0 + t < E) {
        const int et = e0 + t;
        float pv[C];
#pragma unroll
        for (int c = 0; c < C; ++c) pv[c] = gp[c * E + et];
        float s = 0.0f;
#pragma unroll
        for (int c = 0; c < C; ++c) s = s + pv[c];
        gp[C * E + et] = s;
    }
    if (primary && t == MAX_E) {
        float s = 0.0f;
        for (int c = 0; c < C; ++c) s = s + sq[c];
        sq[C] = s;
    }
    __syncthreads();
    stamp<DBG>(P, sl, 22);
    if (pred) {
        if (t <= E) st_tag(dst + g * (E + 1) + t, tag, __float_as_uint(t < E ? gp[C * E + t] : sq[C]));
        return;
    }
    const int n = E + 1 + P.qw;
    for (int i = t; i < n * NREP; i += FT_THREADS) {
        const int rep = i / n, k = i - rep * n;
        if (k < E ? (k < e0 || k >= e0 + NE) : !primary) continue;  // another unit's words
        const uint32_t v = k < E ? __float_as_uint(gp[C * E + k]) : (k == E ? __float_as_uint(sq[C]) : q8w[k - E - 1]);
        st_tag(dst + rep * P.rs_gq + (int64_t)g * P.gq_stride + k, tag, v);
    }
}

// The bias of thread t's expert (t < E) for `layer`, or 0 without a bias;
// issued early so that the load is back by the time routing needs it.
__device__ __forceinline__ float ld_bias(const FusedParams& P, int layer) {
    const int t = threadIdx.x;
    return (P.bias && t < P.E) ? P.bias[(int64_t)layer * P.E + t] : 0.0f;
}

// Outputs of a launch that aborted (or ran on a poisoned workspace): group
// unit g sets its H/8 rows of x_out to NaN, and group unit 0 sets every
// routing record to id -1 / weight NaN, so a caller that does not poll
// ft_hip_fused_status cannot take stale values for results.
__device__ __forceinline__ void poison_outputs(const FusedParams& P, int g) {
    const int HG = P.H / NGROUP;
    const float qnan = __int_as_float(0x7fc00000);
    for (int i = threadIdx.x; i < HG; i += FT_THREADS) P.x_out[(int64_t)g * HG + i] = qnan;
    if (g == 0)
        for (int i = threadIdx.x; i < P.L * P.K; i += FT_THREADS) {
            if (P.ids_out) P.ids_out[i] = -1;
            if (P.wts_out) P.wts_out[i] = qnan;
        }
}

// BPW: gate|up blocks per wave, exactly H/32/8; DB: down blocks per thread,
// ceil(I/32/4) (surplus blocks re-read a valid one and are masked); CPT:
// router chunks per group-unit thread, ceil(H/128/4). Loads are
// unconditional so that they issue back to back.
template <int BPW, int DB, int CPT, bool DBG>
__global__ __launch_bounds__(FT_THREADS, 1) void k_moe_stack_fused(FusedParams P) {
    // Gate|up blocks per wave prefetched before the broadcast wait; the rest
    // are issued once the broadcast is in, and land during the routing. A
    // CU returns loads in order, so every prefetch load issued before the
    // broadcast polls delays them; the whole prefetch there held the
    // broadcast read ~2 us behind its publication. Measured (us/token):
    // all 11 blocks early 396, 10: 392, 9: 383, 8: 374, 7: 381, 6: 383;
    // the down rows late as well: 387 (with 8 early; with 9, 10, 11 early:
    // 383, 387, 388), half or a third of them late: 383 or 380: issued after
    // the broadcast, they sit in front of the act hand-over's polls instead.
    constexpr int PF_EARLY = BPW > 3 ? BPW - 3 : BPW;
    constexpr int C = 2 * BPW;  // router chunks per group = H/128
    // words per thread of each wait (H = 256 * BPW, E <= 128, K <= 8):
    constexpr int UW_GA = (NGROUP * (MAX_E + 1) + FT_THREADS - 1) / FT_THREADS;       // all 8 groups' sums (+ squares)
    // group units: the experts of one split, LPE threads each
    constexpr int LPE_G = FT_THREADS / (MAX_E / GSPLIT), CPT_G = (C + LPE_G - 1) / LPE_G;
    static_assert(CPT_G <= CPT, "a split's router registers fit the pred units' array");
    constexpr int UW_Y = (BPW + 1) / 2;                                            // y of a group's rows
    constexpr int UW_X = (NGROUP * (MAX_E + 1 + 10 * BPW) + FT_THREADS - 1) / FT_THREADS;  // sums + q8 of x
    extern __shared__ __align__(16) uint8_t lds[];
    uint8_t* act8 = lds + P.o_act8;
    float* red = reinterpret_cast<float*>(lds + P.o_red);
    // expert units: [E+1][NGROUP] group sums (row E: sums of squares), then
    // the q8 of x as [H/32][8] qs words (16-byte aligned) and [H/32] (d, qsum) pairs
    uint32_t* gq = reinterpret_cast<uint32_t*>(lds + P.o_gq);
    const uint4* xq4 = reinterpret_cast<const uint4*>(gq + NGROUP * (P.E + 1));
    const int2* xdp = reinterpret_cast<const int2*>(gq + NGROUP * (P.E + 1) + (P.H >> 5) * 8);
    float* gx = reinterpret_cast<float*>(lds + P.o_gx);
    float* gy = reinterpret_cast<float*>(lds + P.o_gy);
    float* gp = reinterpret_cast<float*>(lds + P.o_gp);
    Misc* m = reinterpret_cast<Misc*>(lds + P.o_misc);

    const int w = blockIdx.x, t = threadIdx.x;
    const int H = P.H, I = P.I, E = P.E, K = P.K, L = P.L;
    const int nb = H >> 5, nbj = I >> 5, HG = H / NGROUP;
    if (t == 0) m->abort_flag = 0;
    if (t < 32) m->exp2[t] = libm::exp2_table().t[t];
    __syncthreads();
    // A workspace whose abort word is set (an earlier launch gave up a wait)
    // is poisoned until ft_hip_fused_workspace_init: its epoch may not have
    // advanced, so stale tags could match. Do nothing; the status reports it.
    if (ld_ctl(P.ctl + CTL_ABORT) != 0) {
        if (w >= P.n_unit && w < P.n_unit + NGROUP) poison_outputs(P, w - P.n_unit);
        return;
    }
    const uint32_t epoch = ld_ctl(P.ctl + CTL_EPOCH);
    // A launch's tags are epoch + 1 .. epoch + 4L + 3 and the next launch
    // starts at epoch + 4(L+1): that must stay below 2^32, or a tag would wrap
    // and could match a word not rewritten since an early launch. The host
    // re-initialises a workspace before that (ft_hip_moe_stack_fused); an
    // epoch it did not track is refused here, uniformly by every workgroup.
    if (epoch > 0xFFFFFFFFu - 4u * (uint32_t)(L + 1)) {
        if (w >= P.n_unit && w < P.n_unit + NGROUP) poison_outputs(P, w - P.n_unit);
        if (w == 0 && t == 0)
            __hip_atomic_store(P.ctl + CTL_ABORT, ABORT_EPOCH_WRAP, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    auto tag_g = [&](int l) { return epoch + 4u * l + 1u; };
    auto tag_a = [&](int l) { return epoch + 4u * l + 2u; };
    auto tag_y = [&](int l) { return epoch + 4u * l + 3u; };
    auto gq_buf = [&](int l) { return P.gq_t + (int64_t)(l % 3) * NREP * P.rs_gq; };
    auto cp_buf = [&](int l) { return P.cp_t + (int64_t)(l & 1) * CP_WORDS; };
    auto pp_buf = [&](int l) { return P.pp_t + (int64_t)(l & 1) * NGROUP * (E + 1); };
    // the prediction: one copy per refiner r (on XCD r), read by the units
    // of the same XCD
    auto pid_buf = [&](int l) { return P.pid_t + (int64_t)(l & 1) * NGROUP * PID_STRIDE; };
    auto y_buf = [&](int l) { return P.y_t + (int64_t)(l & 1) * K * H; };
    const int prep = w % NGROUP;  // the refiner whose copies this workgroup reads
    auto ident = [](int i) { return (int64_t)i; };
    const int rep = w % NREP;  // workgroups are dealt to the 8 XCDs round-robin
    const bool pf = P.prefetch != 0;
    if (t == 0) st_tag(P.pl_t + w, tag_g(0), xcc_id());

    if (w >= P.n_unit + (GSPLIT + 1) * NGROUP) {
        // ============ refiner unit r: the prediction of layer l+1 ============
        // Runs beside unit group r (workgroup n_unit + 3*NGROUP + r, on XCD r).
        // Every pred unit's group sums of R_{l+1} x_l (pp) give the early
        // logits of layer l+1 (times the input norm's scale of x_l, plus the
        // bias of l+1). Without a table their K best are the prediction,
        // published once the routing words of l are in. With a table
        // (ft_hip_fused_build_predictor: M_{l,e} = R_{l+1} D_{l,e}, int8 per
        // 32 columns with an f32 scale) the prediction is refined: layer l+1's
        // logits are linear in x_{l+1} = x_l + sum_p w_p D_p a_p, so
        // R_{l+1} x_{l+1} = R_{l+1} x_l + sum_p w_p M_p a_p. The refiner
        // publishes the early logits' NCAND best as candidate words at once;
        // once unit group r has published the act blocks of the slot it runs
        // in layer l, it publishes its share w M a for the candidates; every
        // expert unit then forms the prediction itself from the candidate
        // words and the 8 shares (cand_pid), one hand-over after the shares,
        // and the refiner does the same for the group and pred units (its pid
        // copy). Results never depend on the prediction (it only decides
        // which unit group holds which expert), so this f32 arithmetic is
        // free-form; all that matters is that every workgroup computes the same.
        const int r = w - P.n_unit - (GSPLIT + 1) * NGROUP;
        if (!pf || L < 2) return;
        const bool refine = P.pred_tab != nullptr;
        const int ES = E + 1;
        auto aidx = [=](int i) { return (int64_t)(i / ES) * P.gq_stride + i % ES; };
        auto adst = [=](int i) { return (i % ES) * NGROUP + i / ES; };
        auto act_dst = [=](int i) {
            const int bi = i / 10, k = i - bi * 10;
            return k >= 2 ? bi * 8 + (k - 2) : nbj * 8 + bi * 2 + k;
        };
        float* gs = reinterpret_cast<float*>(gq);         // [E+1][NGROUP]
        float* lg = gy;                                     // [E][NGROUP]: the early logit in column 0
        float* bs = gx;                                     // [E] the early sums
        uint32_t* cwl = reinterpret_cast<uint32_t*>(red);  // candidate words, then (at +CD_STRIDE) the shares
        int* cid = reinterpret_cast<int*>(gp);              // [NCAND] candidates in rank order
        const uint4* aq4 = reinterpret_cast<const uint4*>(act8);
        const int2* adp = reinterpret_cast<const int2*>(act8 + nbj * 32);
        const int64_t rec_bytes = (int64_t)E * nbj * 36;
        static_assert(NCAND * 32 <= FT_THREADS && CW <= CD_STRIDE, "32 lanes per candidate's share");
        for (int l = 0; l + 1 < L; ++l) {
            stamp<DBG>(P, l, 0);
            const float bias_l = ld_bias(P, l), bias_n1 = ld_bias(P, l + 1);
            // the early sums: every group's sums of R_{l+1} x_l and of x_l . x_l
            if (!wait_words<DBG, UW_GA>(P, m, epoch, pp_buf(l + 1), NGROUP * ES, ident, tag_g(l + 1), gq, adst, l, 27))
                return;
            float ir = 1.0f;
            if (tid_here() < E) {
                const float4 a = reinterpret_cast<const float4*>(gs + tid_here() * NGROUP)[0];
                const float4 b = reinterpret_cast<const float4*>(gs + tid_here() * NGROUP)[1];
                const float base = ((((((a.x + a.y) + a.z) + a.w) + b.x) + b.y) + b.z) + b.w;
                if (P.input_norm) {
                    const float4 c = reinterpret_cast<const float4*>(gs + E * NGROUP)[0];
                    const float4 d = reinterpret_cast<const float4*>(gs + E * NGROUP)[1];
                    const float ss = ((((((c.x + c.y) + c.z) + c.w) + d.x) + d.y) + d.z) + d.w;
                    int Hs = P.H;
                    asm volatile("" : "+s"(Hs));
                    ir = 1.0f / sqrtf(ss / (float)Hs + 1e-6f);
                }
                bs[tid_here()] = base;
                float4* o = reinterpret_cast<float4*>(lg + tid_here() * NGROUP);
                o[0] = make_float4(base * ir, 0.0f, 0.0f, 0.0f);
                o[1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
            __syncthreads();
            // early prediction (no table) or the candidates (table): rank the early logits
            route_rank(P, m, lg, bias_n1, (l + 1) & 1, nullptr, refine ? cid : nullptr, NCAND);
            if (refine) {
                const int k = tid_here();
                if (k < CW) {
                    const int c = k % NCAND, e = min(max(cid[c], 0), E - 1);
                    const uint32_t v = k < NCAND ? (uint32_t)e
                                     : k < 2 * NCAND ? __float_as_uint(bs[e])
                                     : k < 3 * NCAND ? __float_as_uint(P.bias ? P.bias[(int64_t)(l + 1) * E + e] : 0.0f)
                                     : __float_as_uint(ir);
                    cwl[k] = v;
                    st_tag(cp_buf(l) + r * CD_STRIDE + k, tag_a(l), v);
                }
            }
            // the routing words of layer l: the slot unit group r runs; this
            // wait also orders the writes below after every group unit's and
            // expert unit's reads (the chains stated at the group units)
            if (!wait_words<DBG, UW_GA>(P, m, epoch, gq_buf(l) + rep * P.rs_gq, NGROUP * ES, aidx, tag_g(l), gq, adst, l,
                                        24))
                return;
            stamp<DBG>(P, l, 12);
            if (refine) {
                const bool first = l == 0;
                route_rank(P, m, gs, bias_l, -1, first ? nullptr : m->pid[l & 1]);
                route_weights(P, m, l, first, false);
                __syncthreads();
                const int slot = unit_slot(m, K, r, first);
                const int eid = min(max(m->ids[slot], 0), E - 1);
                const float wr = m->wts[slot];
                // M_{l, eid} rows of the candidates: thread (candidate c, block b) for b < I/32
                const int tq = tid_here();
                const int c = tq >> 5, b = tq & 31, bb = min(b, nbj - 1);
                const int ec = min(max((int)cwl[c], 0), E - 1);
                const uint8_t* rec = P.pred_tab + ((int64_t)l * E + eid) * rec_bytes;
                const uint4* q = reinterpret_cast<const uint4*>(rec + ((int64_t)ec * nbj + bb) * 32);
                const uint4 mq0 = q[0], mq1 = q[1];
                const float md = *reinterpret_cast<const float*>(rec + (int64_t)E * nbj * 32 + ((int64_t)ec * nbj + bb) * 4);
                if (!wait_words<DBG, 1, true>(P, m, epoch, P.act_t + (int64_t)r * nbj * 10, nbj * 10, ident, tag_a(l),
                                              reinterpret_cast<uint32_t*>(act8), act_dst, l, 25))
                    return;
                stamp<DBG>(P, l, 4);
                const uint4 lo = aq4[bb * 2], hi = aq4[bb * 2 + 1];
                const int2 ap = adp[bb];
                int d = 0;
                d = __builtin_amdgcn_sdot4((int)mq0.x, (int)lo.x, d, false);
                d = __builtin_amdgcn_sdot4((int)mq0.y, (int)lo.y, d, false);
                d = __builtin_amdgcn_sdot4((int)mq0.z, (int)lo.z, d, false);
                d = __builtin_amdgcn_sdot4((int)mq0.w, (int)lo.w, d, false);
                d = __builtin_amdgcn_sdot4((int)mq1.x, (int)hi.x, d, false);
                d = __builtin_amdgcn_sdot4((int)mq1.y, (int)hi.y, d, false);
                d = __builtin_amdgcn_sdot4((int)mq1.z, (int)hi.z, d, false);
                d = __builtin_amdgcn_sdot4((int)mq1.w, (int)hi.w, d, false);
                float v = b < nbj ? (float)d * (md * __int_as_float(ap.x)) : 0.0f;
#pragma unroll
                for (int o = 1; o < 32; o <<= 1) v += __shfl_xor(v, o, 32);
                if (b == 0) st_tag(cp_buf(l) + NGROUP * CD_STRIDE + r * NCAND + c, tag_a(l), __float_as_uint(v * wr));
                stamp<DBG>(P, l, 5);
                // every refiner's share -> the prediction, as every expert unit forms it
                if (!wait_words<DBG, 1>(P, m, epoch, cp_buf(l) + NGROUP * CD_STRIDE, NGROUP * NCAND, ident, tag_a(l),
                                        cwl + CD_STRIDE, l, 26))
                    return;
                stamp<DBG>(P, l, 8);
                if (tid_here() < 64) cand_pid(cwl, cwl + CD_STRIDE, m->keys, m->pid[(l + 1) & 1], K);
                __syncthreads();
            }
            if (tid_here() < K)
                st_tag(pid_buf(l + 1) + r * PID_STRIDE + tid_here(), tag_g(l + 1), (uint32_t)m->pid[(l + 1) & 1][tid_here()]);
            stamp<DBG>(P, l, 14);
        }
        return;
    }

    if (w >= P.n_unit) {
        // ============ group unit (routing) or pred unit (early sums) ============
        // Both combine the same rows bit for bit. A group unit then applies the
        // router of layer l+1 (true routing of l+1, q8 of x_{l+1}); a pred unit
        // the router of layer l+2 and publishes its group's sums (pp), the base
        // of the refiners' prediction of layer l+2.
        // Reused words are rewritten only after every reader has read them:
        //   act_t, hp_t (one buffer): rewritten for l+1 after the routing of
        //     l+1, which needs every y of l, produced after the down units'
        //     reads; refiner u reads act(l) of unit group u before publishing
        //     its share (table) or, without a table, does not read it; every
        //     unit of u takes the shares before it writes act(l+1);
        //   y_t (by parity): rewritten for l+2 after the writer took the
        //     prediction of l+2 (or its candidate words) from its refiner,
        //     published after reading every pred unit's sums of l+2, each
        //     computed after reading y(l); group units read y(l) before
        //     publishing the routing of l+1;
        //   gq_t (by layer mod 3): rewritten for l+3 after every y(l+2). An
        //     expert unit reads gq(l) before its y(l); a group unit before
        //     publishing gq(l+1), which the routing of l+2 needs; every
        //     refiner before publishing the prediction of l+1, and every
        //     expert unit takes the prediction of l+2 (published after it)
        //     before writing y(l+2); a pred unit before publishing its sums
        //     of l+2, which every refiner reads before publishing the
        //     prediction of l+2;
        //   pp_t (by parity): rewritten for l+2 after every y(l); each expert
        //     unit wrote y(l) after taking the prediction of l (or its
        //     candidate words) from its refiner, which had read every group's
        //     pp(l);
        //   pid_t (by parity, one copy per refiner): refiner r rewrites it
        //     for l+3 after the routing words of l+2 (every group unit read
        //     pid(l+1) before publishing them, and they follow every y(l+1),
        //     which each expert unit wrote after taking pid(l+1)) and after
        //     every pred unit's sums of l+3 (each pred unit read pid(l+1)
        //     before computing them);
        //   cp_t (by parity): refiner r rewrites its candidate words for l+2
        //     after every pred unit's sums of l+3, i.e. after every y(l+1),
        //     which each expert unit wrote after reading cp(l); and its share
        //     after the routing words of l+2, published by the group units
        //     after the prediction of l+1 from every refiner, each formed
        //     after reading every share of cp(l).
        // Group units: GSPLIT per group, w - n_unit = sp * NGROUP + g (all on
        // XCD g); split sp publishes the router sums of experts sp*E/GSPLIT..,
        // split 0 also the sum of squares and the q8 blocks, and it writes
        // x_out and the debug records. Every split combines the same rows
        // bit for bit and computes the same routing.
        const int ngu = NGROUP * GSPLIT;
        const bool pu = w >= P.n_unit + ngu;
        const int gi = w - P.n_unit;
        const int g = pu ? gi - ngu : gi % NGROUP, r0 = g * HG;
        const int e0 = pu ? 0 : (gi / NGROUP) * (MAX_E / GSPLIT);  // first expert of this split
        const bool primary = !pu && gi < NGROUP;
        const bool record = primary && g == 0;  // writes ids/wts
        auto fail = [&]() __attribute__((always_inline)) {  // a wait gave up: mark the outputs
            if (primary) poison_outputs(P, g);
        };
        if (pu && (!pf || L < 2)) return;    // nothing to predict
        uint32_t* q8w = reinterpret_cast<uint32_t*>(gp + (C + 1) * E);
        float4 wv[CPT][4];
        // The routing words -> LDS [E+1][NGROUP] (row E: the sums of squares):
        // every group's slot of the broadcast (its own group's too, which the
        // other splits write).
        const int ES = E + 1;
        auto aidx = [=](int i) { return (int64_t)(i / ES) * P.gq_stride + i % ES; };
        auto adst = [=](int i) { return (i % ES) * NGROUP + i / ES; };
        // a split's router weights: the first CPT_G rows of wv
        auto& wvg = reinterpret_cast<float4(&)[CPT_G][4]>(wv);
        auto load_router = [&](int layer) __attribute__((always_inline)) {
            if (pu) group_load_router<CPT, C, 4>(P, layer, g, 0, wv);
            else group_load_router<CPT_G, C, LPE_G>(P, layer, g, e0, wvg);
        };
        // publishes the sums of the router just applied to x (gx): a pred unit
        // layer rl's sums to pp, a group unit its broadcast words
        auto publish = [&](int rl, int sl) __attribute__((always_inline)) {
            if (pu) group_publish<CPT, C, 4, DBG>(P, g, 0, wv, gx, gp, q8w, pp_buf(rl), tag_g(rl), sl, true, true);
            else group_publish<CPT_G, C, LPE_G, DBG>(P, g, e0, wvg, gx, gp, q8w, gq_buf(rl), tag_g(rl), sl, false,
                                                     primary);
        };
        stamp<DBG>(P, -1, 0);
        load_router(pu ? 1 : 0);
        float bias_n = ld_bias(P, 0);
        for (int i = t; i < HG; i += FT_THREADS) {
            gx[i] = P.x_in[r0 + i];
            if (DBG && P.dbg_x && primary) P.dbg_x[r0 + i] = gx[i];
        }
        __syncthreads();
        publish(pu ? 1 : 0, -1);
        stamp<DBG>(P, -1, 11);
        if (!wait_words<DBG, UW_GA>(P, m, epoch, gq_buf(0) + rep * P.rs_gq, NGROUP * ES, aidx, tag_g(0), gq, adst)) {
            fail();
            return;
        }
        stamp<DBG>(P, -1, 12);
        route_rank(P, m, reinterpret_cast<const float*>(gq), bias_n, -1, nullptr);
        route_weights(P, m, 0, true, record);
        stamp<DBG>(P, -1, 14);
        for (int l = 0; l < L; ++l) {
            // a pred unit's last sums (layer L-1's router) were published at
            // l = L-3: nothing of its work after that is read
            if (pu && l + 2 >= L) return;
            stamp<DBG>(P, l, 0);
            const int rl = pu ? l + 2 : l + 1;  // the router layer applied after this layer's combine
            if (rl < L) load_router(rl);
            if (l + 1 < L) bias_n = ld_bias(P, l + 1);
            stamp<DBG>(P, l, 1);
            // y of every unit group for this group's rows, [u][HG] in LDS
            auto yidx = [=](int i) { return (int64_t)(i / HG) * H + r0 + i % HG; };
            if (!wait_words<DBG, UW_Y>(P, m, epoch, y_buf(l), K * HG, yidx, tag_y(l), reinterpret_cast<uint32_t*>(gy), l, 26)) { fail(); return; }
            stamp<DBG>(P, l, 8);
            // x_{l+1} = x_l + sum_p (y_p * w_p), pairs in routing order
            // (ft-model/src/lib.rs:1634-1646); slot p ran on unit group pown[p]
            int own[MAX_K];
#pragma unroll
            for (int q = 0; q < MAX_K; ++q) own[q] = m->pown[min(q, K - 1)];
            for (int r = t; r < HG; r += FT_THREADS) {
                float yv[MAX_K], wk[MAX_K];
#pragma unroll
                for (int q = 0; q < MAX_K; ++q) {
                    yv[q] = gy[own[q] * HG + r];
                    wk[q] = m->wts[q];
                }
                float h = 0.0f;
#pragma unroll
                for (int q = 0; q < MAX_K; ++q) {
                    const float part = yv[q] * wk[q];
                    h = q < K ? h + part : h;
                }
                const float xn = gx[r] + h;
                gx[r] = xn;
                if (primary) {
                    if (l == L - 1) P.x_out[r0 + r] = xn;
                    if (DBG && P.dbg_x) P.dbg_x[(int64_t)(l + 1) * H + r0 + r] = xn;
                }
            }
            __syncthreads();
            stamp<DBG>(P, l, 9);
            if (l + 1 == L) break;
            publish(rl, l);
            stamp<DBG>(P, l, 11);
            if (!wait_words<DBG, UW_GA>(P, m, epoch, gq_buf(l + 1) + rep * P.rs_gq, NGROUP * ES, aidx, tag_g(l + 1), gq,
                                        adst, l, 24)) {
                fail();
                return;
            }
            stamp<DBG>(P, l, 12);
            // the prediction of layer l+1, for the slot -> unit group map
            if (pf && !wait_words<DBG, 1>(P, m, epoch, pid_buf(l + 1) + prep * PID_STRIDE, K, ident, tag_g(l + 1),
                                          reinterpret_cast<uint32_t*>(m->pid[(l + 1) & 1]), l, 27)) {
                fail();
                return;
            }
            route_rank(P, m, reinterpret_cast<const float*>(gq), bias_n, -1, pf ? m->pid[(l + 1) & 1] : nullptr);
            route_weights(P, m, l + 1, !pf, record);
            stamp<DBG>(P, l, 14);
        }
        return;
    }

    // ======================= expert unit =======================
    const int u = w % K, j = w / K;
    const bool refine = P.pred_tab != nullptr;  // the refined prediction (see the refiner units)
    const bool gm = w < P.n_gu, dm = w < P.n_dn;  // false: that part of the unit is idle
    const int dn_tile = nbj * 288;               // bytes of one 16-row down tile
    const int ES = E + 1, nq = ES + P.qw;  // per group: E sums, the sum of squares, q8 words
    auto xidx = [=](int i) {
        const int g = i / nq;
        return (int64_t)g * P.gq_stride + (i - g * nq);
    };
    auto xdst = [=](int i) {
        const int g = i / nq, k = i - g * nq;
        const int kk = k - ES, bl = kk / 10, wd = kk - bl * 10, blk = g * (P.qw / 10) + bl;
        return k < ES ? k * NGROUP + g : NGROUP * ES + (wd >= 2 ? blk * 8 + (wd - 2) : nb * 8 + blk * 2 + wd);
    };
    stamp<DBG>(P, -1, 0);
    float bias_n = ld_bias(P, 0);
    if (!wait_words<DBG, UW_X>(P, m, epoch, gq_buf(0) + rep * P.rs_gq, NGROUP * nq, xidx, tag_g(0), gq, xdst)) return;
    // The act hand-over of unit group u stays in the XCD's L2 (plain stores,
    // agent-scope polls) when every unit of group u, and refiner u (which
    // reads the act too), runs on this workgroup's XCD; otherwise its stores
    // write through.
    bool act_local;
    {
        const int upe = P.n_unit / K;  // units per unit group
        const int64_t ref_w = P.n_unit + (GSPLIT + 1) * NGROUP + u;
        uint32_t* xw = reinterpret_cast<uint32_t*>(red);
        if (!wait_words<DBG, 1>(P, m, epoch, P.pl_t, upe + 1,
                                [=](int i) { return i < upe ? (int64_t)(u + K * i) : ref_w; }, tag_g(0), xw))
            return;
        act_local = __syncthreads_and(t > upe || xw[t] == xcc_id()) != 0;
        trace_value<DBG>(P, -1, 27, act_local ? 1u : 0u);
        trace_value<DBG>(P, -1, 28, xcc_id());
    }
    stamp<DBG>(P, -1, 12);
    route_units(P, m, reinterpret_cast<const float*>(gq), bias_n, nullptr);

    // This unit's share of its expert, in registers from the load to the dots
    // (a prefetch holds it across the end of the previous layer):
    //   gate|up tile j, 64 rows x BPW blocks per wave: qv (16 B of nibbles per
    //   row and block), sc (the dword holding the row's f16 scale and its
    //   neighbour row's);
    //   down rows 128j + 16*wave + rr, blocks s4, s4+4, ...: dq, dsc (the
    //   same pairing of scales).
    // Missed tiles (K == 8): the gate|up tile j of a unit group whose held
    // expert was not routed is computed by the 8 units with index j, one wave
    // slice (64 rows x BPW blocks) each, in a wave of theirs otherwise idle
    // (hq, hs); each publishes its slice's per-row partial, the fma chain of
    // exactly that wave of the unit that owns the tile, and the owner sums the
    // 8 partials in wave order as for its own dots: the same bits. A missed
    // tile's 101 KB thus arrives as 8 loads of 12.7 KB on 8 CUs instead of one
    // 101 KB load on one CU (a CU keeps only ~40 KB of loads in flight).
    uint32_t sc[BPW];
    uint4 qv[BPW];
    uint32_t dsc[DB];
    uint4 dq[DB];
    uint32_t hs[BPW];
    uint4 hq[BPW];
    const bool helpers = K == FT_WAVES;
    // per-thread offsets from an opaque thread index: hoisted out of the layer
    // loop they would stay live (and spill) for the whole kernel
    // blocks [i0, i1) of the wave's share (compile-time bounds)
    auto load_gu = [&](int layer, int eid, int s, uint4 (&q)[BPW], uint32_t (&c)[BPW], auto i0, auto i1)
                       __attribute__((always_inline)) {
        constexpr int I0 = decltype(i0)::value, I1 = decltype(i1)::value;
        const int tl = tid_here();
        const uint8_t* xb = P.banks + ((int64_t)layer * E + eid) * P.expert_bytes;
        const int r = tl & 63, b0 = s * BPW;
        // a unit without a gate|up tile re-reads tile 0 of expert 0 of layer 0
        // (shared by all such units, so it stays in cache)
        const uint8_t* T = gm ? xb + (int64_t)j * nb * 1152 : P.banks;
        const uint8_t* Ts = T + b0 * 128 + r * 2;
        const uint8_t* Tq = T + nb * 128 + b0 * 1024 + r * 16;
        // all 16-byte loads first, then the scales: interleaving them more
        // than doubled the time to stream a layer in a probe. A lane loads
        // the aligned dword holding its row's f16 scale and its neighbour's
        // (rows r & ~1 and r | 1, one cache line either way) and picks its
        // half in the dots: a 2-byte load is widened by a separate
        // instruction, which makes the wave wait for the load at once.
#pragma unroll
        for (int i = I0; i < I1; ++i) q[i] = *reinterpret_cast<const uint4*>(Tq + i * 1024);
#pragma unroll
        for (int i = I0; i < I1; ++i) c[i] = *reinterpret_cast<const uint32_t*>(Ts - (r & 1) * 2 + i * 128);
        asm volatile("" ::: "memory");  // issued here, not sunk towards the first use
    };
    auto load_dn = [&](int layer, int eid) __attribute__((always_inline)) {
        const int tl = tid_here();
        const uint8_t* xb = P.banks + ((int64_t)layer * E + eid) * P.expert_bytes;
        const int wave = tl >> 6, s4 = tl & 3, rr = (tl >> 2) & 15;
        const uint8_t* D = (dm ? xb + (int64_t)(j * FT_WAVES + wave) * dn_tile : P.banks) + P.gu_bytes;
#pragma unroll
        for (int k = 0; k < DB; ++k) {
            const int b = min(s4 + 4 * k, nbj - 1);
            dq[k] = *reinterpret_cast<const uint4*>(D + nbj * 32 + b * 256 + rr * 16);
        }
        asm volatile("" ::: "memory");  // keep the scale loads behind the 16-byte loads
#pragma unroll
        for (int k = 0; k < DB; ++k) {
            const int b = min(s4 + 4 * k, nbj - 1);
            dsc[k] = *reinterpret_cast<const uint32_t*>(D + b * 32 + (rr & ~1) * 2);  // rows rr & ~1, rr | 1
        }
        asm volatile("" ::: "memory");
    };
    // Routing of `layer` known (after route_rank): this unit's slot and
    // expert, the missed unit groups, and the wave slice this unit computes
    // for a missed tile (loaded now: it is on the critical path). With no
    // helpers a missed unit loads its whole tile now; with helpers its down
    // tile is loaded after its slice is computed (a CU keeps ~40 KB of loads
    // in flight, and the down tile is needed only after the act hand-over).
    int p = u, eid = 0, hug = 0, hslot = 0;  // hslot: the missed tile's slot (debug records only)
    bool own_miss = true, hm = false;
    auto decide = [&](int layer, bool first) __attribute__((always_inline)) {
        p = m->ufor[u];
        // the routed id is in [0, E) by construction; the clamp keeps any
        // future logic error from turning into an out-of-bounds weight read
        eid = min(max(m->sel_i[p], 0), E - 1);
        own_miss = first || m->uslot[u] < 0;
        hm = false;
        if (helpers) {
            const int mc = m->mcount, wv = tid_here() >> 6;
            const int mi = mc == FT_WAVES ? wv : wv - 1;  // wave 0 keeps the GELU tail unless all missed
            if (mi >= 0 && mi < mc) {
                hm = true;
                hug = m->mlist[mi];
                if (DBG) hslot = m->mslot[mi];
                load_gu(layer, min(max(m->mexp[mi], 0), E - 1), (u - hug) & (FT_WAVES - 1), hq, hs, IC<0>{}, IC<BPW>{});
            }
        } else if (own_miss) {
            load_gu(layer, eid, tid_here() >> 6, qv, sc, IC<0>{}, IC<BPW>{});
            load_dn(layer, eid);
        }
    };
    decide(0, true);
    trace_value<DBG>(P, 0, 10, own_miss ? 1u : 0u);
    int pe = 0;  // the predicted expert of the next layer
    stamp<DBG>(P, -1, 14);

    for (int l = 0; l < L; ++l) {
        stamp<DBG>(P, l, 0);
        const int tl = tid_here();
        const int wave = tl >> 6, r = tl & 63, s4 = tl & 3, rr = (tl >> 2) & 15;
        // ---- gate|up dots -> GELU*up -> q8 block, published ----
        if (gm) {
            // lane t < 32: gate row j*32+t and up row I+j*32+t, the 8 wave
            // partials in red summed in wave order; GELU*up; the q8 block of
            // the 32 lanes, published as {d, qsum, 8 words of qs}
            auto tail = [&]() __attribute__((always_inline)) {
                float gv[FT_WAVES], uv[FT_WAVES];
#pragma unroll
                for (int v = 0; v < FT_WAVES; ++v) {
                    gv[v] = red[v * 64 + t];
                    uv[v] = red[v * 64 + 32 + t];
                }
                float sg = 0.0f, su = 0.0f;
#pragma unroll
                for (int v = 0; v < FT_WAVES; ++v) {
                    sg = sg + gv[v];
                    su = su + uv[v];
                }
                const float ir = m->inv_r;  // input RMS norm: the sums of rmsnorm(x)
                sg = sg * ir;
                su = su * ir;
                if (DBG && P.dbg_gu) {
                    float* dg = P.dbg_gu + ((int64_t)l * K + p) * 2 * I;
                    dg[j * 32 + t] = sg;
                    dg[I + j * 32 + t] = su;
                }
                stamp<DBG>(P, l, 17);
                const float a = gelu_tanh(sg) * su;
                stamp<DBG>(P, l, 18);
                float d;
                int qsum;
                const uint32_t wq = q8_quantize_lanes32(a, &d, &qsum);
                uint64_t* dst = P.act_t + ((int64_t)u * nbj + j) * 10;
                // the word index from the opaque lane index: hoisted out of the
                // layer loop, the store's address was spilled and reloaded (with a
                // vmcnt(0) in front of the hand-over)
                const int ta = tid_here();
                const int k = (ta & 3) == 0 ? 2 + (ta >> 2) : (ta == 1 ? 0 : (ta == 2 ? 1 : -1));
                const uint32_t v = ta == 1 ? __float_as_uint(d) : (ta == 2 ? (uint32_t)qsum : wq);
                if (k >= 0) {
                    if (act_local) st_tag_local(dst + k, tag_a(l), v);
                    else st_tag(dst + k, tag_a(l), v);
                    if (DBG && P.dbg_act)
                        reinterpret_cast<uint32_t*>(P.dbg_act + (((int64_t)l * K + p) * nbj + j) * Q8_BLK)[k] = v;
                }
                stamp<DBG>(P, l, 19);
            };
            // one wave's partial for row r: the fma chain over the BPW blocks
            // s*BPW.. of the tile in (q, c) against q8(x)
            auto wave_partial = [&](const uint4 (&q)[BPW], const uint32_t (&c)[BPW], int s, int slot)
                                    __attribute__((always_inline)) {
                const int b0 = s * BPW;
                float acc = 0.0f;
#pragma unroll
                for (int i = 0; i < BPW; ++i) {
                    const uint4 lo = xq4[(b0 + i) * 2], hi = xq4[(b0 + i) * 2 + 1];
                    const int2 dq8 = xdp[b0 + i];
                    const int diff = block_dot_v(q[i], lo, hi, dq8.y);
                    acc = fmaf((float)diff, h2f((uint16_t)(c[i] >> ((r & 1) * 16))) * __int_as_float(dq8.x), acc);
                    if (DBG && P.rec_gu) {  // test record: the block's int32 dot
                        const int row = r < 32 ? j * 32 + r : I + j * 32 + (r - 32);
                        P.rec_gu[(((int64_t)l * K + slot) * 2 * I + row) * nb + b0 + i] = diff;
                    }
                }
                return acc;
            };
            // the slice this wave computes for a missed tile, to its owner
            auto help = [&]() __attribute__((always_inline)) {
                if (hm) {
                    const int sl = (u - hug) & (FT_WAVES - 1);
                    const float a2 = wave_partial(hq, hs, sl, hslot);
                    st_tag(P.hp_t + (((int64_t)hug * nbj + j) * FT_WAVES + sl) * 64 + r, tag_a(l), __float_as_uint(a2));
                    if (DBG && P.trace && r == 0 && wave == 1)  // slot 29: wave 1's slice published
                        P.trace[((int64_t)blockIdx.x * (P.L + 1) + (l + 1)) * TRACE_SLOTS + 29] = wall_clock64();
                }
            };
            if (!(helpers && own_miss)) {
                red[wave * 64 + r] = wave_partial(qv, sc, wave, p);
                stamp<DBG>(P, l, 2);
                __syncthreads();
                if (t < 32) tail();
                help();
            } else {
                help();
                load_dn(l, eid);
                if (!wait_words<DBG, 1>(P, m, epoch, P.hp_t + ((int64_t)u * nbj + j) * FT_WAVES * 64, FT_WAVES * 64,
                                        ident, tag_a(l), reinterpret_cast<uint32_t*>(red), l, 26))
                    return;
                stamp<DBG>(P, l, 2);
                if (t < 32) tail();
            }
            stamp<DBG>(P, l, 3);
        }
        // the early prediction of layer l+1 (published before this layer
        // started): loaded now, checked after the down dots, when every older
        // load of this wave has landed anyway, so it never stalls the chain
        uint64_t pid_raw = 0;
        if (pf && !refine && l + 1 < L && tid_here() < K)
            pid_raw = ld_tag(pid_buf(l + 1) + prep * PID_STRIDE + tid_here());
        // ---- down: the act blocks of unit group u, then y of 128 rows ----
        if (dm) {
            // act8: [nbj blocks x 32 B qs][nbj (d, qsum) pairs] (16-B aligned qs)
            auto act_dst = [=](int i) {
                const int bi = i / 10, k = i - bi * 10;
                return k >= 2 ? bi * 8 + (k - 2) : nbj * 8 + bi * 2 + k;
            };
            if (!wait_words<DBG, 1, true>(P, m, epoch, P.act_t + (int64_t)u * nbj * 10, nbj * 10, ident, tag_a(l),
                                       reinterpret_cast<uint32_t*>(act8), act_dst, l, 25))
                return;
            stamp<DBG>(P, l, 4);
            const uint4* aq4 = reinterpret_cast<const uint4*>(act8);
            const int2* adp = reinterpret_cast<const int2*>(act8 + nbj * 32);
            int s4o = threadIdx.x & 3;
            asm volatile("" : "+v"(s4o));
            uint4 alo[DB], ahi[DB];
            int2 ap[DB];
#pragma unroll
            for (int k = 0; k < DB; ++k) {  // all LDS operands first: one wait
                const int bi = min(s4o + 4 * k, nbj - 1);
                alo[k] = aq4[bi * 2];
                ahi[k] = aq4[bi * 2 + 1];
                ap[k] = adp[bi];
            }
            float acc = 0.0f;
#pragma unroll
            for (int k = 0; k < DB; ++k) {
                const int dot = block_dot_v(dq[k], alo[k], ahi[k], ap[k].y);
                const float v = (float)dot * (h2f((uint16_t)(dsc[k] >> ((rr & 1) * 16))) * __int_as_float(ap[k].x));
                acc = s4o + 4 * k < nbj ? acc + v : acc;
                if (DBG && P.rec_dn && s4o + 4 * k < nbj)  // test record: the block's int32 dot
                    P.rec_dn[(((int64_t)l * K + p) * H + j * DN_UNIT + wave * DN_ROWS + rr) * nbj + s4o + 4 * k] = dot;
            }
            acc += quad_xor1(acc);
            acc += quad_xor2(acc);
            stamp<DBG>(P, l, 5);
            if (s4 == 0)
                st_tag(y_buf(l) + (int64_t)u * H + j * DN_UNIT + wave * DN_ROWS + rr, tag_y(l), __float_as_uint(acc));
            stamp<DBG>(P, l, 6);
        }
        if (l + 1 == L) break;
        bias_n = ld_bias(P, l + 1);
        // ---- prefetch: the predicted expert of layer l+1 for this unit group ----
        if (pf) {
            if (refine) {
                // the refined prediction, formed here from this XCD's copy of
                // the candidate words and every refiner's share (one hand-over
                // after the shares, as the refiners form it)
                auto cidx = [=](int i) {
                    return (int64_t)(i < CW ? prep * CD_STRIDE + i : NGROUP * CD_STRIDE + (i - CW));
                };
                auto cdst = [=](int i) { return i < CW ? i : CD_STRIDE + (i - CW); };
                uint32_t* cw = reinterpret_cast<uint32_t*>(red);
                if (!wait_words<DBG, 1>(P, m, epoch, cp_buf(l), CW + NGROUP * NCAND, cidx, tag_a(l), cw, cdst, l, 27))
                    return;
                if (tid_here() < 64) cand_pid(cw, cw + CD_STRIDE, m->keys, m->pid[(l + 1) & 1], K);
                __syncthreads();
            } else {
                bool ok = true;
                const int tq = tid_here();  // the lane tests and the LDS address formed here (hoisted, they spilled)
                if (tq < K) {
                    ok = (uint32_t)(pid_raw >> 32) == tag_g(l + 1);
                    m->pid[(l + 1) & 1][tq] = (int)(uint32_t)pid_raw;
                }
                // not yet published (late refiner): the bounded wait
                if (!__syncthreads_and(ok) &&
                    !wait_words<DBG, 1>(P, m, epoch, pid_buf(l + 1) + prep * PID_STRIDE, K, ident, tag_g(l + 1),
                                     reinterpret_cast<uint32_t*>(m->pid[(l + 1) & 1]), l, 27))
                    return;
            }
            pe = min(max(m->pid[(l + 1) & 1][u], 0), E - 1);
            load_gu(l + 1, pe, wave, qv, sc, IC<0>{}, IC<PF_EARLY>{});
            load_dn(l + 1, pe);
            stamp<DBG>(P, l, 7);
        }
        // ---- routing of layer l+1 and the q8 of x_{l+1}, from the group units ----
        if (!wait_words<DBG, UW_X>(P, m, epoch, gq_buf(l + 1) + rep * P.rs_gq, NGROUP * nq, xidx, tag_g(l + 1), gq, xdst, l, 24))
            return;
        stamp<DBG>(P, l, 12);
        if (pf && PF_EARLY < BPW) load_gu(l + 1, pe, wave, qv, sc, IC<PF_EARLY>{}, IC<BPW>{});  // the rest
        route_units(P, m, reinterpret_cast<const float*>(gq), bias_n, pf ? m->pid[(l + 1) & 1] : nullptr);
        stamp<DBG>(P, l, 13);
        decide(l + 1, !pf);
        trace_value<DBG>(P, l + 1, 10, own_miss ? 1u : 0u);
        stamp<DBG>(P, l, 14);
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

// Refined-prediction table (setup): record (l, e), l < L-1, holds
// M = R_{l+1} D_{l,e} (E router rows x I columns; R_{l+1} from the fused
// router layout, D_{l,e} the expert's down rows dequantized from the fused
// layout), each row quantized per 32 columns like a q8 block: [E][I/32][32]
// int8, then [E][I/32] f32 scales (d = amax / 127, q = rint(v / d)). One
// workgroup per (l, e, 64 columns); f32 products summed over the H rows in
// steps of 32. Only the refiners' predictions read it, so its rounding is
// free-form.
constexpr int PT_STEP = 32;  // D rows (R columns) per step
__global__ __launch_bounds__(256) void k_pred_table(const uint8_t* banks, const float* routers, uint8_t* out, int H,
                                                    int I, int64_t expert_bytes, int64_t gu_bytes) {
    constexpr int E = MAX_E;  // the fused shape's expert count (checked by the host)
    __shared__ float Rs[E][PT_STEP + 1];
    __shared__ float Ds[PT_STEP][64];
    __shared__ float Ms[E][65];
    const int kt = blockIdx.x, e = blockIdx.y, l = blockIdx.z, t = threadIdx.x;
    const int nbj = I >> 5, C = H / DN_ROWS;
    const uint8_t* D0 = banks + ((int64_t)l * E + e) * expert_bytes + gu_bytes;
    const float* R = routers + (int64_t)(l + 1) * C * E * DN_ROWS;
    const int tr = t >> 4, tc = t & 15;  // router rows tr*8.., columns tc*4..
    float acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
    for (int h0 = 0; h0 < H; h0 += PT_STEP) {
        for (int i = t; i < E * PT_STEP; i += 256) {  // chunks h0/16 and h0/16+1, [E][16] each
            const int c = i / (E * DN_ROWS), rem = i % (E * DN_ROWS), er = rem / DN_ROWS, ii = rem % DN_ROWS;
            Rs[er][c * DN_ROWS + ii] = R[((int64_t)(h0 / DN_ROWS + c) * E + er) * DN_ROWS + ii];
        }
        if (t < 64) {  // D rows h0.., blocks 2kt and 2kt+1: one (row, block) per thread
            const int rrow = t >> 1, blk = t & 1, h = h0 + rrow, jt = h / DN_ROWS, rr = h % DN_ROWS, b = 2 * kt + blk;
            const uint8_t* T = D0 + (int64_t)jt * nbj * 288;
            const float d = h2f(*reinterpret_cast<const uint16_t*>(T + b * 32 + rr * 2));
            const uint4 q = *reinterpret_cast<const uint4*>(T + nbj * 32 + b * 256 + rr * 16);
            const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int byte = (int)((qw[i >> 2] >> ((i & 3) * 8)) & 0xFF);
                Ds[rrow][blk * 32 + i] = d * (float)((byte & 15) - 8);
                Ds[rrow][blk * 32 + i + 16] = d * (float)((byte >> 4) - 8);
            }
        }
        __syncthreads();
#pragma unroll 4
        for (int hh = 0; hh < PT_STEP; ++hh) {
            float a[8], b[4];
#pragma unroll
            for (int i = 0; i < 8; ++i) a[i] = Rs[tr * 8 + i][hh];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = Ds[hh][tc * 4 + j];
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) Ms[tr * 8 + i][tc * 4 + j] = acc[i][j];
    __syncthreads();
    // row er, block 2kt + blk: amax, scale, quants
    const int er = t >> 1, blk = t & 1, b = 2 * kt + blk;
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(Ms[er][blk * 32 + i]));
    const float d = amax / 127.0f;
    uint32_t w[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        uint32_t v = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float x = Ms[er][blk * 32 + 4 * k + i];
            const int q = d > 0.0f ? (int)fminf(fmaxf(rintf(x / d), -127.0f), 127.0f) : 0;
            v |= (uint32_t)(q & 0xFF) << (8 * i);
        }
        w[k] = v;
    }
    uint8_t* rec = out + ((int64_t)l * E + e) * ((int64_t)E * nbj * 36);
    uint4* qd = reinterpret_cast<uint4*>(rec + ((int64_t)er * nbj + b) * 32);
    qd[0] = make_uint4(w[0], w[1], w[2], w[3]);
    qd[1] = make_uint4(w[4], w[5], w[6], w[7]);
    *reinterpret_cast<float*>(rec + (int64_t)E * nbj * 32 + ((int64_t)er * nbj + b) * 4) = d;
}

__global__ void k_fill_u32(uint32_t* p, int64_t n, uint32_t v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
struct WsLayout {
    int64_t ctl, act, hp, y, gq, pp, pid, pl, cp, total;
    int gq_stride, qw;
    int64_t rs_gq;  // words
};

WsLayout ws_layout(int64_t H, int64_t I, int64_t E, int64_t K) {
    auto up = [](int64_t v) { return (v + 255) / 256 * 256; };
    WsLayout w{};
    w.qw = (int)(H / NGROUP / 32 * 10);
    w.gq_stride = (int)((E + 1 + w.qw + 31) / 32 * 32);
    w.rs_gq = NGROUP * (int64_t)w.gq_stride;
    int64_t off = 0;
    w.ctl = off; off += 256;
    w.act = off; off += up(K * (I / 32) * 10 * 8);
    w.hp = off; off += up(K * (I / 32) * FT_WAVES * 64 * 8);
    w.y = off; off += 2 * up(K * H * 8);
    w.gq = off; off += 3 * NREP * up(w.rs_gq * 8);
    w.pp = off; off += 2 * up(NGROUP * (E + 1) * 8);
    w.pid = off; off += 2 * up(NGROUP * PID_STRIDE * 8);
    w.pl = off; off += up(((int64_t)std::max(K * (I / 32), K * (H / DN_UNIT)) + (GSPLIT + 2) * NGROUP) * 8);
    w.cp = off; off += 2 * up(CP_WORDS * 8);
    w.total = off;
    return w;
}

int fused_units(int64_t H, int64_t I, int64_t K, int* n_gu, int* n_dn) {
    *n_gu = (int)(K * (I / 32));
    *n_dn = (int)(K * (H / DN_UNIT));
    return std::max(*n_gu, *n_dn);
}

// The fused kernel is built and tested for the Gemma shape only (the unit
// layout, helper slices and LDS plan are exercised by the tests at that
// shape alone); other shapes take ft_hip_moe_layer / ft_hip_moe_layer_grouped.
int check_fused_shape(const char* nm, int64_t H, int64_t I, int64_t E, int64_t K, int64_t L) {
    if (H != 2816 || I != 704 || E != 128 || K != 8)
        return fail(FT_HIP_E_SHAPE,
                    "%s: hidden=%lld inter=%lld n_experts=%lld top_k=%lld: the fused kernel is built for the Gemma "
                    "shape (2816, 704, 128, 8); use ft_hip_moe_layer for others",
                    nm, (long long)H, (long long)I, (long long)E, (long long)K);
    if (L <= 0) return fail(FT_HIP_E_SHAPE, "%s: n_layers must be positive", nm);
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

extern "C" int ft_hip_fused_workgroups(int64_t hidden, int64_t inter, int64_t n_experts, int64_t top_k) {
    if (hidden <= 0 || hidden % 256 || inter <= 0 || inter % 32 || n_experts <= 0 || top_k <= 0) return -1;
    int n_gu, n_dn;
    return fused_units(hidden, inter, top_k, &n_gu, &n_dn) + (GSPLIT + 2) * NGROUP;
}

extern "C" int ft_hip_fused_workspace_init(ft_hip_ctx* ctx, void* stream, void* workspace, size_t workspace_bytes) {
    clear_error();
    if (!ctx || !workspace) return fail(FT_HIP_E_INVALID, "fused_workspace_init: null argument");
    if (workspace_bytes % 4) return fail(FT_HIP_E_SHAPE, "fused_workspace_init: size not a multiple of 4");
    if (workspace_bytes < 256) return fail(FT_HIP_E_SHAPE, "fused_workspace_init: workspace too small");
    const int64_t n = (int64_t)(workspace_bytes / 4);
    hipLaunchKernelGGL(k_fill_u32, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       (uint32_t*)workspace, n, 0u);
    if (int rc = launch_status("fused_workspace_init")) return rc;
    // epoch 1: tags of zero-filled words never match
    hipLaunchKernelGGL(k_fill_u32, dim3(1), dim3(1), 0, reinterpret_cast<hipStream_t>(stream),
                       (uint32_t*)workspace + CTL_EPOCH, (int64_t)1, 1u);
    if (int rc = launch_status("fused_workspace_init")) return rc;
    ctx->fused_epochs[workspace] = 1;
    return FT_HIP_OK;
}

extern "C" int ft_hip_fused_workspace_set_epoch(ft_hip_ctx* ctx, void* stream, void* workspace, uint32_t epoch) {
    clear_error();
    if (!ctx || !workspace) return fail(FT_HIP_E_INVALID, "fused_workspace_set_epoch: null argument");
    if (epoch == 0) return fail(FT_HIP_E_SHAPE, "fused_workspace_set_epoch: epoch 0 is reserved");
    hipLaunchKernelGGL(k_fill_u32, dim3(1), dim3(1), 0, reinterpret_cast<hipStream_t>(stream),
                       (uint32_t*)workspace + CTL_EPOCH, (int64_t)1, epoch);
    if (int rc = launch_status("fused_workspace_set_epoch")) return rc;
    ctx->fused_epochs[workspace] = epoch;
    return FT_HIP_OK;
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

extern "C" int64_t ft_hip_fused_predictor_bytes(int64_t hidden, int64_t inter, int64_t n_experts, int64_t n_layers) {
    if (hidden <= 0 || hidden % 32 || inter <= 0 || inter % 64 || n_experts <= 0 || n_layers <= 0) return -1;
    return (n_layers - 1) * n_experts * n_experts * (inter / 32) * 36;
}

extern "C" int ft_hip_fused_build_predictor(ft_hip_ctx* ctx, void* stream, const void* banks, const float* routers,
                                            int64_t hidden, int64_t inter, int64_t n_experts, int64_t n_layers,
                                            void* table, size_t table_bytes) {
    clear_error();
    const char* nm = "fused_build_predictor";
    if (int rc = check_fused_shape(nm, hidden, inter, n_experts, MAX_K, n_layers)) return rc;
    const int64_t need = ft_hip_fused_predictor_bytes(hidden, inter, n_experts, n_layers);
    if ((int64_t)table_bytes < need)
        return fail(FT_HIP_E_SHAPE, "%s: table_bytes=%zu < %lld", nm, table_bytes, (long long)need);
    if (!ctx || !banks || !routers || (need > 0 && !table)) return fail(FT_HIP_E_INVALID, "%s: null argument", nm);
    if ((reinterpret_cast<uintptr_t>(banks) | reinterpret_cast<uintptr_t>(routers) | reinterpret_cast<uintptr_t>(table)) & 15)
        return fail(FT_HIP_E_SHAPE, "%s: banks, routers and table must be 16-byte aligned", nm);
    if (need == 0) return FT_HIP_OK;
    hipLaunchKernelGGL(k_pred_table, dim3((unsigned)(inter / 64), (unsigned)n_experts, (unsigned)(n_layers - 1)),
                       dim3(256), 0, reinterpret_cast<hipStream_t>(stream), (const uint8_t*)banks, routers,
                       (uint8_t*)table, (int)hidden, (int)inter, ft_hip_fused_expert_bytes(hidden, inter),
                       2 * inter * (hidden / 32) * 18);
    return launch_status(nm);
}

extern "C" int ft_hip_fused_set_predictor(ft_hip_ctx* ctx, const void* table, size_t table_bytes, int64_t n_layers) {
    clear_error();
    if (!ctx) return fail(FT_HIP_E_INVALID, "fused_set_predictor: null ctx");
    if (table && (n_layers <= 0 || (reinterpret_cast<uintptr_t>(table) & 15)))
        return fail(FT_HIP_E_SHAPE, "fused_set_predictor: n_layers must be positive and the table 16-byte aligned");
    ctx->fused_pred = table;
    ctx->fused_pred_bytes = table ? table_bytes : 0;
    ctx->fused_pred_layers = table ? n_layers : 0;
    return FT_HIP_OK;
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
    P.n_unit = fused_units(hidden, inter, top_k, &P.n_gu, &P.n_dn);
    const int nw = P.n_unit + (GSPLIT + 2) * NGROUP;  // + group, pred and refiner units
    P.gq_stride = wl.gq_stride;
    P.qw = wl.qw;
    P.rs_gq = (wl.rs_gq * 8 + 255) / 256 * 256 / 8;
    // LDS plan (expert units and group units use disjoint regions)
    const int C = (int)(hidden / 128), HG = (int)(hidden / NGROUP), nbj = (int)(inter / 32);
    auto up16 = [](int v) { return (v + 15) / 16 * 16; };
    int off = 0;
    P.o_act8 = off; off += up16(nbj * Q8_BLK);
    P.o_red = off; off += up16(FT_WAVES * 64 * 4);
    P.o_gq = off; off += up16((NGROUP * ((int)n_experts + 1) + (int)(hidden / 32) * 10) * 4);
    P.o_gx = off; off += up16(HG * 4);
    P.o_gy = off; off += up16((int)top_k * HG * 4);
    P.o_gp = off; off += up16(((C + 1) * (int)n_experts + wl.qw + C + 1) * 4);
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
    P.act_t = (uint64_t*)(ws + wl.act);
    P.hp_t = (uint64_t*)(ws + wl.hp);
    P.y_t = (uint64_t*)(ws + wl.y);
    P.gq_t = (uint64_t*)(ws + wl.gq);
    P.pp_t = (uint64_t*)(ws + wl.pp);
    P.pid_t = (uint64_t*)(ws + wl.pid);
    P.pl_t = (uint64_t*)(ws + wl.pl);
    P.cp_t = (uint64_t*)(ws + wl.cp);
    P.ctl = (uint32_t*)(ws + wl.ctl);
    P.dbg_gu = dbg_gu;
    P.dbg_act = (uint8_t*)dbg_act;
    P.dbg_x = dbg_x;
    P.trace = dbg_trace;
    P.rec_gu = ctx->rec_gu;
    P.rec_dn = ctx->rec_dn;
    P.expert_bytes = ft_hip_fused_expert_bytes(hidden, inter);
    P.gu_bytes = 2 * inter * (hidden / 32) * 18;
    P.spin_limit = ctx->fused_spin_limit;
    P.prefetch = ctx->fused_prefetch;
    // the refined-prediction table (ft_hip_fused_set_predictor): it must cover
    // this launch's layers; it only steers the prefetch, never the results
    if (ctx->fused_pred) {
        const int64_t need = ft_hip_fused_predictor_bytes(hidden, inter, n_experts, n_layers);
        if (n_layers > ctx->fused_pred_layers || (int64_t)ctx->fused_pred_bytes < need)
            return fail(FT_HIP_E_SHAPE, "%s: the predictor table was built for %lld layers (%zu B); this launch has %lld",
                        nm, (long long)ctx->fused_pred_layers, ctx->fused_pred_bytes, (long long)n_layers);
        P.pred_tab = (const uint8_t*)ctx->fused_pred;
    }
    P.input_norm = ctx->input_norm;
    // The epoch guard: a launch advances the workspace's epoch by 4(L+1) and
    // its tags must stay below 2^32. For a workspace this context initialised
    // (ft_hip_fused_workspace_init) the epoch is tracked here, and a launch
    // that would pass the limit is preceded by a re-initialisation on the same
    // stream (every ~2^32/(4(L+1)) launches: 34.6M for 30 layers, 4 h of
    // decode at 420 us). An untracked workspace near the limit is refused by
    // the kernel (ft_hip_fused_status).
    const uint64_t step = 4ull * (uint64_t)(n_layers + 1);
    if (step > 0xFFFFFFFFull / 2) return fail(FT_HIP_E_SHAPE, "%s: n_layers=%lld too large", nm, (long long)n_layers);
    auto ep = ctx->fused_epochs.find(workspace);
    if (ep != ctx->fused_epochs.end() && ep->second > 0xFFFFFFFFull - step) {
        if (int rc = ft_hip_fused_workspace_init(ctx, stream, workspace, workspace_bytes)) return rc;
        clear_error();
        ep = ctx->fused_epochs.find(workspace);
    }
    void* args[] = {&P};
    // the Gemma shape (check_fused_shape): 11 gate|up blocks per wave, 6 down
    // blocks per thread, 6 router chunks per group-unit thread; debug records
    // and the phase trace are compiled in only when asked for
    const bool dbg = dbg_gu || dbg_act || dbg_x || dbg_trace || (ctx->rec_gu && ctx->rec_dn);
    const void* kern = dbg ? reinterpret_cast<const void*>(k_moe_stack_fused<11, 6, 6, true>)
                           : reinterpret_cast<const void*>(k_moe_stack_fused<11, 6, 6, false>);
    // Plain launch (default): every workgroup must be resident at once, which
    // holds when the kernel has the device to itself (nw <= CUs, one
    // workgroup per CU). A cooperative launch (ft_hip_fused_set_cooperative)
    // guarantees it when kernels of other streams share the device, at ~19 us
    // more per launch measured here. If residency ever fails in a plain
    // launch, the resident workgroups give up their bounded waits and the
    // launch reports FT_HIP_E_TIMEOUT through ft_hip_fused_status; nothing
    // hangs.
    hipError_t e = ctx->fused_cooperative
                       ? hipLaunchCooperativeKernel(kern, dim3((unsigned)nw), dim3(FT_THREADS), args,
                                                    (unsigned)P.lds_bytes, reinterpret_cast<hipStream_t>(stream))
                       : hipLaunchKernel(kern, dim3((unsigned)nw), dim3(FT_THREADS), args, (size_t)P.lds_bytes,
                                         reinterpret_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(FT_HIP_E_LAUNCH, "%s: launch failed: %s", nm, hipGetErrorString(e));
    if (ep != ctx->fused_epochs.end()) ep->second += step;
    return FT_HIP_OK;
}

extern "C" int ft_hip_fused_set_spin_limit(ft_hip_ctx* ctx, int polls) {
    clear_error();
    if (!ctx) return fail(FT_HIP_E_INVALID, "fused_set_spin_limit: null ctx");
    if (polls < 0) return fail(FT_HIP_E_SHAPE, "fused_set_spin_limit: polls=%d < 0", polls);
    ctx->fused_spin_limit = polls;
    return FT_HIP_OK;
}

extern "C" int ft_hip_fused_set_prefetch(ft_hip_ctx* ctx, int on) {
    clear_error();
    if (!ctx) return fail(FT_HIP_E_INVALID, "fused_set_prefetch: null ctx");
    if (on != 0 && on != 1) return fail(FT_HIP_E_SHAPE, "fused_set_prefetch: on=%d is not 0 or 1", on);
    ctx->fused_prefetch = on;
    return FT_HIP_OK;
}

extern "C" int ft_hip_fused_set_cooperative(ft_hip_ctx* ctx, int on) {
    clear_error();
    if (!ctx) return fail(FT_HIP_E_INVALID, "fused_set_cooperative: null ctx");
    if (on != 0 && on != 1) return fail(FT_HIP_E_SHAPE, "fused_set_cooperative: on=%d is not 0 or 1", on);
    ctx->fused_cooperative = on;
    return FT_HIP_OK;
}

extern "C" int ft_hip_fused_status(ft_hip_ctx* ctx, void* workspace, int* aborted) {
    clear_error();
    if (!ctx || !workspace || !aborted) return fail(FT_HIP_E_INVALID, "fused_status: null argument");
    uint32_t ctl[64];
    hipError_t e = hipMemcpy(ctl, workspace, sizeof ctl, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return fail(FT_HIP_E_LAUNCH, "fused_status: %s", hipGetErrorString(e));
    *aborted = ctl[CTL_ABORT] != 0;
    if (ctl[CTL_ABORT] == ABORT_EPOCH_WRAP)
        return fail(FT_HIP_E_TIMEOUT, "fused kernel refused a launch whose tags would pass 2^32 (epoch %u); "
                                      "re-initialise the workspace (ft_hip_fused_workspace_init)", ctl[CTL_EPOCH]);
    if (*aborted) return fail(FT_HIP_E_TIMEOUT, "fused kernel aborted a bounded wait (epoch %u)", ctl[CTL_ABORT]);
    return FT_HIP_OK;
}
