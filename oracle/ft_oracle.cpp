// ft_oracle.cpp -- CPU restatement of freeToken-rs's MoE expert-FFN decode
// arithmetic, used ONLY as the checker in tests/, __graft_entry__.smoke() and
// bench.py's cpu_baseline leg. It is test infrastructure, never a product
// path: the HIP library in freetoken-rs_amd/ never links or calls it.
//
// Every function cites the reference source it restates (paths relative to
// the freeToken-rs repository root). Build flags (oracle/Makefile) are
// -O2 -mavx2 -mfma -mf16c -ffp-contract=off: Rust never contracts a*b+c into
// an FMA, so neither may this file, except where the Rust source itself calls
// an FMA intrinsic (_mm256_fmadd_ps in dot_q4_q8_avx2).
//
// Three functions have no counterpart in the reference and are definitions of
// this build, shared bit-for-bit with the GPU kernels (the input RMS norm,
// orc_rms_inv, is the third; see its comment):
//   * orc_router_logits: the reference computes router logits only on its GPU
//     (ft-cuda/src/q4.cu:1153-1174) in an order tied to its launch shape; this
//     build defines one order (the "R-order", below) that CPU and GPU follow.
//
// GELU's tanh and the routing softmax's exp are the host libm's tanhf / expf,
// the functions Rust's f32::tanh / f32::exp call on Linux (ft-model/src/
// lib.rs:436, :1495). The kernels compute the same bits with a restatement of
// glibc's algorithms (freetoken-rs_amd/csrc/ft_libm.hpp, swept against this
// libm over every f32 input by tests/test_libm.py).

#include <immintrin.h>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>
#include <algorithm>
#include <functional>
#include <condition_variable>
#include <memory>
#include <mutex>

extern "C" {

// ---------------------------------------------------------------------------
// q4_0 format: ft-core/src/q4_0.rs:9-16
// ---------------------------------------------------------------------------
static const int64_t QK = 32;
static const int64_t BLOCK_BYTES = 18;

int64_t orc_row_bytes(int64_t k) { return (k % QK) ? -1 : k / QK * BLOCK_BYTES; }

static inline float f16_to_f32(uint16_t h) { return _cvtsh_ss(h); }
static inline uint16_t f32_to_f16(float f) {
    // IEEE round-to-nearest-even, as half::f16::from_f32 (half 2.7.1).
    return (uint16_t)_cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT);
}

// ft-core/src/q4_0.rs:20-40 (quantize_row): per 32 values, maxv is the first
// value of largest magnitude, d = maxv / -8, id = 1/d (from the unrounded
// f32 d), q = clamp(trunc(x*id + 8.5), 0, 15), byte i = q_i | q_{i+16} << 4.
void orc_quantize_row(const float* row, int64_t k, uint8_t* out) {
    for (int64_t b = 0; b < k / QK; ++b) {
        const float* xb = row + b * QK;
        uint8_t* blk = out + b * BLOCK_BYTES;
        float amax = 0.0f, maxv = 0.0f;
        for (int i = 0; i < QK; ++i) {
            float a = std::fabs(xb[i]);
            if (a > amax) { amax = a; maxv = xb[i]; }
        }
        float d = maxv / -8.0f;
        float id = (d != 0.0f) ? 1.0f / d : 0.0f;
        uint16_t h = f32_to_f16(d);
        blk[0] = (uint8_t)(h & 0xFF);
        blk[1] = (uint8_t)(h >> 8);
        for (int i = 0; i < QK / 2; ++i) {
            float t0 = xb[i] * id;            // separate mul and add: no FMA
            float t1 = xb[i + QK / 2] * id;
            float v0 = t0 + 8.5f, v1 = t1 + 8.5f;
            int q0 = (int)v0, q1 = (int)v1;   // Rust `as i32`: truncation
            q0 = std::min(15, std::max(0, q0));
            q1 = std::min(15, std::max(0, q1));
            blk[2 + i] = (uint8_t)(q0 | (q1 << 4));
        }
    }
}

// ft-core/src/q4_0.rs:43-52 (dequantize_row): w = (q - 8) * d.
void orc_dequantize_row(const uint8_t* row, int64_t k, float* out) {
    for (int64_t b = 0; b < k / QK; ++b) {
        const uint8_t* blk = row + b * BLOCK_BYTES;
        float d = f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        for (int i = 0; i < QK / 2; ++i) {
            out[b * QK + i] = (float)((int)(blk[2 + i] & 0xF) - 8) * d;
            out[b * QK + i + QK / 2] = (float)((int)(blk[2 + i] >> 4) - 8) * d;
        }
    }
}

// ft-core/src/q4_0.rs:62-78 (Q8Vec::quantize): d = amax/127 in f32,
// inv = 1/d, q = clamp(round_half_away(v*inv), -127, 127). Zero block: d=0,
// q=0. The scale stays f32 (it is NOT ggml's fp16 block_q8_0 scale).
// Non-finite values follow Rust: f32::max ignores NaN in the amax fold (as
// fmax does); a NaN product (inf*0 when the block holds inf, so inv = 0;
// 0*inf when amax/127 is subnormal, so inv = inf; NaN input) stays NaN
// through round() and clamp(), and `as i8` maps NaN to 0.
void orc_q8_quantize(const float* x, int64_t k, float* d, int8_t* qs) {
    for (int64_t b = 0; b < k / QK; ++b) {
        const float* xb = x + b * QK;
        float amax = 0.0f;
        for (int i = 0; i < QK; ++i) amax = std::fmax(amax, std::fabs(xb[i]));
        float s = amax > 0.0f ? amax / 127.0f : 0.0f;
        float inv = s > 0.0f ? 1.0f / s : 0.0f;
        d[b] = s;
        for (int i = 0; i < QK; ++i) {
            float r = std::round(xb[i] * inv);   // half away from zero
            r = r == r ? std::fmin(127.0f, std::fmax(-127.0f, r)) : 0.0f;  // NaN as i8 = 0
            qs[b * QK + i] = (int8_t)r;
        }
    }
}

// ft-core/src/q4_0.rs:105-118 (dot_q4_q8_scalar): acc += (d4*d8) * float(s),
// separate multiply and add.
float orc_dot_q4_q8_scalar(const uint8_t* row, const float* d8, const int8_t* qs8, int64_t k) {
    float acc = 0.0f;
    for (int64_t b = 0; b < k / QK; ++b) {
        const uint8_t* blk = row + b * BLOCK_BYTES;
        float d4 = f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        int32_t s = 0;
        for (int i = 0; i < QK / 2; ++i) {
            int lo = (int)(blk[2 + i] & 0xF) - 8;
            int hi = (int)(blk[2 + i] >> 4) - 8;
            s += lo * qs8[b * QK + i] + hi * qs8[b * QK + i + QK / 2];
        }
        float sc = d4 * d8[b];
        float t = sc * (float)s;
        acc = acc + t;
    }
    return acc;
}

// The integer core of one block of dot_q4_q8_avx2 (ft-core/src/q4_0.rs:133-150):
// 8 i32 lanes, lane j = sum over elements 4j..4j+3 of q4u*q8 - 8*q8.
static inline __m256i avx2_block_diff(const uint8_t* qs16, const int8_t* q8p) {
    const __m256i low_mask = _mm256_set1_epi8(0x0F);
    const __m256i ones16 = _mm256_set1_epi16(1);
    const __m256i eights = _mm256_set1_epi8(8);
    __m128i packed = _mm_loadu_si128((const __m128i*)qs16);
    __m256i q4 = _mm256_and_si256(_mm256_set_m128i(_mm_srli_epi16(packed, 4), packed), low_mask);
    __m256i q8 = _mm256_loadu_si256((const __m256i*)q8p);
    __m256i prod32 = _mm256_madd_epi16(_mm256_maddubs_epi16(q4, q8), ones16);
    __m256i off32 = _mm256_madd_epi16(_mm256_maddubs_epi16(eights, q8), ones16);
    return _mm256_sub_epi32(prod32, off32);
}

// ft-core/src/q4_0.rs:153-159: ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)).
static inline float avx2_hsum(__m256 acc) {
    __m128 hi = _mm256_extractf128_ps(acc, 1);
    __m128 lo = _mm256_castps256_ps128(acc);
    __m128 s = _mm_add_ps(lo, hi);
    s = _mm_hadd_ps(s, s);
    s = _mm_hadd_ps(s, s);
    return _mm_cvtss_f32(s);
}

// ft-core/src/q4_0.rs:123-160 (dot_q4_q8_avx2): per block, scale = d4*d8 (f32
// mul), acc_j = fma(float(diff_j), scale, acc_j) over 8 lane chains.
float orc_dot_q4_q8_avx2(const uint8_t* row, const float* d8, const int8_t* qs8, int64_t k) {
    __m256 acc = _mm256_setzero_ps();
    for (int64_t b = 0; b < k / QK; ++b) {
        const uint8_t* blk = row + b * BLOCK_BYTES;
        float d4 = f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        __m256 scale = _mm256_set1_ps(d4 * d8[b]);
        __m256i diff = avx2_block_diff(blk + 2, qs8 + b * QK);
        acc = _mm256_fmadd_ps(_mm256_cvtepi32_ps(diff), scale, acc);
    }
    return avx2_hsum(acc);
}

// Per-(block) int32 dots sum_i (q4_i - 8) * q8_i, taken from the same AVX2
// integer lanes as orc_dot_q4_q8_avx2 (their exact sum). Used to pin the
// GPU's per-block integer dots bit for bit.
void orc_block_dots(const uint8_t* row, const int8_t* qs8, int64_t k, int32_t* out) {
    for (int64_t b = 0; b < k / QK; ++b) {
        __m256i diff = avx2_block_diff(row + b * BLOCK_BYTES + 2, qs8 + b * QK);
        alignas(32) int32_t lanes[8];
        _mm256_store_si256((__m256i*)lanes, diff);
        int32_t s = 0;
        for (int j = 0; j < 8; ++j) s += lanes[j];
        out[b] = s;
    }
}

// ---------------------------------------------------------------------------
// q4r repacked rows: ft-core/src/q4_0.rs:234-323
// ---------------------------------------------------------------------------
int64_t orc_q4r_scales_bytes(int64_t k) { int64_t n = k / QK * 2; return (n + 15) / 16 * 16; }
int64_t orc_q4r_row_bytes(int64_t k) { return orc_q4r_scales_bytes(k) + k / QK * 16; }

// ft-core/src/q4_0.rs:248-258 (repack_row_q4r). Padding bytes are zeroed.
void orc_repack_row_q4r(const uint8_t* src, uint8_t* dst, int64_t k) {
    int64_t nb = k / QK, qs_off = orc_q4r_scales_bytes(k);
    std::memset(dst, 0, (size_t)qs_off);
    for (int64_t b = 0; b < nb; ++b) {
        dst[b * 2] = src[b * 18];
        dst[b * 2 + 1] = src[b * 18 + 1];
        std::memcpy(dst + qs_off + b * 16, src + b * 18 + 2, 16);
    }
}

// ft-core/src/q4_0.rs:276-292 (dot_q4r_q8_scalar)
float orc_dot_q4r_q8_scalar(const uint8_t* row, const float* d8, const int8_t* qs8, int64_t k) {
    int64_t nb = k / QK, qs_off = orc_q4r_scales_bytes(k);
    float acc = 0.0f;
    for (int64_t b = 0; b < nb; ++b) {
        float d4 = f16_to_f32((uint16_t)(row[b * 2] | (row[b * 2 + 1] << 8)));
        const uint8_t* q = row + qs_off + b * 16;
        int32_t s = 0;
        for (int i = 0; i < 16; ++i) {
            int lo = (int)(q[i] & 0xF) - 8;
            int hi = (int)(q[i] >> 4) - 8;
            s += lo * qs8[b * QK + i] + hi * qs8[b * QK + i + 16];
        }
        float sc = d4 * d8[b];
        float t = sc * (float)s;
        acc = acc + t;
    }
    return acc;
}

// ft-core/src/q4_0.rs:294-323 (dot_q4r_q8_avx2)
float orc_dot_q4r_q8_avx2(const uint8_t* row, const float* d8, const int8_t* qs8, int64_t k) {
    int64_t nb = k / QK, qs_off = orc_q4r_scales_bytes(k);
    __m256 acc = _mm256_setzero_ps();
    for (int64_t b = 0; b < nb; ++b) {
        float d4 = f16_to_f32((uint16_t)(row[b * 2] | (row[b * 2 + 1] << 8)));
        __m256 scale = _mm256_set1_ps(d4 * d8[b]);
        __m256i diff = avx2_block_diff(row + qs_off + b * 16, qs8 + b * QK);
        acc = _mm256_fmadd_ps(_mm256_cvtepi32_ps(diff), scale, acc);
    }
    return avx2_hsum(acc);
}

// ---------------------------------------------------------------------------
// Row-parallel GEMV (rayon par_iter_mut over rows, ft-core/src/q4_0.rs:90-103
// and :261-274), with a plain std::thread split of the output rows.
// ---------------------------------------------------------------------------
// A persistent worker pool (rayon keeps its pool alive too), so per-call cost
// is a hand-off, not a thread spawn. Idle workers spin on the job counter
// for a while before sleeping (rayon's workers also spin between jobs), so
// back-to-back GEMVs of one token do not pay a futex wake-up each; the
// caller spins until every worker has checked out of the job, so no worker
// can still hold it when run() returns.
namespace {
struct Pool {
    std::vector<std::thread> workers;
    std::mutex m;
    std::condition_variable cv;
    const std::function<void(int64_t, int64_t)>* job = nullptr;
    std::atomic<int64_t> next{0};
    int64_t n = 0, chunk = 16;
    std::atomic<int> busy{0};
    std::atomic<uint64_t> gen{0};
    std::atomic<bool> stop{false};

    explicit Pool(int nthreads) {
        for (int t = 0; t < nthreads - 1; ++t) workers.emplace_back([this] { loop(); });
    }
    ~Pool() {
        {
            std::lock_guard<std::mutex> g(m);
            stop.store(true);
        }
        cv.notify_all();
        for (auto& w : workers) w.join();
    }
    void drain() {
        for (;;) {
            int64_t s = next.fetch_add(chunk);
            if (s >= n) break;
            (*job)(s, std::min(n, s + chunk));
        }
    }
    void loop() {
        uint64_t seen = 0;
        for (;;) {
            int spins = 0;
            while (gen.load(std::memory_order_acquire) == seen && !stop.load(std::memory_order_acquire)) {
                if (++spins < (1 << 18)) {
                    _mm_pause();
                } else {
                    std::unique_lock<std::mutex> g(m);
                    cv.wait(g, [&] { return stop.load() || gen.load() != seen; });
                }
            }
            if (stop.load()) return;
            seen = gen.load(std::memory_order_acquire);
            drain();
            busy.fetch_sub(1, std::memory_order_acq_rel);
        }
    }
    void run(int64_t total, const std::function<void(int64_t, int64_t)>& f) {
        job = &f;
        n = total;
        next.store(0);
        busy.store((int)workers.size());
        {
            std::lock_guard<std::mutex> g(m);
            gen.fetch_add(1, std::memory_order_acq_rel);
        }
        cv.notify_all();
        drain();
        while (busy.load(std::memory_order_acquire) != 0) _mm_pause();
    }
};
std::mutex g_pool_mu;
std::unique_ptr<Pool> g_pool;
int g_pool_size = 0;
}  // namespace

static void parallel_rows(int64_t n, int threads, const std::function<void(int64_t, int64_t)>& f) {
    if (threads <= 1 || n < 64) { f(0, n); return; }
    std::lock_guard<std::mutex> g(g_pool_mu);
    if (!g_pool || g_pool_size != threads) {
        g_pool.reset();
        g_pool.reset(new Pool(threads));
        g_pool_size = threads;
    }
    g_pool->run(n, f);
}

// layout 0 = q4_0 rows, 1 = q4r rows.
void orc_gemv_q8(const uint8_t* w, int64_t n_rows, int layout, const float* d8, const int8_t* qs8,
                 int64_t k, float* y, int threads) {
    int64_t rb = layout == 0 ? orc_row_bytes(k) : orc_q4r_row_bytes(k);
    parallel_rows(n_rows, threads, [&](int64_t r0, int64_t r1) {
        for (int64_t r = r0; r < r1; ++r)
            y[r] = layout == 0 ? orc_dot_q4_q8_avx2(w + r * rb, d8, qs8, k)
                               : orc_dot_q4r_q8_avx2(w + r * rb, d8, qs8, k);
    });
}

// ---------------------------------------------------------------------------
// GELU-tanh: ft-model/src/lib.rs:435-437
//   0.5 * g * (1.0 + (0.7978845608 * (g + 0.044715 * g * g * g)).tanh())
// evaluated left to right in f32 with no contraction.
// ---------------------------------------------------------------------------
static inline float gelu_arg(float g) {
    float c = 0.044715f * g;
    c = c * g;
    c = c * g;
    float inner = g + c;
    return 0.7978845608f * inner;
}

float orc_gelu_tanh(float g) {
    float t = tanhf(gelu_arg(g));
    float h = 0.5f * g;
    return h * (1.0f + t);
}

// act[j] = gelu_tanh(gate[j]) * up[j], gate = gu[0..inter), up = gu[inter..2inter)
// (ft-model/src/lib.rs:1625-1628), then Q8Vec::quantize (:1632).
void orc_gelu_mul_q8(const float* gu, int64_t inter, float* act, float* d, int8_t* qs) {
    std::vector<float> tmp;
    if (!act) { tmp.resize((size_t)inter); act = tmp.data(); }
    for (int64_t j = 0; j < inter; ++j) {
        float g = gu[j];
        float ge = orc_gelu_tanh(g);
        act[j] = ge * gu[j + inter];
    }
    orc_q8_quantize(act, inter, d, qs);
}

// ---------------------------------------------------------------------------
// The grouped activations and combines of Q4Gemv's batched MoE surface, as
// their CPU counterparts compute them, one f32 op at a time:
// SiLU*up (ft-bench/src/bin/decode.rs:300, the CPU twin of silu_mul_grouped,
// ft-cuda/src/q4.cu:169-179): g / (1.0 + (-g).exp()) * up, exp = libm expf;
// GELU*up per expert (gelu_mul_grouped, q4.cu:289-300, with ft-model's CPU
// GELU of lib.rs:435-437 and :1625-1628).
// gu [n][2*inter] (gate then up rows), out [n][inter].
// ---------------------------------------------------------------------------
void orc_silu_mul_grouped(const float* gu, int64_t inter, int64_t n, float* out) {
    for (int64_t e = 0; e < n; ++e)
        for (int64_t j = 0; j < inter; ++j) {
            const float g = gu[e * 2 * inter + j];
            const float t = expf(-g);
            const float den = 1.0f + t;
            const float sg = g / den;
            out[e * inter + j] = sg * gu[e * 2 * inter + inter + j];
        }
}

void orc_gelu_mul_grouped(const float* gu, int64_t inter, int64_t n, float* out) {
    for (int64_t e = 0; e < n; ++e)
        for (int64_t j = 0; j < inter; ++j)
            out[e * inter + j] = orc_gelu_tanh(gu[e * 2 * inter + j]) * gu[e * 2 * inter + inter + j];
}

// reduce_expert_weighted (q4.cu:303-314): out[i] = out[i] + s, s = sum over
// experts in order from 0.0f of (w[e] * y[e][i]) (f32 mul, then add: the
// pair combine of ft-model/src/lib.rs:1634-1646, without contraction).
void orc_reduce_expert_weighted(const float* y, const float* w, int64_t H, int64_t n, float* out) {
    for (int64_t i = 0; i < H; ++i) {
        float s = 0.0f;
        for (int64_t e = 0; e < n; ++e) {
            const float part = w[e] * y[e * H + i];
            s = s + part;
        }
        out[i] = out[i] + s;
    }
}

// reduce_weighted (q4.cu:182-192): out[i] = out[i] + a * s, s = sum over
// experts in order from 0.0f of y[e][i] (definition of this build: the
// reference's GPU expression order, with no contraction).
void orc_reduce_weighted(const float* y, float a, int64_t H, int64_t n, float* out) {
    for (int64_t i = 0; i < H; ++i) {
        float s = 0.0f;
        for (int64_t e = 0; e < n; ++e) s = s + y[e * H + i];
        const float as = a * s;
        out[i] = out[i] + as;
    }
}

// ---------------------------------------------------------------------------
// Router logits in the R-order (definition of this build; the reference has
// no CPU router and its GPU order is q4.cu:1160-1173).
//   logit[e] = sum over 8 groups g (in order, from 0.0f) of
//              G_g = sum over the C = H/128 chunks c of group g (in order, from 0.0f) of
//              P_c = fma chain over the 16 elements i of chunk c (in order, from 0.0f):
//                    P = fma(W[e][i], x[i], P)
//   chunk c covers x[16c .. 16c+16); group g covers chunks [g*C, (g+1)*C).
// Then logit[e] += bias[e] when a bias is given (the skewed-routing config).
// ---------------------------------------------------------------------------
int orc_router_logits(const float* W, const float* x, int E, int H, const float* bias, float* logits) {
    if (H % 128) return -1;
    int C = H / 128;
    for (int e = 0; e < E; ++e) {
        const float* w = W + (int64_t)e * H;
        float total = 0.0f;
        for (int g = 0; g < 8; ++g) {
            float gs = 0.0f;
            for (int c = g * C; c < (g + 1) * C; ++c) {
                float p = 0.0f;
                for (int i = 16 * c; i < 16 * c + 16; ++i) p = std::fma(w[i], x[i], p);
                gs = gs + p;
            }
            total = total + gs;
        }
        if (bias) total = total + bias[e];
        logits[e] = total;
    }
    return 0;
}

// Input RMS norm of the synthetic layer chain (definition of this build).
// The reference model feeds its router and its routed experts rmsnorm(x)
// (router: unweighted, ft-model/src/lib.rs:1398-1399; experts: :1362-1365);
// the stack here is unweighted on both. The scale of x is
//   ss    = R-order dot of x with itself (orc_router_logits with W = x)
//   inv_r = 1.0f / sqrtf(ss / (float)H + 1e-6f)   (each op rounded once, f32)
// and orc_moe_layer with input_norm applies it where the section is linear
// in its input (router logits, gate|up sums), so that the q8 quants and the
// int32 dots stay those of x itself.
// ---------------------------------------------------------------------------
float orc_rms_inv(const float* x, int H) {
    if (H % 128) return -1.0f;
    float ss = 0.0f;
    orc_router_logits(x, x, 1, H, nullptr, &ss);
    return 1.0f / std::sqrt(ss / (float)H + 1e-6f);
}

// ft-model/src/lib.rs:1487-1504: stable sort by descending logit (ties keep
// the lower expert index first), take k, w_j = exp(l_j - l_max) / sum (sum in
// top-k order from 0.0f), times per_expert_scale[e] (NULL = 1).
int orc_topk_softmax(const float* logits, int E, int k, const float* expert_scale, int32_t* ids, float* wts) {
    if (k > E || k <= 0) return -1;
    std::vector<int> order((size_t)E);
    for (int i = 0; i < E; ++i) order[(size_t)i] = i;
    // descending and stable (ties keep index order); NaN after every number,
    // where the reference's partial_cmp().unwrap() would panic
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) {
        const float x = logits[a], y = logits[b];
        if (std::isnan(x)) return false;
        if (std::isnan(y)) return true;
        return y < x;
    });
    float mx = logits[order[0]];
    std::vector<float> ex((size_t)k);
    float denom = 0.0f;
    for (int j = 0; j < k; ++j) {
        float dl = logits[order[(size_t)j]] - mx;
        ex[(size_t)j] = expf(dl);
        denom = denom + ex[(size_t)j];
    }
    for (int j = 0; j < k; ++j) {
        int e = order[(size_t)j];
        ids[j] = e;
        float w = ex[(size_t)j] / denom;
        if (expert_scale) w = w * expert_scale[e];
        wts[j] = w;
    }
    return 0;
}

// Weighted combine of one token's pairs (ft-model/src/lib.rs:1634-1646):
// part_p = y_p * w_p (f32 mul), h = ((0 + part_0) + part_1) + ... in pair
// order; then the residual of the synthetic layer chain: out = resid + h
// (resid may be NULL, then out = h).
void orc_combine(const float* y, const float* w, int n_pairs, int64_t H, const float* resid, float* out) {
    for (int64_t j = 0; j < H; ++j) {
        float h = 0.0f;
        for (int p = 0; p < n_pairs; ++p) {
            float part = y[(int64_t)p * H + j] * w[p];
            h = h + part;
        }
        out[j] = resid ? resid[j] + h : h;
    }
}

// ---------------------------------------------------------------------------
// One MoE layer for one token (the CPU pair twin, ft-model/src/lib.rs:1609-1653,
// with the router of ft-model/src/lib.rs:1487-1504 and the residual chain of
// the synthetic stack: x_out = x + sum_p w_p * down_p(q8(gelu(gate_p)*up_p))).
//   gu[e], dn[e]: expert e's gate|up rows ([2I x H]) and down rows ([H x I]) in
//   `layout` (0 q4_0, 1 q4r); NULL for experts that are not available.
// input_norm != 0: the layer runs on rmsnorm(x) in the form of orc_rms_inv:
//   logits[e] = R-order(W_r[e], x) * inv_r (+ bias[e]), and the gate|up sums
//   y_gu = gemv_q8(W_gu, q8(x)) * inv_r (f32 mul) before GELU*up; the
//   residual stays x.
// Optional stage outputs (NULL to skip): logits[E], ids[k], wts[k],
//   y_gu[k][2I] (after the scale), act[k][I], act_d[k][I/32], act_qs[k][I], y_dn[k][H].
// Returns 0, or -1 on a bad shape, -2 if a routed expert's bytes are missing.
// ---------------------------------------------------------------------------
int orc_moe_layer(const float* x, int H, int I, int E, int k,
                  const float* W_r, const float* bias, const float* expert_scale,
                  const uint8_t* const* gu, const uint8_t* const* dn, int layout,
                  int threads, int input_norm,
                  float* x_out, float* logits, int32_t* ids, float* wts,
                  float* y_gu, float* act, float* act_d, int8_t* act_qs, float* y_dn) {
    if (H % 128 || I % 32 || k <= 0 || k > E) return -1;
    std::vector<float> lg((size_t)E), w((size_t)k);
    std::vector<int32_t> id((size_t)k);
    const float inv_r = input_norm ? orc_rms_inv(x, H) : 1.0f;
    if (orc_router_logits(W_r, x, E, H, nullptr, lg.data())) return -1;
    for (int e = 0; e < E; ++e) {
        if (input_norm) lg[(size_t)e] = lg[(size_t)e] * inv_r;
        if (bias) lg[(size_t)e] = lg[(size_t)e] + bias[e];
    }
    orc_topk_softmax(lg.data(), E, k, expert_scale, id.data(), w.data());
    for (int j = 0; j < k; ++j)
        if (!gu[id[(size_t)j]] || !dn[id[(size_t)j]]) return -2;
    std::vector<float> xd((size_t)H / 32);
    std::vector<int8_t> xq((size_t)H);
    orc_q8_quantize(x, H, xd.data(), xq.data());
    std::vector<float> ygu((size_t)k * 2 * I), ydn((size_t)k * H), av((size_t)k * I), ad((size_t)k * I / 32);
    std::vector<int8_t> aq((size_t)k * I);
    // The pairs run concurrently, their rows too (ft-model's par_iter over the
    // pairs around ft-core's row-parallel gemv_q8_r): one parallel pass over
    // the k*2I gate|up rows, the GELU*up q8 per pair, one pass over the k*H
    // down rows. Every row's dot is the same call on the same inputs as in a
    // pair-by-pair loop, so the bits are those of one.
    const int64_t rb_h = layout == 0 ? orc_row_bytes(H) : orc_q4r_row_bytes(H);
    const int64_t rb_i = layout == 0 ? orc_row_bytes(I) : orc_q4r_row_bytes(I);
    auto dot = [&](const uint8_t* row, const float* d8, const int8_t* qs8, int64_t kk) {
        return layout == 0 ? orc_dot_q4_q8_avx2(row, d8, qs8, kk) : orc_dot_q4r_q8_avx2(row, d8, qs8, kk);
    };
    parallel_rows((int64_t)k * 2 * I, threads, [&](int64_t r0, int64_t r1) {
        for (int64_t r = r0; r < r1; ++r) {
            const int64_t p = r / (2 * I), rr = r % (2 * I);
            ygu[(size_t)r] = dot(gu[id[(size_t)p]] + rr * rb_h, xd.data(), xq.data(), H);
        }
    });
    for (int p = 0; p < k; ++p) {
        float* yg = ygu.data() + (size_t)p * 2 * I;
        if (input_norm)
            for (int r = 0; r < 2 * I; ++r) yg[r] = yg[r] * inv_r;
        orc_gelu_mul_q8(yg, I, av.data() + (size_t)p * I, ad.data() + (size_t)p * I / 32,
                        aq.data() + (size_t)p * I);
    }
    parallel_rows((int64_t)k * H, threads, [&](int64_t r0, int64_t r1) {
        for (int64_t r = r0; r < r1; ++r) {
            const int64_t p = r / H, rr = r % H;
            ydn[(size_t)r] = dot(dn[id[(size_t)p]] + rr * rb_i, ad.data() + (size_t)p * I / 32,
                                 aq.data() + (size_t)p * I, I);
        }
    });
    orc_combine(ydn.data(), w.data(), k, H, x, x_out);
    if (logits) std::memcpy(logits, lg.data(), sizeof(float) * (size_t)E);
    if (ids) std::memcpy(ids, id.data(), sizeof(int32_t) * (size_t)k);
    if (wts) std::memcpy(wts, w.data(), sizeof(float) * (size_t)k);
    if (y_gu) std::memcpy(y_gu, ygu.data(), sizeof(float) * ygu.size());
    if (act) std::memcpy(act, av.data(), sizeof(float) * av.size());
    if (act_d) std::memcpy(act_d, ad.data(), sizeof(float) * ad.size());
    if (act_qs) std::memcpy(act_qs, aq.data(), aq.size());
    if (y_dn) std::memcpy(y_dn, ydn.data(), sizeof(float) * ydn.size());
    return 0;
}

// ---------------------------------------------------------------------------
// Seeded synthetic inputs (definition of this build; the GPU weight generator
// in the HIP library computes the same bits).
//   key(seed, cfg, layer, expert, tensor) chains splitmix64's finaliser;
//   value i of a tensor: h = mix64(key + (i+1)*0x9E3779B97F4A7C15); the four
//   16-bit fields of h are summed (Irwin-Hall, n=4), centred, and scaled:
//   v = float(sum - 131070) * scale, scale = sigma*sqrt(3)/65536 rounded to f32.
//   (Var of the centred sum is 65536^2/3, so v has standard deviation sigma.)
// ---------------------------------------------------------------------------
static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

uint64_t orc_tensor_key(uint64_t seed, uint32_t cfg, uint32_t layer, uint32_t expert, uint32_t tensor) {
    uint64_t h = mix64(seed + 0x9E3779B97F4A7C15ULL);
    h = mix64(h ^ ((uint64_t)cfg << 32 | tensor));
    h = mix64(h ^ ((uint64_t)layer << 32 | expert));
    return h;
}

static inline float gen_value(uint64_t key, uint64_t i, float scale) {
    uint64_t h = mix64(key + (i + 1) * 0x9E3779B97F4A7C15ULL);
    int32_t s = (int32_t)(h & 0xFFFF) + (int32_t)((h >> 16) & 0xFFFF) + (int32_t)((h >> 32) & 0xFFFF) +
                (int32_t)(h >> 48);
    return (float)(s - 131070) * scale;
}

float orc_gen_scale(double sigma) { return (float)(sigma * std::sqrt(3.0) / 65536.0); }

void orc_gen_values(uint64_t key, int64_t start, int64_t n, float scale, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = gen_value(key, (uint64_t)(start + i), scale);
}

// q4_0 rows [row0, row0+n_rows) of a seeded [*, k] matrix: element (r, c) is
// value r*k + c of the tensor, quantized by orc_quantize_row.
void orc_gen_q4_rows(uint64_t key, int64_t row0, int64_t n_rows, int64_t k, float scale, uint8_t* out, int threads) {
    int64_t rb = orc_row_bytes(k);
    parallel_rows(n_rows, threads, [&](int64_t r0, int64_t r1) {
        std::vector<float> buf((size_t)k);
        for (int64_t r = r0; r < r1; ++r) {
            orc_gen_values(key, (row0 + r) * k, k, scale, buf.data());
            orc_quantize_row(buf.data(), k, out + r * rb);
        }
    });
}

}  // extern "C"
