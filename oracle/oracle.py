"""ctypes binding of the CPU oracle (oracle/ft_oracle.cpp).

TEST INFRASTRUCTURE ONLY. This module is the checker used by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg. The product library
(freetoken-rs_amd/) never imports it, and nothing here is a fallback for the
GPU path.

Each wrapper names the reference function it restates (paths relative to the
freeToken-rs repository root); the C++ source carries the same citations.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None

QK = 32
BLOCK_BYTES = 18

# Tensor ids of the seeded synthetic inputs (shared with the GPU generator).
T_HIDDEN, T_GU, T_DN, T_ROUTER = 1, 2, 3, 4
SEED = 0xF7EE2026


def build():
    """Compile the oracle with its Makefile (g++, a few seconds)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(L):
    P = ctypes.c_void_p
    i64, i32, u32, u64, f32, f64 = (ctypes.c_int64, ctypes.c_int, ctypes.c_uint32,
                                     ctypes.c_uint64, ctypes.c_float, ctypes.c_double)
    sig = {
        "orc_row_bytes": (i64, [i64]),
        "orc_quantize_row": (None, [P, i64, P]),
        "orc_dequantize_row": (None, [P, i64, P]),
        "orc_q8_quantize": (None, [P, i64, P, P]),
        "orc_dot_q4_q8_scalar": (f32, [P, P, P, i64]),
        "orc_dot_q4_q8_avx2": (f32, [P, P, P, i64]),
        "orc_block_dots": (None, [P, P, i64, P]),
        "orc_q4r_scales_bytes": (i64, [i64]),
        "orc_q4r_row_bytes": (i64, [i64]),
        "orc_repack_row_q4r": (None, [P, P, i64]),
        "orc_dot_q4r_q8_scalar": (f32, [P, P, P, i64]),
        "orc_dot_q4r_q8_avx2": (f32, [P, P, P, i64]),
        "orc_gemv_q8": (None, [P, i64, i32, P, P, i64, P, i32]),
        "orc_gelu_tanh": (f32, [f32]),
        "orc_gelu_mul_q8": (None, [P, i64, P, P, P]),
        "orc_router_logits": (i32, [P, P, i32, i32, P, P]),
        "orc_topk_softmax": (i32, [P, i32, i32, P, P, P]),
        "orc_combine": (None, [P, P, i32, i64, P, P]),
        "orc_silu_mul_grouped": (None, [P, i64, i64, P]),
        "orc_gelu_mul_grouped": (None, [P, i64, i64, P]),
        "orc_reduce_expert_weighted": (None, [P, P, i64, i64, P]),
        "orc_reduce_weighted": (None, [P, f32, i64, i64, P]),
        "orc_moe_layer": (i32, [P, i32, i32, i32, i32, P, P, P, P, P, i32, i32, i32,
                                P, P, P, P, P, P, P, P, P]),
        "orc_rms_inv": (f32, [P, i32]),
        "orc_tensor_key": (u64, [u64, u32, u32, u32, u32]),
        "orc_gen_scale": (f32, [f64]),
        "orc_gen_values": (None, [u64, i64, i64, f32, P]),
        "orc_gen_q4_rows": (None, [u64, i64, i64, i64, f32, P, i32]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- q4_0 format: ft-core/src/q4_0.rs ----

def row_bytes(k):
    """ft-core/src/q4_0.rs:13-16"""
    assert k % QK == 0
    return k // QK * BLOCK_BYTES


def quantize_row(x):
    """ft-core/src/q4_0.rs:20-40. x: f32 [k] or [n, k] -> uint8 rows."""
    x = _f32(x)
    k = x.shape[-1]
    rows = x.reshape(-1, k)
    out = np.zeros((rows.shape[0], row_bytes(k)), np.uint8)
    for r in range(rows.shape[0]):
        lib().orc_quantize_row(_p(rows[r]), k, _p(out[r]))
    return out.reshape(x.shape[:-1] + (row_bytes(k),))


def dequantize_row(q, k):
    """ft-core/src/q4_0.rs:43-52."""
    q = np.ascontiguousarray(q, dtype=np.uint8)
    rows = q.reshape(-1, row_bytes(k))
    out = np.zeros((rows.shape[0], k), np.float32)
    for r in range(rows.shape[0]):
        lib().orc_dequantize_row(_p(rows[r]), k, _p(out[r]))
    return out.reshape(q.shape[:-1] + (k,))


def q8_quantize(x):
    """ft-core/src/q4_0.rs:62-78 (Q8Vec::quantize) -> (d f32 [k/32], qs i8 [k])."""
    x = _f32(x).ravel()
    k = x.size
    d = np.zeros(k // QK, np.float32)
    qs = np.zeros(k, np.int8)
    lib().orc_q8_quantize(_p(x), k, _p(d), _p(qs))
    return d, qs


def dot_avx2(row, d8, qs8, k):
    """ft-core/src/q4_0.rs:123-160."""
    return lib().orc_dot_q4_q8_avx2(_p(row), _p(d8), _p(qs8), k)


def dot_scalar(row, d8, qs8, k):
    """ft-core/src/q4_0.rs:105-118."""
    return lib().orc_dot_q4_q8_scalar(_p(row), _p(d8), _p(qs8), k)


def block_dots(w, qs8, k):
    """Per-(row, block) int32 dots sum (q4-8)*q8 from the AVX2 integer lanes."""
    w = np.ascontiguousarray(w, np.uint8).reshape(-1, row_bytes(k))
    out = np.zeros((w.shape[0], k // QK), np.int32)
    for r in range(w.shape[0]):
        lib().orc_block_dots(_p(w[r]), _p(qs8), k, _p(out[r]))
    return out


def q4r_scales_bytes(k):
    """ft-core/src/q4_0.rs:238-241"""
    return (k // QK * 2 + 15) // 16 * 16


def q4r_row_bytes(k):
    """ft-core/src/q4_0.rs:243-245"""
    return q4r_scales_bytes(k) + k // QK * 16


def repack_q4r(w, k):
    """ft-core/src/q4_0.rs:248-258, over a [n, row_bytes] array."""
    w = np.ascontiguousarray(w, np.uint8).reshape(-1, row_bytes(k))
    out = np.zeros((w.shape[0], q4r_row_bytes(k)), np.uint8)
    for r in range(w.shape[0]):
        lib().orc_repack_row_q4r(_p(w[r]), _p(out[r]), k)
    return out


def dot_q4r_avx2(row, d8, qs8, k):
    """ft-core/src/q4_0.rs:294-323."""
    return lib().orc_dot_q4r_q8_avx2(_p(row), _p(d8), _p(qs8), k)


def dot_q4r_scalar(row, d8, qs8, k):
    """ft-core/src/q4_0.rs:276-292."""
    return lib().orc_dot_q4r_q8_scalar(_p(row), _p(d8), _p(qs8), k)


def gemv_q8(w, n_rows, d8, qs8, k, layout=0, threads=1):
    """ft-core/src/q4_0.rs:90-103 (layout 0) / :261-274 (layout 1, q4r)."""
    w = np.ascontiguousarray(w, np.uint8)
    y = np.zeros(n_rows, np.float32)
    lib().orc_gemv_q8(_p(w), n_rows, layout, _p(d8), _p(qs8), k, _p(y), threads)
    return y


def gemv(w, x, n_rows, layout=0, threads=1):
    """ft-core/src/q4_0.rs:84-86: quantize x, then gemv_q8."""
    d, qs = q8_quantize(x)
    return gemv_q8(w, n_rows, d, qs, len(qs), layout, threads)


# ---- expert activation, router, combine ----

def gelu_mul_q8(gu, inter):
    """ft-model/src/lib.rs:435-437 and :1625-1632 -> (act f32 [I], d [I/32], qs [I]);
    tanh is the host libm's tanhf, as Rust's f32::tanh."""
    gu = _f32(gu).ravel()
    act = np.zeros(inter, np.float32)
    d = np.zeros(inter // QK, np.float32)
    qs = np.zeros(inter, np.int8)
    lib().orc_gelu_mul_q8(_p(gu), inter, _p(act), _p(d), _p(qs))
    return act, d, qs


def silu_mul_grouped(gu, inter):
    """ft-bench/src/bin/decode.rs:300 per expert: gu [n, 2*inter] -> [n, inter],
    g / (1 + expf(-g)) * up in f32 (exp is the host libm's expf, as Rust's f32::exp)."""
    gu = _f32(gu).reshape(-1, 2 * inter)
    out = np.zeros((gu.shape[0], inter), np.float32)
    lib().orc_silu_mul_grouped(_p(gu), inter, gu.shape[0], _p(out))
    return out


def gelu_mul_grouped(gu, inter):
    """ft-model/src/lib.rs:435-437, :1625-1628 per expert: gu [n, 2*inter] -> [n, inter]."""
    gu = _f32(gu).reshape(-1, 2 * inter)
    out = np.zeros((gu.shape[0], inter), np.float32)
    lib().orc_gelu_mul_grouped(_p(gu), inter, gu.shape[0], _p(out))
    return out


def reduce_expert_weighted(y, w, out):
    """out + sum_e w[e] * y[e] (experts in order; q4.cu:303-314, no contraction)."""
    y = _f32(y)
    n, H = y.shape
    out = _f32(out).ravel().copy()
    lib().orc_reduce_expert_weighted(_p(y), _p(_f32(w).ravel()), H, n, _p(out))
    return out


def reduce_weighted(y, a, out):
    """out + a * (sum_e y[e]) (experts in order; q4.cu:182-192, no contraction)."""
    y = _f32(y)
    n, H = y.shape
    out = _f32(out).ravel().copy()
    lib().orc_reduce_weighted(_p(y), np.float32(a), H, n, _p(out))
    return out


def router_logits(W, x, bias=None):
    """R-order router logits (definition of this build). W [E, H], x [H]."""
    W = _f32(W)
    x = _f32(x).ravel()
    E, H = W.shape
    out = np.zeros(E, np.float32)
    b = None if bias is None else _f32(bias)
    rc = lib().orc_router_logits(_p(W), _p(x), E, H, _p(b), _p(out))
    if rc:
        raise ValueError("H must be a multiple of 128")
    return out


def topk_softmax(logits, k, expert_scale=None):
    """ft-model/src/lib.rs:1487-1504 -> (ids i32 [k], wts f32 [k]); exp is the
    host libm's expf, as Rust's f32::exp."""
    lg = _f32(logits).ravel()
    ids = np.zeros(k, np.int32)
    wts = np.zeros(k, np.float32)
    es = None if expert_scale is None else _f32(expert_scale)
    rc = lib().orc_topk_softmax(_p(lg), lg.size, k, _p(es), _p(ids), _p(wts))
    if rc:
        raise ValueError("bad k")
    return ids, wts


def combine(y, w, resid=None):
    """ft-model/src/lib.rs:1634-1646 plus the synthetic residual: resid + sum_p w_p y_p."""
    y = _f32(y)
    w = _f32(w).ravel()
    n, H = y.shape
    out = np.zeros(H, np.float32)
    r = None if resid is None else _f32(resid).ravel()
    lib().orc_combine(_p(y), _p(w), n, H, _p(r), _p(out))
    return out


def rms_inv(x):
    """Scale of the stack's input RMS norm: 1/sqrt(R-order(x.x)/H + 1e-6) in f32
    (definition of this build; the reference model's router and experts take
    rmsnorm(x), ft-model/src/lib.rs:1362-1365, :1398-1399)."""
    x = _f32(x).ravel()
    return np.float32(lib().orc_rms_inv(_p(x), x.size))


def moe_layer(x, W_r, gu_banks, dn_banks, H, I, k, bias=None, expert_scale=None,
              layout=0, threads=1, input_norm=False):
    """One MoE layer for one token (ft-model/src/lib.rs:1487-1504, :1609-1653).
    input_norm: run on rmsnorm(x) in the form of rms_inv (logits and gate|up
    sums scaled by it; q8 quants and int32 dots those of x).

    gu_banks / dn_banks: dict expert -> uint8 array (that expert's gate|up rows /
    down rows in `layout`); experts the router may pick must be present.
    Returns a dict with x_out and every stage output.
    """
    x = _f32(x).ravel()
    W_r = _f32(W_r)
    E = W_r.shape[0]
    gu_ptrs = (ctypes.c_void_p * E)()
    dn_ptrs = (ctypes.c_void_p * E)()
    keep = []
    for e, a in gu_banks.items():
        a = np.ascontiguousarray(a, np.uint8)
        keep.append(a)
        gu_ptrs[e] = a.ctypes.data
    for e, a in dn_banks.items():
        a = np.ascontiguousarray(a, np.uint8)
        keep.append(a)
        dn_ptrs[e] = a.ctypes.data
    r = dict(
        x_out=np.zeros(H, np.float32), logits=np.zeros(E, np.float32),
        ids=np.zeros(k, np.int32), wts=np.zeros(k, np.float32),
        y_gu=np.zeros((k, 2 * I), np.float32), act=np.zeros((k, I), np.float32),
        act_d=np.zeros((k, I // QK), np.float32), act_qs=np.zeros((k, I), np.int8),
        y_dn=np.zeros((k, H), np.float32))
    b = None if bias is None else _f32(bias)
    es = None if expert_scale is None else _f32(expert_scale)
    rc = lib().orc_moe_layer(
        _p(x), H, I, E, k, _p(W_r), _p(b), _p(es),
        ctypes.cast(gu_ptrs, ctypes.c_void_p), ctypes.cast(dn_ptrs, ctypes.c_void_p),
        layout, threads, int(bool(input_norm)),
        _p(r["x_out"]), _p(r["logits"]), _p(r["ids"]), _p(r["wts"]), _p(r["y_gu"]),
        _p(r["act"]), _p(r["act_d"]), _p(r["act_qs"]), _p(r["y_dn"]))
    if rc == -2:
        raise KeyError("a routed expert's bank is missing")
    if rc:
        raise ValueError("bad shape")
    return r


# ---- seeded synthetic inputs ----

def tensor_key(cfg, layer, expert, tensor, seed=SEED):
    return lib().orc_tensor_key(seed, cfg, layer, expert, tensor)


def gen_scale(sigma):
    return lib().orc_gen_scale(sigma)


def gen_values(key, start, n, sigma):
    out = np.zeros(n, np.float32)
    lib().orc_gen_values(key, start, n, gen_scale(sigma), _p(out))
    return out


def gen_q4_rows(key, row0, n_rows, k, sigma, threads=1):
    out = np.zeros((n_rows, row_bytes(k)), np.uint8)
    lib().orc_gen_q4_rows(key, row0, n_rows, k, gen_scale(sigma), _p(out), threads)
    return out
