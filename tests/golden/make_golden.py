#!/usr/bin/env python3
"""Writes tests/golden/moe_tiny.npz: small input/expected-output vectors for
every stage of the MoE expert-FFN decode path, computed by the CPU oracle
(oracle/ft_oracle.cpp, a restatement of ft-core/src/q4_0.rs and
ft-model/src/lib.rs:1487-1504, :1609-1653).

The reference ships no fixture files (its tests build inline xorshift32
data), so these vectors are the oracle's own outputs, frozen: the CPU suite
checks that the oracle still reproduces them bit-for-bit and the GPU suite
checks the HIP path against them. Inputs are stored whole, so a test needs
nothing but this file.

Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle as orc  # noqa: E402

CFG = 100  # generator config id reserved for the fixtures


def q4_inputs():
    """Four 64-value rows: seeded Irwin-Hall(4) of sd 1, a zero block, a single spike, a
    negative-extreme block and exact-.5 values after scaling."""
    x = orc.gen_values(orc.tensor_key(CFG, 0, 0, orc.T_HIDDEN), 0, 4 * 64, 1.0).reshape(4, 64)
    x[1, :32] = 0.0
    x[1, 32:] = 0.0
    x[1, 40] = 3.0
    x[2, :32] = np.linspace(-8.0, 7.0, 32, dtype=np.float32)
    x[3, 32:] = np.float32(-1.0) * np.arange(32, dtype=np.float32) / 4
    return x.astype(np.float32)


def main():
    orc.build()
    out = {}

    # a1: quantize_row
    x = q4_inputs()
    out["q4_x"] = x
    out["q4_bytes"] = orc.quantize_row(x)

    # a2: Q8Vec::quantize on a 2816-value hidden row with a zero block and exact ties
    h = orc.gen_values(orc.tensor_key(CFG, 0, 1, orc.T_HIDDEN), 0, 2816, 1.0)
    h[:32] = 0.0
    h[32:64] = np.array([127.0, 2.5, -2.5, 0.5, -0.5, 126.5] + [1.5] * 26, np.float32)
    out["q8_x"] = h
    d8, qs8 = orc.q8_quantize(h)
    out["q8_d"], out["q8_qs"] = d8, qs8

    # a3/a4/a5: per-block int32 dots and AVX2-order dot of 8 q4r rows (K 2816)
    w = orc.gen_q4_rows(orc.tensor_key(CFG, 0, 2, orc.T_GU), 0, 8, 2816, 0.02)
    wr = orc.repack_q4r(w, 2816)
    out["dot_w_q4r"] = wr
    out["dot_blocks"] = orc.block_dots(w, qs8, 2816)
    out["dot_y"] = orc.gemv_q8(wr, 8, d8, qs8, 2816, layout=1)

    # a6: GELU*up -> q8 (libm tanhf, as ft-core) from a 2 x 704 gate|up row
    gu = orc.gen_values(orc.tensor_key(CFG, 0, 3, orc.T_HIDDEN), 0, 2 * 704, 2.0)
    out["gelu_gu"] = gu
    act, ad, aqs = orc.gelu_mul_q8(gu, 704)
    out["gelu_act"], out["gelu_d"], out["gelu_qs"] = act, ad, aqs

    # a7-a11: one whole layer (H 128, I 64, E 8, top-2), q4r banks [E][gate|up | down]
    H, I, E, K = 128, 64, 8, 2
    xl = orc.gen_values(orc.tensor_key(CFG, 1, 0, orc.T_HIDDEN), 0, H, 1.0)
    Wr = orc.gen_values(orc.tensor_key(CFG, 1, 0, orc.T_ROUTER), 0, E * H, 0.02).reshape(E, H)
    gu_b, dn_b, bank = {}, {}, []
    for e in range(E):
        g = orc.repack_q4r(orc.gen_q4_rows(orc.tensor_key(CFG, 1, e, orc.T_GU), 0, 2 * I, H, 0.02), H)
        dn = orc.repack_q4r(orc.gen_q4_rows(orc.tensor_key(CFG, 1, e, orc.T_DN), 0, H, I, 0.02), I)
        gu_b[e], dn_b[e] = g.ravel(), dn.ravel()
        bank.append(np.concatenate([g.ravel(), dn.ravel()]))
    out["layer_shape"] = np.array([H, I, E, K], np.int32)
    out["layer_x"], out["layer_Wr"], out["layer_bank"] = xl, Wr, np.stack(bank)
    out["layer_bias"] = np.array([0.0, -1.5, 0.75, 0.0, 2.0, -0.25, 0.0, 1.0], np.float32)
    for tag, bias in (("layer_", None), ("layerb_", out["layer_bias"])):
        r = orc.moe_layer(xl, Wr, gu_b, dn_b, H, I, K, bias=bias, layout=1)
        for key in ("logits", "ids", "wts", "act_d", "act_qs", "x_out"):
            out[tag + key] = r[key]

    path = os.path.join(HERE, "moe_tiny.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} B, {len(out)} arrays)")


if __name__ == "__main__":
    main()
