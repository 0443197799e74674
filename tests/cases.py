"""Input cases shared by the CPU oracle tests and the GPU parity tests."""
import numpy as np


def nonfinite_q8_blocks():
    """Blocks whose q8 quants are fixed by Rust's f32 semantics
    (ft-core/src/q4_0.rs:67-73): `m.max(v.abs())` skips NaN, a block holding
    inf gets s = inf and inv = 0, `(v*inv).round().clamp(-127.0, 127.0) as i8`
    maps a NaN product to 0 (a saturating float->int cast), and a subnormal
    s = amax/127 has 1/s = inf, so its zeros give 0*inf = NaN -> 0.
    Returns (x [n*32] f32, expected d [n], expected q [n*32])."""
    inf, nan = np.float32(np.inf), np.float32(np.nan)
    tiny = np.float32(127.0 * 2.0 ** -140)          # subnormal amax; amax/127 = 2^-140, 1/that = inf
    blocks, ds, qs = [], [], []

    def add(vals, d, q):
        v = np.zeros(32, np.float32); v[:len(vals)] = vals
        e = np.zeros(32, np.int8); e[:len(q)] = q
        blocks.append(v); ds.append(np.float32(d)); qs.append(e)

    add([inf, 1.0, -2.0, nan, 5.0], inf, [0, 0, 0, 0, 0])           # +inf: every product NaN or 0
    add([-3.0, -inf, 0.0], inf, [0, 0, 0])                          # -inf
    add([nan, 127.0, -63.5, 0.49, nan], 1.0, [0, 127, -64, 0, 0])   # NaN skipped by the amax fold
    add([nan] * 32, 0.0, [])                                        # all NaN: amax = 0, zero block
    add([tiny, 0.0, -tiny / 2, 0.0], 2.0 ** -140, [127, 0, -127, 0])  # inv = inf: 0*inf = NaN -> 0
    return np.concatenate(blocks), np.array(ds, np.float32), np.concatenate(qs)


def q4r_to_q4_0(raw, n_rows, k):
    """q4r rows ([nb f16 scales, zero-padded to 16 B][nb x 16 B qs],
    ft-core/src/q4_0.rs:234-258) back to q4_0 rows (18 B blocks), for the
    oracle's integer block dots, which read q4_0."""
    nb = k // 32
    so = (nb * 2 + 15) // 16 * 16
    raw = np.asarray(raw, np.uint8).reshape(n_rows, so + nb * 16)
    q40 = np.zeros((n_rows, nb, 18), np.uint8)
    q40[:, :, :2] = raw[:, :2 * nb].reshape(n_rows, nb, 2)
    q40[:, :, 2:] = raw[:, so:].reshape(n_rows, nb, 16)
    return q40.reshape(n_rows, nb * 18)
