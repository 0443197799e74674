"""The GGUF reader (ft_gguf_*, the counterpart of ft-gguf's Gguf,
ft-gguf/src/lib.rs:141-206) on files written here byte by byte from the GGUF
v3 layout: the reference's own hand-crafted test file
(parses_handcrafted_file, lib.rs:215-256), a Gemma-like expert-section file,
and malformed files for every error path. Host only: no GPU."""
import struct

import numpy as np
import pytest

import ft_hip

T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 = range(13)
GG_F32, GG_F16, GG_Q4_0 = 0, 1, 2


def _s(x):
    b = x.encode() if isinstance(x, str) else x
    return struct.pack("<Q", len(b)) + b


def _val(ty, v):
    if ty == T_ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_val(et, x) for x in items)
    if ty == T_STR:
        return _s(v)
    fmt = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i", T_F32: "<f",
           T_BOOL: "<?", T_U64: "<Q", T_I64: "<q", T_F64: "<d"}[ty]
    return struct.pack(fmt, v)


def gguf_bytes(kvs, tensors, version=3, align=32):
    """kvs: [(key, type, value)]; tensors: [(name, dims, ggml_type, data bytes)]
    laid out in order, each at an `align`-aligned offset of the data section."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs))
    for k, ty, v in kvs:
        head += _s(k) + struct.pack("<I", ty) + _val(ty, v)
    off, offs = 0, []
    for name, dims, ty, data in tensors:
        offs.append(off)
        off += (len(data) + align - 1) // align * align
    for (name, dims, ty, data), o in zip(tensors, offs):
        head += _s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", ty, o)
    head += b"\0" * (-len(head) % align)
    data_start = len(head)
    body = b""
    for (name, dims, ty, data), o in zip(tensors, offs):
        body += b"\0" * (o - len(body)) + data
    return head + body, data_start


def write(tmp_path, name, blob):
    p = tmp_path / name
    p.write_bytes(blob)
    return str(p)


def test_reference_handcrafted_file(tmp_path):
    """The file of ft-gguf's parses_handcrafted_file (lib.rs:215-256): one KV
    (general.alignment = u32 32), one q4_0 tensor "t" [64, 2] of 72 bytes of
    0xAB; the same assertions."""
    buf = b"GGUF" + struct.pack("<I", 3) + struct.pack("<Q", 1) + struct.pack("<Q", 1)
    key = b"general.alignment"
    buf += struct.pack("<Q", len(key)) + key + struct.pack("<I", 4) + struct.pack("<I", 32)
    buf += struct.pack("<Q", 1) + b"t" + struct.pack("<I", 2) + struct.pack("<Q", 64) + struct.pack("<Q", 2)
    buf += struct.pack("<I", 2) + struct.pack("<Q", 0)
    buf += b"\0" * (-len(buf) % 32)
    data_start = len(buf)
    buf += b"\xAB" * 72
    g = ft_hip.Gguf(write(tmp_path, "tiny.gguf", buf))
    assert g.data_start == data_start
    t = g.tensor("t")
    assert t.dims == [64, 2]
    assert t.nbytes == 72
    assert np.all(g.tensor_data("t") == 0xAB)
    assert g.meta["general.alignment"] == 32
    assert g.version == 3


def q4_0_rows(rng, n_rows, k):
    """Random q4_0 rows: f16 scales of moderate size, random nibbles."""
    nb = k // 32
    out = np.zeros((n_rows, nb, 18), np.uint8)
    d = (rng.uniform(0.001, 0.01, (n_rows, nb)) * rng.choice([-1, 1], (n_rows, nb))).astype(np.float16)
    out[:, :, :2] = d.view(np.uint8).reshape(n_rows, nb, 2)
    out[:, :, 2:] = rng.integers(0, 256, (n_rows, nb, 16), dtype=np.uint8)
    return out.reshape(n_rows, nb * 18)


def expert_file(tmp_path, H=256, I=64, E=8, L=2, seed=0, extra_kv=(), align=32):
    rng = np.random.default_rng(seed)
    kvs = [("general.architecture", T_STR, "gemma4"),
           ("gemma4.block_count", T_U32, L),
           ("gemma4.expert_count", T_U32, E),
           ("gemma4.expert_used_count", T_U32, 2),
           ("gemma4.expert_feed_forward_length", T_U64, I),
           ("gemma4.attention.layer_norm_rms_epsilon", T_F32, 1e-6),
           ("gemma4.attention.head_count_kv", T_ARR, (T_U32, [8, 8, 2])),
           ("gemma4.attention.sliding_window_pattern", T_ARR, (T_BOOL, [True, False, True])),
           ("gemma4.some_i32", T_I32, -5),
           ("gemma4.some_f64", T_F64, 0.25),
           ("tokenizer.ggml.tokens", T_ARR, (T_STR, ["<pad>", "a", "bc", "déf"])),
           ("general.alignment", T_U32, align)] + list(extra_kv)
    tensors, raw = [], {}
    for l in range(L):
        gu = np.concatenate([q4_0_rows(rng, 2 * I, H) for _ in range(E)])
        dn = np.concatenate([q4_0_rows(rng, H, I) for _ in range(E)])
        wr = rng.standard_normal((E, H)).astype(np.float32) * 0.02
        sc = rng.uniform(0.5, 1.5, H).astype(np.float32)
        es = rng.uniform(0.5, 2.0, E).astype(np.float16)
        raw[l] = (gu, dn, wr, sc, es)
        tensors += [(f"blk.{l}.ffn_gate_up_exps.weight", [H, 2 * I, E], GG_Q4_0, gu.tobytes()),
                    (f"blk.{l}.ffn_down_exps.weight", [I, H, E], GG_Q4_0, dn.tobytes()),
                    (f"blk.{l}.ffn_gate_inp.weight", [H, E], GG_F32, wr.tobytes()),
                    (f"blk.{l}.ffn_gate_inp.scale", [H], GG_F32, sc.tobytes()),
                    (f"blk.{l}.ffn_down_exps.scale", [E], GG_F16, es.tobytes())]
    blob, ds = gguf_bytes(kvs, tensors, align=align)
    return write(tmp_path, f"experts_{seed}_{align}.gguf", blob), raw, ds


@pytest.mark.parametrize("align", [32, 64])
def test_expert_file_metadata_and_tensors(tmp_path, align):
    path, raw, ds = expert_file(tmp_path, align=align)
    g = ft_hip.Gguf(path)
    assert g.data_start == ds
    m = g.meta
    assert m["general.architecture"] == "gemma4"
    assert m["gemma4.block_count"] == 2 and m["gemma4.expert_count"] == 8
    assert m["gemma4.expert_feed_forward_length"] == 64
    assert m["gemma4.attention.layer_norm_rms_epsilon"] == pytest.approx(1e-6)
    assert m["gemma4.attention.head_count_kv"] == [8, 8, 2]
    assert m["gemma4.attention.sliding_window_pattern"] == [True, False, True]
    assert m["tokenizer.ggml.tokens"] == ["<pad>", "a", "bc", "déf"]
    assert m["gemma4.some_i32"] == ("negative", T_I32)  # as_u64 refuses negative ints
    t = g.tensor("blk.1.ffn_gate_up_exps.weight")
    assert t.dims == [256, 128, 8] and t.ggml_type == GG_Q4_0 and t.nbytes == 8 * 128 * 8 * 18
    assert np.array_equal(g.tensor_data("blk.1.ffn_gate_up_exps.weight"), raw[1][0].ravel())
    assert np.array_equal(g.tensor_data("blk.0.ffn_down_exps.weight"), raw[0][1].ravel())
    assert np.array_equal(g.to_f32("blk.0.ffn_gate_inp.weight"), raw[0][2].ravel())
    assert np.array_equal(g.to_f32("blk.1.ffn_down_exps.scale"), raw[1][4].astype(np.float32))
    g.close()


def test_router_fold(tmp_path):
    """ft-model's router fold (lib.rs:506-514): W[e][j] * (scale[j] * H^-1/2)
    in f32, H^-1/2 from powf."""
    path, raw, _ = expert_file(tmp_path)
    g = ft_hip.Gguf(path)
    H, E = 256, 8
    wr, sc = raw[1][2], raw[1][3]
    root = np.float32(np.float32(H) ** np.float32(-0.5))
    ref = (wr * (sc * root).astype(np.float32)[None, :]).astype(np.float32)
    assert np.array_equal(g.router_f32(1, H, E), ref)


def test_q4_0_to_f32_matches_oracle(tmp_path, orc):
    """to_f32 of a q4_0 tensor is ft-core's dequantize_row (q4_0.rs:43-52)."""
    rng = np.random.default_rng(3)
    rows = q4_0_rows(rng, 4, 128)
    blob, _ = gguf_bytes([], [("w", [128, 4], GG_Q4_0, rows.tobytes())])
    g = ft_hip.Gguf(write(tmp_path, "q4.gguf", blob))
    ref = np.concatenate([orc.dequantize_row(rows[r], 128) for r in range(4)])
    assert np.array_equal(g.to_f32("w"), ref)


def test_f16_to_f32_all_values(tmp_path):
    """Every f16 bit pattern widens exactly (numpy's f16 -> f32 is exact)."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    blob, _ = gguf_bytes([], [("h", [65536], GG_F16, h.tobytes())])
    g = ft_hip.Gguf(write(tmp_path, "f16.gguf", blob))
    got = g.to_f32("h")
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    # NaN payloads are kept (quiet bit included)
    assert np.array_equal(got[nan].view(np.uint32) & 0x7FFFFF, (h[nan].astype(np.uint32) & 0x3FF) << 13)


def _err(path):
    with pytest.raises(ft_hip.FtHipError) as ei:
        ft_hip.Gguf(path)
    return ei.value.code


def test_errors(tmp_path):
    good, _ = gguf_bytes([("a", T_U32, 1)], [("t", [32], GG_Q4_0, b"\0" * 18)])
    assert _err(str(tmp_path / "missing.gguf")) == ft_hip.E_IO
    assert _err(write(tmp_path, "magic.gguf", b"GGUX" + good[4:])) == ft_hip.E_FORMAT
    v1, _ = gguf_bytes([("a", T_U32, 1)], [], version=1)
    assert _err(write(tmp_path, "v1.gguf", v1)) == ft_hip.E_FORMAT
    v2, _ = gguf_bytes([("a", T_U32, 1)], [], version=2)
    assert ft_hip.Gguf(write(tmp_path, "v2.gguf", v2)).version == 2
    for cut in (3, 10, 30, 45, len(good) - 80):
        assert _err(write(tmp_path, f"cut{cut}.gguf", good[:cut])) == ft_hip.E_FORMAT, cut
    bad_type = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + _s("k") + struct.pack("<I", 13) + b"\0" * 8
    assert _err(write(tmp_path, "vt.gguf", bad_type)) == ft_hip.E_FORMAT
    bad_ggml, _ = gguf_bytes([], [("t", [32], 99, b"\0" * 32)])
    assert _err(write(tmp_path, "gt.gguf", bad_ggml)) == ft_hip.E_FORMAT
    ragged, _ = gguf_bytes([], [("t", [33], GG_Q4_0, b"\0" * 18)])
    assert _err(write(tmp_path, "rag.gguf", ragged)) == ft_hip.E_FORMAT
    # byte sizes that would wrap 64 bits: an f32 tensor of 2^62 elements (the
    # element count fits, elements x 4 bytes does not), and an alignment so
    # large that rounding the data start up wraps
    huge, _ = gguf_bytes([], [("t", [1 << 31, 1 << 31], 0, b"\0" * 4)])
    assert _err(write(tmp_path, "huge.gguf", huge)) == ft_hip.E_FORMAT
    big_align, _ = gguf_bytes([("general.alignment", T_U64, (1 << 64) - 8)], [])
    assert _err(write(tmp_path, "align.gguf", big_align)) == ft_hip.E_FORMAT
    # a tensor whose data runs past the end of the file: open succeeds (as the
    # reference's), tensor_data fails
    short, _ = gguf_bytes([], [("t", [64], GG_Q4_0, b"\0" * 36)])
    g = ft_hip.Gguf(write(tmp_path, "short.gguf", short[:-10]))
    with pytest.raises(ft_hip.FtHipError) as ei:
        g.tensor_data("t")
    assert ei.value.code == ft_hip.E_FORMAT
    with pytest.raises(ft_hip.FtHipError) as ei:
        g.tensor_data("nope")
    assert ei.value.code == ft_hip.E_NOT_FOUND
    with pytest.raises(ft_hip.FtHipError):
        g.router_f32(0, 64, 1)  # no router tensors in this file
