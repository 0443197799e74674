"""The ft-hip Rust crate (freetoken-rs_amd/ft-hip) against the C header.

No cargo in this image, so the crate is checked as text: every prototype of
include/ft_hip.h has exactly one `extern` item in src/ffi.rs with the same
name, the same argument names and the C-equivalent Rust types (int <-> c_int,
int64_t <-> i64, uint64_t <-> u64, size_t <-> usize, constness of pointers
kept), and the same return type; no item exists that the header lacks; the
wrapper (src/lib.rs) calls only declared items; the constants agree.
"""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HDR = os.path.join(ROOT, "include", "ft_hip.h")
CRATE = os.path.join(ROOT, "freetoken-rs_amd", "ft-hip")

C2R = {"int": "c_int", "int64_t": "i64", "uint64_t": "u64", "size_t": "usize", "float": "f32", "void": "c_void",
       "int32_t": "i32", "uint32_t": "u32", "char": "c_char", "ft_hip_ctx": "FtHipCtx", "uint8_t": "u8",
       "ft_gguf": "FtGguf"}


def c_type_to_rust(t):
    t = " ".join(t.split())
    const = t.startswith("const ")
    base = t[6:] if const else t
    stars = base.count("*")
    base = base.replace("*", "").strip()
    r = C2R[base]
    for i in range(stars):
        r = ("*const " if const and i == 0 else "*mut ") + r
    return r


def header_protos():
    src = re.sub(r"/\*.*?\*/", "", open(HDR).read(), flags=re.S)
    out = {}
    for ret, name, args in re.findall(r"^\s*((?:const\s+)?\w+\s*\**)\s*(ft_(?:hip|gguf)_\w+)\s*\(([^)]*)\)\s*;", src, re.M):
        params = []
        args = " ".join(args.split())
        if args and args != "void":
            for a in args.split(","):
                m = re.match(r"\s*(.*?)\s*(\w+)\s*$", a)
                params.append((m.group(2), c_type_to_rust(m.group(1))))
        out[name] = (params, c_type_to_rust(ret))
    return out


def rust_decls():
    src = open(os.path.join(CRATE, "src", "ffi.rs")).read()
    block = src[src.index('extern "C" {'):]
    out = {}
    for name, args, ret in re.findall(r"pub fn (ft_(?:hip|gguf)_\w+)\((.*?)\)\s*->\s*([^;]+);", block, re.S):
        params = []
        for a in [x for x in args.split(",") if x.strip()]:
            n, t = a.split(":", 1)
            params.append((n.strip(), " ".join(t.split())))
        assert name not in out, f"{name} declared twice"
        out[name] = (params, " ".join(ret.split()))
    return out


def test_every_header_prototype_has_a_matching_rust_item():
    h, r = header_protos(), rust_decls()
    assert len(h) >= 36
    assert sorted(h) == sorted(r), (sorted(set(h) - set(r)), sorted(set(r) - set(h)))
    for name, (params, ret) in h.items():
        assert r[name][1] == ret, (name, r[name][1], ret)
        assert r[name][0] == params, (name, r[name][0], params)


def test_wrapper_calls_only_declared_items_and_constants_agree():
    decl = rust_decls()
    lib = open(os.path.join(CRATE, "src", "lib.rs")).read()
    called = set(re.findall(r"ffi::(ft_(?:hip|gguf)_\w+)\(", lib))
    assert called and called <= set(decl), called - set(decl)
    # every Q4Gemv method the reference's MoE path uses is present by name
    for m in ["new", "quantize_q8", "quantize_q8_view", "gemv_grouped_q8_ptr", "gemv_q4r_ptr", "gemv_q4r_idx",
              "gelu_mul_q8", "gemv_f32_rows_dev", "topk_router_dev", "reduce_pairs_weighted"]:
        assert re.search(rf"pub fn {m}\(", lib), m
    hdr = open(HDR).read()
    ffi = open(os.path.join(CRATE, "src", "ffi.rs")).read()
    for c in ["FT_HIP_OK", "FT_HIP_E_INVALID", "FT_HIP_E_SHAPE", "FT_HIP_E_DEVICE", "FT_HIP_E_LAUNCH",
              "FT_HIP_E_TIMEOUT", "FT_HIP_E_IO", "FT_HIP_E_FORMAT", "FT_HIP_E_NOT_FOUND", "FT_Q8_BLK",
              "FT_LAYOUT_Q4_0", "FT_LAYOUT_Q4R", "FT_HIP_NOALLOC_SCRATCH_BYTES"]:
        hv = re.search(rf"#define {c} \(?([^)\n/]+)\)?", hdr).group(1).strip()
        rv = re.search(rf"pub const {c}: \w+ = ([^;]+);", ffi).group(1).strip()
        assert eval(hv.replace("(", "").replace(")", "")) == eval(rv), (c, hv, rv)


def test_build_script_builds_and_links_the_library():
    b = open(os.path.join(CRATE, "build.rs")).read()
    assert "build.py" in b and "rustc-link-lib=dylib=fthip" in b
    toml = open(os.path.join(CRATE, "Cargo.toml")).read()
    assert 'name = "ft-hip"' in toml
