"""The Rust FFI crate (rust/moe-hip-sys) against include/moe_hip.h, on the CPU.

There is no Rust toolchain in this image, so the crate is checked as text:
every function the header declares is in the crate's extern "C" block with the
same parameter names in the same order, the #[repr(C)] structs hold the
header's fields in the header's order (the ctypes mirror, itself checked
against a C compiler in test_abi.py), and the status and dtype constants have
the header's values.
"""
import os
import re

from oxidizr_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "moe_hip.h")
CRATE = os.path.join(ROOT, "rust", "moe-hip-sys")


def _strip_c_comments(text):
    return re.sub(r"/\*.*?\*/", "", text, flags=re.S)


def _c_functions():
    text = _strip_c_comments(open(HEADER).read())
    out = {}
    for m in re.finditer(r"\b(moe_[a-z_]+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        params = [p.strip() for p in m.group(2).split(",") if p.strip() and p.strip() != "void"]
        out[m.group(1)] = [re.findall(r"([A-Za-z_][A-Za-z0-9_]*)\s*$", p)[0] for p in params]
    return out


def _rust_functions():
    text = open(os.path.join(CRATE, "src", "lib.rs")).read()
    block = text[text.index('extern "C" {'):]
    block = block[:block.index("\n    }\n")]
    out = {}
    for m in re.finditer(r"pub fn (moe_[a-z_]+)\s*\((.*?)\)", block, flags=re.S):
        params = [p.strip() for p in m.group(2).split(",") if p.strip()]
        out[m.group(1)] = [p.split(":")[0].strip() for p in params]
    return out


def test_every_header_function_is_bound_with_the_same_parameters():
    c, rust = _c_functions(), _rust_functions()
    assert set(c) == set(_lib.EXPORTED)
    assert set(c) == set(rust), (set(c) ^ set(rust))
    for name, params in c.items():
        assert rust[name] == params, (name, rust[name], params)


def _rust_struct_fields(name):
    text = open(os.path.join(CRATE, "src", "lib.rs")).read()
    m = re.search(r"pub struct " + name + r"\s*\{(.*?)\}", text, flags=re.S)
    return re.findall(r"pub ([a-z_]+):", m.group(1))


def test_repr_c_structs_follow_the_header():
    for rust_name, mirror in (("MoeConfigC", _lib.MoeConfigC), ("MoeWeightsC", _lib.MoeWeightsC),
                              ("MoeGradsC", _lib.MoeGradsC)):
        assert _rust_struct_fields(rust_name) == [f for f, _ in mirror._fields_], rust_name


def test_constants_match_the_header():
    text = open(os.path.join(CRATE, "src", "lib.rs")).read()
    header = _strip_c_comments(open(HEADER).read())
    for name in ("MOE_OK", "MOE_ERR_INVALID", "MOE_ERR_OOM", "MOE_ERR_HIP", "MOE_ERR_UNSUPPORTED",
                 "MOE_DTYPE_F32", "MOE_DTYPE_BF16"):
        rust_val = int(re.search(r"const " + name + r": [a-zA-Z0-9]+ = (\d+);", text).group(1))
        c_val = int(re.search(name + r"\s*=\s*(\d+)", header).group(1))
        assert rust_val == c_val, name
    saved = re.search(r"typedef enum \{(.*?)\} moe_saved_field;", header, flags=re.S).group(1)
    fields = re.findall(r"(MOE_SAVED_[A-Z_]+)", saved)
    for i, name in enumerate(fields[:10]):
        assert int(re.search(r"const " + name + r": i32 = (\d+);", text).group(1)) == i, name
    assert f"MOE_NUM_STAGES: usize = {_lib.NUM_STAGES};" in text


def test_crate_layout():
    for f in ("Cargo.toml", "build.rs", "src/lib.rs", "src/grad.rs"):
        assert os.path.exists(os.path.join(CRATE, f)), f
    cargo = open(os.path.join(CRATE, "Cargo.toml")).read()
    assert 'links = "moe_hip"' in cargo
    assert "rustc-link-lib=dylib=moe_hip" in open(os.path.join(CRATE, "build.rs")).read()
