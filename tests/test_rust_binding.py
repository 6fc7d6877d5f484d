"""The Rust FFI crate (rust/moe-hip-sys) against include/moe_hip.h, on the CPU.

There is no Rust toolchain in this image, so the crate is checked as text:
every function the header declares is in the crate's extern "C" block with the
same parameter names in the same order and the Rust type each C type maps to
(pointer constness, integer widths, return type), the #[repr(C)] structs hold
the header's fields in the header's order with the mapped types, the status
and dtype constants have the header's values, and the backward neither
allocates its scratch nor copies a device buffer to the host synchronously.
"""
import os
import re

from oxidizr_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "moe_hip.h")
CRATE = os.path.join(ROOT, "rust", "moe-hip-sys")

# C base types of the header -> Rust types of the crate
_BASE = {"void": "c_void", "int32_t": "i32", "int": "i32", "int64_t": "i64", "float": "f32",
         "uint8_t": "u8", "size_t": "usize", "char": "c_char", "moe_config": "MoeConfigC",
         "moe_plan": "MoePlan", "moe_weights": "MoeWeightsC", "moe_grads": "MoeGradsC",
         "moe_status": "MoeStatus"}


def c_to_rust(ctype):
    """The Rust spelling of a C type: `const T*` -> `*const T`, `T*` -> `*mut T`,
    `const void* const*` -> `*const *const c_void`, `T` -> its Rust name."""
    toks = re.findall(r"\*|[A-Za-z_][A-Za-z0-9_]*", ctype)
    const = False
    if toks and toks[0] == "const":
        const, toks = True, toks[1:]
    rust = _BASE[toks[0]]
    rest = toks[1:]
    i = 0
    while i < len(rest):
        assert rest[i] == "*", ctype
        rust = ("*const " if const else "*mut ") + rust
        const = i + 1 < len(rest) and rest[i + 1] == "const"
        i += 2 if const else 1
    return rust


def test_type_mapping_itself():
    assert c_to_rust("const void*") == "*const c_void"
    assert c_to_rust("void*") == "*mut c_void"
    assert c_to_rust("moe_plan**") == "*mut *mut MoePlan"
    assert c_to_rust("const void* const*") == "*const *const c_void"
    assert c_to_rust("void* const*") == "*const *mut c_void"
    assert c_to_rust("int64_t") == "i64"
    assert c_to_rust("const char*") == "*const c_char"


def _strip_c_comments(text):
    return re.sub(r"/\*.*?\*/", "", text, flags=re.S)


def _split_decl(p):
    """'const float* d_aux' -> ('const float*', 'd_aux')."""
    name = re.findall(r"([A-Za-z_][A-Za-z0-9_]*)\s*$", p)[0]
    return p[:p.rindex(name)].strip(), name


def _c_functions():
    text = _strip_c_comments(open(HEADER).read())
    out = {}
    for m in re.finditer(r"([A-Za-z_][A-Za-z0-9_ ]*?\**)\s*\b(moe_[a-z_]+)\s*\(([^;{]*?)\)\s*;",
                         text, flags=re.S):
        ret = m.group(1).split("\n")[-1].strip()
        params = [p.strip() for p in m.group(3).split(",") if p.strip() and p.strip() != "void"]
        out[m.group(2)] = (ret, [_split_decl(p) for p in params])
    return out


def _rust_functions():
    text = open(os.path.join(CRATE, "src", "lib.rs")).read()
    block = text[text.index('extern "C" {'):]
    block = block[:block.index("\n    }\n")]
    out = {}
    for m in re.finditer(r"pub fn (moe_[a-z_]+)\s*\((.*?)\)\s*(->\s*([^;]+))?;", block, flags=re.S):
        params = [p.strip() for p in m.group(2).split(",") if p.strip()]
        ret = (m.group(4) or "void").strip()
        out[m.group(1)] = (ret, [(p.split(":", 1)[1].strip(), p.split(":")[0].strip())
                                 for p in params])
    return out


def test_every_header_function_is_bound_with_the_same_parameters_and_types():
    c, rust = _c_functions(), _rust_functions()
    assert set(c) == set(_lib.EXPORTED)
    assert set(c) == set(rust), (set(c) ^ set(rust))
    for name, (c_ret, c_params) in c.items():
        r_ret, r_params = rust[name]
        assert [n for _, n in r_params] == [n for _, n in c_params], name
        for (c_t, n), (r_t, _) in zip(c_params, r_params):
            assert re.sub(r"\s+", " ", r_t) == c_to_rust(c_t), (name, n, c_t, r_t)
        want_ret = "void" if c_ret == "void" else c_to_rust(c_ret)
        assert r_ret == want_ret, (name, c_ret, r_ret)


def _c_struct_fields(name):
    text = _strip_c_comments(open(HEADER).read())
    body = re.search(r"typedef struct \{([^{}]*)\}\s*" + name + r";", text).group(1)
    return [_split_decl(d.strip()) for d in body.split(";") if d.strip()]


def _rust_struct_fields(name):
    text = open(os.path.join(CRATE, "src", "lib.rs")).read()
    m = re.search(r"pub struct " + name + r"\s*\{(.*?)\}", text, flags=re.S)
    return re.findall(r"pub ([a-z_]+):\s*([^,]+),", m.group(1))


def test_repr_c_structs_follow_the_header():
    for rust_name, c_name, mirror in (("MoeConfigC", "moe_config", _lib.MoeConfigC),
                                      ("MoeWeightsC", "moe_weights", _lib.MoeWeightsC),
                                      ("MoeGradsC", "moe_grads", _lib.MoeGradsC)):
        rust = _rust_struct_fields(rust_name)
        c = _c_struct_fields(c_name)
        assert [f for f, _ in rust] == [f for f, _ in mirror._fields_], rust_name
        assert [f for f, _ in rust] == [n for _, n in c], rust_name
        for (f, r_t), (c_t, _) in zip(rust, c):
            assert r_t.strip() == c_to_rust(c_t), (rust_name, f, c_t, r_t)


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


def _fn_body(text, name):
    start = text.index(f"fn {name}(")
    depth, i = 0, text.index("{", text.index(")", start))
    for j in range(i, len(text)):
        depth += {"{": 1, "}": -1}.get(text[j], 0)
        if depth == 0:
            return text[i:j + 1]
    raise AssertionError(name)


def test_grad_fn_backward_neither_allocates_scratch_nor_waits_on_the_stream():
    """The backward takes its scratch from the shared per-stream workspace and
    its expert mask from the forward's pinned counts copy (src/trainer.rs:
    556-566, :1087-1111): no per-call workspace allocation, no synchronous
    device-to-host copy, no has_grad buffer read back."""
    text = open(os.path.join(CRATE, "src", "grad.rs")).read()
    code = re.sub(r"//[^\n]*", "", text)
    body = _fn_body(code, "backward")
    assert "workspace.ensure(" in body
    assert "alloc(plan.workspace_bytes" not in re.sub(r"\s+", "", body).replace("alloc.alloc", "alloc(")
    assert "copy_to_host" not in code
    assert "self.routed.mask(" in body
    # moe_backward gets has_grad = NULL: the last argument of plan.backward
    call = re.search(r"plan\.backward\((.*?)\)\?;", body, flags=re.S).group(1)
    assert call.split(",")[-1].strip() == "std::ptr::null_mut()"
    fwd = _fn_body(code, "forward")
    assert "RoutedExperts::record(" in fwd and "workspace.ensure(" in fwd
    rec = _fn_body(code, "record")
    assert "copy_to_pinned_async" in rec and "record_event" in rec
    assert "event_synchronize" not in rec


def test_crate_layout():
    for f in ("Cargo.toml", "build.rs", "src/lib.rs", "src/grad.rs"):
        assert os.path.exists(os.path.join(CRATE, f)), f
    cargo = open(os.path.join(CRATE, "Cargo.toml")).read()
    assert 'links = "moe_hip"' in cargo
    assert "rustc-link-lib=dylib=moe_hip" in open(os.path.join(CRATE, "build.rs")).read()
