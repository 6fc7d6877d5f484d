"""CPU checks of the drop-in boundary: the C-ABI library loads, exports every
entry point include/moe_hip.h declares, its structs match the ctypes mirror,
and the host-side config validation follows the reference's messages
(src/model.rs:1927-1958, src/config_convert.rs:380-404). No GPU calls."""
import ctypes
import os
import re
import subprocess

import pytest

from oxidizr_amd import _lib
from oxidizr_amd.moe import ModelError, MoeConfig

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "moe_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(moe_[a-z_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = _lib.load()
    names = _declared()
    assert "moe_forward" in names and "moe_backward" in names
    for n in names:
        assert hasattr(L, n), f"{n} declared in moe_hip.h but not exported"
    assert sorted(_lib.EXPORTED) == names


def test_struct_layouts_match_header(tmp_path):
    # every field offset and struct size of the ctypes mirror equals what a C
    # compiler makes of include/moe_hip.h
    structs = {"moe_config": _lib.MoeConfigC, "moe_weights": _lib.MoeWeightsC,
               "moe_grads": _lib.MoeGradsC}
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "moe_hip.h"', "int main(void) {"]
    for cname, py in structs.items():
        lines.append(f'  printf("{cname} size %zu\\n", sizeof({cname}));')
        for f, _ in py._fields_:
            lines.append(f'  printf("{cname} {f} %zu\\n", offsetof({cname}, {f}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)],
                   check=True)
    got = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True,
                               text=True).stdout.splitlines():
        cname, f, v = line.split()
        got[(cname, f)] = int(v)
    for cname, py in structs.items():
        assert got[(cname, "size")] == ctypes.sizeof(py), cname
        for f, _ in py._fields_:
            assert got[(cname, f)] == getattr(py, f).offset, (cname, f)


def test_config_defaults_and_names():
    L = _lib.load()
    c = _lib.MoeConfigC()
    L.moe_config_default(ctypes.byref(c), 2048, 16, 2, 1408, 2816)
    assert (c.hidden, c.num_experts, c.experts_per_tok, c.intermediate, c.shared_intermediate) == \
        (2048, 16, 2, 1408, 2816)
    assert c.dtype == _lib.MOE_DTYPE_BF16
    assert c.router_temperature == 1.0 and c.shared_expert_scale == 1.0
    assert c.aux_switch_coef == 1.0 and c.aux_sqprob_coef == 1.0
    assert c.norm_topk_prob == 0 and c.has_router_bias == 0
    assert c.recompute_activations == 0 and c.fused_block == 0
    names = [L.moe_stage_name(i).decode() for i in range(_lib.NUM_STAGES)]
    assert names[0] == "router_gemm" and names[-4:] == ["dx", "recompute", "norm_fwd", "norm_bwd"]
    assert len(set(names)) == len(names)
    assert L.moe_stage_name(_lib.NUM_STAGES).decode() == "unknown"
    assert b"gfx950" in L.moe_version()


def test_null_plan_is_an_error_not_a_crash():
    L = _lib.load()
    assert L.moe_saved_bytes(None, 16) == 0
    assert L.moe_plan_set_profiling(None, 1) == 1
    assert b"NULL" in L.moe_last_error()
    w = _lib.MoeWeightsC()
    assert L.moe_forward(None, None, 4, None, ctypes.byref(w), None, None, None, None, None) == 1


def test_invalid_config_rejected_before_any_device_call():
    L = _lib.load()
    c = _lib.MoeConfigC()
    L.moe_config_default(ctypes.byref(c), 64, 4, 5, 32, 0)  # k > E
    h = ctypes.c_void_p()
    assert L.moe_plan_create(ctypes.byref(c), 0, ctypes.byref(h)) == 1
    assert b"must not exceed num_experts" in L.moe_last_error()
    L.moe_config_default(ctypes.byref(c), 64, 4, 2, 0, 0)
    assert L.moe_plan_create(ctypes.byref(c), 0, ctypes.byref(h)) == 1
    assert b"intermediate_size must be non-zero" in L.moe_last_error()
    L.moe_config_default(ctypes.byref(c), 60, 4, 2, 32, 0)
    assert L.moe_plan_create(ctypes.byref(c), 0, ctypes.byref(h)) == 1


def test_required_moe_dims_messages():
    with pytest.raises(ModelError, match="must not exceed num_experts"):
        MoeConfig(64, 4, 5, 32).required_moe_dims()
    with pytest.raises(ModelError, match="intermediate_size must be non-zero"):
        MoeConfig(64, 4, 2, 0).required_moe_dims()
    with pytest.raises(ModelError, match="requires cfg.moe.intermediate_size"):
        MoeConfig(64, 4, 2, None).required_moe_dims()
    with pytest.raises(ModelError, match="experts_per_tok is missing"):
        MoeConfig(64, 4, None, 32).required_moe_dims()
    assert MoeConfig(64, 4, 2, 32).required_moe_dims() == (4, 2, 32)
    # shared_expert_enabled: None means true (src/config.rs:127-129)
    assert MoeConfig(64, 4, 2, 32).shared_width() == 32
    assert MoeConfig(64, 4, 2, 32, shared_expert_enabled=False).shared_width() == 0


def test_c_caller_of_the_header(tmp_path):
    # tests/c_abi_check.c: a plain C program compiled against include/moe_hip.h
    # and linked with libmoe_hip.so, as a Rust FFI crate would bind it
    _lib.load()
    exe = tmp_path / "c_abi_check"
    libdir = os.path.dirname(_lib.LIB_PATH)
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"),
                    os.path.join(ROOT, "tests", "c_abi_check.c"), "-L", libdir, "-lmoe_hip",
                    f"-Wl,-rpath,{libdir}", "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failure(s)" in r.stdout


def _check_tokens(H, E, k, I, S, T, dtype=_lib.MOE_DTYPE_BF16):
    L = _lib.load()
    c = _lib.MoeConfigC()
    L.moe_config_default(ctypes.byref(c), H, E, k, I, S)
    c.dtype = dtype
    return L.moe_check_tokens(ctypes.byref(c), T)


def test_token_limit_follows_the_widest_operand():
    # every operand tile is read through a buffer resource with 32-bit byte
    # offsets: T * max(H, I, S, E rounded to 8) * bytes must stay below 2^31
    for H, E, I, S in [(7168, 256, 2048, 2048), (2048, 64, 1408, 2816), (1024, 16, 4096, 0),
                       (512, 1000, 256, 0)]:
        for dt, b in ((_lib.MOE_DTYPE_BF16, 2), (_lib.MOE_DTYPE_F32, 4)):
            wide = max(H, I, S, (E + 7) // 8 * 8)
            limit = (2**31 - 1) // (wide * b)  # largest T with T * wide * b < 2^31
            assert _check_tokens(H, E, 2, I, S, limit, dt) == 0, (H, E, I, S, dt)
            if limit + 1 <= 2**24:
                assert _check_tokens(H, E, 2, I, S, limit + 1, dt) == 4, (H, E, I, S, dt)
    assert _check_tokens(32, 4, 2, 32, 0, 2**24) == 0     # 2^24 * 32 * 2 = 2^30 bytes
    assert _check_tokens(32, 4, 2, 32, 0, 2**24 + 1) == 4  # above 2^24 tokens
    assert _check_tokens(64, 4, 2, 32, 0, -1) == 1
    assert _check_tokens(64, 4, 5, 32, 0, 8) == 1   # invalid config first


def _cfg(H, E, k, I, S, bf16=True, **kw):
    L = _lib.load()
    c = _lib.MoeConfigC()
    L.moe_config_default(ctypes.byref(c), H, E, k, I, S)
    c.dtype = _lib.MOE_DTYPE_BF16 if bf16 else _lib.MOE_DTYPE_F32
    for n, v in kw.items():
        setattr(c, n, v)
    return c


# BASELINE configs 1-5 (H, E, k, I, S, bf16) and a few edge shapes
_WS_CONFIGS = {
    "cfg1": (384, 8, 2, 1024, 0, False), "cfg2": (2048, 16, 2, 1408, 2816, True),
    "cfg3": (2048, 64, 6, 1408, 2816, True), "cfg4": (4096, 128, 8, 1536, 0, True),
    "cfg5": (7168, 256, 8, 2048, 2048, True), "e1k1": (64, 1, 1, 32, 0, True),
    "e1000": (128, 1000, 16, 64, 64, True), "f32wide": (2048, 64, 6, 1408, 2816, False),
}


def _token_limit(c):
    """The largest token count moe_check_tokens accepts (T <= 2^24 and
    T * max(H, I, S, 8 ceil(E / 8)) * b < 2^31)."""
    b = 2 if c.dtype == _lib.MOE_DTYPE_BF16 else 4
    wide = max(c.hidden, c.intermediate, c.shared_intermediate, (c.num_experts + 7) // 8 * 8)
    return min(1 << 24, ((1 << 31) - 1) // (wide * b))


@pytest.mark.parametrize("name", sorted(_WS_CONFIGS))
@pytest.mark.parametrize("flags", [{}, {"recompute_activations": 1}, {"fused_block": 1},
                                   {"has_router_bias": 1, "norm_topk_prob": 1}])
def test_every_launch_fits_its_workspace_region(name, flags):
    # The split-K partials of the dense weight gradients were once planned
    # with one tiling and launched with another (the launch then wrote past its
    # region); moe_workspace_check recomputes every launch's scratch need from
    # the launches' own sizing and compares it with the plan, on the CPU.
    H, E, k, I, S, bf16 = _WS_CONFIGS[name]
    if flags.get("fused_block") and H > 8192:
        pytest.skip("fused_block supports H <= 8192")
    c = _cfg(H, E, k, I, S, bf16, **flags)
    L = _lib.load()
    limit = _token_limit(c)
    assert L.moe_check_tokens(ctypes.byref(c), limit) == 0
    assert L.moe_check_tokens(ctypes.byref(c), limit + 1) == 4
    for T in sorted({0, 1, 16, 63, 64, 65, 255, 256, 257, 1024, 4097, 8192, 16384, 65536,
                     limit}):
        if T > limit:
            continue
        st = L.moe_workspace_check(ctypes.byref(c), T)
        assert st == 0, (name, flags, T, L.moe_last_error().decode())
    assert L.moe_workspace_check(ctypes.byref(c), limit + 1) == 4
    assert L.moe_workspace_check(ctypes.byref(c), -1) == 1


def test_workspace_check_refuses_bad_input():
    # the config and token checks come before any layout arithmetic
    L = _lib.load()
    bad = _cfg(64, 4, 2, 32, 0, True)
    bad.experts_per_tok = 9  # k > E: required_moe_dims refuses it
    assert L.moe_workspace_check(ctypes.byref(bad), 64) == 1
    assert b"experts_per_tok" in L.moe_last_error()
    good = _cfg(64, 4, 2, 32, 0, True)
    assert L.moe_workspace_check(ctypes.byref(good), -5) == 1
    assert L.moe_workspace_check(ctypes.byref(good), (1 << 24) + 1) == 4


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    """With no built libmoe_hip.so there is no CPU fallback: loading raises and
    names the build step."""
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "libmoe_hip.so"))
    with pytest.raises(RuntimeError, match="is missing: build it"):
        _lib.load()
