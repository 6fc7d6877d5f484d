"""ctypes binding of include/moe_hip.h (the C ABI in libmoe_hip.so).

The library is built in-tree by oxidizr_amd.build (hipcc, gfx950). Loading
fails loudly when it is missing: there is no CPU fallback.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmoe_hip.so")

MOE_DTYPE_F32 = 0
MOE_DTYPE_BF16 = 1

SAVED_FIELDS = ["logits", "probs", "lse", "topk_idx", "topk_w", "counts", "offsets", "perm",
                "inv_perm", "mean_prob", "x_perm", "gate_act", "up_act", "swiglu", "expert_out",
                "rstd", "norm_x"]

EXPORTED = [
    "moe_config_default", "moe_plan_create", "moe_plan_destroy", "moe_saved_bytes",
    "moe_workspace_bytes", "moe_forward", "moe_backward", "moe_route_from_logits",
    "moe_saved_field_range", "moe_stage_name", "moe_plan_set_profiling", "moe_plan_stage_times",
    "moe_plan_set_shared_overlap", "moe_block_forward", "moe_block_backward",
    "moe_last_error", "moe_version", "moe_check_tokens", "moe_forward_noalloc",
    "moe_workspace_check",
]
NUM_STAGES = 20


class MoeConfigC(ctypes.Structure):
    _fields_ = [
        ("hidden", ctypes.c_int32), ("num_experts", ctypes.c_int32),
        ("experts_per_tok", ctypes.c_int32), ("intermediate", ctypes.c_int32),
        ("shared_intermediate", ctypes.c_int32), ("dtype", ctypes.c_int32),
        ("norm_topk_prob", ctypes.c_int32), ("has_router_bias", ctypes.c_int32),
        ("router_temperature", ctypes.c_float), ("shared_expert_scale", ctypes.c_float),
        ("aux_switch_coef", ctypes.c_float), ("aux_sqprob_coef", ctypes.c_float),
        ("recompute_activations", ctypes.c_int32), ("fused_block", ctypes.c_int32),
        ("rms_norm_eps", ctypes.c_float),
    ]


_vp = ctypes.c_void_p


class MoeWeightsC(ctypes.Structure):
    _fields_ = [("router", _vp), ("router_bias", _vp), ("gate", _vp), ("up", _vp), ("down", _vp),
                ("shared_gate", _vp), ("shared_up", _vp), ("shared_down", _vp)]


class MoeGradsC(ctypes.Structure):
    _fields_ = [("router", _vp), ("router_bias", _vp), ("gate", _vp), ("up", _vp), ("down", _vp),
                ("shared_gate", _vp), ("shared_up", _vp), ("shared_down", _vp)]


_lib = None


class MoeError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__(f"moe status {status}: {msg}")
        self.status = status


def load():
    """Load libmoe_hip.so (raises if it was not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -c 'import "
                           f"__graft_entry__ as g; g.build()'` (hipcc, gfx950)")
    L = ctypes.CDLL(LIB_PATH)
    i32, sz, i64 = ctypes.c_int32, ctypes.c_size_t, ctypes.c_int64
    P = ctypes.POINTER
    L.moe_config_default.argtypes = [P(MoeConfigC), i32, i32, i32, i32, i32]
    L.moe_config_default.restype = None
    L.moe_plan_create.argtypes = [P(MoeConfigC), ctypes.c_int, P(_vp)]
    L.moe_plan_create.restype = i32
    L.moe_plan_destroy.argtypes = [_vp]
    L.moe_plan_destroy.restype = i32
    L.moe_check_tokens.argtypes = [P(MoeConfigC), i64]
    L.moe_check_tokens.restype = i32
    L.moe_workspace_check.argtypes = [P(MoeConfigC), i64]
    L.moe_workspace_check.restype = i32
    L.moe_saved_bytes.argtypes = [_vp, i64]
    L.moe_saved_bytes.restype = sz
    L.moe_workspace_bytes.argtypes = [_vp, i64]
    L.moe_workspace_bytes.restype = sz
    L.moe_forward.argtypes = [_vp, _vp, i64, _vp, P(MoeWeightsC), _vp, _vp, _vp, _vp, _vp]
    L.moe_forward.restype = i32
    L.moe_forward_noalloc.argtypes = [_vp, _vp, i64, _vp, P(MoeWeightsC), _vp, _vp, _vp]
    L.moe_forward_noalloc.restype = i32
    L.moe_backward.argtypes = [_vp, _vp, i64, _vp, _vp, _vp, _vp, P(MoeWeightsC), _vp, _vp, _vp,
                               P(MoeGradsC), _vp]
    L.moe_backward.restype = i32
    L.moe_block_forward.argtypes = [_vp, _vp, i64, _vp, _vp, P(MoeWeightsC), _vp, _vp, _vp, _vp,
                                    _vp]
    L.moe_block_forward.restype = i32
    L.moe_block_backward.argtypes = [_vp, _vp, i64, _vp, _vp, _vp, _vp, _vp, P(MoeWeightsC), _vp,
                                     _vp, _vp, _vp, P(MoeGradsC), _vp]
    L.moe_block_backward.restype = i32
    L.moe_route_from_logits.argtypes = [_vp, _vp, i64, _vp, _vp, _vp]
    L.moe_route_from_logits.restype = i32
    L.moe_saved_field_range.argtypes = [_vp, i64, i32, P(sz), P(sz)]
    L.moe_saved_field_range.restype = i32
    L.moe_stage_name.argtypes = [i32]
    L.moe_stage_name.restype = ctypes.c_char_p
    L.moe_plan_set_profiling.argtypes = [_vp, i32]
    L.moe_plan_set_profiling.restype = i32
    L.moe_plan_set_shared_overlap.argtypes = [_vp, i32]
    L.moe_plan_set_shared_overlap.restype = i32
    L.moe_plan_stage_times.argtypes = [_vp, P(ctypes.c_float), P(i32), i32]
    L.moe_plan_stage_times.restype = i32
    L.moe_last_error.argtypes = []
    L.moe_last_error.restype = ctypes.c_char_p
    L.moe_version.argtypes = []
    L.moe_version.restype = ctypes.c_char_p
    _lib = L
    return L


def check(status):
    if status != 0:
        raise MoeError(status, load().moe_last_error().decode())


def ptr_array(ptrs):
    arr = (ctypes.c_void_p * len(ptrs))(*ptrs)
    return arr
