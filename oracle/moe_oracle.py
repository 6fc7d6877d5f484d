"""ctypes bindings for the MoE CPU oracle -- TEST INFRASTRUCTURE ONLY.

The oracle (oracle/moe_oracle.cpp) is a CPU restatement of oxidizr's MoE layer
(src/model.rs:1385-1958 in the reference, arithmetic from boostr::nn::moe with
its constants made explicit parameters). Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg may import this module, as the checker or the
timed CPU baseline. The product package (oxidizr_amd) never imports it.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libmoe_oracle.so")
_lib = None


class OracleCfg(ctypes.Structure):
    _fields_ = [
        ("T", ctypes.c_int32), ("H", ctypes.c_int32), ("E", ctypes.c_int32),
        ("k", ctypes.c_int32), ("I", ctypes.c_int32), ("S", ctypes.c_int32),
        ("norm_topk", ctypes.c_int32), ("has_bias", ctypes.c_int32),
        ("tau", ctypes.c_double), ("shared_scale", ctypes.c_double),
        ("aux_switch", ctypes.c_double), ("aux_sqprob", ctypes.c_double),
    ]


def build():
    """Compile the oracle with its Makefile (gcc + OpenMP)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        vp = ctypes.c_void_p
        L.oracle_create.restype = vp
        L.oracle_create.argtypes = [ctypes.POINTER(OracleCfg), ctypes.c_int]
        L.oracle_destroy.argtypes = [vp]
        L.oracle_set_threads.argtypes = [ctypes.c_int]
        L.oracle_max_threads.restype = ctypes.c_int
        L.oracle_forward.argtypes = [vp, ctypes.c_int] + [vp] * 9 + [vp, vp]
        L.oracle_backward.argtypes = [vp, vp, ctypes.c_double, ctypes.c_double] + [vp] * 10
        L.oracle_get.argtypes = [vp, ctypes.c_char_p, vp]
        L.oracle_route_f64.argtypes = [ctypes.POINTER(OracleCfg), ctypes.c_int] + [vp] * 5
        L.oracle_dispatch.argtypes = [ctypes.c_int] * 3 + [vp] * 5
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def make_cfg(T, H, E, k, I, S=0, norm_topk=False, has_bias=False, tau=1.0,
             shared_scale=1.0, aux_switch=1.0, aux_sqprob=1.0):
    return OracleCfg(T, H, E, k, I, S, int(norm_topk), int(has_bias), tau,
                     shared_scale, aux_switch, aux_sqprob)


def set_threads(n):
    lib().oracle_set_threads(int(n))


def max_threads():
    return lib().oracle_max_threads()


def route(cfg, logits):
    """Softmax + top-k of fp64 logits [T, E] -> probs, lse, idx, w."""
    logits = np.ascontiguousarray(logits, dtype=np.float64)
    T, E = logits.shape
    probs = np.empty((T, E)); lse = np.empty(T)
    idx = np.empty((T, cfg.k), np.int32); w = np.empty((T, cfg.k))
    lib().oracle_route_f64(ctypes.byref(cfg), T, _ptr(logits), _ptr(probs), _ptr(lse),
                           _ptr(idx), _ptr(w))
    return probs, lse, idx, w


def dispatch(idx, E):
    """Stable expert-major permutation of the [T, k] assignments."""
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    T, k = idx.shape
    counts = np.empty(E, np.int32); offsets = np.empty(E + 1, np.int32)
    perm = np.empty(T * k, np.int32); inv = np.empty(T * k, np.int32)
    rc = lib().oracle_dispatch(T, k, E, _ptr(idx), _ptr(counts), _ptr(offsets), _ptr(perm),
                               _ptr(inv))
    if rc != 0:
        raise ValueError("expert index out of range")
    return counts, offsets, perm, inv


class MoeOracle:
    """One layer's forward/backward on the CPU. Weights packed per expert:
    wg, wu [E, I, H]; wd [E, H, I]; shared swg, swu [S, H]; swd [H, S]."""

    def __init__(self, cfg, precision=64):
        self.cfg = cfg
        self.dt = np.float64 if precision == 64 else np.float32
        # kept on the instance: at interpreter exit the module globals may be
        # gone before the last oracle is collected
        self._destroy = lib().oracle_destroy
        self.h = lib().oracle_create(ctypes.byref(cfg), precision)
        if not self.h:
            raise ValueError("invalid oracle configuration")
        self._keep = None
        self.T = 0

    def __del__(self):
        if getattr(self, "h", None):
            self._destroy(self.h)
            self.h = None

    def _c(self, a):
        return None if a is None else np.ascontiguousarray(a, dtype=self.dt)

    def forward(self, x, wr, wg, wu, wd, bias=None, swg=None, swu=None, swd=None,
                logits_in=None):
        c = self.cfg
        x = self._c(x).reshape(-1, c.H)
        T = x.shape[0]
        arrs = [x, self._c(wr), self._c(bias), self._c(wg), self._c(wu), self._c(wd),
                self._c(swg), self._c(swu), self._c(swd)]
        li = None if logits_in is None else np.ascontiguousarray(logits_in, dtype=np.float32)
        out = np.empty((T, c.H), self.dt)
        self._keep = arrs + [li]
        self.T = T
        lib().oracle_forward(self.h, T, *[_ptr(a) for a in arrs], _ptr(li), _ptr(out))
        return out, float(self.get("aux")), float(self.get("z"))

    def get(self, name):
        c, T = self.cfg, self.T
        TK = T * c.k
        shapes = {
            "logits": ((T, c.E), self.dt), "probs": ((T, c.E), self.dt), "lse": ((T,), self.dt),
            "topk_idx": ((T, c.k), np.int32), "topk_w": ((T, c.k), self.dt),
            "counts": ((c.E,), np.int32), "offsets": ((c.E + 1,), np.int32),
            "perm": ((TK,), np.int32), "inv_perm": ((TK,), np.int32),
            "x_perm": ((TK, c.H), self.dt), "G": ((TK, c.I), self.dt), "U": ((TK, c.I), self.dt),
            "A": ((TK, c.I), self.dt), "Y": ((TK, c.H), self.dt),
            "shared_Y": ((T, c.H) if c.S > 0 else (0,), self.dt),
            "aux": ((1,), self.dt), "z": ((1,), self.dt),
        }
        shp, dt = shapes[name]
        dst = np.empty(shp, dt)
        if lib().oracle_get(self.h, name.encode(), _ptr(dst)) != 0:
            raise KeyError(name)
        return dst[0] if name in ("aux", "z") else dst

    def grad_buffers(self, fill=np.nan):
        c, T = self.cfg, self.T
        return {
            "x": np.empty((T, c.H), self.dt),
            "router": np.empty((c.E, c.H), self.dt),
            "router_bias": np.empty(c.E, self.dt) if c.has_bias else None,
            "gate": np.full((c.E, c.I, c.H), fill, self.dt),
            "up": np.full((c.E, c.I, c.H), fill, self.dt),
            "down": np.full((c.E, c.H, c.I), fill, self.dt),
            "shared_gate": np.empty((c.S, c.H), self.dt) if c.S else None,
            "shared_up": np.empty((c.S, c.H), self.dt) if c.S else None,
            "shared_down": np.empty((c.H, c.S), self.dt) if c.S else None,
        }

    def backward(self, dout, d_aux=0.0, d_z=0.0, fill=np.nan, out=None):
        """Returns a dict of gradients. Experts with no routed token keep the
        `fill` value in their buffers and report has_grad == 0. `out` may pass
        buffers from grad_buffers() to reuse."""
        c, T = self.cfg, self.T
        dout = self._c(dout).reshape(T, c.H)
        g = out if out is not None else self.grad_buffers(fill)
        has_grad = np.zeros(c.E, np.uint8)
        lib().oracle_backward(self.h, _ptr(dout), float(d_aux), float(d_z), _ptr(g["x"]),
                              _ptr(g["router"]), _ptr(g["router_bias"]), _ptr(g["gate"]),
                              _ptr(g["up"]), _ptr(g["down"]), _ptr(g["shared_gate"]),
                              _ptr(g["shared_up"]), _ptr(g["shared_down"]), _ptr(has_grad))
        g["has_grad"] = has_grad
        return g


# ---------------------------------------------------------------- block path
# The MoE sub-block of a decoder block (reference src/model.rs:2792-2800 MLA
# arm, :2822-2826 legacy arm): residual = h; x = post_attention_layernorm(h);
# (y, aux, z) = MoE(x); out = y + residual.  post_attention_layernorm is
# boostr::nn::RmsNorm (src/model.rs:500-512: weight [H], eps = cfg.rms_norm_eps);
# its formula is restated as x = h * rstd * w, rstd = 1 / sqrt(mean(h^2) + eps).

def rmsnorm_forward(h, w, eps):
    """(x, rstd) in float64, per row of h [T, H]."""
    h = np.asarray(h, np.float64)
    w = np.asarray(w, np.float64)
    rstd = 1.0 / np.sqrt((h * h).mean(axis=-1) + eps)
    return h * rstd[:, None] * w, rstd


def rmsnorm_backward(dx, h, w, rstd):
    """(dh, dw) of x = h * rstd * w for the upstream gradient dx."""
    h = np.asarray(h, np.float64)
    w = np.asarray(w, np.float64)
    xh = h * rstd[:, None]
    gw = np.asarray(dx, np.float64) * w
    mean = (xh * gw).mean(axis=-1, keepdims=True)
    return rstd[:, None] * (gw - xh * mean), (np.asarray(dx, np.float64) * xh).sum(axis=0)


class MoeBlockOracle:
    """post_attention_layernorm -> MoE layer (MoeOracle) -> residual add."""

    def __init__(self, cfg, eps, precision=64):
        self.moe = MoeOracle(cfg, precision)
        self.eps = eps

    def forward(self, h, norm_weight, wr, wg, wu, wd, bias=None, swg=None, swu=None, swd=None,
                logits_in=None):
        self.hin = np.asarray(h, np.float64).reshape(-1, self.moe.cfg.H)
        self.nw = np.asarray(norm_weight, np.float64)
        x, self.rstd = rmsnorm_forward(self.hin, self.nw, self.eps)
        y, aux, z = self.moe.forward(x, wr, wg, wu, wd, bias, swg, swu, swd, logits_in=logits_in)
        return y + self.hin, aux, z

    def backward(self, dout, d_aux=0.0, d_z=0.0, fill=np.nan):
        g = self.moe.backward(dout, d_aux, d_z, fill)
        dh, dw = rmsnorm_backward(g["x"], self.hin, self.nw, self.rstd)
        g["h"] = np.asarray(dout, np.float64).reshape(dh.shape) + dh
        g["norm_weight"] = dw
        return g
