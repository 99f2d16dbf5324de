"""ctypes access to the CPU oracle (libmoe_ref.so) and to the reference's own
scalar twins compiled from /root/reference/qwasar_cpu.c (_ref/libqwasar_cpu.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product package.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmoe_ref.so")
REF_PATH = os.path.join(HERE, "_ref", "libqwasar_cpu.so")

_P = C.c_void_p
_I = C.c_int32


def build() -> None:
    """Compile the oracle (and _ref where the reference tree is present)."""
    subprocess.run(["make", "-B", "-s", "-C", HERE], check=True)


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


class _Q4(C.Structure):
    _fields_ = [("w", _P), ("s", _P), ("b", _P), ("group", _I)]


class _Moe(C.Structure):
    _fields_ = [("H", _I), ("E", _I), ("K", _I), ("I", _I), ("SI", _I),
                ("norm", _I), ("split", _I), ("router", _P),
                ("gate_up", _Q4), ("gate", _Q4), ("up", _Q4), ("down", _Q4),
                ("sh_gate", _Q4), ("sh_up", _Q4), ("sh_down", _Q4),
                ("sh_gate_w", _P)]


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        L.qr_bf16_to_f32.restype = C.c_float
        L.qr_bf16_to_f32.argtypes = [C.c_uint16]
        L.qr_exp.restype = C.c_float
        L.qr_exp.argtypes = [C.c_float]
        L.qr_exp_vec.argtypes = [_P, _P, C.c_int64]
        L.qr_dot_bf16.restype = C.c_float
        L.qr_dot_bf16.argtypes = [_P, _P, _I]
        L.qr_dequant_row.argtypes = [_P, _P, _P, _P, _I, _I, _I]
        L.qr_qmv_q4.argtypes = [_P, _P, _P, _P, _P, _I, _I, _I, _I]
        L.qr_dmat_bf16.argtypes = [_P, _P, _P, _I, _I, _I]
        L.qr_route.argtypes = [_P, _P, _P, _I, _I, _I, _I]
        L.qr_route_literal.argtypes = [_P, _P, _P, _I, _I, _I, _I]
        L.qr_max_tiles.restype = _I
        L.qr_max_tiles.argtypes = [_I, _I, _I]
        L.qr_moe_group.restype = _I
        L.qr_moe_group.argtypes = [_P, _P, _P, _I, _I, _I, _I]
        L.qr_silu.restype = C.c_float
        L.qr_silu.argtypes = [C.c_float]
        L.qr_moe_forward.argtypes = [_P, _P, _P, _P, _I, C.POINTER(_Moe)]
        L.qr_rms_norm.argtypes = [_P, _P, _I, _I, C.c_float]
        L.qr_rms_norm_grouped.argtypes = [_P, _P, _P, _I, _I, _I, C.c_float]
        L.qr_silu_scale.argtypes = [_P, C.c_int64, C.c_float]
        L.qr_hc_mix.argtypes = [_P, _P, _P, _I, _I, _I]
        L.qr_hc_inject.argtypes = [_P, _P, _P, _I, _I, _I]
        L.qr_repeat_cols.argtypes = [_P, _P, _I, _I, _I]
        _lib = L
    return _lib


def reflib():
    """The reference's qwasar_cpu.c, or None where it was never built."""
    global _ref
    if _ref is None and os.path.exists(REF_PATH):
        R = C.CDLL(REF_PATH)
        R.qw_cpu_qmv_q4.argtypes = [_P, _P, _P, _P, _P, _I, _I, _I, _I]
        R.qw_cpu_dequant_row.argtypes = [_P, _P, _P, _P, _I, _I, _I]
        R.qw_cpu_dmv_bf16.argtypes = [_P, _P, _P, _I, _I, _I]
        R.qw_cpu_swiglu.argtypes = [_P, _P, _P, _I]
        R.qw_bf16_to_f32_c.restype = C.c_float
        R.qw_bf16_to_f32_c.argtypes = [C.c_uint16]
        R.qw_cpu_rms_norm.argtypes = [_P, _P, _P, _I, _I, C.c_float, C.c_float]
        _ref = R
    return _ref


# ---- numpy-level helpers -----------------------------------------------------

def exp_vec(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().qr_exp_vec(_ptr(out), _ptr(x), x.size)
    return out


def qmv_q4(x, w, s, b, k, n, rows, group):
    y = np.zeros((rows, n), np.float32)
    x = np.ascontiguousarray(x, np.float32)
    lib().qr_qmv_q4(_ptr(y), _ptr(x), _ptr(w), _ptr(s), _ptr(b), k, n, rows, group)
    return y


def dmat_bf16(x, w, k, n, rows):
    y = np.zeros((rows, n), np.float32)
    x = np.ascontiguousarray(x, np.float32)
    lib().qr_dmat_bf16(_ptr(y), _ptr(x), _ptr(w), k, n, rows)
    return y


def route(logits, rows, E, K, norm=True, literal=False):
    idx = np.zeros((rows, K), np.int32)
    w = np.zeros((rows, K), np.float32)
    lg = np.ascontiguousarray(logits, np.float32)
    fn = lib().qr_route_literal if literal else lib().qr_route
    fn(_ptr(idx), _ptr(w), _ptr(lg), rows, E, K, 1 if norm else 0)
    return idx, w


def max_tiles(pairs, E, bm):
    return lib().qr_max_tiles(pairs, E, bm)


def moe_group(idx, E, bm):
    idx = np.ascontiguousarray(idx, np.int32).ravel()
    pairs = idx.size
    mt = max_tiles(pairs, E, bm)
    perm = np.zeros(max(pairs, 1), np.int32)
    tiles = np.zeros(1 + 3 * max(mt, 1), np.int32)
    lib().qr_moe_group(_ptr(perm), _ptr(tiles), _ptr(idx), pairs, E, bm, mt)
    return perm[:pairs], tiles


def _q4(t):
    if t is None:
        return _Q4(None, None, None, 0)
    return _Q4(t.w.ctypes.data, t.s.ctypes.data, t.b.ctypes.data, t.group)


def moe_forward(layer, x, rows=None):
    """The whole MoE block on the CPU.  `layer` is a qwasar_amd.synth.MoeLayer."""
    x = np.ascontiguousarray(x, np.float32)
    rows = x.shape[0] if rows is None else rows
    L = layer
    m = _Moe(L.H, L.E, L.K, L.I, L.SI, 1 if L.norm else 0, 1 if L.split else 0,
             L.router.ctypes.data, _q4(L.gate_up), _q4(L.gate), _q4(L.up), _q4(L.down),
             _q4(L.sh_gate), _q4(L.sh_up), _q4(L.sh_down), L.sh_gate_w.ctypes.data)
    out = np.zeros((rows, L.H), np.float32)
    idx = np.zeros((rows, L.K), np.int32)
    w = np.zeros((rows, L.K), np.float32)
    lib().qr_moe_forward(_ptr(out), _ptr(idx), _ptr(w), _ptr(x), rows, C.byref(m))
    return out, idx, w


# ---- the layer stack -------------------------------------

STACK_EPS = 1e-6


def rms_norm(x: np.ndarray, eps: float = STACK_EPS) -> np.ndarray:
    """Unit-weight RMS norm of fp32 rows, qwasar_cpu.c:68-82's form."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().qr_rms_norm(_ptr(y), _ptr(x), x.shape[-1], x.size // x.shape[-1], eps)
    return y


def _bf16(a: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def residual_norm(h: np.ndarray, y=None, eps: float = STACK_EPS):
    """(h', x): h' = bf16(h + y) (h when y is None), x = rms_norm(h').
    h, h' are bf16 bits (uint16), y and x fp32."""
    if y is not None:
        h = _bf16(_f32(h) + np.asarray(y, np.float32))
    return h, rms_norm(_f32(h), eps)


def stack_forward(layers, h0: np.ndarray, eps: float = STACK_EPS):
    """The stack on the CPU: x = norm(h); per layer y = MoE(x), h = bf16(h + y),
    x = norm(h).  Returns the final h (bf16 bits) and each layer's (x, y)."""
    h, x = residual_norm(h0, None, eps)
    trace = []
    for L in layers:
        y, _, _ = moe_forward(L, x)
        trace.append((x, y))
        h, x = residual_norm(h, y, eps)
    return h, trace


# ---- the hyper-connection mixer -------------------------------

def rms_norm_grouped(x: np.ndarray, w: np.ndarray, dim: int, groups: int, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.uint16)
    y = np.empty_like(x)
    rows = x.size // (dim * groups)
    lib().qr_rms_norm_grouped(_ptr(y), _ptr(x), _ptr(w), dim, groups, rows, eps)
    return y


def silu_scale(y: np.ndarray, scale: float) -> np.ndarray:
    y = np.array(y, np.float32, copy=True)
    lib().qr_silu_scale(_ptr(y), y.size, scale)
    return y


def hc_mix(n: np.ndarray, m: np.ndarray, rows: int, H: int, S: int) -> np.ndarray:
    n = np.ascontiguousarray(n, np.float32)
    m = np.ascontiguousarray(m, np.float32)
    x = np.empty((rows, H), np.float32)
    lib().qr_hc_mix(_ptr(x), _ptr(n), _ptr(m), rows, H, S)
    return x


def hc_inject(h4: np.ndarray, out: np.ndarray, inj: np.ndarray, rows: int, H: int, S: int) -> np.ndarray:
    h4 = np.array(h4, np.float32, copy=True)
    out = np.ascontiguousarray(out, np.float32)
    inj = np.ascontiguousarray(inj, np.float32)
    lib().qr_hc_inject(_ptr(h4), _ptr(out), _ptr(inj), rows, H, S)
    return h4


def repeat_cols(x: np.ndarray, rows: int, H: int, S: int) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    h4 = np.empty((rows, S * H), np.float32)
    lib().qr_repeat_cols(_ptr(h4), _ptr(x), rows, H, S)
    return h4


def hc_mix_up(d, n4, w, s, b, k, H, S, rows, scale, group):
    """x = mean_s sigmoid(W_s . silu(scale * d)) * n4_s: the reference's
    silu_scale, the up-projection's matvec (qwasar_flash_cpu.c:272-273) and
    hc_mix, composed."""
    ds = silu_scale(np.asarray(d, np.float32).reshape(rows, k), scale)
    m = qmv_q4(ds, w, s, b, k, S * H, rows, group)
    return hc_mix(n4, m, rows, H, S)
