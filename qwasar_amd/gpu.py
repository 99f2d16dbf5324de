"""ctypes binding of include/qwasar_gpu.h (libqwasar_hip.so).

The functions keep the C names and argument order (qw_op_*, qw_buf_*,
qw_cmd_*), so a test written against this module reads like the reference's
own C tests (tests/test_sparse.c).  There is no fallback: if the library is
missing, importing raises.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("QWASAR_HIP_LIB") or os.path.join(HERE, "lib", "libqwasar_hip.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build() "
                      "(make -C qwasar_amd/csrc)")

_lib = C.CDLL(LIB_PATH)

_P = C.c_void_p
_I = C.c_int32
_B = C.c_bool


class qw_ref(C.Structure):
    _fields_ = [("buf", _P), ("off", C.c_size_t)]


def qw_ref_at(buf, off: int = 0) -> qw_ref:
    return qw_ref(buf.handle if isinstance(buf, Buf) else buf, off)


NULL_REF = qw_ref(None, 0)


class qw_qmv_part(C.Structure):
    _fields_ = [("y", qw_ref), ("w", qw_ref), ("scales", qw_ref), ("biases", qw_ref), ("n", _I)]


class qw_q4_ref(C.Structure):
    _fields_ = [("w", qw_ref), ("scales", qw_ref), ("biases", qw_ref), ("group", _I)]


class qw_moe_layer(C.Structure):
    _fields_ = [("H", _I), ("E", _I), ("K", _I), ("I", _I), ("SI", _I),
                ("norm", _B), ("split", _B), ("router", qw_ref),
                ("gate_up", qw_q4_ref), ("gate", qw_q4_ref), ("up", qw_q4_ref),
                ("down", qw_q4_ref), ("sh_gate", qw_q4_ref), ("sh_up", qw_q4_ref),
                ("sh_down", qw_q4_ref), ("sh_gate_w", qw_ref)]


class qw_gdn_prep(C.Structure):
    _fields_ = [("a", qw_ref), ("b", qw_ref), ("A_log", qw_ref), ("dt_bias", qw_ref),
                ("l2eps", C.c_float), ("q_scale", C.c_float), ("k_scale", C.c_float)]


_R = qw_ref
_F = C.c_float


def _sig(name, res, *args):
    f = getattr(_lib, name)
    f.restype = res
    f.argtypes = list(args)
    globals()[name] = f
    return f


_sig("qw_gpu_init", _B, C.c_char_p, C.c_size_t)
_sig("qw_gpu_shutdown", None)
_sig("qw_gpu_name", C.c_char_p)
_sig("qw_gpu_working_set_limit", C.c_uint64)
_sig("qw_gpu_max_buffer_length", C.c_uint64)
_sig("qw_buf_wrap", _P, _P, C.c_size_t)
_sig("qw_buf_alloc", _P, C.c_size_t)
_sig("qw_buf_free", None, _P)
_sig("qw_buf_contents", _P, _P)
_sig("qw_buf_length", C.c_size_t, _P)
_sig("qw_cmd_begin", _P)
_sig("qw_cmd_commit", None, _P)
_sig("qw_cmd_wait", None, _P)
_sig("qw_cmd_flush", None, _P)
_sig("qw_cmd_parallel", None, _P, _B)
_sig("qw_cmd_free", None, _P)
_sig("qw_cmd_error", C.c_char_p, _P)
_sig("qw_residency_new", _P, _P, _I)
_sig("qw_residency_free", None, _P)
_sig("qw_prof_enabled", _B)
_sig("qw_cmd_mark", None, _P, C.c_char_p)
_sig("qw_prof_reset", None)
_sig("qw_prof_set_enabled", None, _B)
_sig("qw_prof_ms", C.c_double, C.c_char_p, C.POINTER(C.c_int64))
_sig("qw_prof_mark_times", _I, C.c_char_p, C.POINTER(C.c_float), _I)
# measurement probe (not a reference entry point): HBM read ceiling
_sig("qw_probe_read", _B, C.POINTER(qw_ref), C.POINTER(C.c_uint64), _I, _I, _I, C.c_uint64, C.POINTER(C.c_float))
_sig("qw_debug_decode_handoff_fail", _B)

_sig("qw_op_qmat_q4", None, _P, _R, _R, _R, _R, _R, _I, _I, _I, _I)
_sig("qw_op_qmv_q4", None, _P, _R, _R, _R, _R, _R, _I, _I, _I, _I)
_sig("qw_op_qmm_q4", None, _P, _R, _R, _R, _R, _R, _I, _I, _I, _I)
_sig("qw_op_qmvb_q4", None, _P, _R, _R, _R, _R, _R, _I, _I, _I, _I)
_sig("qw_op_qmv_q4_multi", _B, _P, _R, _I, _I, _I, C.POINTER(qw_qmv_part))
_sig("qw_op_dmat_bf16", None, _P, _R, _R, _R, _I, _I, _I)
_sig("qw_op_swiglu", None, _P, _R, _R, _R, _I)
_sig("qw_op_add_inplace", None, _P, _R, _R, _I)
_sig("qw_op_moe_combine_shared", None, _P, _R, _R, _R, _R, _R, _I, _I, _I)
_sig("qw_op_moe_route", None, _P, _R, _R, _R, _I, _I, _I, _B)
_sig("qw_op_qmv_q4_bank", None, _P, _R, _R, _R, _R, _R, _R, _I, _I, _I, _I, _B, _I)
_sig("qw_op_qmv_q4_bank2", _B, _P, _R, _R, _R, _R, _R, _R, _R, _R, _R, _I, _I, _I, _I, _I)
_sig("qw_op_qmv_q4_swiglu", None, _P, _R, _R, _R, _I, _R, _R, _R, _R, _I, _I, _I, _I)
_sig("qw_moe_max_tiles", _I, _I, _I)
_sig("qw_moe_tile_rows", _I, _I, _I)
_sig("qw_op_moe_group", None, _P, _R, _R, _R, _R, _I, _I)
_sig("qw_op_qmm_q4_gather", None, _P, _R, _R, _R, _R, _R, _R, _R, _I, _I, _I, _I, _I, _B, _I)
_sig("qw_op_swiglu_split", None, _P, _R, _R, _I, _I)
_sig("qw_op_moe_combine", None, _P, _R, _R, _R, _I, _I, _I)
_sig("qw_op_scale_rows_sigmoid", None, _P, _R, _R, _I, _I)
_sig("qw_checkpoint_open", _P, C.c_char_p, C.c_char_p, C.c_size_t)
_sig("qw_checkpoint_close", None, _P)
_sig("qw_checkpoint_layers", _I, _P)
_sig("qw_checkpoint_tensor", _B, _P, C.c_char_p, C.POINTER(_P), C.POINTER(C.c_size_t), C.POINTER(_I),
     C.POINTER(C.c_int64), C.c_char_p)
_sig("qw_moe_layer_load", _B, _P, _I, C.POINTER(qw_moe_layer), C.c_char_p, C.c_size_t)
_sig("qw_moe_layer_free", None, C.POINTER(qw_moe_layer))
_sig("qw_op_moe_layer", _B, _P, _R, _R, _R, _R, C.POINTER(qw_moe_layer), _I)
_sig("qw_op_moe_layer_noalloc", _B, _P, _R, _R, _R, _R, C.POINTER(qw_moe_layer), _I)
_sig("qw_op_moe_layer_residual", _B, _P, _R, _R, _R, _R, _R, _R, _R, C.POINTER(qw_moe_layer), _I, C.c_float)
_sig("qw_op_rms_norm", None, _P, _R, _R, _R, _I, _I, C.c_float, C.c_float)
_sig("qw_op_hc_inject_norm", None, _P, _R, _R, _R, _R, _R, _I, _I, _I, C.c_float)
_sig("qw_op_hc_pre_decode", _B, _P, _R, _R, _R, _R, _R, _R, _R, _R, _R, _R, _R, _R, _I, _I, _I, _I, C.c_float)
_sig("qw_op_hc_mix_up", _B, _P, _R, _R, _R, _R, _R, _R, _I, _I, _I, _I, C.c_float, _I)
_sig("qw_op_hc_decode", _B, _P, _R, _R, _R, _R, _R, _R, _R, _R, _R, _R, _R, _R, _R, _R, _R, _R, _I, _I, _I, _I, C.c_float, C.c_float)
_sig("qw_op_repeat_cols", None, _P, _R, _R, _I, _I, _I)
_sig("qw_op_rms_norm_grouped", None, _P, _R, _R, _R, _I, _I, _I, C.c_float)
_sig("qw_op_silu_scale", None, _P, _R, _I, C.c_float)
_sig("qw_op_hc_mix", None, _P, _R, _R, _R, _I, _I, _I)
_sig("qw_op_hc_inject", None, _P, _R, _R, _R, _I, _I, _I)
_sig("qw_op_residual_rms_norm_bf16", None, _P, _R, _R, _R, _I, _I, C.c_float)
_sig("qw_op_synth", None, _P, _R, _I, C.c_int64, C.c_uint64, C.c_float, C.c_float)
_sig("qw_op_conv1d_causal_silu", None, _P, _R, _R, _R, _R, _I, _I, _I, _R, _I, _I)
_sig("qw_op_gdn_gates", None, _P, _R, _R, _R, _R, _R, _R, _I, _I)
_sig("qw_op_gated_delta", None, _P, _R, _R, _R, _R, _R, _R, _R, _I, _I, _I, _I, _I, _R, _I, _I)
_sig("qw_op_gated_delta_prep", None, _P, _R, _R, _R, _R, C.POINTER(qw_gdn_prep), _R, _I, _I, _I, _I, _I, _R, _I,
     _I)
_sig("qw_op_gdn_decode", _B, _P, _R, _R, _R, _R, _R, C.POINTER(qw_gdn_prep), _R, _I, _I, _I, _I)
_sig("qw_op_rms_norm_gated_sigmoid", None, _P, _R, _R, _R, _R, _I, _I, _F, _F)
_sig("qw_op_qsa_scores", None, _P, _R, _R, _R, _R, _R, _I, _I, _I, _I, _I, _I, _I, _F)
_sig("qw_op_qsa_pool", None, _P, _R, _R, _R, _R, _I, _I, _I, _I, _I, _F)
_sig("qw_op_qsa_scores_pooled", None, _P, _R, _R, _R, _I, _I, _I, _I, _I, _I)
_sig("qw_op_qsa_select", None, _P, _R, _R, _R, _I, _I, _I, _I, _I, _I)
_sig("qw_op_attn_masked", None, _P, _R, _R, _R, _R, _R, _I, _I, _I, _I, _I, _I, _F, _I, _I)
_sig("qw_op_attn_masked_gated", None, _P, _R, _R, _R, _R, _R, _R, _I, _I, _I, _I, _I, _I, _F, _I, _I)


def qw_qsa_list_cap(block_topk: int, ratio: int) -> int:
    """The header's static inline (qwasar_gpu.h): entries after the count in
    one row of the selection's position list."""
    return block_topk * ratio + ratio


EXPORTED = [n for n in dir() if n.startswith(("qw_op_", "qw_buf_", "qw_cmd_", "qw_gpu_", "qw_prof_",
                                              "qw_residency_", "qw_moe_"))
            and callable(globals()[n])]


def init() -> None:
    err = C.create_string_buffer(256)
    if not qw_gpu_init(err, 256):
        raise RuntimeError(f"qw_gpu_init: {err.value.decode()}")


# ---- numpy convenience ---------------------------------------------------------

class Buf:
    """A qw_buf with numpy views of its host mirror.  Owns the buffer unless
    it wraps caller memory, in which case the array is kept alive here."""

    def __init__(self, nbytes: int = 0, wrap: np.ndarray | None = None):
        if wrap is not None:
            self._keep = np.ascontiguousarray(wrap)
            self.handle = qw_buf_wrap(self._keep.ctypes.data, self._keep.nbytes)
            self.nbytes = self._keep.nbytes
        else:
            self._keep = None
            self.handle = qw_buf_alloc(max(int(nbytes), 1))
            self.nbytes = int(nbytes)
        if not self.handle:
            raise MemoryError(f"qw_buf allocation of {self.nbytes} bytes failed")

    @classmethod
    def of(cls, a: np.ndarray) -> "Buf":
        b = cls(a.nbytes)
        b.write(a)
        return b

    def view(self, dtype, shape=None) -> np.ndarray:
        p = qw_buf_contents(self.handle)
        n = self.nbytes // np.dtype(dtype).itemsize
        arr = np.ctypeslib.as_array((C.c_byte * self.nbytes).from_address(p)).view(dtype)[:n]
        return arr.reshape(shape) if shape is not None else arr

    def write(self, a: np.ndarray, off_bytes: int = 0) -> None:
        a = np.ascontiguousarray(a)
        v = self.view(np.uint8)
        v[off_bytes:off_bytes + a.nbytes] = a.view(np.uint8).ravel()

    def read(self, dtype, shape) -> np.ndarray:
        return self.view(dtype).ravel()[:int(np.prod(shape))].reshape(shape).copy()

    def ref(self, off: int = 0) -> qw_ref:
        return qw_ref(self.handle, off)

    def free(self) -> None:
        if self.handle:
            qw_buf_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def run(c, label: str = "") -> None:
    """qw_cmd_wait + error check + free, as tests/test_sparse.c:50-54 does."""
    qw_cmd_wait(c)
    e = qw_cmd_error(c)
    qw_cmd_free(c)
    if e:
        raise RuntimeError(f"{label}: {e.decode()}")


class Q4Bufs:
    """Device copies of one qwasar_amd.synth.Q4."""

    def __init__(self, q):
        self.w, self.s, self.b = Buf(wrap=q.w), Buf(wrap=q.s), Buf(wrap=q.b)
        self.group = q.group

    def ref(self) -> qw_q4_ref:
        return qw_q4_ref(self.w.ref(), self.s.ref(), self.b.ref(), self.group)


class LayerBufs:
    """Device copies of a qwasar_amd.synth.MoeLayer and its qw_moe_layer."""

    def __init__(self, L):
        self.L = L
        self.router = Buf(wrap=L.router)
        self.sh_gate_w = Buf(wrap=L.sh_gate_w)
        self.q = {}
        for name in ("gate_up", "gate", "up", "down", "sh_gate", "sh_up", "sh_down"):
            t = getattr(L, name)
            self.q[name] = Q4Bufs(t) if t is not None else None
        empty = qw_q4_ref(NULL_REF, NULL_REF, NULL_REF, 0)
        self.desc = qw_moe_layer(
            L.H, L.E, L.K, L.I, L.SI, bool(L.norm), bool(L.split), self.router.ref(),
            *[self.q[n].ref() if self.q[n] else empty
              for n in ("gate_up", "gate", "up", "down", "sh_gate", "sh_up", "sh_down")],
            self.sh_gate_w.ref())

    def free(self):
        self.router.free()
        self.sh_gate_w.free()
        for q in self.q.values():
            if q:
                q.w.free(); q.s.free(); q.b.free()
