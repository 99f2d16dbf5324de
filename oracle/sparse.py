"""numpy-level access to the QSA and gated-DeltaNet oracle (sparse_ref.c in
libmoe_ref.so) and to the reference's own scalar twins of the same ops
(qwasar_cpu.c, compiled into _ref/ where the reference tree was present).

TEST INFRASTRUCTURE ONLY: imported by tests/, never by the product package.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import ref

_P = C.c_void_p
_I = C.c_int32
_F = C.c_float
_done = set()


def _lib():
    L = ref.lib()
    if "lib" not in _done:
        L.qr_f16_to_f32.restype = _F
        L.qr_f16_to_f32.argtypes = [C.c_uint16]
        L.qr_rope_tables.argtypes = [_P, _P, _I, _F, _P]
        L.qr_rope_at.argtypes = [_P, _I, _P, _I, _I, _I]
        L.qr_qsa_block_key.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I, _F]
        L.qr_qsa_scores.argtypes = [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F]
        L.qr_qsa_pool.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I, _I, _F]
        L.qr_qsa_scores_pooled.argtypes = [_P, _P, _P, _I, _I, _I, _I, _I, _I]
        L.qr_qsa_select.argtypes = [_P, _P, _P, _I, _I, _I, _I, _I, _I]
        L.qr_attn_masked.argtypes = [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I]
        L.qr_conv1d_causal_silu.argtypes = [_P, _P, _P, _P, _I, _I, _I, _P, _I, _I]
        L.qr_gdn_gates.argtypes = [_P, _P, _P, _P, _P, _P, _I, _I]
        L.qr_gated_delta.argtypes = [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _I, _I]
        L.qr_gated_delta_prep.argtypes = [_P, _P, _P, _P, _P, _P, _P, _P, _F, _F, _F, _P,
                                          _I, _I, _I, _I, _I, _P, _I, _I]
        L.qr_rms_norm_gated_sigmoid.argtypes = [_P, _P, _P, _P, _I, _I, _F, _F]
        _done.add("lib")
    return L


def reflib():
    R = ref.reflib()
    if R is not None and "ref" not in _done:
        R.qw_rope_tables.argtypes = [_P, _P, _I, _F, _P]
        R.qw_cpu_rope_partial.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I]
        R.qw_cpu_conv1d_causal_silu.argtypes = [_P, _P, _P, _P, _I, _I, _I]
        R.qw_cpu_gdn_gates.argtypes = [_P, _P, _P, _P, _P, _P, _I, _I]
        R.qw_cpu_gated_delta.argtypes = [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I]
        R.qw_cpu_attn_decode.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F]
        R.qw_cpu_kv_write.argtypes = [_P, _P, _P, _P, _I, _I, _I, _I, _I]
        R.qw_f16_to_f32_c.restype = _F
        R.qw_f16_to_f32_c.argtypes = [C.c_uint16]
        _done.add("ref")
    return R


def _p(a):
    return None if a is None else ref._ptr(a)


def _f32(a):
    return np.ascontiguousarray(a, np.float32)


def list_cap(block_topk: int, ratio: int) -> int:
    """Entries after the count in one row of the selection's position list
    (qwasar_gpu.h:637-639)."""
    return block_topk * ratio + ratio


def rope_tables(rotary_dim, theta, section):
    axis = np.zeros(max(rotary_dim // 2, 1), np.uint8)
    inv = np.zeros(max(rotary_dim // 2, 1), np.float32)
    sec = np.ascontiguousarray(section, np.int32)
    _lib().qr_rope_tables(_p(axis), _p(inv), rotary_dim, theta, _p(sec))
    return axis, inv


def qsa_scores(qn, ikeys, k_norm, inv_freq, rows, nq, d, ratio, base_pos, rotary_dim, max_blocks, eps):
    sc = np.zeros((rows, max_blocks), np.float32)
    qn, ikeys, inv_freq = _f32(qn), _f32(ikeys), _f32(inv_freq)
    _lib().qr_qsa_scores(_p(sc), _p(qn), _p(ikeys), _p(k_norm), _p(inv_freq), rows, nq, d, ratio, base_pos,
                         rotary_dim, max_blocks, eps)
    return sc


def qsa_pool(pool, ikeys, k_norm, inv_freq, d, ratio, b0, b1, rotary_dim, eps):
    ikeys, inv_freq = _f32(ikeys), _f32(inv_freq)
    _lib().qr_qsa_pool(_p(pool), _p(ikeys), _p(k_norm), _p(inv_freq), d, ratio, b0, b1, rotary_dim, eps)
    return pool


def block_key(ikeys, k_norm, inv_freq, b, d, ratio, rotary_dim, eps):
    kn = np.zeros(d, np.float32)
    _lib().qr_qsa_block_key(_p(kn), _p(_f32(ikeys)), _p(k_norm), _p(_f32(inv_freq)), b, d, ratio,
                            rotary_dim, eps)
    return kn


def qsa_scores_pooled(qn, pool, rows, nq, d, ratio, base_pos, max_blocks):
    sc = np.zeros((rows, max_blocks), np.float32)
    _lib().qr_qsa_scores_pooled(_p(sc), _p(_f32(qn)), _p(_f32(pool)), rows, nq, d, ratio, base_pos, max_blocks)
    return sc


def qsa_select(scores, rows, ratio, base_pos, block_topk, max_ctx, max_blocks):
    mask = np.zeros((rows, max_ctx), np.uint8)
    lst = np.zeros((rows, 1 + list_cap(block_topk, ratio)), np.uint32)
    _lib().qr_qsa_select(_p(mask), _p(lst), _p(_f32(scores)), rows, ratio, base_pos, block_topk, max_ctx,
                         max_blocks)
    return mask, lst


def attn_masked(q, kc, vc, lst, rows, q_heads, kv_heads, head_dim, max_ctx, scale, cap, gate=None):
    out = np.zeros((rows, q_heads, head_dim), np.float32)
    g = None if gate is None else _f32(gate)
    _lib().qr_attn_masked(_p(out), _p(g), _p(_f32(q)), _p(kc), _p(vc), _p(np.ascontiguousarray(lst, np.uint32)),
                          rows, q_heads, kv_heads, head_dim, max_ctx, scale, cap)
    return out


def conv1d_causal_silu(x, state, w, channels, rows, ksize, n_snap=0):
    """Returns (y, new state, snapshots [n_snap, ksize-1, channels])."""
    y = np.zeros((rows, channels), np.float32)
    st = _f32(state).copy()
    stride = (ksize - 1) * channels
    snap = np.zeros((max(n_snap, 1), ksize - 1, channels), np.float32)
    _lib().qr_conv1d_causal_silu(_p(y), _p(_f32(x)), _p(st), _p(w), channels, rows, ksize, _p(snap), n_snap, stride)
    return y, st, snap[:n_snap]


def gdn_gates(a, b, A_log, dt_bias, hv, rows):
    g = np.zeros((rows, hv), np.float32)
    beta = np.zeros((rows, hv), np.float32)
    _lib().qr_gdn_gates(_p(g), _p(beta), _p(_f32(a)), _p(_f32(b)), _p(A_log), _p(dt_bias), hv, rows)
    return g, beta


def gated_delta(q, k, v, g, beta, state, hk, hv, dk, dv, rows, n_snap=0):
    """Returns (y [rows, hv, dv], new state, snapshots [n_snap, hv, dv, dk])."""
    y = np.zeros((rows, hv, dv), np.float32)
    st = _f32(state).copy()
    snap = np.zeros((max(n_snap, 1), hv, dv, dk), np.float32)
    _lib().qr_gated_delta(_p(y), _p(_f32(q)), _p(_f32(k)), _p(_f32(v)), _p(_f32(g)), _p(_f32(beta)), _p(st),
                          hk, hv, dk, dv, rows, _p(snap), n_snap, hv * dv * dk)
    return y, st, snap[:n_snap]


def gated_delta_prep(q, k, v, a, b, A_log, dt_bias, l2eps, q_scale, k_scale, state, hk, hv, dk, dv, rows,
                     n_snap=0):
    y = np.zeros((rows, hv, dv), np.float32)
    st = _f32(state).copy()
    snap = np.zeros((max(n_snap, 1), hv, dv, dk), np.float32)
    _lib().qr_gated_delta_prep(_p(y), _p(_f32(q)), _p(_f32(k)), _p(_f32(v)), _p(_f32(a)), _p(_f32(b)),
                               _p(A_log), _p(dt_bias), l2eps, q_scale, k_scale, _p(st), hk, hv, dk, dv, rows,
                               _p(snap), n_snap, hv * dv * dk)
    return y, st, snap[:n_snap]


def rms_norm_gated_sigmoid(x, w, gate, dim, rows, eps, out_scale=1.0):
    y = np.zeros((rows, dim), np.float32)
    _lib().qr_rms_norm_gated_sigmoid(_p(y), _p(_f32(x)), _p(w), _p(_f32(gate)), dim, rows, eps, out_scale)
    return y


def f16_bits(a) -> np.ndarray:
    """fp32 -> fp16 bit patterns, round to nearest even (numpy's cast)."""
    return np.ascontiguousarray(np.asarray(a, np.float32).astype(np.float16)).view(np.uint16)
