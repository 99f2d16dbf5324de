"""The C-ABI library without a GPU: it loads, exports every function that
include/qwasar_gpu.h declares, and honours the reference's host-side
conventions (NULL command -> nothing encoded; bool ops' shape answers)."""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qwasar_gpu.h")


def declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = set()
    for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b(qw_\w+)\s*\(", src, flags=re.M):
        line = src[m.start():src.index("\n", m.start())]
        if "static inline" in line or line.lstrip().startswith("typedef"):
            continue
        names.add(m.group(1))
    return sorted(names)


def test_header_declares_the_moe_boundary():
    names = declared()
    for n in ("qw_gpu_init", "qw_buf_alloc", "qw_cmd_begin", "qw_op_moe_route", "qw_op_qmv_q4_bank",
              "qw_op_qmv_q4_bank2", "qw_op_qmv_q4_swiglu", "qw_op_moe_group", "qw_op_qmm_q4_gather",
              "qw_op_moe_combine_shared", "qw_op_dmat_bf16", "qw_op_qmat_q4", "qw_op_moe_layer"):
        assert n in names


def test_library_exports_every_declared_function():
    from qwasar_amd import gpu
    lib = C.CDLL(gpu.LIB_PATH)
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_null_command_encodes_nothing():
    from qwasar_amd import gpu
    r = gpu.NULL_REF
    # void ops return at once with no command (reference QW_BEGIN, qwasar_metal.m:1606-1611)
    gpu.qw_op_swiglu(None, r, r, r, 10)
    gpu.qw_op_qmv_q4_bank(None, r, r, r, r, r, r, 64, 8, 1, 1, False, 64)
    gpu.qw_op_moe_group(None, r, r, r, r, 4, 4)
    # bool ops still answer whether the shape applies
    assert not gpu.qw_op_qmv_q4_bank2(None, r, r, r, r, r, r, r, r, r, 1024, 8, 1, 1, 64)
    assert gpu.qw_op_qmv_q4_bank2(None, r, r, r, r, r, r, r, r, r, 2048, 8, 1, 1, 64)
    assert not gpu.qw_op_qmv_q4_multi(None, r, 2048, 64, 5, None)
    assert not gpu.qw_op_qmv_q4_multi(None, r, 1024, 64, 2, None)   # too short to take (reference :105-107)
    assert gpu.qw_op_qmv_q4_multi(None, r, 2048, 64, 2, None)


def test_tile_bounds():
    from qwasar_amd import gpu
    from oracle import ref
    for pairs, E in ((5120, 512), (20480, 512), (10, 16), (80, 512)):
        bm = gpu.qw_moe_tile_rows(pairs, E)
        assert bm in (16, 32, 64)
        assert ref.max_tiles(pairs, E, bm) <= gpu.qw_moe_max_tiles(pairs, E)
    assert gpu.qw_moe_tile_rows(20480, 512) == 64
    assert gpu.qw_moe_tile_rows(5120, 512) == 16


def test_init_reports_a_missing_gpu():
    from qwasar_amd import gpu
    err = C.create_string_buffer(256)
    if gpu.qw_gpu_init(err, 256):
        pytest.skip("a gfx950 GPU is present")
    assert err.value


def test_hc_pre_decode_refuses_overlaps():
    """No output of qw_op_hc_pre_decode may share a byte with an input or with
    another output (its workgroups read every input while others write);
    checked on the shape alone, with no command and no device."""
    from qwasar_amd import gpu
    H, S, lr = 256, 4, 32
    HH = S * H
    A, B = 0x1000, 0x2000          # two stand-in buffer handles, never dereferenced
    r = lambda buf, off=0: gpu.qw_ref(buf, off)
    N = gpu.NULL_REF

    def call(h4_out, n4, d, inj_out, h4, out, inj):
        return gpu.qw_op_hc_pre_decode(None, h4_out, n4, d, inj_out, h4, out, inj, N, N, N, N, N,
                                       H, S, lr, 64, 1e-6)

    # outputs laid end to end in A, inputs in B: accepted
    o = [0, 4 * HH, 8 * HH, 8 * HH + 4 * lr]
    i = [0, 4 * HH, 4 * HH + 4 * H]
    ok = dict(h4_out=r(A, o[0]), n4=r(A, o[1]), d=r(A, o[2]), inj_out=r(A, o[3]),
              h4=r(B, i[0]), out=r(B, i[1]), inj=r(B, i[2]))
    assert call(**ok)
    for name, bad in (("n4", r(B, 4 * HH - 4)),          # n4's first float is h4's last
                      ("d", r(B, 4 * HH + 4 * H - 8)),   # d over out's tail
                      ("inj_out", r(B, i[2])),           # inj_out is inj
                      ("h4_out", r(B, 16)),              # h4_out inside h4
                      ("n4", r(A, o[0] + 4 * HH - 4))):  # two outputs sharing a float
        args = dict(ok)
        args[name] = bad
        assert not call(**args), name


def test_c_caller_compiles_as_c99():
    """include/qwasar_gpu.h and the C caller of the boundary are plain C99
    (gcc -std=c99 -pedantic -Werror), as the reference's C drivers need."""
    import subprocess
    here = os.path.dirname(os.path.abspath(__file__))
    src = os.path.join(here, "c_boundary", "encode_moe.c")
    inc = os.path.join(os.path.dirname(here), "include")
    r = subprocess.run(["gcc", "-std=c99", "-pedantic", "-Wall", "-Wextra", "-Werror", "-fsyntax-only",
                        "-I", inc, src], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_gdn_decode_refuses_overlapping_windows():
    """qw_op_gdn_decode's window out may not share a byte with the window in
    or with x (its workgroups read the old window while one writes the new);
    checked on the shape alone, with no command and no device."""
    from qwasar_amd import gpu
    hk, hv, d = 2, 4, 128
    ch = 2 * hk * d + hv * d
    A, B = 0x1000, 0x2000          # two stand-in buffer handles, never dereferenced
    r = lambda buf, off=0: gpu.qw_ref(buf, off)
    N = gpu.NULL_REF
    prep = gpu.qw_gdn_prep(N, N, N, N, 1e-6, 1.0, 1.0)

    def call(x, win, wout, dk=d):
        return gpu.qw_op_gdn_decode(None, N, x, win, wout, N, prep, N, hk, hv, dk, d)

    assert call(r(B), r(A), r(A, 12 * ch))
    assert not call(r(B), r(A), r(A, 12 * ch - 4)), "window out over the window in's tail"
    assert not call(r(B), r(A), r(B, 4 * ch - 4)), "window out over x"
    assert not call(r(B), r(A), r(A)), "the same window"
    assert not call(r(B), r(A), r(A, 12 * ch), dk=64), "head dims other than 128"
