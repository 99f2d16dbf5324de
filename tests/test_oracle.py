"""Pins the CPU oracle (oracle/moe_ref.c) before anything is held to it.

Each function is checked against something independent of its own code: the
reference's own scalar twins compiled from /root/reference/qwasar_cpu.c
(oracle/_ref, bit-exact), hand-built vectors with known answers, fp64 brute
force, closed forms and invariants -- chosen so a plausible slip (a dropped
term, a wrong index, a swapped operand, a different summation order) fails
one of them."""
import math
import os

import numpy as np
import pytest

from oracle import ref
from qwasar_amd import synth
from tests.fixture_layers import layer_from_npz

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
P = ref._ptr


def need_ref():
    R = ref.reflib()
    if R is None:
        pytest.skip("oracle/_ref (the reference's qwasar_cpu.c) is not built here")
    return R


# ---- bf16 and dequantisation ------------------------------------------------------

def test_bf16_all_patterns_match_reference():
    R = need_ref()
    L = ref.lib()
    for v in range(0, 65536, 7):
        a, b = L.qr_bf16_to_f32(v), R.qw_bf16_to_f32_c(v)
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32) or (math.isnan(a) and math.isnan(b))


def test_dequant_hand_vectors():
    # nibbles 0..7 in word 0, 8..15 in word 1: element i at bit 4*(i%8)
    w = np.array([[0x76543210, 0xFEDCBA98]], np.uint32)
    one, zero = synth.to_bf16(np.float32(1.0)), synth.to_bf16(np.float32(0.0))
    s = np.array([[one]], np.uint16)
    b = np.array([[zero]], np.uint16)
    out = np.zeros(16, np.float32)
    # group 16 here: one scale/bias for the row
    ref.lib().qr_dequant_row(P(out), P(w), P(s), P(b), 16, 0, 16)
    assert list(out) == list(range(16))
    # bias = -8 * scale: symmetric about zero
    sc = np.float32(0.0078125)
    s[0, 0] = synth.to_bf16(sc)
    b[0, 0] = synth.to_bf16(-8 * sc)
    ref.lib().qr_dequant_row(P(out), P(w), P(s), P(b), 16, 0, 16)
    assert np.array_equal(out, (np.arange(16) - 8).astype(np.float32) * sc)


@pytest.mark.parametrize("G", [64, 32])
def test_qmv_bit_exact_against_reference(G):
    R = need_ref()
    k, n, rows = 512, 48, 3
    q = synth.make_q4(3 + G, "w", n, k, G)
    x = synth.normal(9, "x", rows * k).astype(np.float32).reshape(rows, k)
    got = ref.qmv_q4(x, q.w, q.s, q.b, k, n, rows, G)
    want = np.zeros((rows, n), np.float32)
    R.qw_cpu_qmv_q4(P(want), P(x), P(q.w), P(q.s), P(q.b), k, n, rows, G)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # and close to an fp64 product of the dequantised matrix
    exact = x.astype(np.float64) @ q.dequant().astype(np.float64).T
    assert np.abs(got - exact).max() / np.abs(exact).max() < 1e-5


@pytest.mark.parametrize("name", ["tiny_q4_layer0.npz", "tiny_mlx_layer0.npz"])
def test_fixture_banks_dequant_against_reference(name):
    """The reference's toy checkpoints' real banks, row by row."""
    R = need_ref()
    L = layer_from_npz(os.path.join(GOLD, name))
    for q in (L.gate_up, L.gate, L.down, L.sh_down):
        if q is None:
            continue
        for row in (0, q.rows // 2, q.rows - 1):
            a = np.zeros(q.cols, np.float32)
            b = np.zeros(q.cols, np.float32)
            ref.lib().qr_dequant_row(P(a), P(q.w), P(q.s), P(q.b), q.cols, row, q.group)
            R.qw_cpu_dequant_row(P(b), P(q.w), P(q.s), P(q.b), q.cols, row, q.group)
            assert np.array_equal(a, b)
            assert np.array_equal(a, q.dequant(row, 1)[0])


# ---- the specified exponential ------------------------------------------------------

def test_exp_within_two_ulp():
    x = np.linspace(-103.9, 88.7, 400001, dtype=np.float32)
    x = np.concatenate([x, -np.geomspace(1e-8, 30, 2001).astype(np.float32),
                        np.geomspace(1e-8, 30, 2001).astype(np.float32)])
    got = ref.exp_vec(x)
    want = np.exp(x.astype(np.float64))
    normal = want > 1.2e-38
    ulp = np.spacing(want[normal].astype(np.float32)).astype(np.float64)
    err = np.abs(got[normal].astype(np.float64) - want[normal]) / ulp
    assert err.max() <= 2.0, f"max error {err.max():.2f} ulp"
    # subnormal results: absolute error within 2 subnormal ulps
    sub = ~normal
    assert np.abs(got[sub].astype(np.float64) - want[sub]).max() <= 2 * 2.0 ** -149
    assert ref.lib().qr_exp(0.0) == 1.0
    assert ref.lib().qr_exp(-200.0) == 0.0
    assert math.isinf(ref.lib().qr_exp(89.0))
    assert np.all(np.diff(got[:400001]) >= 0), "not monotone"


# ---- order R ---------------------------------------------------------------------

def dot(w, x):
    w = np.ascontiguousarray(w, np.uint16)
    x = np.ascontiguousarray(x, np.float32)
    return ref.lib().qr_dot_bf16(P(w), P(x), x.size)


def test_order_r_chunks_then_left_to_right():
    """2^24 in chunk 0, then 1 + 1 in chunk 1: order R adds the chunk
    partial 2 to 2^24 (exact); a serial sum loses both ones to rounding."""
    k = 128
    w = np.zeros(k, np.uint16)
    x = np.zeros(k, np.float32)
    w[[0, 64, 65]] = synth.to_bf16(np.array([1.0], np.float32))[0]
    x[0], x[64], x[65] = 2.0 ** 24, 1.0, 1.0
    assert dot(w, x) == 2.0 ** 24 + 2.0
    R = ref.reflib()
    if R is not None:
        y = np.zeros(1, np.float32)
        R.qw_cpu_dmv_bf16(P(y), P(x), P(w), k, 1, 1)
        assert y[0] == 2.0 ** 24


def test_order_r_partials_are_fused():
    """Within a chunk each step is an fma: -1 + (1+2^-7)(1+2^-23) keeps its
    2^-30 term, which an unfused multiply-then-add would drop."""
    w = synth.to_bf16(np.array([-1.0, 1.0 + 2.0 ** -7], np.float32))
    x = np.array([1.0, 1.0 + 2.0 ** -23], np.float32)
    assert dot(w, x) == np.float32(2.0 ** -7 + 2.0 ** -23 + 2.0 ** -30)


def test_order_r_close_to_brute_force_and_reference():
    k, n = 3072, 64
    w = synth.to_bf16(synth.normal(1, "w", n * k, 0.02).astype(np.float32)).reshape(n, k)
    x = synth.bf16_round(synth.normal(2, "x", k).astype(np.float32))[None]
    got = ref.dmat_bf16(x, w, k, n, 1)[0]
    exact = synth.bf16_to_f32(w).astype(np.float64) @ x[0].astype(np.float64)
    bound = 3072 * 2.0 ** -24 * (np.abs(synth.bf16_to_f32(w)).astype(np.float64) @ np.abs(x[0]))
    assert np.all(np.abs(got - exact) <= bound)
    R = ref.reflib()
    if R is not None:
        y = np.zeros(n, np.float32)
        R.qw_cpu_dmv_bf16(P(y), P(x), P(w), k, n, 1)
        assert np.all(np.abs(got - y) <= 2 * bound)


# ---- routing ----------------------------------------------------------------------

@pytest.mark.parametrize("E,K", [(16, 4), (512, 10), (1000, 32), (8, 8)])
def test_route_matches_full_sort(E, K):
    rows = 16
    lg = synth.normal(E + K, "lg", rows * E, 2.0).astype(np.float32).reshape(rows, E)
    idx, w = ref.route(lg, rows, E, K)
    for r in range(rows):
        order = np.lexsort((np.arange(E), -lg[r].astype(np.float64)))
        assert list(idx[r]) == list(order[:K])
        assert len(set(idx[r])) == K
        assert np.all(np.diff(w[r]) <= 0)
        assert abs(float(w[r].astype(np.float64).sum()) - 1.0) <= K * 2.0 ** -23
        p = np.exp(lg[r].astype(np.float64) - lg[r].max())
        p /= p.sum()
        want = p[idx[r]] / p[idx[r]].sum()
        assert np.allclose(w[r], want, rtol=1e-5, atol=1e-7)
    li, lw = ref.route(lg, rows, E, K, literal=True)
    assert np.array_equal(idx, li)
    assert np.allclose(w, lw, rtol=1e-5, atol=1e-7)


def test_route_ties_and_norm():
    E, K = 64, 5
    lg = np.zeros((2, E), np.float32)
    lg[1, [9, 3, 40]] = 1.0
    idx, w = ref.route(lg, 2, E, K)
    assert list(idx[0]) == [0, 1, 2, 3, 4]
    assert np.allclose(w[0], 1.0 / K)
    assert list(idx[1]) == [3, 9, 40, 0, 1]
    _, wn = ref.route(lg, 2, E, K, norm=False)
    assert np.allclose(wn[0], 1.0 / E)


# ---- the dispatch permutation -------------------------------------------------------

@pytest.mark.parametrize("pairs,E,bm", [(2560, 64, 16), (20480, 512, 64), (37, 16, 32), (1, 8, 16), (0, 4, 16)])
def test_group_is_stable_sort_with_tiles(pairs, E, bm):
    r = synth.raw64(pairs + E, "g", max(pairs, 1))[:pairs]
    idx = np.where(r % np.uint64(5) < np.uint64(2), 0, (r >> np.uint64(8)) % np.uint64(E)).astype(np.int32)
    perm, tiles = ref.moe_group(idx, E, bm)
    assert np.array_equal(perm, np.argsort(idx, kind="stable"))
    nt = int(tiles[0])
    assert nt <= ref.max_tiles(pairs, E, bm)
    pos = 0
    for t in range(nt):
        e, s, ln = tiles[1 + 3 * t:4 + 3 * t]
        assert s == pos and 1 <= ln <= bm
        assert np.all(idx[perm[s:s + ln]] == e)
        pos += ln
    assert pos == pairs
    counts = np.bincount(idx, minlength=E)
    assert nt == int(np.sum((counts + bm - 1) // bm))


# ---- the whole block -----------------------------------------------------------------

def fp64_layer(L, x, idx, w):
    """fp64 restatement of qwasar_flash_cpu.c:524-552 on dequantised weights."""
    sig = lambda v: 1.0 / (1.0 + np.exp(-v))
    out = np.zeros((x.shape[0], L.H))
    for r in range(x.shape[0]):
        xr = x[r].astype(np.float64)
        for n in range(L.K):
            e = int(idx[r, n])
            if L.split:
                g = L.gate.dequant(e * L.I, L.I) @ xr
                u = L.up.dequant(e * L.I, L.I) @ xr
            else:
                gu = L.gate_up.dequant(e * 2 * L.I, 2 * L.I) @ xr
                g, u = gu[:L.I], gu[L.I:]
            act = g * sig(g) * u
            out[r] += float(w[r, n]) * (L.down.dequant(e * L.H, L.H).astype(np.float64) @ act)
        sg = L.sh_gate.dequant() @ xr
        su = L.sh_up.dequant() @ xr
        sh = L.sh_down.dequant().astype(np.float64) @ (sg * sig(sg) * su)
        gate = synth.bf16_to_f32(L.sh_gate_w).astype(np.float64) @ xr
        out[r] += sig(gate) * sh
    return out


@pytest.mark.parametrize("split", [True, False])
def test_forward_against_fp64(split):
    L, x = synth.make_config(0, split=split, rows=3, seed=5)
    out, idx, w = ref.moe_forward(L, x)
    want = fp64_layer(L, x, idx, w)
    assert np.sqrt(((out - want) ** 2).sum() / (want ** 2).sum()) < 1e-5
    logits = ref.dmat_bf16(x, L.router, L.H, L.E, 3)
    i2, w2 = ref.route(logits, 3, L.E, L.K)
    assert np.array_equal(idx, i2) and np.array_equal(w, w2)


def test_fixture_layer_against_fp64():
    L = layer_from_npz(os.path.join(GOLD, "tiny_mlx_layer0.npz"))
    x = synth.make_x(3, 4, L.H)
    out, idx, w = ref.moe_forward(L, x)
    want = fp64_layer(L, x, idx, w)
    assert np.sqrt(((out - want) ** 2).sum() / (want ** 2).sum()) < 1e-5


def test_golden_regression():
    g = np.load(os.path.join(GOLD, "c0_golden.npz"))
    L, x = synth.make_config(0)
    assert np.array_equal(x, g["c0_x"]), "synthetic generator changed"
    out, idx, w = ref.moe_forward(L, x)
    assert np.array_equal(idx, g["c0_idx"]) and np.array_equal(w, g["c0_w"])
    assert np.array_equal(out, g["c0_out"])
    for tag, name in (("q4", "tiny_q4_layer0.npz"), ("mlx", "tiny_mlx_layer0.npz")):
        TL = layer_from_npz(os.path.join(GOLD, name))
        o, i, ww = ref.moe_forward(TL, g[f"{tag}_x"])
        assert np.array_equal(i, g[f"{tag}_idx"]) and np.array_equal(o, g[f"{tag}_out"])
