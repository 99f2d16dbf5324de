"""QSA (block scores, stored keys, selection, masked attention) and the gated
DeltaNet (conv, gates, delta rule, prep, output gate) on the GPU, through the
C ABI, against the CPU oracle (oracle/sparse_ref.c, pinned in
tests/test_oracle_sparse.py).  The cases follow the reference's own tests
(tests/test_sparse.c:348-470,562-620,887-915; tests/test_gdn.c) with the toy
checkpoint's weights and shapes, then the full model's shapes.

Bars, written per test:
- selection: bit-exact (mask and position list) on the same scores;
- scores: |diff| <= 1e-5 * (1 + |score|) -- the GPU sums the rms norm and the
  head dots in another order than the oracle's serial loops, and rounds the
  rotation as one fma; stored-key scores bit-identical to direct scores;
- attention: 2e-6 absolute on O(1) outputs (online softmax in chunks of 256
  against the oracle's two-pass form);
- delta rule: rel-L2 5e-6 on outputs and state (the reference's own bar,
  tests/test_gdn.c:197-198), and a run of single steps bit-identical to one
  batched call;
- conv, gates, output gate: 2e-6 relative (fma and the device's expf)."""
import os

import numpy as np
import pytest

from oracle import sparse
from qwasar_amd import synth

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FX = dict(np.load(os.path.join(GOLD, "tiny_q4_sparse.npz")))
EPS = float(FX["eps"])


def rnd(shape, seed, lo=-1.0, hi=1.0):
    return np.random.default_rng(seed).uniform(lo, hi, shape).astype(np.float32)


def rel_l2(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.sqrt(((a - b) ** 2).sum() / max((b * b).sum(), 1e-300)))


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def rope_inv():
    _, inv = sparse.rope_tables(int(FX["rotary_dim"]), float(FX["rope_theta"]), FX["mrope_section"])
    return inv


# ---- QSA scores ------------------------------------------------------------------

def gpu_scores(gpu, qn, ikeys, kw, inv, rows, nq, d, ratio, base, max_blocks, pooled=False):
    B = gpu.Buf
    qb, kb, wb, ib = B.of(qn), B.of(ikeys), B.of(np.ascontiguousarray(kw)), B.of(inv)
    sb = B.of(np.full((rows, max_blocks), np.nan, np.float32))
    c = gpu.qw_cmd_begin()
    if pooled:
        pb = B(max_blocks * d * 4)
        allb = (base + rows) // ratio
        gpu.qw_op_qsa_pool(c, pb.ref(), kb.ref(), wb.ref(), ib.ref(), d, ratio, 0, allb // 2, 64, EPS)
        gpu.qw_op_qsa_pool(c, pb.ref(), kb.ref(), wb.ref(), ib.ref(), d, ratio, allb // 2, allb, 64, EPS)
        gpu.qw_op_qsa_scores_pooled(c, sb.ref(), qb.ref(), pb.ref(), rows, nq, d, ratio, base, max_blocks)
    else:
        gpu.qw_op_qsa_scores(c, sb.ref(), qb.ref(), kb.ref(), wb.ref(), ib.ref(), rows, nq, d, ratio, base, 64,
                             max_blocks, EPS)
    gpu.run(c, "qsa scores")
    out = sb.read(np.float32, (rows, max_blocks))
    pool = pb.read(np.float32, (max_blocks, d)) if pooled else None
    return out, pool


@pytest.mark.parametrize("rows,base,max_ctx,d", [(5, 13, 64, 128), (3, 4000, 4096, 128), (40, 0, 64, 128),
                                                 (2, 700, 1024, 256), (9, 130, 256, 96)])
def test_qsa_scores_and_pooled(gpu, rows, base, max_ctx, d):
    """The reference's case (tests/test_sparse.c:348-421: 5 rows at 13, 64
    keys), a long context, a prefill from position 0 and the widest and an
    odd head size; then the same scores from keys stored in two stretches."""
    nq, ratio = int(FX["nq"]), int(FX["ratio"])
    mb = max_ctx // ratio
    kw = FX["k_norm"] if d == 128 else synth.to_bf16(1.0 + 0.1 * rnd(d, d))
    qn, ik, inv = rnd((rows, nq, d), 51 + d), rnd((max_ctx, d), 52 + d), rope_inv()
    got, _ = gpu_scores(gpu, qn, ik, kw, inv, rows, nq, d, ratio, base, mb)
    want = sparse.qsa_scores(qn, ik, kw, inv, rows, nq, d, ratio, base, 64, mb, EPS)
    for r in range(rows):
        nb = (base + r + 1) // ratio
        assert np.all(np.abs(got[r, :nb] - want[r, :nb]) <= 1e-5 * (1 + np.abs(want[r, :nb]))), f"row {r}"
        assert np.isnan(got[r, nb:]).all(), "entries past the row's complete blocks are left alone"
    got2, pool = gpu_scores(gpu, qn, ik, kw, inv, rows, nq, d, ratio, base, mb, pooled=True)
    for r in range(rows):
        nb = (base + r + 1) // ratio
        assert same_bits(got2[r, :nb], got[r, :nb]), f"pooled row {r}"
    allb = (base + rows) // ratio
    wp = np.zeros((mb, d), np.float32)
    sparse.qsa_pool(wp, ik, kw, inv, d, ratio, 0, allb, 64, EPS)
    assert np.allclose(pool[:allb], wp[:allb], rtol=1e-5, atol=1e-6)


# ---- selection -------------------------------------------------------------------

@pytest.mark.parametrize("nq,d,base,rows", [(16, 128, 4000, 48), (12, 96, 130, 40), (16, 64, 0, 33)])
@pytest.mark.parametrize("pooled", [False, True])
def test_qsa_scores_matrix_cores_match_rowwise(gpu, nq, d, base, rows, pooled):
    """From 16 rows on (nq <= 16, d <= 128) the scores run on the fp32 matrix
    cores; one row at a time they take the per-thread fma chains.  Both are
    the same chain of fmas per head, so every score agrees bit for bit:
    rows that straddle block boundaries, a ragged last row group, fewer heads
    than the instruction's rows and a head size under 128."""
    ratio = int(FX["ratio"])
    mb = (base + rows) // ratio + 3
    kw = FX["k_norm"] if d == 128 else synth.to_bf16(1.0 + 0.1 * rnd(d, d + nq))
    qn, ik, inv = rnd((rows, nq, d), 61 + d), rnd((mb * ratio, d), 62 + d), rope_inv()
    got, _ = gpu_scores(gpu, qn, ik, kw, inv, rows, nq, d, ratio, base, mb, pooled=pooled)
    assert rows >= 16
    for r in range(rows):
        one, _ = gpu_scores(gpu, qn[r:r + 1], ik, kw, inv, 1, nq, d, ratio, base + r, mb, pooled=pooled)
        nb = (base + r + 1) // ratio
        assert same_bits(got[r, :nb], one[0, :nb]), f"row {r}"
        assert np.isnan(got[r, nb:]).all(), f"row {r}: entries past the row's complete blocks are left alone"
    want = sparse.qsa_scores(qn, ik, kw, inv, rows, nq, d, ratio, base, 64, mb, EPS)
    for r in range(rows):
        nb = (base + r + 1) // ratio
        assert np.all(np.abs(got[r, :nb] - want[r, :nb]) <= 1e-5 * (1 + np.abs(want[r, :nb]))), f"row {r}"


def gpu_select(gpu, scores, rows, ratio, base, topk, max_ctx, max_blocks):
    B = gpu.Buf
    cap = gpu.qw_qsa_list_cap(topk, ratio)
    sb = B.of(np.ascontiguousarray(scores, np.float32))
    mb = B.of(np.full((rows, max_ctx), 7, np.uint8))
    lb = B.of(np.zeros((rows, 1 + cap), np.uint32))
    c = gpu.qw_cmd_begin()
    gpu.qw_op_qsa_select(c, mb.ref(), lb.ref(), sb.ref(), rows, ratio, base, topk, max_ctx, max_blocks)
    gpu.run(c, "qsa select")
    return mb.read(np.uint8, (rows, max_ctx)), lb.read(np.uint32, (rows, 1 + cap))


def check_select(gpu, scores, rows, ratio, base, topk, max_ctx, max_blocks):
    m, lst = gpu_select(gpu, scores, rows, ratio, base, topk, max_ctx, max_blocks)
    wm, wl = sparse.qsa_select(scores, rows, ratio, base, topk, max_ctx, max_blocks)
    for r in range(rows):
        n = base + r + 1
        assert np.array_equal(m[r, :n], wm[r, :n]), f"mask row {r}"
        assert (m[r, n:] == 7).all(), "positions past the row's keys are left alone"
        assert np.array_equal(lst[r, :1 + wl[r, 0]], wl[r, :1 + wl[r, 0]]), f"list row {r}"
    return m, lst


def test_qsa_select_reference_case(gpu):
    """tests/test_sparse.c:423-458: random distinct scores, budget 2 blocks."""
    rows, base, max_ctx, ratio = 5, 13, 64, 4
    check_select(gpu, rnd((rows, 16), 53), rows, ratio, base, 2, max_ctx, 16)


@pytest.mark.parametrize("base", [2047, 2051, 2052, 4164, 9000, 40001])
def test_qsa_select_at_scale_with_ties(gpu, base):
    """tests/test_sparse.c:562-620: budget 512 blocks, 97 score levels, so
    many blocks tie at the cut."""
    rows, ratio, topk = 3, 4, 512
    max_ctx = base + rows + 8
    mb = max_ctx // ratio
    st = np.random.default_rng(base).integers(0, 97, (rows, mb))
    check_select(gpu, (st * 0.25).astype(np.float32), rows, ratio, base, topk, max_ctx, mb)


@pytest.mark.parametrize("ratio,base,max_ctx", [(4, 32766, 32768), (4, 32764, 32771), (4, 8190, 8208),
                                                (3, 24574, 24580), (1, 4000, 4096), (4, 40001, 40016)])
def test_qsa_select_distinct_scores(gpu, ratio, base, max_ctx):
    """Continuous scores (the decode shape among them: 32K keys, 8192 blocks,
    top 512): the search ends early when a bin holds exactly the blocks still
    needed; rows whose mask start is or is not 16-byte aligned."""
    rows, topk = 2, 512
    mb = max_ctx // ratio
    check_select(gpu, rnd((rows, mb), base + ratio), rows, ratio, base, topk, max_ctx, mb)


def test_qsa_select_edges(gpu):
    ratio = 4
    # every score equal: the lowest blocks win
    check_select(gpu, np.ones((2, 64), np.float32), 2, ratio, 200, 10, 256, 64)
    # negative zero ties with zero; -FLT_MAX, -inf and NaN are never taken
    s = rnd((1, 64), 3)
    s[0, :5] = [0.0, -0.0, -np.finfo(np.float32).max, -np.inf, np.nan]
    check_select(gpu, s, 1, ratio, 255, 60, 256, 64)
    s = np.full((1, 64), -np.finfo(np.float32).max, np.float32)
    s[0, [3, 40]] = [1.0, -1e30]
    check_select(gpu, s, 1, ratio, 255, 8, 256, 64)
    # +inf is the best score; -inf, -NaN and NaN among the rest stay unselected
    # when the budget exceeds the selectable blocks
    s = rnd((1, 64), 7)
    s[0, [5, 9, 20, 33, 50]] = [np.inf, -np.inf, np.nan, -np.nan, np.inf]
    check_select(gpu, s, 1, ratio, 255, 62, 256, 64)
    check_select(gpu, s, 1, ratio, 255, 3, 256, 64)
    # the budget covers every block; no complete block at all
    check_select(gpu, rnd((3, 16), 4), 3, ratio, 9, 8, 64, 16)
    check_select(gpu, rnd((3, 16), 5), 3, ratio, 0, 8, 64, 16)
    # large magnitudes of both signs
    check_select(gpu, rnd((2, 1024), 6, -1e30, 1e30), 2, ratio, 4090, 100, 4096, 1024)


# ---- masked attention ----------------------------------------------------------------

def attn_case(gpu, rows, qh, kvh, base, topk, ratio, seed, gated=False):
    D = 256
    max_ctx = base + rows + 4
    mb = max_ctx // ratio
    scores = rnd((rows, mb), seed)
    m, lst = check_select(gpu, scores, rows, ratio, base, topk, max_ctx, mb)
    cap = gpu.qw_qsa_list_cap(topk, ratio)
    q = rnd((rows, qh, D), seed + 1)
    kc = sparse.f16_bits(rnd((kvh, max_ctx, D), seed + 2))
    vc = sparse.f16_bits(rnd((kvh, max_ctx, D), seed + 3))
    gate = rnd((rows, qh, D), seed + 4, -4, 4) if gated else None
    B = gpu.Buf
    qb, kb, vb, lb, ob = B.of(q), B.of(kc), B.of(vc), B.of(lst), B(rows * qh * D * 4)
    c = gpu.qw_cmd_begin()
    scale = 1.0 / 16.0
    if gated:
        gb = B.of(gate)
        gpu.qw_op_attn_masked_gated(c, ob.ref(), gb.ref(), qb.ref(), kb.ref(), vb.ref(), lb.ref(), rows, qh, kvh, D,
                                    max_ctx, base, scale, topk, ratio)
    else:
        gpu.qw_op_attn_masked(c, ob.ref(), qb.ref(), kb.ref(), vb.ref(), lb.ref(), rows, qh, kvh, D, max_ctx, base,
                              scale, topk, ratio)
    gpu.run(c, "attn masked")
    got = ob.read(np.float32, (rows, qh, D))
    want = sparse.attn_masked(q, kc, vc, lst, rows, qh, kvh, D, max_ctx, scale, cap, gate=gate)
    assert np.abs(got - want).max() < 2e-6, f"max |diff| {np.abs(got - want).max():.3g}"


@pytest.mark.parametrize("qh,kvh", [(4, 1), (1, 1), (4, 2), (8, 1), (24, 2), (16, 1)])
def test_attn_masked_small(gpu, qh, kvh):
    """The toy model's heads (4 query, 1 kv), the full model's (24, 2) and the
    other supported ratios, 5 rows at position 13 with a budget of 2 blocks."""
    attn_case(gpu, 5, qh, kvh, 13, 2, 4, 71 + qh + kvh)


def test_attn_masked_long_list_and_gate(gpu):
    """A budget of 512 blocks at 9000 keys: lists of 2048+ positions walk
    nine chunks of the online softmax; and the gated form."""
    attn_case(gpu, 2, 4, 1, 9000, 512, 4, 81)
    attn_case(gpu, 3, 8, 2, 300, 16, 4, 82, gated=True)


@pytest.mark.parametrize("rows,qh,kvh,base", [(1, 24, 2, 32767), (1, 8, 1, 9000), (2, 16, 2, 4000),
                                               (3, 16, 4, 2500)])
def test_attn_masked_split_merge(gpu, rows, qh, kvh, base):
    """The split launch at decode shapes (the model's 24/2 heads over a
    2048-position list among them) and its ordered merge; twice in a row."""
    for _ in range(2):
        attn_case(gpu, rows, qh, kvh, base, 512, 4, 90 + qh + rows, gated=True)


# ---- gated DeltaNet ----------------------------------------------------------------

@pytest.mark.parametrize("channels,rows,n_snap", [(1024, 1, 1), (1024, 7, 7), (10240, 3, 3), (1024, 2, 2),
                                                 (320, 40, 40), (1000, 53, 20), (256, 17, 0)])
def test_conv1d_causal_silu(gpu, channels, rows, n_snap):
    """Steps run in parallel runs of 16: a run's window comes from the
    inputs before it, the first run's from the carried window (fewer rows
    than the window among the cases), snapshots for the first n_snap rows."""
    w = np.ascontiguousarray(FX["conv1d"]) if channels == 1024 else synth.to_bf16(0.3 * rnd((channels, 4), 9))
    x, st = rnd((rows, channels), 81), rnd((3, channels), 82)
    B = gpu.Buf
    xb, sb, wb, yb = B.of(x), B.of(st), B.of(w), B(rows * channels * 4)
    nb = B(max(n_snap, 1) * 3 * channels * 4)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_conv1d_causal_silu(c, yb.ref(), xb.ref(), sb.ref(), wb.ref(), channels, rows, 4,
                                 nb.ref() if n_snap else gpu.NULL_REF, n_snap, 3 * channels)
    gpu.run(c, "conv1d")
    y, s1, snap = sparse.conv1d_causal_silu(x, st, w, channels, rows, 4, n_snap=n_snap)
    assert np.allclose(yb.read(np.float32, (rows, channels)), y, rtol=2e-6, atol=1e-7)
    assert same_bits(sb.read(np.float32, (3, channels)), s1), "the window is a copy of inputs"
    if n_snap:
        assert same_bits(nb.read(np.float32, (n_snap, 3, channels)), snap[:n_snap])


def test_conv1d_prefill_equals_split_calls(gpu):
    """One 2048-row call at the model's 10240 channels against the same rows
    in three calls (1000, 1, 1047) carrying the window: the same bits."""
    channels, rows = 10240, 2048
    w = synth.to_bf16(0.3 * rnd((channels, 4), 19))
    x, st = rnd((rows, channels), 83), rnd((3, channels), 84)
    B = gpu.Buf
    xb, wb, yb, y2 = B.of(x), B.of(w), B(rows * channels * 4), B(rows * channels * 4)
    s_one, s_split = B.of(st), B.of(st)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_conv1d_causal_silu(c, yb.ref(), xb.ref(), s_one.ref(), wb.ref(), channels, rows, 4, gpu.NULL_REF, 0, 0)
    t = 0
    for n in (1000, 1, 1047):
        off = t * channels * 4
        gpu.qw_op_conv1d_causal_silu(c, y2.ref(off), xb.ref(off), s_split.ref(), wb.ref(), channels, n, 4,
                                     gpu.NULL_REF, 0, 0)
        t += n
    gpu.run(c, "conv1d split")
    assert same_bits(yb.read(np.float32, (rows, channels)), y2.read(np.float32, (rows, channels)))
    assert same_bits(s_one.read(np.float32, (3, channels)), s_split.read(np.float32, (3, channels)))
    assert same_bits(s_one.read(np.float32, (3, channels)), x[-3:])
    yo = sparse.conv1d_causal_silu(x[:64], st, w, channels, 64, 4)[0]
    assert np.allclose(yb.read(np.float32, (rows, channels))[:64], yo, rtol=2e-6, atol=1e-7)


def test_gdn_gates(gpu):
    hv, rows = int(FX["hv"]), 9
    a, b = rnd((rows, hv), 91, -30, 30), rnd((rows, hv), 92, -8, 8)
    a[0, 0] = 25.0
    B = gpu.Buf
    ab, bb, Al, dt = B.of(a), B.of(b), B.of(np.ascontiguousarray(FX["A_log"])), B.of(np.ascontiguousarray(FX["dt_bias"]))
    gb, tb = B(rows * hv * 4), B(rows * hv * 4)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_gdn_gates(c, gb.ref(), tb.ref(), ab.ref(), bb.ref(), Al.ref(), dt.ref(), hv, rows)
    gpu.run(c, "gdn gates")
    g, beta = sparse.gdn_gates(a, b, FX["A_log"], FX["dt_bias"], hv, rows)
    assert np.allclose(gb.read(np.float32, (rows, hv)), g, rtol=4e-6, atol=1e-30)
    assert np.allclose(tb.read(np.float32, (rows, hv)), beta, rtol=2e-6)


def delta_inputs(hk, hv, rows, seed):
    dk = dv = 128
    q, k = rnd((rows, hk, dk), seed), rnd((rows, hk, dk), seed + 1)
    q /= np.linalg.norm(q, axis=-1, keepdims=True) * np.sqrt(dk)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rnd((rows, hv, dv), seed + 2)
    g = (0.9 + 0.09 * np.abs(rnd((rows, hv), seed + 3))).astype(np.float32)
    beta = (0.3 + 0.4 * (np.arange(rows * hv).reshape(rows, hv) % 7) / 7.0).astype(np.float32)
    s0 = rnd((hv, dv, dk), seed + 4) * np.float32(0.05)
    return [np.ascontiguousarray(a, np.float32) for a in (q, k, v, g, beta, s0)]


def gpu_delta(gpu, q, k, v, g, beta, s0, hk, hv, rows, n_snap=0):
    B = gpu.Buf
    qb, kb, vb, gb, bb, sb = B.of(q), B.of(k), B.of(v), B.of(g), B.of(beta), B.of(s0)
    yb = B(rows * hv * 128 * 4)
    nb = B(max(n_snap, 1) * hv * 128 * 128 * 4)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_gated_delta(c, yb.ref(), qb.ref(), kb.ref(), vb.ref(), gb.ref(), bb.ref(), sb.ref(), hk, hv, 128, 128,
                          rows, nb.ref(), n_snap, hv * 128 * 128)
    gpu.run(c, "gated delta")
    return (yb.read(np.float32, (rows, hv, 128)), sb.read(np.float32, (hv, 128, 128)),
            nb.read(np.float32, (max(n_snap, 1), hv, 128, 128))[:n_snap])


@pytest.mark.parametrize("hk,hv,rows", [(2, 4, 1), (2, 4, 3), (2, 4, 40), (16, 48, 1), (16, 48, 64)])
def test_gated_delta(gpu, hk, hv, rows):
    """The toy model's heads (2 key, 4 value) and the full model's (16, 48),
    one step, a few, and runs past one 16-step chunk; snapshots of the first
    steps; and one step at a time lands on the batched call's bits."""
    q, k, v, g, beta, s0 = delta_inputs(hk, hv, rows, 7 + rows)
    ns = min(rows, 3)
    y, s1, snap = gpu_delta(gpu, q, k, v, g, beta, s0, hk, hv, rows, n_snap=ns)
    wy, ws, wsnap = sparse.gated_delta(q, k, v, g, beta, s0, hk, hv, 128, 128, rows, n_snap=ns)
    assert rel_l2(y, wy) < 5e-6 and rel_l2(s1, ws) < 5e-6, (rel_l2(y, wy), rel_l2(s1, ws))
    for t in range(ns):
        assert rel_l2(snap[t], wsnap[t]) < 5e-6
    if rows > 1 and rows <= 40:
        st = s0
        for t in range(rows):
            yt, st, _ = gpu_delta(gpu, q[t:t + 1], k[t:t + 1], v[t:t + 1], g[t:t + 1], beta[t:t + 1], st, hk, hv, 1)
            assert same_bits(yt[0], y[t]), f"step {t}"
            if t < ns:
                assert same_bits(snap[t], st)
        assert same_bits(st, s1)


@pytest.mark.parametrize("hk,hv", [(2, 4), (16, 48)])
def test_gdn_decode_one_launch(gpu, hk, hv):
    """The fused decode step (conv, then the prepared delta rule on the
    conv's q, k and v channels) against the two ops it replaces, bit for bit
    in y, the state and the conv window, over three steps that alternate
    the two windows; and the first step's y against the oracle."""
    dk = dv = 128
    ch = 2 * hk * dk + hv * dv
    B = gpu.Buf
    wq = synth.to_bf16(rnd((ch, 4), 60, -0.5, 0.5))
    w = B.of(wq)
    Al = np.ascontiguousarray(np.resize(FX["A_log"], hv))
    dt = np.ascontiguousarray(np.resize(FX["dt_bias"], hv))
    Ab, db = B.of(Al), B.of(dt)
    eps, qs, ks = 1e-6 / dk, 1.0 / dk, 1.0 / np.sqrt(dk)
    s0 = rnd((hv, dv, dk), 61) * np.float32(0.05)
    c0 = rnd((3, ch), 62)
    sA, sB = B.of(s0), B.of(s0)                      # fused, reference
    wA0, wA1, wB = B.of(c0), B(3 * ch * 4), B.of(c0)  # windows: fused alternate, reference in place
    yA, yB, mix = B(hv * dv * 4), B(hv * dv * 4), B(ch * 4)
    for step in range(3):
        x = rnd((1, ch), 70 + step)
        a, bg = rnd((1, hv), 80 + step), rnd((1, hv), 90 + step)
        xb, ab, bb = B.of(x), B.of(a), B.of(bg)
        prep = gpu.qw_gdn_prep(ab.ref(), bb.ref(), Ab.ref(), db.ref(), eps, qs, ks)
        win_in, win_out = (wA0, wA1) if step % 2 == 0 else (wA1, wA0)
        c = gpu.qw_cmd_begin()
        assert gpu.qw_op_gdn_decode(c, yA.ref(), xb.ref(), win_in.ref(), win_out.ref(), w.ref(), prep, sA.ref(),
                                    hk, hv, dk, dv)
        gpu.qw_op_conv1d_causal_silu(c, mix.ref(), xb.ref(), wB.ref(), w.ref(), ch, 1, 4, gpu.NULL_REF, 0, 0)
        kd = hk * dk
        gpu.qw_op_gated_delta_prep(c, yB.ref(), mix.ref(0), mix.ref(4 * kd), mix.ref(8 * kd), prep, sB.ref(), hk, hv,
                                   dk, dv, 1, gpu.NULL_REF, 0, 0)
        gpu.run(c, "gdn decode")
        ya, yb = yA.read(np.float32, (hv, dv)), yB.read(np.float32, (hv, dv))
        assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32)), f"y, step {step}"
        assert np.array_equal(sA.read(np.uint32, (hv, dv, dk)), sB.read(np.uint32, (hv, dv, dk))), f"state, step {step}"
        assert np.array_equal(win_out.read(np.uint32, (3, ch)), wB.read(np.uint32, (3, ch))), f"window, step {step}"
        if step == 0:
            m = sparse.conv1d_causal_silu(x, c0, wq, ch, 1, 4)[0]
            wy, _, _ = sparse.gated_delta_prep(m[:, :kd].reshape(1, hk, dk), m[:, kd:2 * kd].reshape(1, hk, dk),
                                               m[:, 2 * kd:].reshape(1, hv, dv), a, bg, Al, dt, eps, qs, ks, s0, hk,
                                               hv, dk, dv, 1)
            assert rel_l2(ya, wy.reshape(hv, dv)) < 5e-6
        for t in (xb, ab, bb):
            t.free()


@pytest.mark.parametrize("hk,hv,rows", [(2, 4, 3), (16, 48, 20), (16, 48, 150)])
def test_gated_delta_prep(gpu, hk, hv, rows):
    """Norms and gates inside the recurrence, against the oracle's prep and
    against the GPU's own composition of rms_norm, gates and the recurrence
    (tests/test_sparse.c:887-915)."""
    dk = dv = 128
    q, k, v = rnd((rows, hk, dk), 41), rnd((rows, hk, dk), 42), rnd((rows, hv, dv), 43)
    a, b = rnd((rows, hv), 44), rnd((rows, hv), 45)
    s0 = rnd((hv, dv, dk), 46) * np.float32(0.05)
    Al = np.ascontiguousarray(np.resize(FX["A_log"], hv))
    dt = np.ascontiguousarray(np.resize(FX["dt_bias"], hv))
    eps, qs, ks = 1e-6 / dk, 1.0 / dk, 1.0 / np.sqrt(dk)
    B = gpu.Buf
    qb, kb, vb, ab, bb, Ab, db = B.of(q), B.of(k), B.of(v), B.of(a), B.of(b), B.of(Al), B.of(dt)
    s1b, s2b = B.of(s0), B.of(s0)
    y1b, y2b = B(rows * hv * dv * 4), B(rows * hv * dv * 4)
    q1b, k1b, gb, tb = B(q.nbytes), B(k.nbytes), B(rows * hv * 4), B(rows * hv * 4)
    c = gpu.qw_cmd_begin()
    prep = gpu.qw_gdn_prep(ab.ref(), bb.ref(), Ab.ref(), db.ref(), eps, qs, ks)
    gpu.qw_op_gated_delta_prep(c, y2b.ref(), qb.ref(), kb.ref(), vb.ref(), prep, s2b.ref(), hk, hv, dk, dv, rows,
                               gpu.NULL_REF, 0, 0)
    gpu.qw_op_rms_norm(c, q1b.ref(), qb.ref(), gpu.NULL_REF, dk, rows * hk, eps, qs)
    gpu.qw_op_rms_norm(c, k1b.ref(), kb.ref(), gpu.NULL_REF, dk, rows * hk, eps, ks)
    gpu.qw_op_gdn_gates(c, gb.ref(), tb.ref(), ab.ref(), bb.ref(), Ab.ref(), db.ref(), hv, rows)
    gpu.qw_op_gated_delta(c, y1b.ref(), q1b.ref(), k1b.ref(), vb.ref(), gb.ref(), tb.ref(), s1b.ref(), hk, hv, dk,
                          dv, rows, gpu.NULL_REF, 0, 0)
    gpu.run(c, "gated delta prep")
    y2, s2 = y2b.read(np.float32, (rows, hv, dv)), s2b.read(np.float32, (hv, dv, dk))
    y1, s1 = y1b.read(np.float32, (rows, hv, dv)), s1b.read(np.float32, (hv, dv, dk))
    wy, ws, _ = sparse.gated_delta_prep(q, k, v, a, b, Al, dt, eps, qs, ks, s0, hk, hv, dk, dv, rows)
    assert rel_l2(y2, wy) < 5e-6 and rel_l2(s2, ws) < 5e-6, (rel_l2(y2, wy), rel_l2(s2, ws))
    assert rel_l2(y2, y1) < 5e-6 and rel_l2(s2, s1) < 5e-6


def test_gated_delta_prep_long_equals_short_calls(gpu):
    """From 64 steps on a prepared call computes every step's norms and
    gates first, in parallel; shorter calls compute them a chunk at a time
    inside the recurrence.  150 steps in one call against 60 + 60 + 30
    carrying the state: the same bits in y and the state."""
    hk, hv, dk, rows = 16, 48, 128, 150
    q, k, v = rnd((rows, hk, dk), 141), rnd((rows, hk, dk), 142), rnd((rows, hv, dk), 143)
    a, b = rnd((rows, hv), 144, -4, 4), rnd((rows, hv), 145, -4, 4)
    s0 = rnd((hv, dk, dk), 146) * np.float32(0.05)
    Al = np.ascontiguousarray(np.resize(FX["A_log"], hv))
    dt = np.ascontiguousarray(np.resize(FX["dt_bias"], hv))
    eps, qs, ks = 1e-6 / dk, 1.0 / dk, 1.0 / np.sqrt(dk)
    B = gpu.Buf
    qb, kb, vb, ab, bb, Ab, db = B.of(q), B.of(k), B.of(v), B.of(a), B.of(b), B.of(Al), B.of(dt)
    s1b, s2b = B.of(s0), B.of(s0)
    y1b, y2b = B(rows * hv * dk * 4), B(rows * hv * dk * 4)
    c = gpu.qw_cmd_begin()
    prep = gpu.qw_gdn_prep(ab.ref(), bb.ref(), Ab.ref(), db.ref(), eps, qs, ks)
    gpu.qw_op_gated_delta_prep(c, y1b.ref(), qb.ref(), kb.ref(), vb.ref(), prep, s1b.ref(), hk, hv, dk, dk, rows,
                               gpu.NULL_REF, 0, 0)
    t = 0
    for n in (60, 60, 30):
        pn = gpu.qw_gdn_prep(ab.ref(t * hv * 4), bb.ref(t * hv * 4), Ab.ref(), db.ref(), eps, qs, ks)
        gpu.qw_op_gated_delta_prep(c, y2b.ref(t * hv * dk * 4), qb.ref(t * hk * dk * 4), kb.ref(t * hk * dk * 4),
                                   vb.ref(t * hv * dk * 4), pn, s2b.ref(), hk, hv, dk, dk, n, gpu.NULL_REF, 0, 0)
        t += n
    gpu.run(c, "gated delta prep, long and short calls")
    assert same_bits(y1b.read(np.float32, (rows, hv, dk)), y2b.read(np.float32, (rows, hv, dk)))
    assert same_bits(s1b.read(np.float32, (hv, dk, dk)), s2b.read(np.float32, (hv, dk, dk)))
    wy, ws, _ = sparse.gated_delta_prep(q, k, v, a, b, Al, dt, eps, qs, ks, s0, hk, hv, dk, dk, rows)
    assert rel_l2(y1b.read(np.float32, (rows, hv, dk)), wy) < 5e-6


def test_rms_norm_gated_sigmoid(gpu):
    dim, rows = 128, 48
    x, gate = rnd((rows, dim), 7), rnd((rows, dim), 8, -6, 6)
    w = np.ascontiguousarray(FX["gdn_norm"])
    B = gpu.Buf
    xb, gb, wb, yb = B.of(x), B.of(gate), B.of(w), B(x.nbytes)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_rms_norm_gated_sigmoid(c, yb.ref(), xb.ref(), wb.ref(), gb.ref(), dim, rows, EPS, 1.0)
    gpu.run(c, "rms norm gated sigmoid")
    want = sparse.rms_norm_gated_sigmoid(x, w, gate, dim, rows, EPS)
    assert np.allclose(yb.read(np.float32, (rows, dim)), want, rtol=3e-6, atol=1e-7)
