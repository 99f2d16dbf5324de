"""Pins the QSA and gated-DeltaNet oracle (oracle/sparse_ref.c) before any
kernel is held to it.

Where the reference has a scalar twin (qwasar_cpu.c, compiled into
oracle/_ref) the oracle must give its bits.  Where it has none -- the QSA
block key and score, the selection, the position list -- the checks are an
fp64 restatement written independently here, a full sort, closed forms and
invariants, chosen so that a plausible slip (a dropped relu, a rope at the
wrong position, a tie broken upward, a snapshot one step late) fails one of
them.  Shapes and weights come from the reference's toy Flash-Next checkpoint
(tests/golden/tiny_q4_sparse.npz)."""
import os

import numpy as np
import pytest

from oracle import ref, sparse
from tests.test_oracle import need_ref

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
P = ref._ptr


@pytest.fixture(scope="module")
def fx():
    return dict(np.load(os.path.join(GOLD, "tiny_q4_sparse.npz")))


def bfv(u16):
    return (np.asarray(u16, np.uint32) << 16).view(np.float32)


def rnd(shape, seed, lo=-1.0, hi=1.0):
    return np.random.default_rng(seed).uniform(lo, hi, shape).astype(np.float32)


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


# ---- rope ------------------------------------------------------------------------

def test_rope_tables_and_rotation_match_reference(fx):
    R = need_ref()
    sparse.reflib()
    rd = int(fx["rotary_dim"])
    axis, inv = sparse.rope_tables(rd, float(fx["rope_theta"]), fx["mrope_section"])
    ra, ri = np.zeros(rd // 2, np.uint8), np.zeros(rd // 2, np.float32)
    R.qw_rope_tables(P(ra), P(ri), rd, float(fx["rope_theta"]), P(np.ascontiguousarray(fx["mrope_section"])))
    assert np.array_equal(axis, ra) and same_bits(inv, ri)
    for pos in (0, 1, 7, 4095, 40000):
        x = rnd((3, 128), pos + 1)
        a = x.copy()
        sparse._lib().qr_rope_at(P(a), pos, P(inv), 3, 128, rd)
        b = x.copy()
        p3 = np.full(3, pos, np.int32)
        R.qw_cpu_rope_partial(P(b), P(p3), P(ra), P(ri), 1, 3, 128, rd)
        assert same_bits(a, b)
        # a rotation: the norm of each (j, j + rd/2) pair is kept, dims past rd untouched
        assert np.array_equal(a[:, rd:], x[:, rd:])
        n0 = x[:, :rd // 2] ** 2 + x[:, rd // 2:rd] ** 2
        n1 = a[:, :rd // 2].astype(np.float64) ** 2 + a[:, rd // 2:rd].astype(np.float64) ** 2
        assert np.allclose(n0, n1, rtol=1e-5)


# ---- QSA scores --------------------------------------------------------------------

def scores64(qn, ikeys, kw, inv_freq, rows, nq, d, ratio, base_pos, rd, max_blocks, eps):
    """fp64 restatement of the indexer's block score, written from the
    reference's description (qwasar_flash_cpu.c:378-392), with its own rope."""
    sc = np.full((rows, max_blocks), np.nan)
    w = bfv(kw).astype(np.float64)
    half = rd // 2
    for b in range((base_pos + rows) // ratio):
        pooled = ikeys[b * ratio:(b + 1) * ratio].astype(np.float64).mean(0)
        kn = pooled / np.sqrt((pooled ** 2).mean() + eps) * w
        ang = float(b * ratio) * inv_freq.astype(np.float64)
        x0, x1 = kn[:half].copy(), kn[half:rd].copy()
        kn[:half] = x0 * np.cos(ang) - x1 * np.sin(ang)
        kn[half:rd] = x1 * np.cos(ang) + x0 * np.sin(ang)
        for r in range(rows):
            if b < (base_pos + r + 1) // ratio:
                dots = qn[r].astype(np.float64) @ kn
                sc[r, b] = dots[dots > 0].sum() / np.sqrt(d)
    return sc


def qsa_case(fx, rows=5, base_pos=37, max_ctx=64, seed=51):
    nq, d, ratio, rd = int(fx["nq"]), int(fx["d"]), int(fx["ratio"]), int(fx["rotary_dim"])
    _, inv = sparse.rope_tables(rd, float(fx["rope_theta"]), fx["mrope_section"])
    qn = rnd((rows, nq, d), seed)
    ikeys = rnd((max_ctx, d), seed + 1)
    return dict(nq=nq, d=d, ratio=ratio, rd=rd, inv=inv, qn=qn, ikeys=ikeys, rows=rows, base_pos=base_pos,
                max_ctx=max_ctx, max_blocks=max_ctx // ratio, kw=fx["k_norm"], eps=float(fx["eps"]))


def test_block_key_matches_reference_composition(fx):
    """The block key is the reference's own rms norm and rope applied to the
    serial mean of the block's raw keys: bit for bit."""
    R = need_ref()
    sparse.reflib()
    c = qsa_case(fx)
    d, ratio, rd = c["d"], c["ratio"], c["rd"]
    axis, _ = sparse.rope_tables(rd, float(fx["rope_theta"]), fx["mrope_section"])
    for b in (0, 3, 9):
        pooled = np.zeros(d, np.float32)
        for t in range(ratio):
            pooled = pooled + c["ikeys"][b * ratio + t]
        pooled = pooled / np.float32(ratio)
        kn = np.zeros(d, np.float32)
        R.qw_cpu_rms_norm(P(kn), P(pooled), P(np.ascontiguousarray(c["kw"])), d, 1, c["eps"], 1.0)
        p3 = np.full(3, b * ratio, np.int32)
        R.qw_cpu_rope_partial(P(kn), P(p3), P(axis), P(c["inv"]), 1, 1, d, rd)
        got = sparse.block_key(c["ikeys"], c["kw"], c["inv"], b, d, ratio, rd, c["eps"])
        assert same_bits(got, kn)


def test_scores_against_fp64(fx):
    c = qsa_case(fx)
    args = (c["rows"], c["nq"], c["d"], c["ratio"], c["base_pos"], c["rd"], c["max_blocks"], c["eps"])
    got = sparse.qsa_scores(c["qn"], c["ikeys"], c["kw"], c["inv"], *args)
    want = scores64(c["qn"], c["ikeys"], c["kw"], c["inv"], *args)
    m = ~np.isnan(want)
    assert m.sum() == sum((c["base_pos"] + r + 1) // c["ratio"] for r in range(c["rows"]))
    assert np.abs(got[m] - want[m]).max() < 1e-5 * max(1.0, np.abs(want[m]).max())


def test_scores_relu_and_scale_invariance(fx):
    """Heads whose dots are all negative add nothing: negating every head's
    query zeroes a score whose dots were all positive.  A block's key is an
    rms norm, so scaling its raw keys by a power of two leaves it unchanged."""
    c = qsa_case(fx, rows=1, base_pos=15)
    kn = sparse.block_key(c["ikeys"], c["kw"], c["inv"], 2, c["d"], c["ratio"], c["rd"], 0.0)
    q = np.stack([kn * (h + 1) for h in range(c["nq"])])[None].astype(np.float32)
    args = (1, c["nq"], c["d"], c["ratio"], c["base_pos"], c["rd"], c["max_blocks"], 0.0)
    s = sparse.qsa_scores(q, c["ikeys"], c["kw"], c["inv"], *args)
    want2 = sum((h + 1) * float(kn.astype(np.float64) @ kn) for h in range(c["nq"])) / np.sqrt(c["d"])
    assert abs(s[0, 2] - want2) < 1e-5 * want2
    s_neg = sparse.qsa_scores(-q, c["ikeys"], c["kw"], c["inv"], *args)
    assert s_neg[0, 2] == 0.0
    ik2 = c["ikeys"].copy()
    ik2[8:12] *= 4.0
    s2 = sparse.qsa_scores(q, ik2, c["kw"], c["inv"], *args)
    assert same_bits(s2[0, :4], s[0, :4])


def test_pooled_scores_identical(fx):
    """Block keys stored in two stretches, then scored, give the same bits as
    scoring from the raw keys (the contract of qwasar_gpu.h:627-629)."""
    c = qsa_case(fx, rows=6, base_pos=41)
    d, ratio = c["d"], c["ratio"]
    args = (c["rows"], c["nq"], d, ratio, c["base_pos"], c["rd"], c["max_blocks"], c["eps"])
    a = sparse.qsa_scores(c["qn"], c["ikeys"], c["kw"], c["inv"], *args)
    pool = np.zeros((c["max_blocks"], d), np.float32)
    allb = (c["base_pos"] + c["rows"]) // ratio
    sparse.qsa_pool(pool, c["ikeys"], c["kw"], c["inv"], d, ratio, 0, allb // 2, c["rd"], c["eps"])
    sparse.qsa_pool(pool, c["ikeys"], c["kw"], c["inv"], d, ratio, allb // 2, allb, c["rd"], c["eps"])
    b = sparse.qsa_scores_pooled(c["qn"], pool, c["rows"], c["nq"], d, ratio, c["base_pos"], c["max_blocks"])
    for r in range(c["rows"]):
        nb = (c["base_pos"] + r + 1) // ratio
        assert same_bits(a[r, :nb], b[r, :nb])


# ---- selection ---------------------------------------------------------------------

def select_by_sort(scores, rows, ratio, base_pos, topk, max_ctx):
    """The selection as a full sort: score descending, block ascending."""
    want = np.zeros((rows, max_ctx), np.uint8)
    for r in range(rows):
        n_keys = base_pos + r + 1
        nb = n_keys // ratio
        order = sorted(range(nb), key=lambda b: (-float(scores[r, b]), b))
        want[r, nb * ratio:n_keys] = 1
        for b in order[:min(topk, nb)]:
            want[r, b * ratio:(b + 1) * ratio] = 1
    return want


def check_list(mask, lst, rows, base_pos, cap):
    for r in range(rows):
        vis = np.nonzero(mask[r, :base_pos + r + 1])[0]
        assert lst[r, 0] == len(vis) <= cap
        assert np.array_equal(lst[r, 1:1 + len(vis)], vis)


@pytest.mark.parametrize("base", [2047, 2051, 4164, 9000])
def test_select_matches_sort_with_ties(base):
    """The reference's scale test (tests/test_sparse.c:562-620): 97 score
    levels, so many blocks tie at the cut; ties go to the lower block."""
    ratio, topk, rows = 4, 512, 3
    max_ctx = base + rows + 8
    mb = max_ctx // ratio
    st = np.random.default_rng(base).integers(0, 97, (rows, mb))
    scores = (st * 0.25).astype(np.float32)
    mask, lst = sparse.qsa_select(scores, rows, ratio, base, topk, max_ctx, mb)
    want = select_by_sort(scores, rows, ratio, base, topk, max_ctx)
    for r in range(rows):
        n = base + r + 1
        assert np.array_equal(mask[r, :n], want[r, :n])
    check_list(mask, lst, rows, base, sparse.list_cap(topk, ratio))


def test_select_small_budget_covers_all_and_tail():
    """Fewer complete blocks than the budget: every block and the tail are
    visible.  No complete block: only the tail."""
    ratio, topk = 4, 8
    scores = rnd((3, 16), 9)
    mask, lst = sparse.qsa_select(scores, 3, ratio, 2, topk, 64, 16)
    assert np.array_equal(mask[0, :3], [1, 1, 1])           # 3 keys, no block
    assert np.array_equal(mask[1, :4], [1, 1, 1, 1])        # one complete block
    assert lst[0, 0] == 3 and lst[1, 0] == 4 and lst[2, 0] == 5
    # exactly -FLT_MAX (the reference's struck value) is never picked
    s = np.full((1, 16), -np.finfo(np.float32).max, np.float32)
    s[0, 5] = 1.0
    mask, lst = sparse.qsa_select(s, 1, ratio, 31, 2, 64, 16)
    assert mask[0, :32].sum() == 4 and mask[0, 20:24].all()


# ---- masked attention --------------------------------------------------------------

def test_attn_masked_full_list_is_reference_decode():
    """With every position listed, masked attention is the reference's plain
    decode attention over the fp16 cache (qw_cpu_attn_decode), bit for bit."""
    R = need_ref()
    sparse.reflib()
    rows, qh, kvh, D, max_ctx, base = 2, 4, 1, 256, 32, 9
    q, k, v = rnd((rows, qh, D), 61), rnd((base + rows, kvh, D), 62), rnd((base + rows, kvh, D), 63)
    kc, vc = np.zeros((kvh, max_ctx, D), np.uint16), np.zeros((kvh, max_ctx, D), np.uint16)
    R.qw_cpu_kv_write(P(kc), P(vc), P(k), P(v), base + rows, kvh, D, max_ctx, 0)
    cap = base + rows
    lst = np.zeros((rows, 1 + cap), np.uint32)
    for r in range(rows):
        lst[r, 0] = base + r + 1
        lst[r, 1:base + r + 2] = np.arange(base + r + 1)
    scale = 1.0 / 16.0
    got = sparse.attn_masked(q, kc, vc, lst, rows, qh, kvh, D, max_ctx, scale, cap)
    want = np.zeros((rows, qh, D), np.float32)
    R.qw_cpu_attn_decode(P(want), P(q), P(kc), P(vc), rows, qh, kvh, D, max_ctx, base, scale)
    assert same_bits(got, want)
    # fp16 cache conversion agrees with the reference's on every pattern
    L = sparse._lib()
    for h in range(0, 65536, 13):
        a, b = L.qr_f16_to_f32(h), R.qw_f16_to_f32_c(h)
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32) or (np.isnan(a) and np.isnan(b))


def test_attn_masked_sparse_list_fp64_and_gate():
    rows, qh, kvh, D, max_ctx = 2, 4, 2, 256, 40
    rng = np.random.default_rng(5)
    q = rnd((rows, qh, D), 71)
    kc = sparse.f16_bits(rnd((kvh, max_ctx, D), 72))
    vc = sparse.f16_bits(rnd((kvh, max_ctx, D), 73))
    cap = 12
    lst = np.zeros((rows, 1 + cap), np.uint32)
    for r in range(rows):
        pos = np.sort(rng.choice(30, 9, replace=False))
        lst[r, 0] = 9
        lst[r, 1:10] = pos
    scale = 0.0625
    got = sparse.attn_masked(q, kc, vc, lst, rows, qh, kvh, D, max_ctx, scale, cap)
    K = kc.view(np.float16).astype(np.float64)
    V = vc.view(np.float16).astype(np.float64)
    for r in range(rows):
        pos = lst[r, 1:1 + lst[r, 0]]
        for h in range(qh):
            g = h // (qh // kvh)
            s = (q[r, h].astype(np.float64) * scale) @ K[g, pos].T
            p = np.exp(s - s.max())
            p /= p.sum()
            assert np.allclose(got[r, h], p @ V[g, pos], atol=2e-6)
    gated = sparse.attn_masked(q, kc, vc, lst, rows, qh, kvh, D, max_ctx, scale, cap,
                               gate=np.zeros((rows, qh, D), np.float32))
    assert same_bits(gated, got * np.float32(0.5))


# ---- gated DeltaNet ----------------------------------------------------------------

def test_conv1d_matches_reference_and_snapshots(fx):
    R = need_ref()
    sparse.reflib()
    w = np.ascontiguousarray(fx["conv1d"])
    ch, ks, rows = w.shape[0], int(fx["conv_k"]), 5
    x, st = rnd((rows, ch), 81), rnd((ks - 1, ch), 82)
    y, st1, snap = sparse.conv1d_causal_silu(x, st, w, ch, rows, ks, n_snap=rows)
    yr, sr = np.zeros((rows, ch), np.float32), st.copy()
    R.qw_cpu_conv1d_causal_silu(P(yr), P(x), P(sr), P(w), ch, rows, ks)
    assert same_bits(y, yr) and same_bits(st1, sr)
    # snapshot t is the state after row t: a run of t+1 rows leaves exactly it
    for t in range(rows):
        _, s_t, _ = sparse.conv1d_causal_silu(x[:t + 1], st, w, ch, t + 1, ks)
        assert same_bits(snap[t], s_t)


def test_gdn_gates_match_reference(fx):
    R = need_ref()
    sparse.reflib()
    hv, rows = int(fx["hv"]), 7
    a, b = rnd((rows, hv), 91, -30, 30), rnd((rows, hv), 92, -8, 8)
    a[0, 0] = 25.0   # softplus's linear branch
    g, beta = sparse.gdn_gates(a, b, fx["A_log"], fx["dt_bias"], hv, rows)
    gr, br = np.zeros_like(g), np.zeros_like(beta)
    R.qw_cpu_gdn_gates(P(gr), P(br), P(a), P(b), P(np.ascontiguousarray(fx["A_log"])),
                       P(np.ascontiguousarray(fx["dt_bias"])), hv, rows)
    assert same_bits(g, gr) and same_bits(beta, br)
    assert (g >= 0).all() and (g <= 1).all() and (beta > 0).all() and (beta < 1).all()


def delta_inputs(hk, hv, dk, dv, rows, seed):
    q, k = rnd((rows, hk, dk), seed), rnd((rows, hk, dk), seed + 1)
    q /= np.linalg.norm(q, axis=-1, keepdims=True) * np.sqrt(dk)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rnd((rows, hv, dv), seed + 2)
    g = (0.9 + 0.09 * np.abs(rnd((rows, hv), seed + 3))).astype(np.float32)
    beta = (0.3 + 0.4 * np.arange(rows * hv).reshape(rows, hv) % 7 / 7.0).astype(np.float32)
    s0 = rnd((hv, dv, dk), seed + 4) * np.float32(0.05)
    return [np.ascontiguousarray(a, np.float32) for a in (q, k, v, g, beta, s0)]


def test_gated_delta_matches_reference_and_streams(fx):
    R = need_ref()
    sparse.reflib()
    hk, hv, dk, dv, rows = int(fx["hk"]), int(fx["hv"]), int(fx["dk"]), int(fx["dv"]), 6
    q, k, v, g, beta, s0 = delta_inputs(hk, hv, dk, dv, rows, 1)
    y, s1, snap = sparse.gated_delta(q, k, v, g, beta, s0, hk, hv, dk, dv, rows, n_snap=3)
    yr, sr = np.zeros_like(y), s0.copy()
    R.qw_cpu_gated_delta(P(yr), P(q), P(k), P(v), P(g), P(beta), P(sr), hk, hv, dk, dv, rows)
    assert same_bits(y, yr) and same_bits(s1, sr)
    # one step at a time lands on the same bits, and the snapshots are the
    # states after steps 0, 1, 2
    st = s0.copy()
    for t in range(rows):
        yt, st, _ = sparse.gated_delta(q[t:t + 1], k[t:t + 1], v[t:t + 1], g[t:t + 1], beta[t:t + 1], st,
                                       hk, hv, dk, dv, 1)
        assert same_bits(yt[0], y[t])
        if t < 3:
            assert same_bits(snap[t], st)
    assert same_bits(st, s1)


def test_gated_delta_closed_form():
    """beta = 1, g = 1, zero state, unit k: one step writes v k^T, so the
    output is v (k . q)."""
    hk, hv, dk, dv = 1, 2, 128, 128
    k = np.zeros((1, hk, dk), np.float32)
    k[0, 0, 5] = 1.0
    q = rnd((1, hk, dk), 3)
    v = rnd((1, hv, dv), 4)
    y, s, _ = sparse.gated_delta(q, k, v, np.ones((1, hv), np.float32), np.ones((1, hv), np.float32),
                                 np.zeros((hv, dv, dk), np.float32), hk, hv, dk, dv, 1)
    assert np.allclose(y[0], v[0] * q[0, 0, 5], rtol=1e-6)
    assert np.allclose(s[:, :, 5], v[0]) and np.count_nonzero(s[:, :, :5]) == 0


def test_gated_delta_prep_is_norms_gates_then_delta(fx):
    """The prep form equals the reference's own rms norm (out_scale as the
    l2 scale), its gates and its recurrence, applied in turn."""
    R = need_ref()
    sparse.reflib()
    hk, hv, dk, dv, rows = int(fx["hk"]), int(fx["hv"]), int(fx["dk"]), int(fx["dv"]), 3
    q, k, v = rnd((rows, hk, dk), 41), rnd((rows, hk, dk), 42), rnd((rows, hv, dv), 43)
    a, b = rnd((rows, hv), 44), rnd((rows, hv), 45)
    s0 = rnd((hv, dv, dk), 46)
    eps, qs, ks = 1e-6 / dk, 1.0 / dk, 1.0 / np.sqrt(dk)
    y, s1, _ = sparse.gated_delta_prep(q, k, v, a, b, fx["A_log"], fx["dt_bias"], eps, qs, ks, s0,
                                       hk, hv, dk, dv, rows)
    q1, k1 = np.zeros_like(q), np.zeros_like(k)
    R.qw_cpu_rms_norm(P(q1), P(q), None, dk, rows * hk, eps, qs)
    R.qw_cpu_rms_norm(P(k1), P(k), None, dk, rows * hk, eps, np.float32(ks))
    g, beta = np.zeros((rows, hv), np.float32), np.zeros((rows, hv), np.float32)
    R.qw_cpu_gdn_gates(P(g), P(beta), P(a), P(b), P(np.ascontiguousarray(fx["A_log"])),
                       P(np.ascontiguousarray(fx["dt_bias"])), hv, rows)
    yr, sr = np.zeros_like(y), s0.copy()
    R.qw_cpu_gated_delta(P(yr), P(q1), P(k1), P(v), P(g), P(beta), P(sr), hk, hv, dk, dv, rows)
    assert same_bits(y, yr) and same_bits(s1, sr)


def test_rms_norm_gated_sigmoid(fx):
    R = need_ref()
    dim, rows = 128, 4
    x, gate = rnd((rows, dim), 7), rnd((rows, dim), 8, -6, 6)
    w = np.ascontiguousarray(fx["gdn_norm"])
    y = sparse.rms_norm_gated_sigmoid(x, w, gate, dim, rows, 1e-6)
    n = np.zeros_like(x)
    R.qw_cpu_rms_norm(P(n), P(x), P(w), dim, rows, 1e-6, 1.0)
    want = n.astype(np.float64) / (1.0 + np.exp(-gate.astype(np.float64)))
    assert np.allclose(y, want, rtol=3e-7, atol=1e-7)
    # gate 0: exactly half the norm
    y0 = sparse.rms_norm_gated_sigmoid(x, w, np.zeros_like(gate), dim, rows, 1e-6)
    assert same_bits(y0, n * np.float32(0.5))
