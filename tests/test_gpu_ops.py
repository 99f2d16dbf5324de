"""The MoE ops of include/qwasar_gpu.h on the GPU, each against the CPU oracle
or against the ops it fuses -- the structure of the reference's
tests/test_sparse.c (test_moe :173-286, test_fused :763-876,
test_bank_splitk :919-971, test_grouped_experts :977-1025).

Integer results (routing ids, the dispatch permutation, tiles) and the
routing weights are compared bit for bit; fp32 products by relative L2 with
the tolerances written next to each check."""
import numpy as np
import pytest

from oracle import ref
from qwasar_amd import synth

pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    den = np.sqrt((b * b).sum())
    num = np.sqrt(((a - b) ** 2).sum())
    return num / den if den > 0 else num


def rnd(shape, seed, scale=1.0):
    return (synth.normal(seed, "t", int(np.prod(shape)), scale).astype(np.float32)).reshape(shape)


def bank(seed, E, n, k, G):
    return synth.make_q4(seed, "bank", E * n, k, G)


def per_pair_ref(q, x, idx, k, n, K, by_pair):
    pairs = idx.size
    y = np.zeros((pairs, n), np.float32)
    words, groups = k // 8, k // q.group
    for p in range(pairs):
        e = int(idx[p])
        xr = x[p] if by_pair else x[p // K]
        y[p] = ref.qmv_q4(xr[None], q.w[e * n:(e + 1) * n], q.s[e * n:(e + 1) * n], q.b[e * n:(e + 1) * n],
                          k, n, 1, q.group)[0]
    return y


# ---- routing -----------------------------------------------------------------

@pytest.mark.parametrize("E,K,rows", [(8, 2, 7), (16, 4, 7), (512, 10, 9), (1000, 32, 3), (64, 1, 5)])
def test_route_bit_exact(gpu, E, K, rows):
    lg = (rnd((rows, E), 21 + E) * 4.0).astype(np.float32)
    # constructed ties: equal logits must go to the lower expert first
    lg[0, 3] = lg[0, 5] = lg[0, 7] = lg[0].max() + 1.0
    lg[1 % rows, :] = 0.25
    if E >= 192 and rows > 2:
        # equal values in one lane's slots (5, 69, 133 share a wave lane) and
        # one more in another lane (131): ascending index order is required
        lg[2, [133, 69, 5, 131]] = lg[2].max() + 2.0
    B = gpu.Buf
    lgb, ib, wb = B.of(lg), B(rows * K * 4), B(rows * K * 4)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_moe_route(c, ib.ref(), wb.ref(), lgb.ref(), rows, E, K, True)
    gpu.run(c, "moe_route")
    idx, w = ref.route(lg, rows, E, K, norm=True)
    got_i = ib.read(np.int32, (rows, K))
    got_w = wb.read(np.float32, (rows, K))
    assert np.array_equal(got_i, idx), "route ids differ from the oracle"
    assert np.array_equal(got_w.view(np.uint32), w.view(np.uint32)), "route weights not bit-exact"
    assert list(got_i[0, :3]) == [3, 5, 7][:min(K, 3)]
    assert list(got_i[1 % rows, :K]) == list(range(K))
    if E >= 192 and rows > 2:
        assert list(got_i[2, :4]) == [5, 69, 131, 133][:K]


@pytest.mark.parametrize("E,K", [(512, 10), (256, 32), (128, 8), (1000, 4)])
def test_route_selection_edges(gpu, E, K):
    """Rows whose candidate set (p at or above the K-th largest lane maximum)
    is exactly 64, 65 or all experts, ties inside one lane's slots, and
    probabilities that underflow to zero: every row bit-exact to the oracle."""
    rows = 8
    g = np.random.default_rng(E * 100 + K)
    lg = (g.standard_normal((rows, E)) * 3.0).astype(np.float32)
    top = np.float32(20.0)
    lg[0, g.choice(E, 64, replace=False)] = top           # 64 tied maxima
    lg[1, g.choice(E, 65, replace=False)] = top           # 65: more than a wave
    lg[2] *= 100.0                                        # most p round to zero
    lg[3, :] = -1.0e4
    lg[3, E - 1] = 0.0                                    # one p = 1, the rest 0
    lg[4, g.choice(E, 40, replace=False)] = top
    lg[4, 3] = top + 1.0                                  # one above forty ties
    lane = [l for l in range(3, E, 64)]                   # one lane's slots
    lg[5, lane] = top
    lg[5, [1, 2]] = top                                   # and two other lanes
    lg[6, :] = 0.0                                        # all equal
    B = gpu.Buf
    lgb, ib, wb = B.of(lg), B(rows * K * 4), B(rows * K * 4)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_moe_route(c, ib.ref(), wb.ref(), lgb.ref(), rows, E, K, True)
    gpu.run(c, "moe_route edges")
    idx, w = ref.route(lg, rows, E, K, norm=True)
    got_i = ib.read(np.int32, (rows, K))
    got_w = wb.read(np.float32, (rows, K))
    for r in range(rows):
        assert np.array_equal(got_i[r], idx[r]), f"row {r}: ids differ from the oracle"
        assert np.array_equal(got_w[r].view(np.uint32), w[r].view(np.uint32)), f"row {r}: weights not bit-exact"
    assert list(got_i[6]) == list(range(K))
    assert got_i[3, 0] == E - 1


def test_route_refuses_oversize(gpu, capfd):
    B = gpu.Buf
    lg, ib, wb = B(4 * 2048), B(4 * 40), B(4 * 40)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_moe_route(c, ib.ref(), wb.ref(), lg.ref(), 1, 2048, 4, True)
    gpu.qw_op_moe_route(c, ib.ref(), wb.ref(), lg.ref(), 1, 64, 40, True)
    gpu.run(c, "route refusals")
    err = capfd.readouterr().err
    assert err.count("unsupported") == 2


@pytest.mark.parametrize("k,n,rows", [(3072, 512, 1), (3072, 512, 8), (3072, 64, 20), (256, 16, 3), (100, 7, 2),
                                      (3072, 512, 70), (2560, 100, 33), (256, 16, 64), (192, 40, 97),
                                      (3072, 1, 2048), (256, 3, 40), (64, 1, 9), (8192, 2, 12),
                                      (3072, 512, 2048), (3072, 515, 1024), (12288, 4, 300), (16384, 7, 9)])
def test_dmat_bf16_order_r_bit_exact(gpu, k, n, rows):
    """Small row counts take one wave per output; from 32 rows on (k % 64 == 0)
    the register-tiled kernel, including ragged row and output blocks (the
    full 2048-row prefill chunk among them); a few outputs (n < 8, the shared
    expert's gate) over many rows one wave per (row, output)."""
    w = synth.to_bf16(rnd((n, k), 5 + k, 0.02))
    x = synth.bf16_round(rnd((rows, k), 6 + n))
    if rows >= 32:
        x = rnd((rows, k), 9 + n).astype(np.float32)   # full fp32 inputs
        x[rows // 2] = 0.0                             # a zero row: signed zeros must match
        x[rows // 3, : k // 2] *= -1e-30               # tiny products
    B = gpu.Buf
    wb, xb, yb = B.of(w), B.of(x), B(rows * n * 4)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_dmat_bf16(c, yb.ref(), xb.ref(), wb.ref(), k, n, rows)
    gpu.run(c, "dmat")
    want = ref.dmat_bf16(x, w, k, n, rows)
    got = yb.read(np.float32, (rows, n))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), "router logits not bit-exact (order R)"


# ---- decode banks ------------------------------------------------------------

@pytest.mark.parametrize("G", [64, 32])
@pytest.mark.parametrize("by_pair", [False, True])
def test_bank(gpu, G, by_pair):
    E, k, n, K, rows = 16, 2560, 640, 10, 2
    pairs = rows * K
    q = bank(17 + G, E, n, k, G)
    x = rnd((pairs if by_pair else rows, k), 71 + G)
    idx = np.array([(p * 7 + 3) % E for p in range(pairs)], np.int32)
    B = gpu.Buf
    wb, sb, bb = B(wrap=q.w), B(wrap=q.s), B(wrap=q.b)
    xb, ib, yb = B.of(x), B.of(idx), B(pairs * n * 4)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_qmv_q4_bank(c, yb.ref(), xb.ref(), ib.ref(), wb.ref(), sb.ref(), bb.ref(), k, n, pairs, K,
                          by_pair, G)
    gpu.run(c, "bank")
    want = per_pair_ref(q, x, idx, k, n, K, by_pair)
    assert rel_l2(yb.read(np.float32, (pairs, n)), want) < 1e-5


@pytest.mark.parametrize("G", [64, 32])
def test_bank2(gpu, G):
    E, k, n, K, rows = 16, 2560, 640, 10, 2
    pairs = rows * K
    q0, q1 = bank(31, E, n, k, G), bank(32, E, n, k, G)
    x = rnd((rows, k), 33)
    idx = np.array([(p * 7 + 3) % E for p in range(pairs)], np.int32)
    B = gpu.Buf
    bufs = [(B(wrap=q.w), B(wrap=q.s), B(wrap=q.b)) for q in (q0, q1)]
    xb, ib, yb = B.of(x), B.of(idx), B(2 * pairs * n * 4)
    c = gpu.qw_cmd_begin()
    ok = gpu.qw_op_qmv_q4_bank2(c, yb.ref(), xb.ref(), ib.ref(), *(b.ref() for b in bufs[0]),
                                *(b.ref() for b in bufs[1]), k, n, pairs, K, G)
    gpu.run(c, "bank2")
    assert ok
    want = np.concatenate([per_pair_ref(q, x, idx, k, n, K, False) for q in (q0, q1)])
    assert rel_l2(yb.read(np.float32, (2 * pairs, n)), want) < 1e-5
    # too short to split: declined, nothing encoded (reference qwasar_metal.m:1700)
    assert not gpu.qw_op_qmv_q4_bank2(None, yb.ref(), xb.ref(), ib.ref(), *(b.ref() for b in bufs[0]),
                                      *(b.ref() for b in bufs[1]), 1024, n, pairs, K, G)


@pytest.mark.parametrize("layout", ["split", "interleaved"])
def test_swiglu_bank(gpu, layout):
    """swiglu . bank == bank(swiglu(gate, up)) (test_fused, tests/test_sparse.c:767-805)."""
    G, k, n, E, K, pairs = 32, 640, 2560, 16, 10, 10
    q = bank(11, E, n, k, G)
    gu = rnd((2 * pairs * k,), 13)
    idx = np.array([(p * 5 + 2) % E for p in range(pairs)], np.int32)
    B = gpu.Buf
    wb, sb, bb = B(wrap=q.w), B(wrap=q.s), B(wrap=q.b)
    gub, ib, actb = B.of(gu), B.of(idx), B(pairs * k * 4)
    y1, y2 = B(pairs * n * 4), B(pairs * n * 4)
    u_off = (k if layout == "interleaved" else pairs * k) * 4
    stride = 2 * k if layout == "interleaved" else k
    c = gpu.qw_cmd_begin()
    if layout == "interleaved":
        gpu.qw_op_swiglu_split(c, actb.ref(), gub.ref(), pairs, k)
    else:
        gpu.qw_op_swiglu(c, actb.ref(), gub.ref(), gub.ref(u_off), pairs * k)
    gpu.qw_op_qmv_q4_bank(c, y1.ref(), actb.ref(), ib.ref(), wb.ref(), sb.ref(), bb.ref(), k, n, pairs, K, True, G)
    gpu.qw_op_qmv_q4_swiglu(c, y2.ref(), gub.ref(), gub.ref(u_off), stride, ib.ref(), wb.ref(), sb.ref(), bb.ref(),
                            k, n, pairs, G)
    gpu.run(c, "swiglu bank")
    assert rel_l2(y2.read(np.float32, (pairs, n)), y1.read(np.float32, (pairs, n))) < 1e-5
    # and the activation itself against the oracle's silu
    g = gu.reshape(-1)
    if layout == "interleaved":
        gg = g.reshape(pairs, 2 * k)
        act = np.array([[ref.lib().qr_silu(float(v)) for v in row[:k]] for row in gg], np.float32) * gg[:, k:]
    else:
        act = np.array([ref.lib().qr_silu(float(v)) for v in g[:pairs * k]], np.float32).reshape(pairs, k) \
            * g[pairs * k:].reshape(pairs, k)
    assert rel_l2(actb.read(np.float32, (pairs, k)), act) < 1e-6
    # the fused product itself against the oracle: pair p's expert idx[p]
    # (rows idx[p] n .. + n of the bank) applied to the oracle's activation
    y2h = y2.read(np.float32, (pairs, n))
    for pr in range(pairs):
        e = int(idx[pr])
        want = ref.qmv_q4(act[pr][None], q.w[e * n:(e + 1) * n], q.s[e * n:(e + 1) * n], q.b[e * n:(e + 1) * n],
                          k, n, 1, G)[0]
        assert rel_l2(y2h[pr], want) < 1e-5, f"pair {pr} (expert {e}) against the oracle"


@pytest.mark.parametrize("count", [1, 2, 3, 4])
def test_multi(gpu, count):
    G, k = 64, 3072
    ns = [512, 512, 48, 1000][:count]
    qs = [synth.make_q4(40 + i, "m", ns[i], k, G) for i in range(count)]
    x = rnd((1, k), 41)
    B = gpu.Buf
    xb = B.of(x)
    bufs = [(B(wrap=q.w), B(wrap=q.s), B(wrap=q.b), B(ns[i] * 4)) for i, q in enumerate(qs)]
    parts = (gpu.qw_qmv_part * count)(*[gpu.qw_qmv_part(b[3].ref(), b[0].ref(), b[1].ref(), b[2].ref(), ns[i])
                                         for i, b in enumerate(bufs)])
    c = gpu.qw_cmd_begin()
    assert gpu.qw_op_qmv_q4_multi(c, xb.ref(), k, G, count, parts)
    gpu.run(c, "multi")
    for i, q in enumerate(qs):
        want = ref.qmv_q4(x, q.w, q.s, q.b, k, ns[i], 1, G)
        assert rel_l2(bufs[i][3].read(np.float32, (1, ns[i])), want) < 1e-5


@pytest.mark.parametrize("rows", [1, 3, 21, 100])
def test_qmat(gpu, rows):
    """qw_op_qmat_q4 across its matvec and MFMA forms (test_qmm_splitk, :740-761)."""
    G, k, n = 32, 2560, 320
    q = synth.make_q4(51 + rows, "qm", n, k, G)
    x = rnd((rows, k), 61 + rows)
    B = gpu.Buf
    wb, sb, bb, xb, yb = B(wrap=q.w), B(wrap=q.s), B(wrap=q.b), B.of(x), B(rows * n * 4)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_qmat_q4(c, yb.ref(), xb.ref(), wb.ref(), sb.ref(), bb.ref(), k, n, rows, G)
    gpu.run(c, "qmat")
    want = ref.qmv_q4(x, q.w, q.s, q.b, k, n, rows, G)
    # f16 activation tiles in the MFMA form, fp32 in the matvec
    tol = 5e-4 if rows >= 8 else 1e-5
    assert rel_l2(yb.read(np.float32, (rows, n)), want) < tol


@pytest.mark.parametrize("k,n,rows,G", [(12288, 320, 300, 64), (1024, 64, 17, 32), (4096, 200, 90, 128),
                                        (640, 96, 40, 64)])
def test_qmm_splitk(gpu, k, n, rows, G):
    """The dense MFMA product with its k range sliced across workgroups (the
    hyper-connection down-projection's shape first; 2 slices; group 128 with a
    ragged column block; and a k too short to split), against the oracle."""
    print(f"qmm splitk k={k} n={n} rows={rows} G={G}", flush=True)
    q = synth.make_q4(71 + rows, "qsk", n, k, G)
    x = rnd((rows, k), 81 + rows)
    B = gpu.Buf
    wb, sb, bb, xb, yb = B(wrap=q.w), B(wrap=q.s), B(wrap=q.b), B.of(x), B(rows * n * 4)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_qmm_q4(c, yb.ref(), xb.ref(), wb.ref(), sb.ref(), bb.ref(), k, n, rows, G)
    gpu.run(c, "qmm splitk")
    want = ref.qmv_q4(x, q.w, q.s, q.b, k, n, rows, G)
    assert rel_l2(yb.read(np.float32, (rows, n)), want) < 5e-4


# ---- elementwise and the combine ----------------------------------------------

def test_combine_shared(gpu):
    """combine_shared == combine + scale_rows_sigmoid + add (tests/test_sparse.c:807-830)."""
    rows, K, H = 3, 10, 2560
    y, w = rnd((rows * K, H), 21), rnd((rows, K), 22)
    sh, g = rnd((rows, H), 23), rnd((rows,), 24)
    B = gpu.Buf
    yb, wb, shb, gb, sh1 = B.of(y), B.of(w), B.of(sh), B.of(g), B.of(sh)
    o1, o2 = B(rows * H * 4), B(rows * H * 4)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_moe_combine_shared(c, o2.ref(), yb.ref(), wb.ref(), shb.ref(), gb.ref(), rows, K, H)
    gpu.qw_op_moe_combine(c, o1.ref(), yb.ref(), wb.ref(), rows, K, H)
    gpu.qw_op_scale_rows_sigmoid(c, sh1.ref(), gb.ref(), rows, H)
    gpu.qw_op_add_inplace(c, o1.ref(), sh1.ref(), rows * H)
    gpu.run(c, "combine")
    got2, got1 = o2.read(np.float32, (rows, H)), o1.read(np.float32, (rows, H))
    assert rel_l2(got2, got1) < 1e-6
    sig = 1.0 / (1.0 + np.exp(-g.astype(np.float64)))
    want = (w.astype(np.float64)[:, :, None] * y.reshape(rows, K, H)).sum(1) + sig[:, None] * sh
    assert rel_l2(got2, want) < 1e-6


# ---- prefill: dispatch permutation and grouped experts -------------------------

def skewed_idx(pairs, E, seed):
    """One expert takes ~40% of the pairs, many get a few, some none
    (tests/test_sparse.c:996-1003)."""
    r = synth.raw64(seed, "skew", pairs)
    a = (r >> np.uint64(16)) % np.uint64(5)
    b = (r >> np.uint64(8)) % np.uint64(max(E - 16, 1))
    return np.where(a < 2, 0, b).astype(np.int32)


@pytest.mark.parametrize("pairs,E", [(2560, 64), (20480, 512), (37, 16), (1, 8), (5120, 1024)])
def test_group_bit_exact(gpu, pairs, E):
    idx = skewed_idx(pairs, E, pairs + E)
    bm = int(gpu.qw_moe_tile_rows(pairs, E))
    mt = int(gpu.qw_moe_max_tiles(pairs, E))
    B = gpu.Buf
    ib, pb, tb, cb = B.of(idx), B(pairs * 4), B((1 + 3 * mt) * 4), B(E * 4)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_moe_group(c, pb.ref(), tb.ref(), cb.ref(), ib.ref(), pairs, E)
    gpu.run(c, "group")
    perm, tiles = ref.moe_group(idx, E, bm)
    got_p = pb.read(np.int32, (pairs,))
    got_t = tb.read(np.int32, (1 + 3 * mt,))
    assert np.array_equal(got_p, perm), "dispatch permutation differs from the stable sort"
    nt = int(tiles[0])
    assert got_t[0] == nt and np.array_equal(got_t[:1 + 3 * nt], tiles[:1 + 3 * nt])
    assert np.array_equal(perm, np.argsort(idx, kind="stable"))


@pytest.mark.parametrize("G", [64, 32])
@pytest.mark.parametrize("by_pair", [False, True])
def test_grouped_experts(gpu, G, by_pair):
    """Grouped (MFMA, prefill) vs per-pair matvec (decode) on one bank, on a
    skewed routing (tests/test_sparse.c:977-1025); tol 1e-3 as there for
    half-precision operand tiles."""
    E, k, n, rows, K = 64, 2560, 640, 256, 10
    pairs = rows * K
    q = bank(99 + G, E, n, k, G)
    x = rnd((pairs, k), 5 + G)
    idx = skewed_idx(pairs, E, 7 + G)
    mt = int(gpu.qw_moe_max_tiles(pairs, E))
    B = gpu.Buf
    wb, sb, bb = B(wrap=q.w), B(wrap=q.s), B(wrap=q.b)
    xb, ib = B.of(x), B.of(idx)
    pb, tb, cb = B(pairs * 4), B((1 + 3 * mt) * 4), B(E * 4)
    yg, yr = B(pairs * n * 4), B(pairs * n * 4)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_moe_group(c, pb.ref(), tb.ref(), cb.ref(), ib.ref(), pairs, E)
    gpu.qw_op_qmm_q4_gather(c, yg.ref(), xb.ref(), pb.ref(), tb.ref(), wb.ref(), sb.ref(), bb.ref(),
                            k, n, pairs, E, K, by_pair, G)
    gpu.qw_op_qmv_q4_bank(c, yr.ref(), xb.ref(), ib.ref(), wb.ref(), sb.ref(), bb.ref(), k, n, pairs, K,
                          by_pair, G)
    gpu.run(c, "grouped experts")
    e = rel_l2(yg.read(np.float32, (pairs, n)), yr.read(np.float32, (pairs, n)))
    assert e < 1e-3, f"grouped vs per-pair rel L2 {e:.3g}"
    tiles = tb.read(np.int32, (1 + 3 * mt,))
    big = sum(1 for t in range(tiles[0]) if tiles[1 + 3 * t] == 0)
    assert big > 10, f"expert 0 should span many tiles, got {big}"
    # spot-check rows against the oracle directly
    sel = np.arange(0, pairs, 97)
    # (A row of pair p: x[p] by pair, else the token's row x[p // K])
    xs = x[sel] if by_pair else x[sel // K]
    want = np.stack([ref.qmv_q4(xs[i][None], q.w[idx[s] * n:(idx[s] + 1) * n],
                                q.s[idx[s] * n:(idx[s] + 1) * n], q.b[idx[s] * n:(idx[s] + 1) * n],
                                k, n, 1, G)[0] for i, s in enumerate(sel)])
    assert rel_l2(yg.read(np.float32, (pairs, n))[sel], want) < 1e-3
