"""The hyper-connection mixer's ops on the GPU against the CPU oracle
(oracle/moe_ref.c restating qwasar_flash_cpu.c:57-70 and 263-293 with the
GPU ops' semantics, metal/sparse.metal:14-189), and the mixer composed around
one MoE layer of config 1's shape, each step fed the GPU's own inputs.

Tolerances: the norms' sums run in another order than the oracle's serial
loops (2e-5 relative per element, the serial fp32 sum's own error at these
lengths); sigmoid and silu use the device's expf (2e-6 relative); the
up-projection's dot and the mix, fmaf chains against the oracle's serial
products (rel-L2 1e-5)."""
import numpy as np
import pytest

from oracle import ref
from qwasar_amd import synth

pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.sqrt(((a - b) ** 2).sum() / (b * b).sum()))


def _rng(seed):
    return np.random.default_rng(seed)


@pytest.mark.parametrize("rows,H,S", [(1, 3072, 4), (5, 2560, 4), (33, 256, 3), (3, 6144, 2), (2, 1000, 2)])
def test_grouped_norm_and_inject_norm(gpu, rows, H, S):
    g = _rng(rows * H + S)
    h4 = (g.standard_normal((rows, S * H)) * 2).astype(np.float32)
    w = synth.to_bf16(1.0 + 0.1 * g.standard_normal(S * H).astype(np.float32))
    out = g.standard_normal((rows, H)).astype(np.float32)
    inj = (g.standard_normal((rows, S)) * 3).astype(np.float32)
    B = gpu.Buf
    hb, wb, nb, ob, ib = B.of(h4), B.of(w), B(h4.nbytes), B.of(out), B.of(inj)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_rms_norm_grouped(c, nb.ref(), hb.ref(), wb.ref(), H, S, rows, 1e-6)
    gpu.run(c, "rms_norm_grouped")
    want = ref.rms_norm_grouped(h4, w, H, S, 1e-6)
    assert np.allclose(nb.read(np.float32, (rows, S * H)), want, rtol=2e-5, atol=0)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_hc_inject_norm(c, hb.ref(), ob.ref(), ib.ref(), wb.ref(), nb.ref(), rows, H, S, 1e-6)
    gpu.run(c, "hc_inject_norm")
    wh = ref.hc_inject(h4, out, inj, rows, H, S)
    gh = hb.read(np.float32, (rows, S * H))
    assert np.allclose(gh, wh, rtol=2e-6, atol=1e-6), "injected streams"
    assert np.allclose(nb.read(np.float32, (rows, S * H)), ref.rms_norm_grouped(gh, w, H, S, 1e-6),
                       rtol=2e-5, atol=0), "normed streams"


@pytest.mark.parametrize("rows,H,S", [(1, 3072, 4), (7, 256, 2)])
def test_mix_inject_repeat_silu(gpu, rows, H, S):
    g = _rng(100 + rows)
    n = g.standard_normal((rows, S * H)).astype(np.float32)
    m = (g.standard_normal((rows, S * H)) * 3).astype(np.float32)
    out = g.standard_normal((rows, H)).astype(np.float32)
    inj = (g.standard_normal((rows, S)) * 3).astype(np.float32)
    B = gpu.Buf
    nb, mb, xb, ob, ib, hb = B.of(n), B.of(m), B(rows * H * 4), B.of(out), B.of(inj), B.of(n)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_hc_mix(c, xb.ref(), nb.ref(), mb.ref(), rows, H, S)
    gpu.qw_op_hc_inject(c, hb.ref(), ob.ref(), ib.ref(), rows, H, S)
    gpu.run(c, "hc_mix, hc_inject")
    assert np.allclose(xb.read(np.float32, (rows, H)), ref.hc_mix(n, m, rows, H, S), rtol=2e-6, atol=1e-7)
    assert np.allclose(hb.read(np.float32, (rows, S * H)), ref.hc_inject(n, out, inj, rows, H, S), rtol=2e-6, atol=1e-6)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_repeat_cols(c, hb.ref(), ob.ref(), rows, H, S)
    gpu.qw_op_silu_scale(c, mb.ref(), rows * S * H, 0.25)
    gpu.run(c, "repeat_cols, silu_scale")
    assert np.array_equal(hb.read(np.float32, (rows, S * H)), ref.repeat_cols(out, rows, H, S))
    assert np.allclose(mb.read(np.float32, (rows, S * H)), ref.silu_scale(m, 0.25), rtol=2e-6, atol=1e-7)


def _q4(seed, name, rows, cols, group):
    return synth.make_q4(seed, name, rows, cols, group)


@pytest.mark.parametrize("rows,H,S,k,G", [(1, 3072, 4, 320, 64), (4, 2560, 4, 320, 32), (2, 256, 3, 64, 64)])
def test_hc_mix_up(gpu, rows, H, S, k, G):
    g = _rng(7 * rows + k)
    q = _q4(11, f"mixup{H}", S * H, k, G)
    d = (g.standard_normal((rows, k)) * 4).astype(np.float32)
    n4 = g.standard_normal((rows, S * H)).astype(np.float32)
    B = gpu.Buf
    wb, sb, bb = B.of(q.w), B.of(q.s), B.of(q.b)
    db, nb, xb = B.of(d), B.of(n4), B(rows * H * 4)
    c = gpu.qw_cmd_begin()
    assert gpu.qw_op_hc_mix_up(c, xb.ref(), db.ref(), nb.ref(), wb.ref(), sb.ref(), bb.ref(), k, H, S, rows,
                               1.0 / S, G)
    gpu.run(c, "hc_mix_up")
    want = ref.hc_mix_up(d, n4, q.w, q.s, q.b, k, H, S, rows, 1.0 / S, G)
    e = rel_l2(xb.read(np.float32, (rows, H)), want)
    assert e < 1e-5, f"rel-L2 {e:.3g}"
    c = gpu.qw_cmd_begin()
    assert not gpu.qw_op_hc_mix_up(c, xb.ref(), db.ref(), nb.ref(), wb.ref(), sb.ref(), bb.ref(), k, H, 5, rows,
                                   0.2, G), "S > 4 must be refused"
    gpu.qw_cmd_free(c)


def test_mixer_around_the_moe_layer(gpu):
    """One Flash-Next MLP sublayer at config 1's shape (H 3072, S 4, low rank
    320): inject the previous block's output and norm the streams, mix down,
    the injection logits, the fused mix-up, the MoE layer on the mixed input,
    then its output into the streams; each step against the oracle on the
    GPU's own inputs (routing ids and weights bit-exact)."""
    H, S, k, G, rows = 3072, 4, 320, 64, 1
    cfg = dict(synth.CONFIGS[1])
    L = synth.make_layer(21, **{kk: cfg[kk] for kk in ("H", "E", "K", "I", "SI", "group")})
    lb = gpu.LayerBufs(L)
    g = _rng(22)
    h4 = (g.standard_normal((rows, S * H))).astype(np.float32)
    prev = g.standard_normal((rows, H)).astype(np.float32)
    pinj = g.standard_normal((rows, S)).astype(np.float32)
    wn = synth.to_bf16(1.0 + 0.05 * g.standard_normal(S * H).astype(np.float32))
    down = _q4(23, "hc.down", k, S * H, G)
    up = _q4(24, "hc.up", S * H, k, G)
    binj = synth.to_bf16((0.02 * g.standard_normal((S, S * H))).astype(np.float32))
    B = gpu.Buf
    hb, pb, ib, wnb = B.of(h4), B.of(prev), B.of(pinj), B.of(wn)
    n4b, db, injb, xb = B(S * H * 4), B(k * 4), B(S * 4), B(H * 4)
    dwb, dsb, dbb = B.of(down.w), B.of(down.s), B.of(down.b)
    uwb, usb, ubb = B.of(up.w), B.of(up.s), B.of(up.b)
    bjb = B.of(binj)
    ob, oib, owb = B(H * 4), B(L.K * 4), B(L.K * 4)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_hc_inject_norm(c, hb.ref(), pb.ref(), ib.ref(), wnb.ref(), n4b.ref(), rows, H, S, 1e-6)
    gpu.qw_op_qmv_q4(c, db.ref(), n4b.ref(), dwb.ref(), dsb.ref(), dbb.ref(), S * H, k, rows, G)
    gpu.qw_op_dmat_bf16(c, injb.ref(), n4b.ref(), bjb.ref(), S * H, S, rows)
    assert gpu.qw_op_hc_mix_up(c, xb.ref(), db.ref(), n4b.ref(), uwb.ref(), usb.ref(), ubb.ref(), k, H, S, rows,
                               1.0 / S, G)
    assert gpu.qw_op_moe_layer(c, ob.ref(), oib.ref(), owb.ref(), xb.ref(), lb.desc, rows)
    gpu.run(c, "mixer and MoE layer")
    gh = hb.read(np.float32, (rows, S * H))
    assert np.allclose(gh, ref.hc_inject(h4, prev, pinj, rows, H, S), rtol=2e-6, atol=1e-6)
    n4 = n4b.read(np.float32, (rows, S * H))
    assert np.allclose(n4, ref.rms_norm_grouped(gh, wn, H, S, 1e-6), rtol=2e-5, atol=0)
    d = db.read(np.float32, (rows, k))
    assert rel_l2(d, ref.qmv_q4(n4, down.w, down.s, down.b, S * H, k, rows, G)) < 1e-5
    inj = injb.read(np.float32, (rows, S))
    assert np.array_equal(inj.view(np.uint32), ref.dmat_bf16(n4, binj, S * H, S, rows).view(np.uint32))
    x = xb.read(np.float32, (rows, H))
    assert rel_l2(x, ref.hc_mix_up(d, n4, up.w, up.s, up.b, k, H, S, rows, 1.0 / S, G)) < 1e-5
    out, idx, w = ref.moe_forward(L, x)
    assert np.array_equal(oib.read(np.int32, (rows, L.K)), idx)
    assert np.array_equal(owb.read(np.float32, (rows, L.K)).view(np.uint32), w.view(np.uint32))
    assert rel_l2(ob.read(np.float32, (rows, H)), out) < 5e-4
    # the block's output into the streams
    c = gpu.qw_cmd_begin()
    gpu.qw_op_hc_inject(c, hb.ref(), ob.ref(), injb.ref(), rows, H, S)
    gpu.run(c, "inject")
    assert np.allclose(hb.read(np.float32, (rows, S * H)),
                       ref.hc_inject(gh, ob.read(np.float32, (rows, H)), inj, rows, H, S), rtol=2e-6, atol=1e-6)
    lb.free()


@pytest.mark.parametrize("H,S,k,G", [(3072, 4, 320, 64), (1024, 4, 96, 32), (256, 2, 64, 128), (7680, 2, 64, 64),
                                     (1536, 3, 40, 32)])
def test_pre_decode_fused(gpu, H, S, k, G):
    """qw_op_hc_pre_decode (one launch) against the separate ops on the same
    inputs: injected streams, normed streams and injection logits bit-exact
    (the same arithmetic in the same order), the down-projection against the
    oracle; then against the oracle end to end."""
    print(f"hc pre decode H={H} S={S} k={k} G={G}", flush=True)
    g = _rng(31 + H)
    h4 = g.standard_normal((1, S * H)).astype(np.float32)
    prev = g.standard_normal((1, H)).astype(np.float32)
    pinj = g.standard_normal((1, S)).astype(np.float32)
    wn = synth.to_bf16(1.0 + 0.05 * g.standard_normal(S * H).astype(np.float32))
    down = _q4(32 + H, "hcf.down", k, S * H, G)
    binj = synth.to_bf16((0.02 * g.standard_normal((S, S * H))).astype(np.float32))
    B = gpu.Buf
    h_sep, pb, ib, wnb, bjb = B.of(h4), B.of(prev), B.of(pinj), B.of(wn), B.of(binj)
    dwb, dsb, dbb = B.of(down.w), B.of(down.s), B.of(down.b)
    n_sep, d_sep, i_sep = B(S * H * 4), B(k * 4), B(S * 4)
    h_in, h_out, n_f, d_f, i_f = B.of(h4), B(S * H * 4), B(S * H * 4), B(k * 4), B(S * 4)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_hc_inject_norm(c, h_sep.ref(), pb.ref(), ib.ref(), wnb.ref(), n_sep.ref(), 1, H, S, 1e-6)
    gpu.qw_op_qmv_q4(c, d_sep.ref(), n_sep.ref(), dwb.ref(), dsb.ref(), dbb.ref(), S * H, k, 1, G)
    gpu.qw_op_dmat_bf16(c, i_sep.ref(), n_sep.ref(), bjb.ref(), S * H, S, 1)
    assert gpu.qw_op_hc_pre_decode(c, h_out.ref(), n_f.ref(), d_f.ref(), i_f.ref(), h_in.ref(), pb.ref(), ib.ref(),
                                   wnb.ref(), dwb.ref(), dsb.ref(), dbb.ref(), bjb.ref(), H, S, k, G, 1e-6)
    assert not gpu.qw_op_hc_pre_decode(c, h_in.ref(), n_f.ref(), d_f.ref(), i_f.ref(), h_in.ref(), pb.ref(),
                                       ib.ref(), wnb.ref(), dwb.ref(), dsb.ref(), dbb.ref(), bjb.ref(), H, S, k, G,
                                       1e-6), "h4_out aliasing h4 is refused"
    gpu.run(c, "hc pre decode")
    u32 = lambda b, n: b.read(np.float32, (1, n)).view(np.uint32)
    assert np.array_equal(u32(h_out, S * H), u32(h_sep, S * H))
    assert np.array_equal(u32(n_f, S * H), u32(n_sep, S * H))
    assert np.array_equal(u32(i_f, S), u32(i_sep, S))
    assert np.array_equal(u32(h_in, S * H), h4.view(np.uint32)), "h4 is left as it was"
    n4 = n_f.read(np.float32, (1, S * H))
    assert rel_l2(d_f.read(np.float32, (1, k)), ref.qmv_q4(n4, down.w, down.s, down.b, S * H, k, 1, G)) < 1e-5
    assert rel_l2(d_f.read(np.float32, (1, k)), d_sep.read(np.float32, (1, k))) < 1e-5
    gh = ref.hc_inject(h4, prev, pinj, 1, H, S)
    assert np.allclose(h_out.read(np.float32, (1, S * H)), gh, rtol=2e-6, atol=1e-6)
    # the norm on the GPU's own injected streams, as the step-by-step test
    assert np.allclose(n4, ref.rms_norm_grouped(h_out.read(np.float32, (1, S * H)), wn, H, S, 1e-6),
                       rtol=2e-5, atol=0)
    assert np.array_equal(u32(i_f, S), ref.dmat_bf16(n4, binj, S * H, S, 1).view(np.uint32))


@pytest.mark.parametrize("H,S,k,G", [(3072, 4, 320, 64), (1024, 4, 96, 32), (256, 2, 128, 128), (7680, 2, 64, 64),
                                     (1536, 3, 64, 32), (2048, 1, 512, 64)])
def test_hc_decode_one_launch(gpu, H, S, k, G):
    """qw_op_hc_decode (the whole step in one launch, d handed over between
    workgroups) against qw_op_hc_pre_decode + qw_op_hc_mix_up on the same
    inputs: h4_out, n4 and the injection logits bit-exact (the same
    arithmetic in the same order); d, summed a stream at a time and the
    streams' partials added in order, against the separate op's (rel-L2
    1e-6) and the oracle's 4-bit matvec of n4 (rel-L2 1e-5); x against the
    oracle on the GPU's own d and n4 (rel-L2 1e-5, as the mix-up op); three
    steps in a row, each on the last one's streams, so every launch takes a
    new epoch."""
    print(f"hc decode H={H} S={S} k={k} G={G}", flush=True)
    g = _rng(41 + H + k)
    h4 = g.standard_normal((1, S * H)).astype(np.float32)
    wn = synth.to_bf16(1.0 + 0.05 * g.standard_normal(S * H).astype(np.float32))
    down = _q4(42 + H, "hcd.down", k, S * H, G)
    up = _q4(43 + H, "hcd.up", S * H, k, G)
    binj = synth.to_bf16((0.02 * g.standard_normal((S, S * H))).astype(np.float32))
    B = gpu.Buf
    wnb, bjb = B.of(wn), B.of(binj)
    dwb, dsb, dbb = B.of(down.w), B.of(down.s), B.of(down.b)
    uwb, usb, ubb = B.of(up.w), B.of(up.s), B.of(up.b)
    u32 = lambda b, n: b.read(np.float32, (1, n)).view(np.uint32)
    cur = h4
    for step in range(3):
        prev = g.standard_normal((1, H)).astype(np.float32)
        pinj = g.standard_normal((1, S)).astype(np.float32)
        hb, pb, ib = B.of(cur), B.of(prev), B.of(pinj)
        h_s, n_s, d_s, i_s, x_s = B(S * H * 4), B(S * H * 4), B(k * 4), B(S * 4), B(H * 4)
        h_f, n_f, d_f, i_f, x_f = B(S * H * 4), B(S * H * 4), B(k * 4), B(S * 4), B(H * 4)
        c = gpu.qw_cmd_begin()
        assert gpu.qw_op_hc_pre_decode(c, h_s.ref(), n_s.ref(), d_s.ref(), i_s.ref(), hb.ref(), pb.ref(), ib.ref(),
                                       wnb.ref(), dwb.ref(), dsb.ref(), dbb.ref(), bjb.ref(), H, S, k, G, 1e-6)
        assert gpu.qw_op_hc_mix_up(c, x_s.ref(), d_s.ref(), n_s.ref(), uwb.ref(), usb.ref(), ubb.ref(), k, H, S, 1,
                                   1.0 / S, G)
        assert gpu.qw_op_hc_decode(c, x_f.ref(), h_f.ref(), n_f.ref(), d_f.ref(), i_f.ref(), hb.ref(), pb.ref(),
                                   ib.ref(), wnb.ref(), dwb.ref(), dsb.ref(), dbb.ref(), bjb.ref(), uwb.ref(),
                                   usb.ref(), ubb.ref(), H, S, k, G, 1e-6, 1.0 / S)
        assert not gpu.qw_op_hc_decode(c, x_f.ref(), hb.ref(), n_f.ref(), d_f.ref(), i_f.ref(), hb.ref(), pb.ref(),
                                       ib.ref(), wnb.ref(), dwb.ref(), dsb.ref(), dbb.ref(), bjb.ref(), uwb.ref(),
                                       usb.ref(), ubb.ref(), H, S, k, G, 1e-6, 1.0 / S), "h4_out aliasing h4"
        gpu.run(c, f"hc decode step {step}")
        assert np.array_equal(u32(h_f, S * H), u32(h_s, S * H)), "injected streams"
        assert np.array_equal(u32(n_f, S * H), u32(n_s, S * H)), "normed streams"
        assert np.array_equal(u32(i_f, S), u32(i_s, S)), "injection logits"
        n4 = n_f.read(np.float32, (1, S * H))
        d = d_f.read(np.float32, (1, k))
        assert rel_l2(d, d_s.read(np.float32, (1, k))) < 1e-6, "down-projection against the separate op"
        assert rel_l2(d, ref.qmv_q4(n4, down.w, down.s, down.b, S * H, k, 1, G)) < 1e-5, "down-projection"
        want = ref.hc_mix_up(d, n4, up.w, up.s, up.b, k, H, S, 1, 1.0 / S, G)
        e = rel_l2(x_f.read(np.float32, (1, H)), want)
        assert e < 1e-5, f"step {step}: rel-L2 {e:.3g}"
        assert rel_l2(x_f.read(np.float32, (1, H)), x_s.read(np.float32, (1, H))) < 1e-5
        cur = h_f.read(np.float32, (1, S * H))


def test_hc_decode_refusals(gpu):
    """Shapes the one launch does not take are refused with nothing encoded
    (no command is needed to ask)."""
    r = gpu.NULL_REF
    args = lambda H, S, k, G: (None, r, r, r, r, r, r, r, r, r, r, r, r, r, r, r, r, H, S, k, G, 1e-6, 0.25)
    assert gpu.qw_op_hc_decode(*args(3072, 4, 320, 64))
    assert not gpu.qw_op_hc_decode(*args(3072, 5, 320, 64)), "S above 4"
    assert not gpu.qw_op_hc_decode(*args(3072, 4, 576, 64)), "lowrank above 512"
    assert not gpu.qw_op_hc_decode(*args(3072, 4, 100, 32)), "lowrank not a multiple of 8 and of the group"
    assert not gpu.qw_op_hc_decode(*args(4096, 4, 320, 64)), "S*H above 15360"


def test_hc_decode_give_up(gpu):
    """With the hand-off error word raised (as if a wait had given up), the
    one launch still ends (its waits see the word and give up at once), the
    command reports the failure, and the next launch runs normally."""
    H, S, k, G = 1024, 4, 96, 32
    g = _rng(4400)
    h4 = g.standard_normal((1, S * H)).astype(np.float32)
    prev = g.standard_normal((1, H)).astype(np.float32)
    pinj = g.standard_normal((1, S)).astype(np.float32)
    wn = synth.to_bf16(1.0 + 0.05 * g.standard_normal(S * H).astype(np.float32))
    down, up = _q4(4401, "hcg.down", k, S * H, G), _q4(4402, "hcg.up", S * H, k, G)
    binj = synth.to_bf16((0.02 * g.standard_normal((S, S * H))).astype(np.float32))
    B = gpu.Buf
    ins = [B.of(a) for a in (h4, prev, pinj, wn, down.w, down.s, down.b, binj, up.w, up.s, up.b)]
    outs = [B(S * H * 4), B(S * H * 4), B(k * 4), B(S * 4), B(H * 4)]
    hb, pb, ib, wnb, dwb, dsb, dbb, bjb, uwb, usb, ubb = ins
    h_f, n_f, d_f, i_f, x_f = outs

    def step():
        c = gpu.qw_cmd_begin()
        assert gpu.qw_op_hc_decode(c, x_f.ref(), h_f.ref(), n_f.ref(), d_f.ref(), i_f.ref(), hb.ref(), pb.ref(),
                                   ib.ref(), wnb.ref(), dwb.ref(), dsb.ref(), dbb.ref(), bjb.ref(), uwb.ref(),
                                   usb.ref(), ubb.ref(), H, S, k, G, 1e-6, 1.0 / S)
        gpu.qw_cmd_wait(c)
        e = gpu.qw_cmd_error(c)
        gpu.qw_cmd_free(c)
        return e

    assert gpu.qw_debug_decode_handoff_fail()
    e = step()
    assert e is not None and b"hand-off wait gave up" in e
    assert step() is None
    want = ref.hc_mix_up(d_f.read(np.float32, (1, k)), n_f.read(np.float32, (1, S * H)), up.w, up.s, up.b, k, H,
                         S, 1, 1.0 / S, G)
    assert rel_l2(x_f.read(np.float32, (1, H)), want) < 1e-5
