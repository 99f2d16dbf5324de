"""The layer stack of BASELINE config 4 on the GPU against the CPU oracle:
the device generator against its host restatement, qw_op_rms_norm and the
residual step against oracle/ref.py, and stacks of MoE layers run both
layer by layer (each layer's GPU input fed to the oracle: routing ids and
weights bit-exact, outputs to the layer tests' tolerance, the bf16 carry
bit-exact) and free-running (final h against the oracle's stack).

Tolerances: the norm is held to 2e-6 relative per element against the same
norm in fp64; against the oracle, whose serial fp32 sum of squares carries
an error growing with the row length (about 2.5e-6 at 3072), to 3e-5.  A MoE
layer to its own bar (rel-L2 5e-4 on the decode path, 1e-3 grouped); the
free-running stack's final h, where the small differences pass through 48
bf16 roundings and renormalisations, to rel-L2 1e-2."""
import numpy as np
import pytest

from oracle import ref
from qwasar_amd import stack, synth

pytestmark = pytest.mark.gpu


def norm64(h_bits):
    """rms_norm of bf16 rows in fp64 (eps 1e-6), the exact value the fp32 norms round."""
    h = synth.bf16_to_f32(h_bits).astype(np.float64)
    return h / np.sqrt((h * h).mean(axis=-1, keepdims=True) + 1e-6)


def check_norm(x, h_bits, want_oracle):
    assert np.allclose(x, norm64(h_bits), rtol=2e-6, atol=0), "norm off its fp64 value"
    assert np.allclose(x, want_oracle, rtol=3e-5, atol=0), "norm off the oracle"


def rel_l2(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.sqrt(((a - b) ** 2).sum() / (b * b).sum()))


@pytest.mark.parametrize("kind,nbytes", [(synth.SYNTH_U32, 4), (synth.SYNTH_BF16_UNIFORM, 2),
                                         (synth.SYNTH_BF16_NEG8, 2), (synth.SYNTH_BF16_NORMAL, 2),
                                         (synth.SYNTH_F32_BF16_NORMAL, 4)])
def test_synth_matches_host(gpu, kind, nbytes):
    n = 300007
    key = synth.sm_key(11, f"kind{kind}")
    a, b = (0.001, 0.02) if kind in (synth.SYNTH_BF16_UNIFORM, synth.SYNTH_BF16_NEG8) else (0.7, 0.0)
    buf = gpu.Buf(n * nbytes)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_synth(c, buf.ref(), kind, n, key, a, b)
    gpu.run(c, "synth")
    dt = {4: np.uint32, 2: np.uint16}[nbytes]
    got = buf.read(dt, (n,))
    want = synth.sm_values(kind, n, key, a, b).view(dt)
    if kind in (synth.SYNTH_BF16_NORMAL, synth.SYNTH_F32_BF16_NORMAL):
        # log and cos in double on the device and on the host may differ in
        # the last bit, which the bf16 rounding almost always absorbs
        diff = got != want
        assert diff.mean() < 1e-4, f"{diff.sum()} of {n} differ"
        g = got[diff].astype(np.int64) >> (16 if nbytes == 4 else 0)
        w = want[diff].astype(np.int64) >> (16 if nbytes == 4 else 0)
        assert np.all(np.abs(g - w) <= 1)
    else:
        assert np.array_equal(got, want)


@pytest.mark.parametrize("dim,rows", [(3072, 5), (256, 3), (64, 1)])
def test_rms_norm_op(gpu, dim, rows):
    g = np.random.default_rng(dim + rows)
    x = (g.standard_normal((rows, dim)) * 2.0).astype(np.float32)
    wt = synth.to_bf16(g.standard_normal(dim).astype(np.float32))
    xb, yb, wb = gpu.Buf.of(x), gpu.Buf(x.nbytes), gpu.Buf.of(wt)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_rms_norm(c, yb.ref(), xb.ref(), gpu.NULL_REF, dim, rows, 1e-6, 1.0)
    gpu.run(c, "rms_norm")
    got = yb.read(np.float32, (rows, dim))
    want = ref.rms_norm(x, 1e-6)
    x64 = x.astype(np.float64)
    assert np.allclose(got, x64 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + 1e-6), rtol=2e-6, atol=0)
    assert np.allclose(got, want, rtol=3e-5, atol=0)
    # weight and out_scale, applied after normalising as the reference does
    c = gpu.qw_cmd_begin()
    gpu.qw_op_rms_norm(c, yb.ref(), xb.ref(), wb.ref(), dim, rows, 1e-6, 0.25)
    gpu.run(c, "rms_norm weighted")
    got = yb.read(np.float32, (rows, dim))
    assert np.allclose(got, want * np.float32(0.25) * synth.bf16_to_f32(wt), rtol=3e-5, atol=0)


@pytest.mark.parametrize("dim,rows", [(3072, 7), (256, 33)])
def test_residual_norm_op(gpu, dim, rows):
    g = np.random.default_rng(dim * rows)
    h = synth.to_bf16(g.standard_normal((rows, dim)).astype(np.float32))
    y = (g.standard_normal((rows, dim)) * 0.3).astype(np.float32)
    hb, xb, yb = gpu.Buf.of(h), gpu.Buf(rows * dim * 4), gpu.Buf.of(y)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_residual_rms_norm_bf16(c, hb.ref(), xb.ref(), yb.ref(), dim, rows, 1e-6)
    gpu.run(c, "residual norm")
    wh, wx = ref.residual_norm(h, y)
    assert np.array_equal(hb.read(np.uint16, (rows, dim)), wh), "bf16 carry not bit-exact"
    check_norm(xb.read(np.float32, (rows, dim)), wh, wx)
    # without y: h untouched
    c = gpu.qw_cmd_begin()
    gpu.qw_op_residual_rms_norm_bf16(c, hb.ref(), xb.ref(), gpu.NULL_REF, dim, rows, 1e-6)
    gpu.run(c, "norm only")
    assert np.array_equal(hb.read(np.uint16, (rows, dim)), wh)
    check_norm(xb.read(np.float32, (rows, dim)), wh, ref.rms_norm(synth.bf16_to_f32(wh)))


def _layerwise(gpu, layers, hosts, h0, rows):
    """Runs the stack one layer per command; checks each layer against the
    oracle on the GPU's own input.  Returns the final h."""
    st = stack.Stack(layers, rows)
    st.h.write(h0)
    c = gpu.qw_cmd_begin()
    gpu.qw_op_residual_rms_norm_bf16(c, st.h.ref(), st.x.ref(), gpu.NULL_REF, st.H, rows, stack.EPS)
    gpu.run(c, "opening norm")
    h = h0
    tol = 5e-4 if rows <= 8 else 1e-3
    for l, L in enumerate(hosts):
        x = st.x.read(np.float32, (rows, st.H))
        c = gpu.qw_cmd_begin()
        st.encode(c, rows, first=l, count=1, start=False)
        gpu.run(c, f"layer {l}")
        y = st.y.read(np.float32, (rows, st.H))
        wy, widx, ww = ref.moe_forward(L, x)
        assert np.array_equal(st.idx.read(np.int32, (rows, L.K)), widx), f"layer {l}: routing ids differ"
        assert np.array_equal(st.w.read(np.float32, (rows, L.K)).view(np.uint32), ww.view(np.uint32)), \
            f"layer {l}: routing weights not bit-exact"
        e = rel_l2(y, wy)
        assert e < tol, f"layer {l}: rel-L2 {e:.3g}"
        wh, wx = ref.residual_norm(h, y)
        h = st.h.read(np.uint16, (rows, st.H))
        assert np.array_equal(h, wh), f"layer {l}: bf16 carry differs"
        check_norm(st.x.read(np.float32, (rows, st.H)), h, wx)
    st.free()
    return h


@pytest.mark.parametrize("rows", [24, 1, 3])
def test_stack_layer_by_layer_config0_shape(gpu, rows):
    """48 layers of config 0's shape (grouped path at 24 rows, decode at 1 and 3)."""
    c0 = dict(synth.CONFIGS[0])
    c0.pop("rows")
    layers = [stack.DeviceLayer(77, l, **c0) for l in range(48)]
    hosts = [L.host() for L in layers]
    h0 = synth.to_bf16(synth.normal(77, f"stack.h0.{rows}", rows * c0["H"]).astype(np.float32)).reshape(rows, -1)
    _layerwise(gpu, layers, hosts, h0, rows)
    for L in layers:
        L.free()


def test_stack_config1_shape_layer_by_layer_and_free_running(gpu):
    """Two layers of config 1's shape: 12 rows (grouped), then one decode row
    through the same layers; then the free-running stack against the oracle's."""
    c1 = dict(synth.CONFIGS[1])
    c1.pop("rows")
    layers = [stack.DeviceLayer(5, l, **c1) for l in range(2)]
    hosts = [L.host() for L in layers]
    for rows in (12, 1):
        h0 = synth.to_bf16(synth.normal(5, f"stack.h0.{rows}", rows * c1["H"]).astype(np.float32)).reshape(rows, -1)
        _layerwise(gpu, layers, hosts, h0, rows)
        st = stack.Stack(layers, rows)
        st.h.write(h0)
        c = gpu.qw_cmd_begin()
        st.encode(c, rows)
        gpu.run(c, "free-running stack")
        got = st.h.read(np.uint16, (rows, c1["H"]))
        want, _ = ref.stack_forward(hosts, h0)
        e = rel_l2(synth.bf16_to_f32(got), synth.bf16_to_f32(want))
        print(f"rows {rows}: free-running final h rel-L2 {e:.3g}")
        assert e < 1e-2
        st.free()
    for L in layers:
        L.free()


def _fused_equals_unfused(gpu, layers, h0, rows):
    """The fused stack (qw_op_moe_layer_residual: each residual step inside
    the next layer's op) gives the unfused stack's bits."""
    st = stack.Stack(layers, rows)
    st.h.write(h0)
    c = gpu.qw_cmd_begin()
    st.encode(c, rows)
    gpu.run(c, "unfused stack")
    want_h = st.h.read(np.uint16, (rows, st.H))
    want_x = st.x.read(np.float32, (rows, st.H))
    st.h.write(h0)
    c = gpu.qw_cmd_begin()
    st.encode_fused(c, rows)
    gpu.run(c, "fused stack")
    got_h = st.h_final.read(np.uint16, (rows, st.H))
    got_x = st.x.read(np.float32, (rows, st.H))
    assert np.array_equal(got_h, want_h), "fused stack h differs from the unfused one"
    assert np.array_equal(got_x.view(np.uint32), want_x.view(np.uint32)), "fused stack x differs"
    st.free()


@pytest.mark.parametrize("rows", [1, 3, 8, 12])
def test_stack_fused_residual_same_bits(gpu, rows):
    """qw_op_moe_layer_residual (the residual step inside the decode launch at
    <= 8 rows; the norm kernel then the grouped layer above) gives the
    unfused stack's bits: 5 layers of config 1's shape, and 48 of config 0's."""
    c1 = dict(synth.CONFIGS[1])
    c1.pop("rows")
    layers = [stack.DeviceLayer(31, l, **c1) for l in range(5)]
    h0 = synth.to_bf16(synth.normal(31, f"stack.h0f.{rows}", rows * c1["H"]).astype(np.float32)).reshape(rows, -1)
    _fused_equals_unfused(gpu, layers, h0, rows)
    for L in layers:
        L.free()
    c0 = dict(synth.CONFIGS[0])
    c0.pop("rows")
    layers = [stack.DeviceLayer(32, l, **c0) for l in range(48)]
    h0 = synth.to_bf16(synth.normal(32, f"stack.h0f0.{rows}", rows * c0["H"]).astype(np.float32)).reshape(rows, -1)
    _fused_equals_unfused(gpu, layers, h0, rows)
    for L in layers:
        L.free()


def test_stack_config4_full_size_decode(gpu):
    """Config 4 at full size: 48 layers of config 1's shape (~65 GB on the
    device), one decode token through all of them, twice: the same bits both
    times and with the residual step folded into each launch, and the first
    and last layers against the oracle on their inputs."""
    c1 = dict(synth.CONFIGS[1])
    c1.pop("rows")
    layers = [stack.DeviceLayer(2026, l, **c1) for l in range(48)]
    st = stack.Stack(layers, 1)
    h0 = synth.to_bf16(synth.normal(2026, "stack.h0.full", c1["H"]).astype(np.float32)).reshape(1, -1)
    outs = []
    for _ in range(2):
        st.h.write(h0)
        c = gpu.qw_cmd_begin()
        st.encode(c, 1)
        gpu.run(c, "48-layer decode")
        outs.append(st.h.read(np.uint16, (1, c1["H"])))
    assert np.array_equal(outs[0], outs[1]), "the stack is not deterministic"
    st.h.write(h0)
    c = gpu.qw_cmd_begin()
    st.encode_fused(c, 1)
    gpu.run(c, "48-layer decode, residual folded in")
    assert np.array_equal(st.h_final.read(np.uint16, (1, c1["H"])), outs[0]), "fused stack differs"
    assert np.isfinite(synth.bf16_to_f32(outs[0])).all()
    # the first and the last layer, each against the oracle on the GPU's input
    for l in (0, 47):
        st.h.write(h0)
        c = gpu.qw_cmd_begin()
        st.encode(c, 1, first=0, count=l)
        gpu.run(c, f"layers before {l}")
        x = st.x.read(np.float32, (1, c1["H"]))
        c = gpu.qw_cmd_begin()
        st.encode(c, 1, first=l, count=1, start=False)
        gpu.run(c, f"layer {l}")
        wy, widx, ww = ref.moe_forward(layers[l].host(), x)
        assert np.array_equal(st.idx.read(np.int32, (1, c1["K"])), widx)
        assert rel_l2(st.y.read(np.float32, (1, c1["H"])), wy) < 5e-4
    st.free()
    for L in layers:
        L.free()


def test_stack_config4_full_size_prefill(gpu):
    """Config 4's prefill at full size: 48 layers of config 1's shape, one
    2048-token chunk, twice (the same bits both times, and with the residual
    step folded into each layer's op); then the first and the last layer on
    their GPU inputs against the oracle: all 2048 x 10 routing ids and
    weights bit-exact, 128 sampled rows of y to the grouped bar, the bf16
    carry bit-exact on every row."""
    from tests import oracle_par
    c1 = dict(synth.CONFIGS[1])
    c1.pop("rows")
    rows = 2048
    layers = [stack.DeviceLayer(2027, l, **c1) for l in range(48)]
    st = stack.Stack(layers, rows)
    H, K = c1["H"], c1["K"]
    h0 = synth.to_bf16(synth.normal(2027, "stack.h0.prefill", rows * H).astype(np.float32)).reshape(rows, -1)
    outs = []
    for _ in range(2):
        st.h.write(h0)
        c = gpu.qw_cmd_begin()
        st.encode(c, rows)
        gpu.run(c, "48-layer prefill")
        outs.append(st.h.read(np.uint16, (rows, H)))
    assert np.array_equal(outs[0], outs[1]), "the prefill stack is not deterministic"
    st.h.write(h0)
    c = gpu.qw_cmd_begin()
    st.encode_fused(c, rows)
    gpu.run(c, "48-layer prefill, residual folded in")
    assert np.array_equal(st.h_final.read(np.uint16, (rows, H)), outs[0]), "fused stack differs"
    assert np.isfinite(synth.bf16_to_f32(outs[0])).all()
    sel = np.arange(3, rows, 16)
    for l in (0, 47):
        st.h.write(h0)
        c = gpu.qw_cmd_begin()
        st.encode(c, rows, first=0, count=l)
        gpu.run(c, f"layers before {l}")
        x = st.x.read(np.float32, (rows, H))
        h_in = st.h.read(np.uint16, (rows, H))
        c = gpu.qw_cmd_begin()
        st.encode(c, rows, first=l, count=1, start=False)
        gpu.run(c, f"layer {l}")
        L = layers[l].host()
        widx, ww = oracle_par.route_rows(L, x)
        idx = st.idx.read(np.int32, (rows, K))
        assert np.array_equal(idx, widx), f"layer {l}: {(idx != widx).sum()} routing ids differ"
        assert np.array_equal(st.w.read(np.float32, (rows, K)).view(np.uint32), ww.view(np.uint32)), \
            f"layer {l}: routing weights not bit-exact"
        y = st.y.read(np.float32, (rows, H))
        wy, _, _ = oracle_par.moe_rows(L, x[sel])
        e = rel_l2(y[sel], wy)
        m = float(np.abs(y[sel] - wy).max())
        ymax = float(np.abs(wy).max())
        print(f"layer {l}: y rel-L2 {e:.3g} max-abs {m:.3g} (max |y| {ymax:.4g}) on {sel.size} rows")
        # The max-abs bar is for outputs of order one.  Deep in the stack the
        # synthetic weights' non-zero mean (bias -8 * scale: mean -scale / 2)
        # has grown h along one direction and |y| reaches the thousands, so
        # there the bar scales with the output's largest magnitude.
        assert e < 1e-3 and m < 2e-2 * max(1.0, ymax), f"layer {l}: rel-L2 {e:.3g} max-abs {m:.3g}"
        wh, wx = ref.residual_norm(h_in, y)
        assert np.array_equal(st.h.read(np.uint16, (rows, H)), wh), f"layer {l}: bf16 carry differs"
        check_norm(st.x.read(np.float32, (rows, H)), wh, wx)
        del L
    st.free()
    for L in layers:
        L.free()
