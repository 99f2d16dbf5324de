"""CPU checks for the hyper-connection mixer's oracle (oracle/moe_ref.c):
the grouped norm bit-exact against the reference's own qw_cpu_rms_norm
(qwasar_cpu.c:68-82, compiled into oracle/_ref) applied group by group with
its weight slice; the mix and the injection against fp64 and their exact
special cases."""
import numpy as np
import pytest

from oracle import ref
from qwasar_amd import synth


def test_rms_norm_grouped_bit_exact_against_reference():
    R = ref.reflib()
    if R is None:
        pytest.skip("oracle/_ref not built")
    g = np.random.default_rng(3)
    rows, S, H = 3, 4, 256
    x = (g.standard_normal((rows, S * H)) * 2).astype(np.float32)
    w = synth.to_bf16(1.0 + 0.1 * g.standard_normal(S * H).astype(np.float32))
    got = ref.rms_norm_grouped(x, w, H, S, 1e-6)
    want = np.empty_like(x)
    for r in range(rows):
        for s in range(S):
            xs = np.ascontiguousarray(x[r, s * H:(s + 1) * H])
            ys = np.empty_like(xs)
            ws = np.ascontiguousarray(w[s * H:(s + 1) * H])
            R.qw_cpu_rms_norm(ys.ctypes.data, xs.ctypes.data, ws.ctypes.data, H, 1, np.float32(1e-6), np.float32(1.0))
            want[r, s * H:(s + 1) * H] = ys
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _sig64(v):
    return 1.0 / (1.0 + np.exp(-np.asarray(v, np.float64)))


def test_hc_mix_against_fp64_and_exact_cases():
    g = np.random.default_rng(4)
    rows, S, H = 2, 4, 64
    n = g.standard_normal((rows, S * H)).astype(np.float32)
    m = (g.standard_normal((rows, S * H)) * 3).astype(np.float32)
    got = ref.hc_mix(n, m, rows, H, S)
    want = (_sig64(m) * n).reshape(rows, S, H).sum(axis=1) / S
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6)
    # sigmoid(100) rounds to exactly 1, and with two equal streams the sum
    # (n + n = 2n) and the mean are exact: the stream itself
    same = np.tile(n[:, :H], (1, 2))
    assert np.array_equal(ref.hc_mix(same, np.full_like(same, 100.0), rows, H, 2), n[:, :H])


def test_hc_inject_and_repeat():
    g = np.random.default_rng(5)
    rows, S, H = 3, 4, 32
    h4 = g.standard_normal((rows, S * H)).astype(np.float32)
    out = g.standard_normal((rows, H)).astype(np.float32)
    inj = (g.standard_normal((rows, S)) * 4).astype(np.float32)
    got = ref.hc_inject(h4, out, inj, rows, H, S)
    wgt = 2 * _sig64(inj / S)
    want = h4.astype(np.float64) + np.repeat(out[:, None, :], S, axis=1).reshape(rows, S * H) * np.repeat(wgt, H, axis=1)
    assert np.allclose(got, want, rtol=1e-6, atol=1e-6)
    # inj = 0: weight 2 * sigmoid(0) = 1 exactly, so h4 + out exactly
    got0 = ref.hc_inject(h4, out, np.zeros_like(inj), rows, H, S)
    assert np.array_equal(got0, h4 + np.tile(out, (1, S)))
    assert np.array_equal(ref.repeat_cols(out, rows, H, S), np.tile(out, (1, S)))


def test_silu_scale():
    y = np.linspace(-8, 8, 1001).astype(np.float32)
    got = ref.silu_scale(y, 0.25)
    v = y.astype(np.float64) * 0.25
    assert np.allclose(got, v * _sig64(v), rtol=2e-6, atol=1e-7)
