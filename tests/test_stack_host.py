"""CPU checks for the layer stack's pieces: the oracle's RMS norm against
the reference's own qw_cpu_rms_norm (qwasar_cpu.c:68-82) and closed forms,
the residual step, and the host restatement of the device's SplitMix64
generator against the sequential algorithm and its published outputs."""
import numpy as np
import pytest

from oracle import ref
from qwasar_amd import synth


def _need_ref():
    R = ref.reflib()
    if R is None:
        pytest.skip("oracle/_ref not built (reference tree absent when it was built)")
    return R


@pytest.mark.parametrize("dim,rows", [(256, 3), (3072, 2), (64, 5), (7, 1)])
def test_rms_norm_bit_exact_against_reference(dim, rows):
    R = _need_ref()
    x = (np.random.default_rng(dim).standard_normal((rows, dim)) * 3.0).astype(np.float32)
    got = ref.rms_norm(x, 1e-6)
    want = np.empty_like(x)
    R.qw_cpu_rms_norm(want.ctypes.data, x.ctypes.data, None, dim, rows, np.float32(1e-6), np.float32(1.0))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_rms_norm_closed_forms():
    # a constant row c: y = c / sqrt(c^2 + eps)
    for c in (1.0, -3.5, 1e-3):
        x = np.full((1, 128), c, np.float32)
        y = ref.rms_norm(x, 1e-6)
        want = np.float32(c) / np.sqrt(np.float32(c) ** 2 + np.float32(1e-6))
        assert np.allclose(y, want, rtol=1e-6, atol=0)
    # unit mean square, and invariance to a power-of-two scale (exact in fp32)
    x = np.random.default_rng(5).standard_normal((4, 3072)).astype(np.float32)
    y = ref.rms_norm(x, 0.0)
    assert np.allclose((y.astype(np.float64) ** 2).mean(axis=1), 1.0, rtol=1e-5)
    assert np.array_equal(ref.rms_norm(x * np.float32(8.0), 0.0), y)


def test_residual_step():
    g = np.random.default_rng(9)
    h = synth.to_bf16(g.standard_normal((3, 256)).astype(np.float32))
    # no y: h unchanged, x its norm
    h2, x = ref.residual_norm(h, None)
    assert np.array_equal(h2, h)
    assert np.array_equal(x, ref.rms_norm(synth.bf16_to_f32(h)))
    # y = 0 keeps h; y exactly representable moves h by exactly y
    h3, _ = ref.residual_norm(h, np.zeros((3, 256), np.float32))
    assert np.array_equal(h3, h)
    y = synth.bf16_to_f32(h)       # h + h = 2h: exact in bf16
    h4, _ = ref.residual_norm(h, y)
    assert np.array_equal(synth.bf16_to_f32(h4), 2.0 * synth.bf16_to_f32(h))


def _splitmix_sequential(seed: int, n: int):
    m = (1 << 64) - 1
    s, out = seed, []
    for _ in range(n):
        s = (s + 0x9E3779B97F4A7C15) & m
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
        out.append(z ^ (z >> 31))
    return out


def test_splitmix_counter_form_is_the_sequential_generator():
    for seed in (0, 1, 1234567, 0xFFFFFFFFFFFFFFFF, synth.sm_key(7, "x")):
        assert [int(v) for v in synth.sm_raw(seed, 40)] == _splitmix_sequential(seed, 40)
        assert [int(v) for v in synth.sm_raw(seed, 5, start=33)] == _splitmix_sequential(seed, 38)[33:]


def test_splitmix_published_outputs():
    # the first outputs of SplitMix64 seeded with 1234567 (Vigna's splitmix64.c)
    assert [int(v) for v in synth.sm_raw(1234567, 5)] == [
        6457827717110365317, 3203168211198807973, 9817491932198370423,
        4593380528125082431, 16408922859458223821]


def test_synth_distributions():
    k = synth.sm_key(3, "t")
    s = synth.bf16_to_f32(synth.sm_values(synth.SYNTH_BF16_UNIFORM, 200000, k, 0.001, 0.02))
    assert s.min() >= 0.00099 and s.max() <= 0.0201 and abs(s.mean() - 0.0105) < 2e-4
    b = synth.bf16_to_f32(synth.sm_values(synth.SYNTH_BF16_NEG8, 200000, k, 0.001, 0.02))
    assert np.array_equal(b, -8.0 * s)
    nv = synth.sm_values(synth.SYNTH_F32_BF16_NORMAL, 200000, k, 1.0)
    assert abs(nv.mean()) < 0.01 and abs(nv.std() - 1.0) < 0.01
    assert np.array_equal(synth.bf16_to_f32(synth.sm_values(synth.SYNTH_BF16_NORMAL, 1000, k, 1.0)), nv[:1000])
    w = synth.sm_values(synth.SYNTH_U32, 100000, k)
    nib = ((w[:, None] >> (np.arange(8, dtype=np.uint32) * 4)) & 0xF).ravel()
    counts = np.bincount(nib, minlength=16)
    assert counts.min() > 0.9 * counts.mean()
