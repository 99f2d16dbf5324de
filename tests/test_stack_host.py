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


def _bits(v):
    return synth.to_bf16(np.array([v], np.float32))[0]


def test_residual_carry_rounds_to_nearest_even():
    """The bf16 carry h' = bf16(h + y) rounds to nearest, ties to even, on the
    fp32 sum.  At h = 1 the bf16 spacing is 2^-7: y = 2^-8 is a tie (even
    keeps 1), y = 3*2^-8 a tie whose even neighbour is above (1 + 2^-6),
    y = 3*2^-9 above the midpoint (up; truncation would go down), y = 2^-9
    below it (down); and the same mirrored.  Truncation, round-half-up or
    round-half-away each fail one of these."""
    u = 2.0 ** -7
    cases = [  # (h, y, expected h')
        (1.0, 2.0 ** -8, 1.0),
        (1.0, 3 * 2.0 ** -8, 1.0 + 2 * u),
        (1.0, 3 * 2.0 ** -9, 1.0 + u),
        (1.0, 2.0 ** -9, 1.0),
        (1.0 + u, 2.0 ** -8, 1.0 + 2 * u),         # a tie from an odd mantissa: up to even
        (-1.0, -(2.0 ** -8), -1.0),
        (-1.0, -3 * 2.0 ** -8, -1.0 - 2 * u),
        (-1.0, -3 * 2.0 ** -9, -1.0 - u),
        (-1.0 - u, -(2.0 ** -8), -1.0 - 2 * u),
        (1.0, -(2.0 ** -9), 1.0),                  # below 1 the spacing halves: 1 - 2^-9 is a tie
        (1.0, -3 * 2.0 ** -10, 1.0 - 2.0 ** -8),   # between 1 - 2^-8 and 1, nearer the former
    ]
    h = np.array([_bits(c[0]) for c in cases], np.uint16).reshape(1, -1)
    y = np.array([c[1] for c in cases], np.float32).reshape(1, -1)
    got, _ = ref.residual_norm(h, y)
    want = np.array([_bits(c[2]) for c in cases], np.uint16)
    assert np.array_equal(got.ravel(), want), f"{got.ravel()} vs {want}"


def test_residual_carry_is_the_nearest_bf16():
    """On random sums: h' is one of the two bf16 values around the fp32 sum
    h + y, the nearer (distances in fp64), the even one at a tie."""
    g = np.random.default_rng(31)
    h = synth.to_bf16(g.standard_normal(200000).astype(np.float32)).reshape(1, -1)
    y = (g.standard_normal(200000) * 0.05).astype(np.float32).reshape(1, -1)
    # some exact ties: y = half a bf16 spacing of h
    hf = synth.bf16_to_f32(h)
    e = np.floor(np.log2(np.abs(hf[0, :1000]) + 1e-30))
    y[0, :1000] = (2.0 ** (e - 8)).astype(np.float32)
    got, _ = ref.residual_norm(h, y)
    s = (synth.bf16_to_f32(h) + y).astype(np.float32).ravel().astype(np.float64)
    lo = (np.asarray(s, np.float32).view(np.uint32) & 0xFFFF0000).view(np.float32).astype(np.float64)
    lo_bits = (np.asarray(s, np.float32).view(np.uint32) >> 16).astype(np.uint16)
    hi_bits = (lo_bits.astype(np.uint32) + 1).astype(np.uint16)
    hi = synth.bf16_to_f32(hi_bits).astype(np.float64)
    d_lo, d_hi = np.abs(s - lo), np.abs(hi - s)
    want = np.where(d_lo < d_hi, lo_bits, np.where(d_hi < d_lo, hi_bits,
                                                   np.where(lo_bits % 2 == 0, lo_bits, hi_bits)))
    assert np.array_equal(got.ravel(), want)
    assert (d_lo == d_hi).sum() >= 900   # the ties were exercised
