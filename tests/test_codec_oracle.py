"""Pins the codec oracle (oracle/codec_oracle.py) on the CPU: convolution padding and tap
direction, LayerNorm, the codec GELU's erf, the x2 upsampling."""
import math

import numpy as np
import pytest

import codec_oracle as co


def _metal_conv1d_same(x, w, b):
    """The index arithmetic of mit2_conv1d_same_f32 (kernels.metal:1397-1426), literally."""
    T, cin = x.shape
    cout, _, k = w.shape
    pad = k // 2
    out = np.zeros((T, cout))
    for t in range(T):
        for o in range(cout):
            acc = b[o]
            for i in range(cin):
                for j in range(k):
                    src = t + j - pad
                    if 0 <= src < T:
                        acc += x[src, i] * w[o, i, j]
            out[t, o] = acc
    return out


@pytest.mark.parametrize("T,cin,cout,k", [(5, 3, 2, 3), (5, 2, 3, 7), (1, 2, 2, 7), (9, 4, 4, 7)])
def test_conv1d_same_matches_kernel_arithmetic(T, cin, cout, k):
    rng = np.random.default_rng(T * 100 + k)
    x, w, b = rng.standard_normal((T, cin)), rng.standard_normal((cout, cin, k)), rng.standard_normal(cout)
    np.testing.assert_allclose(co.conv1d_same(x, w, b), _metal_conv1d_same(x, w, b), rtol=0, atol=1e-12)


@pytest.mark.parametrize("k,tap", [(7, 3), (7, 0), (7, 6), (3, 1), (3, 2)])
def test_conv1d_same_impulse_is_a_shift(k, tap):
    """An identity channel map at tap j gives out[t] = x[t + j - k/2] (zero outside [0, T))."""
    rng = np.random.default_rng(k + tap)
    T, c = 11, 4
    x = rng.standard_normal((T, c))
    w = np.zeros((c, c, k))
    w[:, :, tap] = np.eye(c)
    out = co.conv1d_same(x, w, np.zeros(c))
    s = tap - k // 2
    for t in range(T):
        exp = x[t + s] if 0 <= t + s < T else np.zeros(c)
        np.testing.assert_array_equal(out[t], exp)
    # the same through the depthwise form
    dw = np.zeros((c, 1, k))
    dw[:, 0, tap] = 1.0
    np.testing.assert_array_equal(co.dwconv_same(x, dw, np.zeros(c)), out)


def test_dwconv_same_is_the_diagonal_of_conv1d_same():
    rng = np.random.default_rng(3)
    T, c, k = 8, 5, 7
    x, dw, b = rng.standard_normal((T, c)), rng.standard_normal((c, 1, k)), rng.standard_normal(c)
    full = np.zeros((c, c, k))
    for i in range(c):
        full[i, i] = dw[i, 0]
    np.testing.assert_allclose(co.dwconv_same(x, dw, b), co.conv1d_same(x, full, b), rtol=0, atol=1e-12)


def test_layernorm_rows_are_standardised():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((6, 384)) * 3 + 1
    y = co.layernorm(x, np.ones(384), np.zeros(384), eps=0.0)
    np.testing.assert_allclose(y.mean(axis=1), 0, atol=1e-12)
    np.testing.assert_allclose(y.var(axis=1), 1, atol=1e-12)
    # eps enters under the square root: a constant row maps to beta
    z = co.layernorm(np.full((1, 384), 2.5), np.full(384, 7.0), np.full(384, 0.25))
    np.testing.assert_array_equal(z, np.full((1, 384), 0.25))


def test_codec_erf_within_published_bound():
    """Abramowitz & Stegun 7.1.26 promises |error| <= 1.5e-7; a coefficient off by 1e-4 breaks it."""
    xs = np.linspace(-6, 6, 24001)
    ref = np.array([math.erf(v) for v in xs])
    assert np.max(np.abs(co.erf_as(xs) - ref)) <= 1.5e-7
    saved = co._AS
    try:
        co._AS = (saved[0], saved[1] + 1e-4, *saved[2:])  # a planted mistake
        assert np.max(np.abs(co.erf_as(xs) - ref)) > 1.5e-7
    finally:
        co._AS = saved
    g = co.codec_gelu(xs)
    exact = 0.5 * xs * (1.0 + np.array([math.erf(v / math.sqrt(2.0)) for v in xs]))
    assert np.max(np.abs(g - exact)) <= 0.5 * 6 * 1.5e-7


def test_nearest_up2_repeats_rows():
    x = np.arange(15.0).reshape(5, 3)
    np.testing.assert_array_equal(co.nearest_up2(x), np.repeat(x, 2, axis=0))


def test_lookup_rejects_out_of_range_codes():
    w = {"codec.quantizer.quantizers.0.codebook.weight": np.zeros((8192, 8)),
         "codec.quantizer.quantizers.0.out_project.weight": np.zeros((1024, 8)),
         "codec.quantizer.quantizers.0.out_project.bias": np.zeros(1024)}
    for bad in ([], [8192], list(range(5001))):
        with pytest.raises(ValueError, match="Codec expects 1..5000 code IDs"):
            co.lookup(w, bad)
    assert co.lookup(w, [0, 8191]).shape == (2, 1024)
