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


# ---------------------------------------------------------------- the composition (codec.cpp:36-48, 64-72)

MUTATIONS = ["no_residual", "up_after_conv", "swap_pw", "norm_first", "gelu_after"]


def _codec_weights(seed, blocks, gamma=None):
    """Random codec decode weights at the real widths for `blocks` ConvNeXt blocks (numpy only)."""
    rng = np.random.default_rng(seed)
    q, d = "codec.quantizer.quantizers.0", "codec.decoder.0"
    H, W, F = co.HIDDEN, co.WIDTH, co.FFN
    n = lambda *s, sd=0.05, m=0.0: m + sd * rng.standard_normal(s)
    w = {f"{q}.codebook.weight": n(64, 8, sd=1.0), f"{q}.out_project.weight": n(W, 8, sd=0.3), f"{q}.out_project.bias": n(W),
         f"{d}.embed.weight": n(H, W, 7, sd=0.02), f"{d}.embed.bias": n(H),
         f"{d}.norm.weight": n(H, sd=0.1, m=1.0), f"{d}.norm.bias": n(H, sd=0.1)}
    for i in range(blocks):
        l = f"{d}.convnext.{i}"
        w.update({f"{l}.dwconv.weight": n(H, 1, 7, sd=0.3), f"{l}.dwconv.bias": n(H),
                  f"{l}.norm.weight": n(H, sd=0.1, m=1.0), f"{l}.norm.bias": n(H, sd=0.1),
                  f"{l}.pwconv1.weight": n(F, H), f"{l}.pwconv1.bias": n(F),
                  f"{l}.pwconv2.weight": n(H, F, sd=0.03), f"{l}.pwconv2.bias": n(H),
                  f"{l}.gamma": n(H, sd=0.1, m=0.5) if gamma is None else np.full(H, gamma)})
    w.update({f"{d}.final_layer_norm.weight": n(H, sd=0.1, m=1.0), f"{d}.final_layer_norm.bias": n(H, sd=0.1),
              "codec.decoder.1.weight": n(W, H), "codec.decoder.1.bias": n(W),
              "codec.up.weight": n(W, W, 3, sd=0.02), "codec.up.bias": n(W)})
    return w


def _torch_vocos_decode(w, codes, blocks):
    """decode() as an independent float64 forward: torch's own conv1d (zero padding k // 2,
    groups = C for the depthwise conv), layer_norm (eps 1e-6), exact-erf gelu, linear and
    nearest interpolate, in the channels-first [1, C, T] layout of the published Vocos backbone
    (VocosBackbone / ConvNeXtBlock: x + gamma * pwconv2(gelu(pwconv1(norm(dwconv(x)))))), then
    the x2 upsampling and the k = 3 convolution of codec.up."""
    import torch
    import torch.nn.functional as F

    t = lambda name: torch.from_numpy(np.asarray(w[name], np.float64))
    q, d, H = "codec.quantizer.quantizers.0", "codec.decoder.0", co.HIDDEN
    ln = lambda x, p: F.layer_norm(x.transpose(1, 2), (H,), t(p + ".weight"), t(p + ".bias"), eps=1e-6).transpose(1, 2)
    e = F.embedding(torch.tensor([int(c) for c in codes]), t(q + ".codebook.weight"))
    x = F.linear(e, t(q + ".out_project.weight"), t(q + ".out_project.bias")).T.unsqueeze(0)
    x = ln(F.conv1d(x, t(d + ".embed.weight"), t(d + ".embed.bias"), padding=3), d + ".norm")
    for i in range(blocks):
        l = f"{d}.convnext.{i}"
        y = ln(F.conv1d(x, t(l + ".dwconv.weight"), t(l + ".dwconv.bias"), padding=3, groups=H), l + ".norm")
        y = F.linear(F.gelu(F.linear(y.transpose(1, 2), t(l + ".pwconv1.weight"), t(l + ".pwconv1.bias"))),
                     t(l + ".pwconv2.weight"), t(l + ".pwconv2.bias"))
        x = x + (t(l + ".gamma") * y).transpose(1, 2)
    x = ln(x, d + ".final_layer_norm")
    x = F.linear(x.transpose(1, 2), t("codec.decoder.1.weight"), t("codec.decoder.1.bias")).transpose(1, 2)
    x = F.interpolate(x, scale_factor=2, mode="nearest")
    return F.conv1d(x, t("codec.up.weight"), t("codec.up.bias"), padding=1)[0].T.numpy()


def _with_mutation(m, fn):
    saved = co.MUTATION
    try:
        co.MUTATION = m
        return fn()
    finally:
        co.MUTATION = saved


def test_decode_with_zero_layer_scales_is_the_outer_chain():
    """gamma = 0 makes every ConvNeXt block x + 0 * h = x, so decode() must reduce to
    up(repeat2(decoder.1(final_LN(norm(embed(lookup)))))) (codec.cpp:40-47, 66-70), composed here
    from the separately pinned pieces and np.repeat.  A dropped residual (x = gamma * h) or the
    upsampling after codec.up breaks it."""
    w = _codec_weights(7, blocks=3, gamma=0.0)
    codes = [3, 17, 0, 63, 5, 9]
    d = "codec.decoder.0"
    x = co.lookup(w, codes)
    x = co.layernorm(co.conv1d_same(x, w[d + ".embed.weight"], w[d + ".embed.bias"]), w[d + ".norm.weight"], w[d + ".norm.bias"])
    x = co.layernorm(x, w[d + ".final_layer_norm.weight"], w[d + ".final_layer_norm.bias"])
    x = x @ w["codec.decoder.1.weight"].T + w["codec.decoder.1.bias"]
    exp = co.conv1d_same(np.repeat(x, 2, axis=0), w["codec.up.weight"], w["codec.up.bias"])
    got = co.decode(w, codes, blocks=3)
    assert got.shape == (12, 1024)
    np.testing.assert_allclose(got, exp, rtol=0, atol=1e-12)
    for m in ("no_residual", "up_after_conv"):
        bad = _with_mutation(m, lambda: co.decode(w, codes, blocks=3))
        assert np.max(np.abs(bad - exp)) > 1e-2, m


def test_decode_equals_independent_torch_vocos_forward():
    """decode() against the torch float64 forward on two blocks with nonzero layer scales, to
    within the codec GELU's erf approximation (|erf error| <= 1.5e-7); every planted mistake
    moves the output by more than 1e-3, far outside that."""
    pytest.importorskip("torch")
    w = _codec_weights(11, blocks=2)
    codes = [1, 2, 40, 63, 7, 7, 30, 0, 12]
    exp = _torch_vocos_decode(w, codes, 2)
    got = co.decode(w, codes, blocks=2)
    err = float(np.max(np.abs(got - exp)))
    assert err < 1e-6 * max(1.0, float(np.max(np.abs(exp)))), err
    for m in MUTATIONS:
        bad = _with_mutation(m, lambda: co.decode(w, codes, blocks=2))
        assert np.max(np.abs(bad - exp)) > 1e-3, m


def test_up_conv_order_by_a_shift_kernel():
    """codec.up as a one-row shift (identity at tap 0: out[t] = in[t - 1]) exposes the order of
    the x2 upsampling and the convolution: row 2i + 1 of the output is hidden row i and row 2i is
    hidden row i - 1 (zero for i = 0).  With the convolution first both rows would be hidden row
    i - 1."""
    w = _codec_weights(5, blocks=1)
    up = np.zeros((1024, 1024, 3))
    up[:, :, 0] = np.eye(1024)
    w["codec.up.weight"], w["codec.up.bias"] = up, np.zeros(1024)
    codes = [4, 8, 15, 16, 23]
    hidden = co.vocos(w, co.lookup(w, codes), "codec.decoder", 1)
    out = co.decode(w, codes, blocks=1)
    for i in range(len(codes)):
        np.testing.assert_array_equal(out[2 * i + 1], hidden[i])
        np.testing.assert_array_equal(out[2 * i], hidden[i - 1] if i else np.zeros(1024))
    bad = _with_mutation("up_after_conv", lambda: co.decode(w, codes, blocks=1))
    assert not np.array_equal(bad[1::2], hidden)
