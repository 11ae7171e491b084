"""CPU restatement of EnhancedCodec::decode (src/codec.cpp:57-72) in float64 numpy.

TEST INFRASTRUCTURE ONLY: imported by tests/, which compare the HIP codec decode against it.

Each function follows the reference op it names:
  * lookup           codec.cpp:57-63: codebook rows (mit2_embedding_f32, kernels.metal:281-294),
                     then out_project, y = x W^T + b (linear_rows_f32).
  * conv1d_same      mit2_conv1d_same_f32 (kernels.metal:1397-1426): pad = k / 2,
                     out[t][o] = b[o] + sum_i sum_j x[t + j - pad][i] * w[o][i][j], zero outside [0, T).
  * dwconv_same      mit2_depthwise_conv1d_same_f32 (kernels.metal:1516-1541), weights [C][1][k].
  * layernorm        mit2_layernorm_f32_rows (kernels.metal:618-669): mean, biased variance of the
                     centred values, 1 / sqrt(var + eps); the codec uses eps 1e-6 (codec.cpp:28).
  * codec_gelu       itts25_codec_gelu (kernels.metal:3133-3137): 0.5 x (1 + erf(x / sqrt 2)) with
                     erf from Abramowitz & Stegun 7.1.26.
  * nearest_up2      mit2_nearest_interpolate_f32 (kernels.metal:1376-1395) with scale in/out = 1/2:
                     row j of the output is row floor(j / 2) of the input.
  * vocos / decode   codec.cpp:36-48 and 64-72.
What pins each one (tests/test_codec_oracle.py): conv kernels that are a unit impulse at tap
j shift the input by j - pad (identity at j = pad) and a brute-force loop over the Metal
kernel's index arithmetic on tiny shapes; LayerNorm rows have zero mean and unit variance;
the GELU's erf is within the published 1.5e-7 bound of math.erf on a dense grid (a wrong
coefficient breaks the bound); the upsampling equals np.repeat(x, 2).
The composition (vocos() and decode(), codec.cpp:36-48 and 64-72) is pinned by two checks:
with every layer scale gamma = 0 the ConvNeXt blocks are the identity and decode() reduces to
up(repeat2(linear(LN(LN(embed(lookup)))))); and decode() equals an independent float64
forward built from torch's conv1d / layer_norm / gelu / linear / interpolate in the published
Vocos backbone's channels-first form.  MUTATION plants one mistake at a time (a dropped
residual, the x2 upsampling after codec.up, pwconv1 and pwconv2 swapped as transposes, the
block's LayerNorm before its depthwise conv, the GELU after pwconv2); each must fail a check.
"""
from __future__ import annotations

import math
from typing import Dict, Sequence

import numpy as np

WIDTH, HIDDEN, FFN, BLOCKS, CODEBOOK = 1024, 384, 2048, 12, 8192
EPS = 1e-6
MUTATION = None  # tests only: None, or one planted mistake (see the module docstring)

_AS = (0.254829592, -0.284496736, 1.421413741, -1.453152027, 1.061405429)  # Abramowitz & Stegun 7.1.26
_AS_P = 0.3275911


def erf_as(x: np.ndarray) -> np.ndarray:
    """erf by Abramowitz & Stegun 7.1.26 (|error| <= 1.5e-7), odd extension."""
    a = np.abs(x)
    t = 1.0 / (1.0 + _AS_P * a)
    poly = ((((_AS[4] * t + _AS[3]) * t + _AS[2]) * t + _AS[1]) * t + _AS[0]) * t
    return np.sign(x) * (1.0 - poly * np.exp(-a * a))


def codec_gelu(x: np.ndarray) -> np.ndarray:
    return 0.5 * x * (1.0 + erf_as(x / math.sqrt(2.0)))


def layernorm(x: np.ndarray, g: np.ndarray, b: np.ndarray, eps: float = EPS) -> np.ndarray:
    mean = x.mean(axis=-1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
    return (x - mean) / np.sqrt(var + eps) * g + b


def conv1d_same(x: np.ndarray, w: np.ndarray, b: np.ndarray) -> np.ndarray:
    """x [T][Cin], w [Cout][Cin][k] -> [T][Cout]."""
    T, k = x.shape[0], w.shape[2]
    pad = k // 2
    xp = np.zeros((T + 2 * pad, x.shape[1]))
    xp[pad:pad + T] = x
    out = np.broadcast_to(b, (T, w.shape[0])).astype(np.float64).copy()
    for j in range(k):
        out += xp[j:j + T] @ w[:, :, j].T
    return out


def dwconv_same(x: np.ndarray, w: np.ndarray, b: np.ndarray) -> np.ndarray:
    """x [T][C], w [C][1][k] -> [T][C]."""
    T, k = x.shape[0], w.shape[2]
    pad = k // 2
    xp = np.zeros((T + 2 * pad, x.shape[1]))
    xp[pad:pad + T] = x
    out = np.broadcast_to(b, x.shape).astype(np.float64).copy()
    for j in range(k):
        out += xp[j:j + T] * w[:, 0, j]
    return out


def nearest_up2(x: np.ndarray) -> np.ndarray:
    T = x.shape[0]
    idx = np.minimum(np.floor(np.arange(2 * T) * 0.5).astype(np.int64), T - 1)
    return x[idx]


def linear(x: np.ndarray, w: np.ndarray, b: np.ndarray) -> np.ndarray:
    return x @ w.T + b


def _w(weights: Dict[str, np.ndarray], name: str) -> np.ndarray:
    return np.asarray(weights[name], dtype=np.float64)


def lookup(weights: Dict[str, np.ndarray], codes: Sequence[int]) -> np.ndarray:
    codes = [int(c) for c in codes]
    if not codes or len(codes) > 5000 or max(codes) >= CODEBOOK or min(codes) < 0:
        raise ValueError("Codec expects 1..5000 code IDs in [0,8192)")
    q = "codec.quantizer.quantizers.0"
    e = _w(weights, q + ".codebook.weight")[codes]
    return linear(e, _w(weights, q + ".out_project.weight"), _w(weights, q + ".out_project.bias"))


def vocos(weights: Dict[str, np.ndarray], x: np.ndarray, prefix: str = "codec.decoder", blocks: int = BLOCKS) -> np.ndarray:
    p = prefix + ".0"
    x = layernorm(conv1d_same(x, _w(weights, p + ".embed.weight"), _w(weights, p + ".embed.bias")),
                  _w(weights, p + ".norm.weight"), _w(weights, p + ".norm.bias"))
    for i in range(blocks):
        l = f"{p}.convnext.{i}"
        dw = (_w(weights, l + ".dwconv.weight"), _w(weights, l + ".dwconv.bias"))
        ln = (_w(weights, l + ".norm.weight"), _w(weights, l + ".norm.bias"))
        w1, w2 = _w(weights, l + ".pwconv1.weight"), _w(weights, l + ".pwconv2.weight")
        if MUTATION == "swap_pw":
            w1, w2 = w2.T, w1.T
        if MUTATION == "norm_first":
            h = dwconv_same(layernorm(x, *ln), *dw)
        else:
            h = layernorm(dwconv_same(x, *dw), *ln)
        h = linear(h, w1, _w(weights, l + ".pwconv1.bias"))
        if MUTATION != "gelu_after":
            h = codec_gelu(h)
        h = linear(h, w2, _w(weights, l + ".pwconv2.bias"))
        if MUTATION == "gelu_after":
            h = codec_gelu(h)
        x = h * _w(weights, l + ".gamma") if MUTATION == "no_residual" else x + h * _w(weights, l + ".gamma")
    x = layernorm(x, _w(weights, p + ".final_layer_norm.weight"), _w(weights, p + ".final_layer_norm.bias"))
    return linear(x, _w(weights, prefix + ".1.weight"), _w(weights, prefix + ".1.bias"))


def decode(weights: Dict[str, np.ndarray], codes: Sequence[int], blocks: int = BLOCKS) -> np.ndarray:
    """[2T][1024] features of T codes (codec.cpp:64-72), float64."""
    hidden = vocos(weights, lookup(weights, codes), "codec.decoder", blocks)
    up = (_w(weights, "codec.up.weight"), _w(weights, "codec.up.bias"))
    if MUTATION == "up_after_conv":
        return nearest_up2(conv1d_same(hidden, *up))
    return conv1d_same(nearest_up2(hidden), *up)
