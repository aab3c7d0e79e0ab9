"""The encoder-layer oracle (oracle/encoder.py) pinned without a GPU.

* layernorm: zero mean and unit variance (to 1e-5 eps) before the affine part,
  and the float64 form;
* GELU: gelu(0) = 0, gelu(t) -> t for large t and -> 0 for very negative t,
  and within 1e-3 of the exact erf form 0.5 t (1 + erf(t / sqrt 2));
* the quantized layer within the activation-quantization error of a float64
  composition of the same steps on the dequantized weights.
"""
import math

import numpy as np
import pytest
from scipy.special import erf

import oracle as O
from oracle.encoder import encoder_layer, encoder_layer_f64, gelu, layernorm


def test_layernorm_normalizes():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((7, 384)) * 3 + 2).astype(np.float32)
    y = layernorm(x, np.ones(384, np.float32), np.zeros(384, np.float32))
    np.testing.assert_allclose(y.mean(axis=1), 0, atol=1e-5)
    np.testing.assert_allclose(y.var(axis=1), 1 / (1 + 1e-5 / x.var(axis=1)), rtol=1e-4)
    w, b = rng.standard_normal(384).astype(np.float32), rng.standard_normal(384).astype(np.float32)
    x64 = x.astype(np.float64)
    ref = (x64 - x64.mean(1, keepdims=True)) / np.sqrt(x64.var(1, keepdims=True) + 1e-5) * w + b
    np.testing.assert_allclose(layernorm(x, w, b), ref, rtol=1e-5, atol=1e-5)


def test_gelu_known_values():
    assert gelu(np.float32([0.0]))[0] == 0.0
    t = np.float32([10.0, 30.0, -10.0, -30.0])
    np.testing.assert_allclose(gelu(t)[:2], t[:2], rtol=1e-6)
    assert np.all(np.abs(gelu(t)[2:]) < 1e-6)
    x = np.linspace(-6, 6, 1001).astype(np.float32)
    exact = 0.5 * x * (1 + erf(x / math.sqrt(2)))
    assert np.max(np.abs(gelu(x) - exact)) < 1e-3  # the tanh form's known deviation


def _params(n, f, dtype, seed):
    rng = np.random.default_rng(seed)

    def w(rows, cols):
        raw = O.quantize(dtype, (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32))
        return {"dtype": dtype, "raw": raw, "n": rows}

    def vec(k, s=0.1, c=0.0):
        return (rng.standard_normal(k) * s + c).astype(np.float32)

    return {"attn_ln_w": vec(n, 0.1, 1.0), "attn_ln_b": vec(n), "q": w(n, n), "k": w(n, n), "v": w(n, n),
            "out": w(n, n), "q_b": vec(n), "v_b": vec(n), "out_b": vec(n), "mlp_ln_w": vec(n, 0.1, 1.0),
            "mlp_ln_b": vec(n), "fc1": w(f, n), "fc1_b": vec(f), "fc2": w(n, f), "fc2_b": vec(n)}


@pytest.mark.parametrize("dtype", [8, 7])
def test_layer_close_to_float64_composition(dtype):
    n, f, heads, t = 128, 512, 2, 40
    p = _params(n, f, dtype, seed=dtype)
    x = np.random.default_rng(3).standard_normal((t, n)).astype(np.float32)
    got = encoder_layer(x, p, heads)
    ref = encoder_layer_f64(x, p, heads)
    err = np.max(np.abs(got - ref), axis=1) / np.linalg.norm(ref, axis=1)
    assert err.max() < 5e-3  # int8 activation quantization of four products
    # the residual stream dominates: the layer changes x but not beyond recognition
    assert np.abs(got - x).max() > 1e-2
