"""The package's vectorized synthetic-weight quantizer against the oracle's
scalar restatement of the reference test quantizers (bitwise bytes)."""
import numpy as np
import pytest

import oracle as O
from rusty_whisper_amd import synth

from _data import DTYPES, NAMES


def test_f16_encoder_matches_oracle():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(50000) * 10.0 ** rng.uniform(-9, 6, 50000)).astype(np.float32)
    x = np.concatenate([x, np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 65504.0, 65520.0, 1e-8,
                                     6.1035156e-5, 1.0 + 2.0 ** -11], np.float32)])
    got = synth.f32_to_f16_bits(x)
    want = np.array([O.f32_to_f16(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: NAMES[d])
def test_quantize_matches_oracle_bitwise(dtype):
    rng = np.random.default_rng(dtype)
    x = (rng.standard_normal(64 * 512) * 0.02).astype(np.float32)
    x[:32] = 0.0  # all-zero block
    x[32:64] = 0.5  # constant block (d = 0 for the _1 formats)
    assert np.array_equal(synth.quantize(dtype, x), O.quantize(dtype, x))


def test_normal_weights_shape_and_spread():
    raw = synth.normal_weights(7, 64, 256, seed=1, spread=True)
    assert raw.size == 64 * 8 * 24
    assert np.array_equal(raw, synth.normal_weights(7, 64, 256, seed=1, spread=True))


def test_layer_shapes():
    enc = synth.encoder_layer_shapes(1280, 5120)
    assert sum(2 * n * k for _, n, k in enc) * 1500 * 32 == 1887436800000  # 1887.4 G-ops
    dec = synth.decoder_layer_shapes(1280, 5120)
    assert len(dec) == 10
