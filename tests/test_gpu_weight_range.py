"""Weights whose values leave f16's range, through both product regimes.

The encoder-shape GEMM multiplies f16 operands.  A weight row's values
d*q + m are divided by a power of two chosen per row at upload (so the row's
largest lands in [2^14, 2^15)) and the output column is multiplied back, so
valid ggml blocks whose values exceed 65504 (a Q8_0 scale near 1000, a Q5_1
min near 60000) or sit in f16's subnormal range (scales near 1e-7) keep full
precision.  The reference computes these in f32 and stays finite
(src/quant.rs:429-490); so must the GPU path.

Bars: 1e-3 of the reference CPU path (max error over the reference row's L2
norm) and the regime's analytic bound against the exact combination, at
m = 9 (the smallest GEMM input) and m = 1500, and at m = 5 (the decode GEMV,
exact integer sums, for comparison)."""
import numpy as np
import pytest

import oracle as O
from rusty_whisper_amd import _abi as A

from _data import activations, check_combine, rel_row_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _device():
    A.init(0)


def _rows(n, k, seed, kind):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, k)).astype(np.float32)
    if kind == "q8_large_d":  # d = amax / 127 near 1000 in every other row
        x[::2] *= np.float32(127000.0 / 3.5)
        x[1::2] *= np.float32(0.02)
    elif kind == "q51_large_m":  # values in [60000, 66000): m ~ 60000, d ~ 190
        x = (60000.0 + 6000.0 * rng.random((n, k))).astype(np.float32)
        x[1::3] = rng.standard_normal((len(x[1::3]), k)).astype(np.float32) * np.float32(0.02)
    elif kind == "tiny":  # scales near 1e-7: f16 subnormal d and m
        x *= np.float32(2e-6)
    elif kind == "mixed_rows":  # rows of 1e-6 and 1e3 scale side by side
        s = np.where(np.arange(n) % 2 == 0, 1e-6, 1e3).astype(np.float32)
        x *= s[:, None]
    elif kind == "spread_in_row":  # blocks of one row over ten decades
        s = (10.0 ** rng.uniform(-6.0, 4.0, size=(n, k // 32, 1))).astype(np.float32)
        x = (x.reshape(n, k // 32, 32) * s).reshape(n, k)
    return x


CASES = [(8, "q8_large_d"), (7, "q51_large_m"), (3, "q51_large_m"), (7, "tiny"), (2, "tiny"), (6, "tiny"),
         (8, "mixed_rows"), (7, "mixed_rows"), (7, "spread_in_row"), (2, "spread_in_row")]


@pytest.mark.parametrize("dtype,kind", CASES, ids=lambda x: str(x))
@pytest.mark.parametrize("m", [5, 9, 1500])
def test_out_of_f16_range_weights(dtype, kind, m):
    n, k = 96, 256
    raw = O.quantize(dtype, _rows(n, k, 7 + dtype, kind))
    a = activations(m, k, 3)
    bias = (np.random.default_rng(2).standard_normal(n) * 0.1).astype(np.float32)
    w = A.DeviceWeight(dtype, n, k, raw)
    got = w.matmul(a, bias)
    ref = O.matmul_emul(a, dtype, raw, n, bias=bias)
    assert np.all(np.isfinite(ref))
    assert np.all(np.isfinite(got))
    err = rel_row_l2(got, ref)
    assert err <= 1e-3, err
    check_combine(got, a, dtype, raw, n, bias)


def test_large_weights_in_a_multi_weight_launch():
    """Three weights of different row scales in one GEMM launch."""
    import torch

    m, n, k = 200, 64, 128
    raws = [O.quantize(8, _rows(n, k, 1, "q8_large_d")), O.quantize(8, _rows(n, k, 2, "tiny")),
            O.quantize(8, _rows(n, k, 3, "none"))]
    a = activations(m, k, 9)
    ws_len = A.workspace_size(m, k)
    ws = torch.empty(ws_len, dtype=torch.uint8, device="cuda:0")
    A.quantize_dev(torch.from_numpy(a).to("cuda:0"), m, k, ws, ws_len)
    ws_w = [A.DeviceWeight(8, n, k, r) for r in raws]
    outs = [torch.empty(m, n, device="cuda:0") for _ in raws]
    A.matmul_prequant_multi_dev(ws_w, ws, m, outs)
    torch.cuda.synchronize()
    for raw, o in zip(raws, outs):
        got = o.cpu().numpy()
        ref = O.matmul_emul(a, 8, raw, n)
        assert rel_row_l2(got, ref) <= 1e-3
        check_combine(got, a, 8, raw, n)
