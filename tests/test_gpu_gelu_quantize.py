"""rw_rocm_matmul_prequant_gelu_quantize_dev: the encoder MLP's middle
(src/encoder.rs:161-171; gelu src/tensor.rs:289-305) -- fc1's product, its
bias and GELU, quantized for fc2 in the product's epilogue.  Followed by
fc2 through rw_rocm_matmul_prequant_dev it matches the oracle's
linear -> gelu -> linear (the reference's int8 path, oracle/encoder.py's
pieces) within the matmul bar (1e-3 of the row norm), and it matches the
same chain with the GELU output written in f32 and quantized by
rw_rocm_quantize_dev within one quantization step's effect (the two GELU
evaluations, numpy's and the device's, may differ in the last bit)."""
import numpy as np
import pytest

import oracle as O
from oracle.encoder import gelu, linear
from rusty_whisper_amd import _abi as A

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as T

    A.init(0)
    return T


def _linear_ref(x, raw, dtype, n, bias):
    return linear(x, {"dtype": dtype, "raw": raw, "n": n}, bias)


@pytest.mark.parametrize("m,d,dtype", [(1500, 1280, 7), (100, 384, 2), (33, 256, 8), (9, 512, 6)],
                         ids=lambda x: str(x))
def test_gelu_quantize_then_fc2_matches_the_oracle(torch, m, d, dtype):
    f = 4 * d
    rng = np.random.default_rng(m + d)
    w1 = (rng.standard_normal((f, d)) * 0.05).astype(np.float32)
    w2 = (rng.standard_normal((d, f)) * 0.05).astype(np.float32)
    raw1, raw2 = O.quantize(dtype, w1), O.quantize(dtype, w2)
    b1 = (rng.standard_normal(f) * 0.1).astype(np.float32)
    b2 = (rng.standard_normal(d) * 0.1).astype(np.float32)
    x = rng.standard_normal((m, d)).astype(np.float32)
    W1, W2 = A.DeviceWeight(dtype, f, d, raw1), A.DeviceWeight(dtype, d, f, raw2)
    dev = lambda a: torch.from_numpy(a).to("cuda:0")  # noqa: E731
    ws1 = torch.empty(A.workspace_size(m, d), dtype=torch.uint8, device="cuda:0")
    n2 = A.gelu_quantize_workspace_size(m, f)
    assert n2 >= A.workspace_size(m, f)
    ws2 = torch.empty(n2, dtype=torch.uint8, device="cuda:0")
    out = torch.empty(m, d, device="cuda:0")
    xd, b1d, b2d = dev(x), dev(b1), dev(b2)
    A.quantize_dev(xd, m, d, ws1, ws1.numel())
    A.matmul_prequant_gelu_quantize_dev(W1, ws1, m, b1d, ws2, n2)
    W2.matmul_prequant_dev(ws2, m, out, b2d)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    # the oracle chain (rows sampled at full size)
    rows = np.arange(m) if m <= 200 else np.random.default_rng(1).choice(m, 48, replace=False)
    h = gelu(_linear_ref(x[rows], raw1, dtype, f, b1))
    want = _linear_ref(h, raw2, dtype, d, b2)
    err = np.max(np.max(np.abs(got[rows] - want), axis=1) / np.linalg.norm(want, axis=1))
    print(f"  gelu+quantize m={m} d={d} dtype={dtype}: error vs oracle {err:.3g}", flush=True)
    assert err <= 1e-3, err
    # the same chain with y in f32: fc1's product, GELU on the host, quantize_dev
    y = torch.empty(m, f, device="cuda:0")
    W1.matmul_prequant_dev(ws1, m, y, b1d)
    torch.cuda.synchronize()
    yh = gelu(y.cpu().numpy())
    ws3 = torch.empty(A.workspace_size(m, f), dtype=torch.uint8, device="cuda:0")
    A.quantize_dev(dev(yh), m, f, ws3, ws3.numel())
    out2 = torch.empty(m, d, device="cuda:0")
    W2.matmul_prequant_dev(ws3, m, out2, b2d)
    torch.cuda.synchronize()
    ref2 = out2.cpu().numpy()
    e2 = np.max(np.max(np.abs(got - ref2), axis=1) / np.linalg.norm(ref2, axis=1))
    assert e2 <= 1e-4, e2


def test_gelu_quantize_rejects_bad_arguments(torch):
    W = A.DeviceWeight(8, 64, 64, O.quantize(8, np.zeros((64, 64), np.float32)))
    ws = torch.empty(A.workspace_size(40, 64), dtype=torch.uint8, device="cuda:0")
    nxt = torch.empty(A.gelu_quantize_workspace_size(40, 64), dtype=torch.uint8, device="cuda:0")
    with pytest.raises(A.RwError, match="more than 8 rows"):
        A.matmul_prequant_gelu_quantize_dev(W, ws, 8, None, nxt, nxt.numel())
    with pytest.raises(A.RwError, match="bytes < "):
        A.matmul_prequant_gelu_quantize_dev(W, ws, 40, None, nxt, nxt.numel() - 1)
    assert A.gelu_quantize_workspace_size(8, 64) == 0 and A.gelu_quantize_workspace_size(40, 48) == 0
