"""rw_rocm_matmul_t_q_dev_noalloc (the entry point that allocates nothing)
against rw_rocm_matmul_t_q_dev, through the C ABI: bit for bit the same
outputs on two calls in a row, the second with a smaller input, in both
product regimes; inputs too large for the fixed scratch are rejected."""
import numpy as np
import pytest

from rusty_whisper_amd import _abi as A

from _data import activations, weights

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as T

    A.init(0)
    return T


def _both(torch, w, a, bias):
    ad = torch.from_numpy(a).to("cuda:0")
    bd = torch.from_numpy(bias).to("cuda:0")
    ref = torch.empty(a.shape[0], w.n, device="cuda:0")
    got = torch.full((a.shape[0], w.n), float("nan"), device="cuda:0")
    w.matmul_dev(ad, a.shape[0], ref, bd)
    w.matmul_dev_noalloc(ad, a.shape[0], got, bd)
    torch.cuda.synchronize()
    return got.cpu().numpy(), ref.cpu().numpy()


@pytest.mark.parametrize("dtype,n,k,ms", [(7, 1280, 1280, (1500, 300)), (8, 768, 3072, (1500, 33)),
                                          (2, 5120, 1280, (200, 9)), (6, 1280, 1280, (5, 1))],
                         ids=lambda x: str(x))
def test_noalloc_matches_matmul_dev(torch, dtype, n, k, ms):
    raw = weights(dtype, n, k, seed=n + k)
    w = A.DeviceWeight(dtype, n, k, raw)
    bias = (np.random.default_rng(1).standard_normal(n) * 0.1).astype(np.float32)
    for i, m in enumerate(ms):  # the second call is smaller: stale scratch contents must not leak in
        print(f"noalloc dtype={dtype} [{n}x{k}] m={m} call {i + 1}", flush=True)
        got, ref = _both(torch, w, activations(m, k, seed=10 * i + m), bias)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_noalloc_rejects_inputs_beyond_the_scratch(torch):
    k = 5120
    w = A.DeviceWeight(8, 64, k, weights(8, 64, k, seed=3))
    m = 4096  # 4096 x 5120 f16 values: 40 MiB of workspace
    a = torch.zeros(m, k, device="cuda:0")
    out = torch.empty(m, 64, device="cuda:0")
    with pytest.raises(A.RwError, match="fixed scratch"):
        w.matmul_dev_noalloc(a, m, out)
