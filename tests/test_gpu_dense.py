"""GPU parity of the dense f32 tier (rw_rocm_matmul_t_f32 / _dev, the
mirror's matmul_t and linear_w's Dense arm) against the oracle's
restatement of tensor::matmul_t (src/tensor.rs:104-238).

Bar: bit for bit.  Every element is tensor::dot's sum (8 lane accumulators,
products and sums rounded separately, lanes and tail summed from -0.0), so
the device result must equal the oracle's in every bit, signed zeros and
infinities included, over shapes with and without a k % 8 tail and with m,
n off the 32 x 32 tile."""
import numpy as np
import pytest

import oracle as O
from rusty_whisper_amd import _abi as A
from rusty_whisper_amd import quant as Q

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    A.init(0)


def bits(x):
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


def test_known_values():
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)  # tensor.rs:377-383
    bt = np.array([[7, 9, 11], [8, 10, 12]], np.float32)
    assert A.matmul_t_f32(a, bt).tolist() == [[58, 64], [139, 154]]
    assert Q.matmul_t(a, bt).tolist() == [[58, 64], [139, 154]]


@pytest.mark.parametrize("m,k,n", [(37, 100, 41), (64, 256, 96), (33, 7, 65), (1, 1280, 3000), (70, 1283, 50),
                                   (5, 8, 1), (200, 64, 33)], ids=str)
def test_bitwise_vs_oracle(m, k, n):
    rng = np.random.default_rng(m * 1000 + k + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    want = O.matmul_t_dense(a, b)
    got = A.matmul_t_f32(a, b)
    assert np.array_equal(bits(got), bits(want)), f"{np.sum(bits(got) != bits(want))} elements differ"


def test_signed_zeros_and_infinities():
    # all-tail rows of negative zeros give -0.0 + ... sums; an infinity
    # propagates; a row of exact cancellations sums to +0.0
    a = np.zeros((4, 20), np.float32)
    a[0] = -0.0
    a[1, :5] = -0.0
    a[2, 3] = np.inf
    a[3, :16] = np.tile([1.5, -1.5], 8)
    b = np.ones((3, 20), np.float32)
    b[1] = -1.0
    b[2, :] = 0.25
    for k in (20, 5):  # with and without a main part
        aa, bb = np.ascontiguousarray(a[:, :k]), np.ascontiguousarray(b[:, :k])
        want = O.matmul_t_dense(aa, bb)
        got = A.matmul_t_f32(aa, bb)
        assert np.array_equal(bits(got), bits(want))


def test_device_entry_matches_host_entry():
    import torch

    rng = np.random.default_rng(7)
    m, k, n = 45, 333, 77
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((n, k)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    host = A.matmul_t_f32(a, b, bias)
    da, db, dbias = (torch.from_numpy(x).to("cuda:0") for x in (a, b, bias))
    out = torch.empty(m, n, device="cuda:0")
    A.matmul_t_f32_dev(da, m, k, db, n, out, dbias, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(bits(out.cpu().numpy()), bits(host))
    want = (O.matmul_t_dense(a, b) + bias).astype(np.float32)  # add_bias: one f32 add per element
    assert np.array_equal(bits(host), bits(want))


def test_linear_w_dense_arm():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((9, 384)).astype(np.float32)
    w = (rng.standard_normal((1536, 384)) * 0.02).astype(np.float32)
    bias = rng.standard_normal(1536).astype(np.float32)
    W = Q.Weight.Dense(w)
    want = O.matmul_t_dense(x, w)
    assert np.array_equal(bits(Q.linear_w(x, W)), bits(want))
    assert np.array_equal(bits(Q.linear_w(x, W, bias)), bits((want + bias).astype(np.float32)))
    assert Q.linear_w(np.zeros((0, 384), np.float32), W).shape == (0, 1536)
