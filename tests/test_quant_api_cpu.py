"""The C++ mirror of the reference API without a device: shape checks panic
with the reference's messages (src/quant.rs:757-758, tensor.rs:266) before any
device work, and a missing device is an error, never a CPU fallback."""
import numpy as np
import pytest

from rusty_whisper_amd import _abi as A
from rusty_whisper_amd import quant as Q


def test_constants():
    assert Q.QK == 32
    assert [Q.block_bytes(d) for d in (2, 3, 6, 7, 8)] == [18, 20, 22, 24, 34]
    assert Q.block_bytes(4) is None


def test_inner_dim_mismatch_panics_like_reference():
    qt = Q.QTensor([4, 32], 8, np.zeros(4 * 34, np.uint8))
    with pytest.raises(Q.Panic, match="matmul_t_q inner dims: 64 vs 32"):
        Q.matmul_t_q(np.zeros((2, 64), np.float32), qt)


def test_k_not_multiple_of_32_panics():
    qt = Q.QTensor([4, 48], 8, np.zeros(4 * 34, np.uint8))
    with pytest.raises(Q.Panic, match="k must be a multiple of 32"):
        Q.matmul_t_q(np.zeros((2, 48), np.float32), qt)


def test_dense_weight_accessors():
    w = Q.Weight.Dense(np.arange(6, dtype=np.float32).reshape(2, 3))
    assert not w.is_quant() and w.shape() == [2, 3]
    assert w.row_f32(1).tolist() == [3.0, 4.0, 5.0]
    # the Dense arm checks shapes as tensor::matmul_t and add_bias do (before any device work)
    with pytest.raises(Q.Panic, match="matmul_t inner dims: 4 vs 3"):
        Q.linear_w(np.zeros((1, 4), np.float32), w)
    with pytest.raises(Q.Panic, match="bias length 3 != 2"):
        Q.linear_w(np.zeros((1, 3), np.float32), w, np.zeros(3, np.float32))
    wq = Q.Weight.Quant([4, 32], 8, np.zeros(4 * 34, np.uint8))
    with pytest.raises(Q.Panic, match="expected dense weight, found quantized"):
        wq.dense()


def test_bias_length_checked():
    wq = Q.Weight.Quant([4, 32], 8, np.zeros(4 * 34, np.uint8))
    with pytest.raises(Q.Panic, match="bias length 3 != 4"):
        Q.linear_w(np.zeros((1, 32), np.float32), wq, np.zeros(3, np.float32))


def test_without_device_is_an_error():
    if A.device_count() > 0:
        pytest.skip("a device is present: covered by the gpu tests")
    qt = Q.QTensor([4, 32], 8, np.zeros(4 * 34, np.uint8))
    with pytest.raises(Q.Panic) as e:
        Q.matmul_t_q(np.zeros((1, 32), np.float32), qt)
    assert e.value.args[1] == A.RW_ENODEV
