"""The reference's own quant tests (src/quant.rs:1125-1384, src/model.rs:348-421)
restated against the C++ mirror of its API on the GPU: same names, seeds,
shapes and tolerances.  The dense reference (matmul_t on to_dense) uses the
oracle's restatement of tensor::matmul_t and the device's bit-exact
to_dense."""
import struct
import threading

import numpy as np
import pytest

import oracle as O
from rusty_whisper_amd import quant as Q

from _data import random_blocks

pytestmark = pytest.mark.gpu


def quantize_q8_0(x):
    return O.quantize(8, x)


def quantize_q5_1(x):
    return O.quantize(7, x)


def test_matrix(n, k, seed):
    return O.test_matrix(n, k, seed)


test_matrix.__test__ = False  # a helper named like the reference's, not a test


def dense_reference(a, qt):
    return O.matmul_t_dense(a, qt.to_dense())


def assert_close_to_dense(fast, reference):
    rms_ref = float(np.sqrt(np.mean(reference.astype(np.float32) ** 2, dtype=np.float32)))
    bad = np.abs(fast - reference) >= 0.05 * max(rms_ref, 1.0)
    assert not bad.any(), f"first mismatch at {np.argwhere(bad)[0]}"


def test_avx2_dequant_bit_identical_to_scalar():
    # quant.rs:1125-1160 -- here: device dequant vs the scalar restatement
    for dtype in (2, 3, 6, 7, 8):
        raw = random_blocks(dtype, 7, seed=0x5678, scale_codes=(0x3555, 0xB555))
        qt = Q.QTensor([1, 7 * 32], dtype, raw)
        fast = qt.to_dense()
        scalar = O.dequant(dtype, raw, 1, 7 * 32)
        assert np.array_equal(fast.view(np.uint32), scalar.view(np.uint32)), dtype


def test_unpack_matches_f32_dequant_reference():
    # quant.rs:1162-1174
    block = bytearray(24)
    block[0:2] = struct.pack("<H", 0x3800)
    block[2:4] = struct.pack("<H", 0x4000)
    block[4:8] = struct.pack("<I", 1)
    block[8] = 0x03
    d = Q.QTensor([1, 32], 7, np.frombuffer(bytes(block), np.uint8)).to_dense()[0]
    assert d[0] == 11.5 and d[1] == 2.0


def test_qtensor_row_roundtrip():
    # quant.rs:1176-1185
    x = test_matrix(3, 64, 7)
    qt = Q.QTensor([3, 64], 8, quantize_q8_0(x))
    row = qt.row_f32(1)
    assert np.all(np.abs(row - x[64:128]) < 0.02)


def test_matmul_t_q_matches_dense_within_quant_error():
    # quant.rs:1187-1206
    m, k, n = 7, 96, 33
    a = test_matrix(1, m * k, 11).reshape(m, k)
    qt = Q.QTensor([n, k], 8, quantize_q8_0(test_matrix(n, k, 13)))
    assert_close_to_dense(Q.matmul_t_q(a, qt), dense_reference(a, qt))


def test_matmul_t_q_real_encoder_shape_q5_1():
    # quant.rs:1213-1232
    m, k, n = 1500, 384, 1536
    a = test_matrix(1, m * k, 41).reshape(m, k)
    qt = Q.QTensor([n, k], 7, quantize_q5_1(test_matrix(n, k, 43)))
    assert_close_to_dense(Q.matmul_t_q(a, qt), dense_reference(a, qt))


def test_matmul_t_q_odd_shape_matches_dense():
    # quant.rs:1236-1255
    m, k, n = 37, 96, 41
    a = test_matrix(1, m * k, 17).reshape(m, k)
    qt = Q.QTensor([n, k], 8, quantize_q8_0(test_matrix(n, k, 19)))
    assert_close_to_dense(Q.matmul_t_q(a, qt), dense_reference(a, qt))


def test_matmul_t_q_odd_shape_matches_dense_q5_1():
    # quant.rs:1259-1278
    m, k, n = 37, 96, 41
    a = test_matrix(1, m * k, 23).reshape(m, k)
    qt = Q.QTensor([n, k], 7, quantize_q5_1(test_matrix(n, k, 29)))
    assert_close_to_dense(Q.matmul_t_q(a, qt), dense_reference(a, qt))


def test_matmul_t_q_parallel_q5_1():
    # quant.rs:1282-1301
    m, k, n = 600, 128, 600
    a = test_matrix(1, m * k, 31).reshape(m, k)
    qt = Q.QTensor([n, k], 7, quantize_q5_1(test_matrix(n, k, 37)))
    assert_close_to_dense(Q.matmul_t_q(a, qt), dense_reference(a, qt))


def test_matmul_t_q_repeated_calls_same_tensor_stay_correct():
    # quant.rs:1311-1331
    k, n = 96, 41
    qt = Q.QTensor([n, k], 7, quantize_q5_1(test_matrix(n, k, 29)))
    for call in range(5):
        m = 1 + call
        a = test_matrix(1, m * k, 100 + call).reshape(m, k)
        assert_close_to_dense(Q.matmul_t_q(a, qt), dense_reference(a, qt))


def test_int8_gemm_matches_scalar_reference():
    # quant.rs:1336-1370
    m, k, n = 5, 128, 20
    a = test_matrix(1, m * k, 41).reshape(m, k)
    raw = quantize_q8_0(test_matrix(n, k, 43))
    fast = Q.matmul_t_q(a, Q.QTensor([n, k], 8, raw))
    qa, da, _ = O.quantize_acts(a)
    nb = k // 32
    for i in range(m):
        for j in range(n):
            acc = np.float32(0.0)
            for bl in range(nb):
                q, db, _ = O.unpack_block(8, raw[(j * nb + bl) * 34:(j * nb + bl + 1) * 34].tobytes())
                s = int(np.dot(qa[i, bl * 32:(bl + 1) * 32].astype(np.int32), q.astype(np.int32)))
                acc = np.float32(acc + np.float32(np.float32(da[i, bl]) * np.float32(db)) * np.float32(s))
            assert abs(fast[i, j] - acc) < 1e-3 * max(abs(float(acc)), 1.0)


def test_matmul_t_q_parallel_matches_serial():
    # quant.rs:1372-1384
    m, k, n = 8, 128, 1200
    a = test_matrix(1, m * k, 21).reshape(m, k)
    qt = Q.QTensor([n, k], 8, quantize_q8_0(test_matrix(n, k, 23)))
    par = Q.matmul_t_q(a, qt)
    serial = Q.matmul_t_q(a[:1].copy(), qt)
    assert np.array_equal(par[0].view(np.uint32), serial[0].view(np.uint32))


def test_dequant_known_blocks_via_qtensor():
    # model.rs:348-381
    raw = bytearray(34)
    raw[0:2] = struct.pack("<H", 0x3800)
    raw[2], raw[3], raw[4] = 0, 1, 0xFE
    raw[5:34] = bytes([3]) * 29
    d = Q.QTensor([1, 32], 8, np.frombuffer(bytes(raw), np.uint8)).to_dense()[0]
    assert d[:3].tolist() == [0.0, 0.5, -1.0] and d[31] == 1.5
    raw = bytearray(18)
    raw[0:2] = struct.pack("<H", 0x3C00)
    raw[2] = 0xF8
    d = Q.QTensor([1, 32], 2, np.frombuffer(bytes(raw), np.uint8)).to_dense()[0]
    assert d[0] == 0.0 and d[16] == 7.0 and d[1] == -8.0
    raw = bytearray(22)
    raw[0:2] = struct.pack("<H", 0x3C00)
    raw[2:6] = struct.pack("<I", 1)
    d = Q.QTensor([1, 32], 6, np.frombuffer(bytes(raw), np.uint8)).to_dense()[0]
    assert d[0] == 0.0 and d[16] == -16.0


def test_loads_quantized_tensor_values():
    # model.rs:400-421: a Q8_0 [1, 32] tensor, d = 1.0, quants all 2
    raw = struct.pack("<H", 0x3C00) + bytes([2]) * 32
    w = Q.Weight.Quant([1, 32], 8, np.frombuffer(raw, np.uint8))
    assert w.is_quant() and w.shape() == [1, 32]
    assert w.row_f32(0).tolist() == [2.0] * 32


def test_linear_w_adds_bias_after_the_product():
    # quant.rs:1054-1063 + tensor.rs:263-271
    m, k, n = 9, 160, 70
    a = test_matrix(1, m * k, 5).reshape(m, k)
    raw = quantize_q5_1(test_matrix(n, k, 6))
    b = test_matrix(1, n, 7)
    w = Q.Weight.Quant([n, k], 7, raw)
    y = Q.linear_w(a, w, b)
    y0 = Q.linear_w(a, w)
    assert np.array_equal(y.view(np.uint32), (y0 + b[None, :]).view(np.uint32))


def test_shared_qtensor_across_threads():
    # transcribe_parallel shares &Model across threads (transcribe.rs:1525-1552)
    m, k, n = 40, 256, 96
    qt = Q.QTensor([n, k], 7, quantize_q5_1(test_matrix(n, k, 9)))
    inputs = [test_matrix(1, m * k, 200 + t).reshape(m, k) for t in range(8)]
    want = [Q.matmul_t_q(x, qt) for x in inputs]
    got = [None] * len(inputs)

    def run(t):
        for _ in range(3):
            got[t] = Q.matmul_t_q(inputs[t], qt)

    threads = [threading.Thread(target=run, args=(t,)) for t in range(len(inputs))]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    for g, w in zip(got, want):
        assert np.array_equal(g.view(np.uint32), w.view(np.uint32))
