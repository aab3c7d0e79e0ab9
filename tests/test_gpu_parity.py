"""GPU parity: librw_rocm.so (through its C ABI) against the oracle.

Bars (written in each test):
  * dequantized weights: bit-exact with dequant_row_scalar (quant.rs:528-537)
  * activation quantization q/d/sum: bit-exact with quantize_acts_i8
    (quant.rs:691-716)
  * per-block integer sums: bit-exact
  * f32 outputs: within 1e-3 of the reference CPU path, max error scaled by
    the reference row's L2 norm; and against the exact (float64) combination:
    decode regime (m <= 8, exact integer block sums) within a few f32
    roundings per block, encoder regime (m > 8, f16 operands) within
    (2^-10 + (k+8) 2^-24) sum|a||w|.
"""
import numpy as np
import pytest

import oracle as O
from rusty_whisper_amd import _abi as A

from _data import DTYPES, NAMES, activations, check_combine, edge_activation_rows, random_blocks, rel_row_l2, weights

pytestmark = pytest.mark.gpu

ROW_L2_TOL = 1e-3


@pytest.fixture(scope="module", autouse=True)
def _device():
    A.init(0)


# ------------------------------------------------------------ dequant


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: NAMES[d])
@pytest.mark.parametrize("n,k", [(64, 256), (33, 96), (7, 32), (100, 416)])
def test_dequant_bit_exact_random_blocks(dtype, n, k):
    raw = random_blocks(dtype, n * k // 32, seed=1000 + dtype + n)
    w = A.DeviceWeight(dtype, n, k, raw)
    got = w.dequant_rows()
    ref = O.dequant(dtype, raw, n, k)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: NAMES[d])
def test_dequant_pinned_scales_like_avx2_test(dtype):
    # quant.rs:1125-1160: 7 random blocks, d = 0x3555, m = 0xb555, bitwise
    raw = random_blocks(dtype, 7, seed=0x12345678 & 0xFFFF, scale_codes=(0x3555, 0xB555))
    w = A.DeviceWeight(dtype, 1, 7 * 32, raw)
    got = w.dequant_rows()
    ref = O.dequant(dtype, raw, 1, 7 * 32)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: NAMES[d])
def test_dequant_row_slices(dtype):
    n, k = 70, 128
    raw = weights(dtype, n, k, seed=5)
    w = A.DeviceWeight(dtype, n, k, raw)
    ref = O.dequant(dtype, raw, n, k)
    for row0, nrows in [(0, 1), (31, 2), (32, 32), (69, 1), (5, 60)]:
        got = w.dequant_rows(row0, nrows)
        assert np.array_equal(got.view(np.uint32), ref[row0:row0 + nrows].view(np.uint32))


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: NAMES[d])
def test_dequant_nonfinite_scales(dtype):
    # inf / NaN scale codes: the reference keeps the NaN payload (model.rs:82);
    # after d*q+m only NaN-ness and inf values are comparable.
    codes = np.array([[0x7C00, 0x3C00], [0xFC00, 0x3C00], [0x7E01, 0x3C00], [0x3C00, 0x7C00]], np.uint16)
    raws = [random_blocks(dtype, 1, seed=7 + i, scale_codes=tuple(c)) for i, c in enumerate(codes)]
    raw = np.concatenate(raws)
    w = A.DeviceWeight(dtype, 4, 32, raw)
    got = w.dequant_rows()
    ref = O.dequant(dtype, raw, 4, 32)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    fin = ~np.isnan(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))


# ----------------------------------------------------- quantize_acts


@pytest.mark.parametrize("m,k", [(37, 96), (1, 32), (64, 384), (70, 1280)])
def test_quantize_acts_bit_exact(m, k):
    a = activations(m, k, seed=m * 7 + k, outliers=0.01)
    edge = edge_activation_rows(k)
    a = np.concatenate([a, edge])
    with np.errstate(all="ignore"):
        q0, d0, s0 = O.quantize_acts(a)
    q1, d1, s1 = A.quantize_acts(a)
    assert np.array_equal(q0, q1)
    assert np.array_equal(d0.view(np.uint32), d1.view(np.uint32))
    assert np.array_equal(s0, s1)


def test_quantize_acts_reference_seed():
    # the activations of quant.rs:1214-1231 (LCG seed 41, [1500, 384])
    a = O.test_matrix(1, 1500 * 384, 41).reshape(1500, 384)
    q0, d0, s0 = O.quantize_acts(a)
    q1, d1, s1 = A.quantize_acts(a)
    assert np.array_equal(q0, q1) and np.array_equal(s0, s1)
    assert np.array_equal(d0.view(np.uint32), d1.view(np.uint32))


# --------------------------------------------------------- block dots


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: NAMES[d])
@pytest.mark.parametrize("m,n,k", [(37, 41, 96), (64, 64, 256), (5, 70, 160), (33, 1, 32)])
def test_block_dots_exact(dtype, m, n, k):
    raw = random_blocks(dtype, n * k // 32, seed=17 + dtype * 3 + m)
    rng = np.random.default_rng(m + n + k)
    qa = rng.integers(-128, 128, size=(m, k), dtype=np.int8)  # full int8 range
    got = A.DeviceWeight(dtype, n, k, raw).block_dots(qa)
    ref = O.block_dots(dtype, raw, n, k, qa)
    assert np.array_equal(got, ref)


# ------------------------------------------------------------- matmul

SHAPES = [
    (7, 96, 33),      # quant.rs:1189
    (37, 96, 41),     # quant.rs:1238
    (1, 384, 1536),   # decode, one row
    (5, 1280, 1280),  # decode, beam 5
    (8, 96, 64),      # largest GEMV m
    (9, 96, 64),      # smallest GEMM m
    (64, 128, 96),
    (65, 160, 70),
    (200, 416, 130),
]


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: NAMES[d])
@pytest.mark.parametrize("m,k,n", SHAPES, ids=lambda s: str(s))
def test_matmul_parity(dtype, m, k, n):
    a = activations(m, k, seed=m * 131 + k)
    raw = weights(dtype, n, k, seed=n * 17 + k)
    bias = np.random.default_rng(3).standard_normal(n).astype(np.float32)
    w = A.DeviceWeight(dtype, n, k, raw)
    got = w.matmul(a)
    ref = O.matmul_emul(a, dtype, raw, n, tier=O.TIER_VNNI)
    assert rel_row_l2(got, ref) <= ROW_L2_TOL
    check_combine(got, a, dtype, raw, n)
    got_b = w.matmul(a, bias)
    assert np.array_equal(got_b.view(np.uint32), (got + bias[None, :]).view(np.uint32))
    ref_b = O.matmul_emul(a, dtype, raw, n, bias=bias, tier=O.TIER_AVX2)
    assert rel_row_l2(got_b, ref_b) <= ROW_L2_TOL


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: NAMES[d])
def test_rows_independent_of_m(dtype):
    k, n = 160, 100
    raw = weights(dtype, n, k, seed=11)
    w = A.DeviceWeight(dtype, n, k, raw)
    a = activations(150, k, seed=12)
    big = w.matmul(a)
    for m in (9, 33, 64, 100):  # GEMM family: bitwise
        assert np.array_equal(w.matmul(a[:m]).view(np.uint32), big[:m].view(np.uint32))
    small = w.matmul(a[:8])
    for m in range(1, 8):  # GEMV family: bitwise
        assert np.array_equal(w.matmul(a[:m]).view(np.uint32), small[:m].view(np.uint32))
    # across the two families: exact block sums vs f16 operands
    assert rel_row_l2(small, big[:8]) <= ROW_L2_TOL


def test_m_zero_is_a_noop():
    w = A.DeviceWeight(8, 4, 32, weights(8, 4, 32, seed=1))
    out = w.matmul(np.zeros((0, 32), np.float32))
    assert out.shape == (0, 4)


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: NAMES[d])
def test_scale_spread_and_outliers(dtype):
    # per-block weight scales spread over 2 decades, 1% x20 activation channels
    m, k, n = 96, 1280, 160
    raw = weights(dtype, n, k, seed=21, spread=True)
    a = activations(m, k, seed=22, outliers=0.01)
    got = A.DeviceWeight(dtype, n, k, raw).matmul(a)
    ref = O.matmul_emul(a, dtype, raw, n)
    assert rel_row_l2(got, ref) <= ROW_L2_TOL
    check_combine(got, a, dtype, raw, n)


# -------------------------------- the reference's own tests, on the GPU


def _dense_check(fast, a, qt_raw, dtype, n, k):
    reference = O.matmul_t_dense(a, O.dequant(dtype, qt_raw, n, k))
    rms_ref = float(np.sqrt(np.mean(reference.astype(np.float32) ** 2, dtype=np.float32)))
    assert np.all(np.abs(fast - reference) < 0.05 * max(rms_ref, 1.0))


def test_matmul_t_q_matches_dense_within_quant_error():
    # quant.rs:1187-1206
    m, k, n = 7, 96, 33
    a = O.test_matrix(1, m * k, 11).reshape(m, k)
    raw = O.quantize(8, O.test_matrix(n, k, 13))
    _dense_check(A.DeviceWeight(8, n, k, raw).matmul(a), a, raw, 8, n, k)


def test_matmul_t_q_real_encoder_shape_q5_1():
    # quant.rs:1213-1232: the tiny-encoder fc1 shape, LCG seeds 41 / 43
    m, k, n = 1500, 384, 1536
    a = O.test_matrix(1, m * k, 41).reshape(m, k)
    raw = O.quantize(7, O.test_matrix(n, k, 43))
    got = A.DeviceWeight(7, n, k, raw).matmul(a)
    _dense_check(got, a, raw, 7, n, k)
    ref = O.matmul_emul(a, 7, raw, n)
    assert rel_row_l2(got, ref) <= ROW_L2_TOL


@pytest.mark.parametrize("dtype,sa,sb", [(8, 17, 19), (7, 23, 29)], ids=["Q8_0", "Q5_1"])
def test_matmul_t_q_odd_shape_matches_dense(dtype, sa, sb):
    # quant.rs:1236-1278
    m, k, n = 37, 96, 41
    a = O.test_matrix(1, m * k, sa).reshape(m, k)
    raw = O.quantize(dtype, O.test_matrix(n, k, sb))
    _dense_check(A.DeviceWeight(dtype, n, k, raw).matmul(a), a, raw, dtype, n, k)


def test_matmul_t_q_parallel_q5_1():
    # quant.rs:1282-1301
    m, k, n = 600, 128, 600
    a = O.test_matrix(1, m * k, 31).reshape(m, k)
    raw = O.quantize(7, O.test_matrix(n, k, 37))
    _dense_check(A.DeviceWeight(7, n, k, raw).matmul(a), a, raw, 7, n, k)


def test_matmul_t_q_repeated_calls_same_tensor_stay_correct():
    # quant.rs:1311-1331: one resident weight, m = 1..5, fresh activations
    k, n = 96, 41
    raw = O.quantize(7, O.test_matrix(n, k, 29))
    w = A.DeviceWeight(7, n, k, raw)
    for call in range(5):
        m = 1 + call
        a = O.test_matrix(1, m * k, 100 + call).reshape(m, k)
        _dense_check(w.matmul(a), a, raw, 7, n, k)


def test_int8_gemm_matches_scalar_reference():
    # quant.rs:1336-1370: against an independent scalar int8 computation,
    # 1e-3 * max(|acc|, 1)
    m, k, n = 5, 128, 20
    a = O.test_matrix(1, m * k, 41).reshape(m, k)
    raw = O.quantize(8, O.test_matrix(n, k, 43))
    fast = A.DeviceWeight(8, n, k, raw).matmul(a)
    qa, da, _ = O.quantize_acts(a)
    S = O.block_dots(8, raw, n, k, qa)
    _, db, _, _ = O.unpack_rows(8, raw, n, k)
    for i in range(m):
        for j in range(n):
            acc = np.float32(0.0)
            for bl in range(k // 32):
                acc = np.float32(acc + np.float32(da[i, bl] * db[j, bl]) * np.float32(S[i, j, bl]))
            assert abs(fast[i, j] - acc) < 1e-3 * max(abs(acc), 1.0)


def test_matmul_t_q_parallel_matches_serial():
    # quant.rs:1372-1384: row 0 of an m = 8 call is bitwise the m = 1 result
    m, k, n = 8, 128, 1200
    a = O.test_matrix(1, m * k, 21).reshape(m, k)
    raw = O.quantize(8, O.test_matrix(n, k, 23))
    w = A.DeviceWeight(8, n, k, raw)
    par = w.matmul(a)
    one = w.matmul(a[:1])
    assert np.array_equal(par[0].view(np.uint32), one[0].view(np.uint32))


# encoder-regime shapes that select each k split of the GEMM (1, 2 and 4
# wavefronts along k, from the weight's 64-row column tiles and its blocks),
# a block count that does not divide evenly over the wavefronts, and splits
# cut back because the row has few blocks
KSPLIT_SHAPES = [
    (70, 512, 3100),   # 49 column tiles: split 1
    (40, 1280, 1600),  # 25 column tiles: split 2
    (40, 5120, 96),    # 2 column tiles, nb 160: split 4
    (33, 5152, 70),    # nb 161: split 4, uneven
    (45, 384, 100),    # nb 12: split cut to 2
    (20, 224, 96),     # nb 7: split cut to 1
]


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: NAMES[d])
@pytest.mark.parametrize("m,k,n", KSPLIT_SHAPES, ids=lambda s: str(s))
def test_gemm_k_splits(dtype, m, k, n):
    a = activations(m, k, seed=m + k + dtype, outliers=0.01)
    raw = weights(dtype, n, k, seed=n + k + dtype)
    bias = np.random.default_rng(5).standard_normal(n).astype(np.float32)
    w = A.DeviceWeight(dtype, n, k, raw)
    got = w.matmul(a, bias)
    ref = O.matmul_emul(a, dtype, raw, n, bias=bias)
    assert rel_row_l2(got, ref) <= ROW_L2_TOL
    check_combine(got, a, dtype, raw, n, bias)
    # a row's result does not depend on m
    assert np.array_equal(w.matmul(a[:9], bias).view(np.uint32), got[:9].view(np.uint32))


def test_gemm_k_split_on_a_tall_ragged_input():
    # the 4-way k split at encoder height: 1500 rows (a partial last row
    # group), 129 blocks (uneven over the 4 wavefronts), 900 columns (an odd
    # number of weight row groups, the last one partial), 128-row tiles.
    # Rows 0..8 are bitwise an m = 9 call's (64-row, 32-column tiles, the
    # same k split); a sample of rows, the last row group's among them,
    # against the oracle
    m, k, n, dtype = 1500, 4128, 900, 7
    a = activations(m, k, seed=41, outliers=0.01)
    raw = weights(dtype, n, k, seed=43)
    bias = np.random.default_rng(45).standard_normal(n).astype(np.float32)
    w = A.DeviceWeight(dtype, n, k, raw)
    got = w.matmul(a, bias)
    assert np.all(np.isfinite(got))
    assert np.array_equal(w.matmul(a[:9], bias).view(np.uint32), got[:9].view(np.uint32))
    rows = np.unique(np.concatenate([np.random.default_rng(47).choice(m - 32, 24, replace=False),
                                     np.arange(m - 28, m, 9), [m - 1]]))
    ref = O.matmul_emul(a[rows], dtype, raw, n, bias=bias)
    assert rel_row_l2(got[rows], ref) <= ROW_L2_TOL
    check_combine(got[rows], a[rows], dtype, raw, n, bias)


@pytest.mark.parametrize("m", [5, 70])
def test_nonfinite_input_stays_in_its_row(m):
    # an inf activation makes its own row non-finite (as in the reference:
    # d_a = inf) and leaves every other row bitwise unchanged
    k, n = 1312, 96  # nb 41: the GEMM reads past the last block
    raw = weights(7, n, k, seed=8)
    w = A.DeviceWeight(7, n, k, raw)
    a = activations(m, k, seed=9)
    clean = w.matmul(a)
    a2 = a.copy()
    a2[3, 1300] = np.inf
    dirty = w.matmul(a2)
    others = [i for i in range(m) if i != 3]
    assert np.array_equal(dirty[others].view(np.uint32), clean[others].view(np.uint32))
    assert not np.all(np.isfinite(dirty[3]))
