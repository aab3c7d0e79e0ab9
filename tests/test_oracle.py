"""Pins the oracle (CPU, no GPU): against the reference's own known-answer
vectors (tests/golden/reference_kats.json), against independent numpy
restatements and brute force, and bitwise against the AVX2 / AVX-512 VNNI
intrinsics restatement in oracle/cpu_baseline.c."""
import json
import os
import struct

import numpy as np
import pytest

import oracle as O

from _data import DTYPES, NAMES, activations, random_blocks, weights

KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))


def h(code: str) -> int:
    return int(code, 16)


# ------------------------------------------------------------------ f16


def test_f16_reference_values():
    kat = KATS["f16_to_f32"]
    for code, val in kat["exact"]:
        assert O.f16_to_f32(h(code)) == np.float32(val)
    for code, val, tol in kat["approx"]:
        assert abs(O.f16_to_f32(h(code)) - val) < tol
    for code in kat["inf"]:
        assert np.isinf(O.f16_to_f32(h(code)))
    for code in kat["nan"]:
        assert np.isnan(O.f16_to_f32(h(code)))


def test_f16_exhaustive_against_numpy():
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.f16_to_f32_bits(codes)
    finite = (codes & 0x7C00) != 0x7C00
    want = codes.view(np.float16).astype(np.float32).view(np.uint32)
    assert np.array_equal(got[finite], want[finite])
    # inf / NaN: sign | 0x7f800000 | frac << 13, payload kept (model.rs:82-83)
    nf = ~finite
    c = codes[nf].astype(np.uint32)
    closed = ((c >> 15) << 31) | 0x7F800000 | ((c & 0x3FF) << 13)
    assert np.array_equal(got[nf], closed)


def test_f16_round_trip_values():
    kat = KATS["f16_round_trip"]
    for v in kat["exact"]:
        assert O.f16_to_f32(O.f32_to_f16(v)) == np.float32(v)
    for v in kat["to_inf"]:
        assert np.isinf(O.f16_to_f32(O.f32_to_f16(v)))


def test_f32_to_f16_matches_numpy_off_ties_and_rounds_ties_up():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(20000) * 10.0 ** rng.uniform(-6, 4, 20000)).astype(np.float32)
    bits = x.view(np.uint32)
    exp = (bits >> 23) & 0xFF
    normal16 = (exp >= 127 - 14) & (exp <= 127 + 15)
    tie = (bits & 0x1FFF) == 0x1000  # exactly half an f16 ulp dropped
    sel = normal16 & ~tie
    got = np.array([O.f32_to_f16(float(v)) for v in x[sel]], dtype=np.uint16)
    assert np.array_equal(got, x[sel].astype(np.float16).view(np.uint16))
    # ties round up in magnitude (model.rs:112-114), unlike numpy's RNE
    assert O.f32_to_f16(1.0 + 2.0 ** -11) == 0x3C01
    assert O.f32_to_f16(-(1.0 + 2.0 ** -11)) == 0xBC01


# --------------------------------------------------------- block codec


def test_block_bytes():
    assert [O.block_bytes(d) for d in DTYPES] == [18, 20, 22, 24, 34]
    assert O.block_bytes(0) == -1 and O.block_bytes(1) == -1 and O.block_bytes(9) == -1


def _blk(size, **fields):
    b = bytearray(size)
    for off, data in fields.values():
        b[off:off + len(data)] = data
    return bytes(b)


def test_known_blocks():
    k = KATS["q8_0_block"]
    raw = bytearray(34)
    raw[0:2] = struct.pack("<H", h(k["d_code"]))
    raw[2:5] = bytes(np.array(k["quants_head"], np.int8).view(np.uint8))
    raw[5:34] = bytes([k["quants_fill"]]) * 29
    d = O.dequant(8, np.frombuffer(bytes(raw), np.uint8), 1, 32)[0]
    assert list(d[:3]) == k["expect_head"] and d[31] == k["expect_last"]

    k = KATS["q4_0_block"]
    raw = bytearray(18)
    raw[0:2] = struct.pack("<H", h(k["d_code"]))
    raw[2] = h(k["byte0"])
    d = O.dequant(2, np.frombuffer(bytes(raw), np.uint8), 1, 32)[0]
    for e, v in k["expect"]:
        assert d[e] == v

    k = KATS["q5_0_block"]
    raw = bytearray(22)
    raw[0:2] = struct.pack("<H", h(k["d_code"]))
    raw[2:6] = struct.pack("<I", k["qh"])
    d = O.dequant(6, np.frombuffer(bytes(raw), np.uint8), 1, 32)[0]
    for e, v in k["expect"]:
        assert d[e] == v

    k = KATS["q5_1_block"]
    raw = bytearray(24)
    raw[0:2] = struct.pack("<H", h(k["d_code"]))
    raw[2:4] = struct.pack("<H", h(k["m_code"]))
    raw[4:8] = struct.pack("<I", k["qh"])
    raw[8] = h(k["byte0"])
    q, dd, mm = O.unpack_block(7, bytes(raw))
    for e, v in k["expect"]:
        assert np.float32(dd) * np.float32(q[e]) + np.float32(mm) == v

    k = KATS["q8_0_file_tensor"]
    raw = struct.pack("<H", h(k["d_code"])) + bytes([k["quant"]]) * 32
    assert np.all(O.dequant(8, np.frombuffer(raw, np.uint8), 1, 32) == k["expect_all"])


def test_unpack_rejects_unknown_dtype():
    with pytest.raises(ValueError):
        O.unpack_block(4, bytes(34))


def _numpy_unpack(dtype, raw, nblk):
    """Independent restatement of the ggml byte maps (ggml-format block layouts)."""
    bb = O.BLOCK_BYTES[dtype]
    b = raw.reshape(nblk, bb)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(nblk)
    m = np.zeros(nblk, np.float32)
    if dtype == 8:
        return b[:, 2:].view(np.int8).astype(np.int32), d, m
    off = {2: 2, 3: 4, 6: 6, 7: 8}[dtype]
    if dtype in (3, 7):
        m = b[:, 2:4].copy().view(np.float16).astype(np.float32).reshape(nblk)
    qs = b[:, off:off + 16].astype(np.int32)
    q = np.concatenate([qs & 0xF, qs >> 4], axis=1)
    if dtype in (6, 7):
        qh = b[:, off - 4:off].copy().view(np.uint32).astype(np.int64).reshape(nblk, 1)
        q = q | (((qh >> np.arange(32)) & 1) << 4).astype(np.int32)
    q = q - {2: 8, 3: 0, 6: 16, 7: 0}[dtype]
    return q, d, m


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: NAMES[d])
def test_dequant_closed_form_all_patterns(dtype):
    # random bytes hit every nibble / high-bit value at every position; the
    # closed form x = d*q + m is evaluated independently in numpy float32
    nblk = 4096
    raw = random_blocks(dtype, nblk, seed=dtype)
    q, d, m = _numpy_unpack(dtype, raw, nblk)
    want = (d[:, None] * q.astype(np.float32)) + m[:, None]
    got = O.dequant(dtype, raw, nblk, 32)
    assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))
    qb, db, mb, sb = O.unpack_rows(dtype, raw, 1, nblk * 32)
    assert np.array_equal(qb.reshape(nblk, 32).astype(np.int32), q)
    assert np.array_equal(sb.reshape(-1), q.sum(axis=1))


def test_q5_0_zero_with_negative_scale_is_positive_zero():
    # H6: d*q + m with m = +0.0 never yields -0.0
    raw = bytearray(22)
    raw[0:2] = struct.pack("<H", 0xBC00)  # d = -1
    raw[2:6] = struct.pack("<I", 0xFFFFFFFF)  # q = 16 everywhere -> 0
    got = O.dequant(6, np.frombuffer(bytes(raw), np.uint8), 1, 32)
    assert np.all(got.view(np.uint32) == 0)


# ---------------------------------------------------- quantize_acts


def _numpy_quantize(a):
    m, k = a.shape
    x = a.reshape(m, k // 32, 32)
    amax = np.nanmax(np.where(np.isnan(x), -np.inf, np.abs(x)), axis=2)
    amax = np.maximum(amax, np.float32(0.0)).astype(np.float32)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore", over="ignore", invalid="ignore"):
        inv = np.where(d > 0, np.float32(1.0) / np.where(d > 0, d, 1), 0).astype(np.float32)
        v = (x * inv[:, :, None]).astype(np.float32).astype(np.float64)
        r = np.sign(v) * np.floor(np.abs(v) + 0.5)  # half away from zero
    r = np.where(np.isnan(r), 0, np.clip(r, -127, 127)).astype(np.int32)
    return r.reshape(m, k).astype(np.int8), d, r.sum(axis=2).astype(np.int32)


def test_quantize_acts_numpy_restatement():
    a = activations(40, 256, seed=3, outliers=0.01)
    rows = np.zeros((6, 256), np.float32)
    rows[1, :4] = [127.0, 0.5, -0.5, 1.5]
    rows[2, :2] = [3.0, -3.0]
    rows[3, :] = 1e-38
    rows[4, 3] = np.nan
    rows[4, 4] = 1.0
    rows[5, 5] = np.inf
    a = np.concatenate([a, rows])
    with np.errstate(all="ignore"):
        q0, d0, s0 = O.quantize_acts(a)
    q1, d1, s1 = _numpy_quantize(a)
    assert np.array_equal(q0, q1) and np.array_equal(s0, s1)
    assert np.array_equal(d0.view(np.uint32), d1.view(np.uint32))
    # closed-form spot checks
    assert list(q0[41, :4]) == [127, 1, -1, 2]  # halves round away from zero
    assert q0[42, 0] == 127 and q0[42, 1] == -127 and s0[42, 0] == 0
    assert np.all(q0[40] == 0) and d0[40, 0] == 0.0


# --------------------------------------------------------- int sums


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: NAMES[d])
def test_block_dots_brute_force(dtype):
    m, n, k = 6, 9, 96
    raw = random_blocks(dtype, n * k // 32, seed=dtype + 50)
    qa = np.random.default_rng(1).integers(-128, 128, size=(m, k), dtype=np.int8)
    S = O.block_dots(dtype, raw, n, k, qa)
    q, _, _ = _numpy_unpack(dtype, raw, n * k // 32)
    qb = q.reshape(n, k // 32, 32).astype(np.int64)
    want = np.einsum("ibe,jbe->ijb", qa.reshape(m, k // 32, 32).astype(np.int64), qb)
    assert np.array_equal(S.astype(np.int64), want)


# ------------------------------------------------ lane emulations


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: NAMES[d])
@pytest.mark.parametrize("m,k,n", [(7, 96, 33), (37, 96, 41), (5, 128, 20), (130, 384, 70)])
def test_emulation_bitwise_equals_intrinsics_port(dtype, m, k, n):
    if O.cpu_tier() != O.TIER_VNNI:
        pytest.skip("this host lacks AVX-512 VNNI")
    a = activations(m, k, seed=m + k)
    raw = weights(dtype, n, k, seed=n + k)
    bias = np.linspace(-1, 1, n).astype(np.float32)
    for tier in (O.TIER_VNNI, O.TIER_AVX2):
        want = O.matmul_emul(a, dtype, raw, n, bias=bias, tier=tier)
        t = O.CpuQTensor(dtype, n, k, raw)
        for threads in (1, 0, 3):  # cold, then packed cache; serial and threaded
            got = t.matmul(a, bias=bias, tier=tier, threads=threads)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (tier, threads)


def test_exact_combine_against_numpy():
    m, k, n = 9, 160, 13
    for dtype in DTYPES:
        a = activations(m, k, seed=dtype)
        raw = weights(dtype, n, k, seed=dtype + 1)
        qa, da, sa = O.quantize_acts(a)
        q, db, mb = _numpy_unpack(dtype, raw, n * k // 32)
        S = np.einsum("ibe,jbe->ijb", qa.reshape(m, -1, 32).astype(np.int64),
                      q.reshape(n, -1, 32).astype(np.int64)).astype(np.float64)
        db = db.reshape(n, -1).astype(np.float64)
        mb = mb.reshape(n, -1).astype(np.float64)
        want = np.einsum("ib,jb,ijb->ij", da.astype(np.float64), db, S) + \
            np.einsum("jb,ib->ij", mb, da.astype(np.float64) * sa)
        got = O.matmul_exact(a, dtype, raw, n)
        assert np.allclose(got, want, rtol=1e-12, atol=1e-12)


def test_dense_matmul_t_known_values():
    a = np.array([[1, 2, 3], [4, 5, 6]], np.float32)  # tensor.rs:377-383
    bt = np.array([[7, 9, 11], [8, 10, 12]], np.float32)
    assert O.matmul_t_dense(a, bt).tolist() == [[58, 64], [139, 154]]
    x = activations(5, 37, seed=1)
    y = activations(6, 37, seed=2)
    assert np.allclose(O.matmul_t_dense(x, y), x.astype(np.float64) @ y.T.astype(np.float64), atol=1e-4)


def test_test_matrix_lcg_closed_form():
    state, vals = 41, []
    for _ in range(5):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        vals.append(np.float32(np.float32(state >> 8) / np.float32(1 << 24)) * np.float32(2.0) - np.float32(1.0))
    assert np.array_equal(O.test_matrix(1, 5, 41), np.array(vals, np.float32))


# ------------------------ the reference's own tests, run on the oracle


def _emul_vs_dense(m, k, n, dtype, sa, sb):
    a = O.test_matrix(1, m * k, sa).reshape(m, k)
    raw = O.quantize(dtype, O.test_matrix(n, k, sb))
    fast = O.matmul_emul(a, dtype, raw, n)
    ref = O.matmul_t_dense(a, O.dequant(dtype, raw, n, k))
    rms = float(np.sqrt(np.mean(ref ** 2)))
    assert np.all(np.abs(fast - ref) < 0.05 * max(rms, 1.0))


def test_reference_tests_on_oracle():
    _emul_vs_dense(7, 96, 33, 8, 11, 13)      # quant.rs:1187-1206
    _emul_vs_dense(37, 96, 41, 8, 17, 19)     # quant.rs:1236-1255
    _emul_vs_dense(37, 96, 41, 7, 23, 29)     # quant.rs:1259-1278
    _emul_vs_dense(600, 128, 600, 7, 31, 37)  # quant.rs:1282-1301


def test_qtensor_row_roundtrip_on_oracle():
    k = KATS["qtensor_row_roundtrip"]  # quant.rs:1176-1185
    n, kk = k["shape"]
    x = O.test_matrix(n, kk, k["seed"]).reshape(n, kk)
    row = O.dequant(8, O.quantize(8, x), n, kk)[k["row"]]
    assert np.all(np.abs(row - x[k["row"]]) < k["tol"])


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: NAMES[d])
def test_quantizers_roundtrip_error(dtype):
    x = activations(16, 256, seed=dtype) * np.float32(0.02)
    deq = O.dequant(dtype, O.quantize(dtype, x), 16, 256)
    blocks = x.reshape(-1, 32)
    amax = np.abs(blocks).max(1)
    step = {
        2: amax / 8, 6: amax / 16, 8: amax / 127,  # symmetric: d = |extreme| / levels
        3: (blocks.max(1) - blocks.min(1)) / 15, 7: (blocks.max(1) - blocks.min(1)) / 31,
    }[dtype]
    err = np.abs(deq.reshape(-1, 32) - blocks).max(1)
    # half a step (a whole step for Q4_0 / Q5_0, whose codes run -8..7 /
    # -16..15 so the extreme opposite the scale's sign clamps one step short),
    # plus the f16 rounding of d (and m) scaled by the largest code
    half = 1.0 if dtype in (2, 6) else 0.5
    assert np.all(err <= step * (half + 32 * 2.0 ** -11) + amax * 2.0 ** -10)
