"""Seeded inputs shared by the tests (weights as ggml bytes, f32 activations)."""
from __future__ import annotations

import numpy as np

import oracle as O

DTYPES = (2, 3, 6, 7, 8)
NAMES = O.DTYPE_NAMES


def weights(dtype: int, n: int, k: int, seed: int, std: float = 0.02, spread: bool = False) -> np.ndarray:
    """N(0, std) weights quantized into ggml blocks; `spread` scales every
    32-block by 10**U(-1, 1) first (a log-uniform spread over two decades)."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, k), dtype=np.float32) * np.float32(std)
    if spread:
        s = (10.0 ** rng.uniform(-1.0, 1.0, size=(n, k // 32, 1))).astype(np.float32)
        x = (x.reshape(n, k // 32, 32) * s).reshape(n, k)
    return O.quantize(dtype, x)


def activations(m: int, k: int, seed: int, outliers: float = 0.0) -> np.ndarray:
    """N(0, 1) activations; `outliers` > 0 scales that fraction of channels x20."""
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((m, k), dtype=np.float32)
    if outliers > 0:
        ch = rng.choice(k, size=max(1, int(round(outliers * k))), replace=False)
        a[:, ch] *= np.float32(20.0)
    return a


def random_blocks(dtype: int, nblocks: int, seed: int, scale_codes=None) -> np.ndarray:
    """Uniformly random block bytes with the f16 scale (and min) fields set to
    finite codes: every nibble / high-bit pattern occurs."""
    rng = np.random.default_rng(seed)
    bb = O.BLOCK_BYTES[dtype]
    raw = rng.integers(0, 256, size=(nblocks, bb), dtype=np.uint8)
    if scale_codes is None:
        # finite f16 codes: normals and subnormals of both signs
        codes = rng.integers(0, 0x7c00, size=(nblocks, 2), dtype=np.uint16)
        codes |= (rng.integers(0, 2, size=(nblocks, 2), dtype=np.uint16) << 15)
    else:
        codes = np.broadcast_to(np.asarray(scale_codes, dtype=np.uint16), (nblocks, 2)).copy()
    raw[:, 0:2] = codes[:, 0:1].view(np.uint8).reshape(nblocks, 2)
    if dtype in (3, 7):
        raw[:, 2:4] = codes[:, 1:2].view(np.uint8).reshape(nblocks, 2)
    return raw.reshape(-1)


def edge_activation_rows(k: int) -> np.ndarray:
    """Rows that hit every special case of quantize_acts_i8 (quant.rs:691-716)."""
    rows = []
    z = np.zeros(k, np.float32)
    rows.append(z)  # d = 0 -> inv = 0 -> q = 0
    h = np.zeros(k, np.float32)
    h[:4] = [127.0, 0.5, -0.5, 1.5]  # amax 127 -> d = 1: exact halves round away from 0
    rows.append(h)
    e = np.zeros(k, np.float32)
    e[0], e[1] = 3.0, -3.0  # +-amax -> +-127
    rows.append(e)
    t = np.full(k, 1e-38, np.float32)  # d subnormal, 1/d overflows to inf
    t[1] = -2e-39
    rows.append(t)
    s = np.full(k, 3e-45, np.float32)  # subnormal inputs
    rows.append(s)
    n = np.ones(k, np.float32)
    n[3] = np.nan  # NaN ignored by the amax fold, quantizes to 0
    rows.append(n)
    nn = np.ones(k, np.float32)
    nn[:32] = np.nan  # a block of NaN: the fold from 0 gives amax = 0 -> d = 0, q = 0
    if k >= 64:
        nn[36:40] = np.nan  # one 4-value lane of a block all NaN
    rows.append(nn)
    i = np.ones(k, np.float32)
    i[5] = np.inf  # amax = inf -> inv = 0 -> q = 0 (inf*0 = NaN -> 0)
    rows.append(i)
    b = np.full(k, 3.4e38, np.float32)
    b[2] = -3.4e38
    rows.append(b)
    return np.stack(rows)


def rel_row_l2(got: np.ndarray, ref: np.ndarray) -> float:
    """max_ij |got-ref| / ||ref_i||_2 -- the output tolerance of the products (1e-3)."""
    ref64 = ref.astype(np.float64)
    norms = np.linalg.norm(ref64, axis=1, keepdims=True)
    norms = np.where(norms > 0, norms, 1.0)
    return float(np.max(np.abs(got.astype(np.float64) - ref64) / norms))


def _abs_terms(a, dtype, raw, n):
    """sum_bl |d_a d_b S| + |m_b d_a sum_a| in float64: the scale of the f32
    combine's rounding error for each output."""
    k = a.shape[1]
    qa, da, sa = O.quantize_acts(a)
    S = O.block_dots(dtype, raw, n, k, qa).astype(np.float64)  # [m, n, nb]
    _, db, mb, _ = O.unpack_rows(dtype, raw, n, k)
    t = np.abs(da[:, None, :].astype(np.float64) * db[None, :, :] * S)
    t += np.abs(mb[None, :, :].astype(np.float64) * (da * sa)[:, None, :])
    return t.sum(axis=2)


def check_exact_combine(got, a, dtype, raw, n, bias=None):
    """Decode regime (exact block sums, f32 combine): within a few f32
    roundings per block of the exact combination."""
    exact = O.matmul_exact(a, dtype, raw, n, bias=bias)
    nb = a.shape[1] // 32
    scale = _abs_terms(a, dtype, raw, n)
    if bias is not None:
        scale = scale + np.abs(bias)[None, :]
    # a few f32 roundings per block on the path (the scale product and the
    # min term may be formed as short sums of exact products)
    bound = (4 * nb + 8) * 2.0 ** -24 * scale + 1e-30
    err = np.abs(got.astype(np.float64) - exact)
    assert np.all(err <= bound), f"max err/bound {np.max(err / bound):.3g}"


def check_f16_combine(got, a, dtype, raw, n, bias=None):
    """Encoder regime: f16 operands A' = d_a q_a and W' = d_b q_b + m_b (one
    rounding each, relative 2^-11), exact products, f32 accumulation.  Per
    output: |y - exact| <= (2^-10 + (k + 8) 2^-24) sum_j |a_j w_j| plus the
    f16 subnormal floor, against the exact combination in float64."""
    exact = O.matmul_exact(a, dtype, raw, n, bias=bias)
    k = a.shape[1]
    qa, da, _ = O.quantize_acts(a)
    av = np.abs(qa.astype(np.float64) * np.repeat(da.astype(np.float64), 32, axis=1))
    wv = np.abs(O.dequant(dtype, raw, n, k).astype(np.float64))
    scale = av @ wv.T
    floor = 2.0 ** -25 * av.sum(axis=1)[:, None] + 2.0 ** -30 * av.max(axis=1)[:, None] * wv.sum(axis=1)[None, :]
    bound = (2.0 ** -10 + (k + 8) * 2.0 ** -24) * scale + floor + 1e-30
    if bias is not None:
        bound = bound + 2.0 ** -24 * np.abs(bias)[None, :]
    err = np.abs(got.astype(np.float64) - exact)
    assert np.all(err <= bound), f"max err/bound {np.max(err / bound):.3g}"


def check_combine(got, a, dtype, raw, n, bias=None):
    from rusty_whisper_amd import _abi as A
    if a.shape[0] <= A.GEMV_MAX_M:
        check_exact_combine(got, a, dtype, raw, n, bias)
    else:
        check_f16_combine(got, a, dtype, raw, n, bias)
