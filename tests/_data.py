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
    i = np.ones(k, np.float32)
    i[5] = np.inf  # amax = inf -> inv = 0 -> q = 0 (inf*0 = NaN -> 0)
    rows.append(i)
    b = np.full(k, 3.4e38, np.float32)
    b[2] = -3.4e38
    rows.append(b)
    return np.stack(rows)


def rel_row_l2(got: np.ndarray, ref: np.ndarray) -> float:
    """max_ij |got-ref| / ||ref_i||_2 -- the north-star output tolerance."""
    ref64 = ref.astype(np.float64)
    norms = np.linalg.norm(ref64, axis=1, keepdims=True)
    norms = np.where(norms > 0, norms, 1.0)
    return float(np.max(np.abs(got.astype(np.float64) - ref64) / norms))
