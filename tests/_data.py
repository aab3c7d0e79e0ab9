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


def rel_row_l2(got: np.ndarray, ref: np.ndarray) -> float:
    """max_ij |got-ref| / ||ref_i||_2 -- the north-star output tolerance."""
    ref64 = ref.astype(np.float64)
    norms = np.linalg.norm(ref64, axis=1, keepdims=True)
    norms = np.where(norms > 0, norms, 1.0)
    return float(np.max(np.abs(got.astype(np.float64) - ref64) / norms))
