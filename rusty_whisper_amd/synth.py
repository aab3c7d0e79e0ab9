"""Synthetic ggml-quantized weights and the Whisper linear shapes they fill.

The reference never produces quantized weights outside its tests; its test
quantizers for Q8_0 (src/quant.rs:1071-1083) and Q5_1 (src/quant.rs:1088-1113)
and the f16 encoder they use (src/model.rs:90-115) are restated here,
vectorized, so benchmarks can build large seeded weight sets quickly.  Q4_0,
Q4_1 and Q5_0 have no reference quantizer; these follow ggml's scheme (the
extreme element of a symmetric block maps to code 0).
"""
from __future__ import annotations

import numpy as np

QK = 32
BLOCK_BYTES = {2: 18, 3: 20, 6: 22, 7: 24, 8: 34}
NAMES = {2: "Q4_0", 3: "Q4_1", 6: "Q5_0", 7: "Q5_1", 8: "Q8_0"}
BY_NAME = {v: k for k, v in NAMES.items()}


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    """src/model.rs:90-115, vectorized (round-half-up on the first dropped bit)."""
    bits = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.int64)
    sign = (bits >> 16) & 0x8000
    exp = (bits >> 23) & 0xFF
    frac = bits & 0x7FFFFF
    e = exp - 127 + 15
    out = np.empty(bits.shape, np.int64)
    nonfinite = exp == 0xFF
    out[nonfinite] = (sign | 0x7C00 | np.where(frac != 0, 0x200, 0))[nonfinite]
    over = ~nonfinite & (e >= 0x1F)
    out[over] = (sign | 0x7C00)[over]
    zero = ~nonfinite & ~over & (e < -10)
    out[zero] = sign[zero]
    sub = ~nonfinite & ~over & ~zero & (e <= 0)
    if np.any(sub):
        f = frac[sub] | 0x800000
        shift = 14 - e[sub]
        half = f >> shift
        rnd = (f >> (shift - 1)) & 1
        out[sub] = sign[sub] | ((half + rnd) & 0xFFFF)
    norm = ~nonfinite & ~over & ~zero & ~sub
    half = (e << 10) | (frac >> 13)
    rnd = (frac >> 12) & 1
    out[norm] = (sign | ((half + rnd) & 0xFFFF))[norm]
    return (out & 0xFFFF).astype(np.uint16)


def _round_away(v: np.ndarray) -> np.ndarray:
    """Rust f32::round (half away from zero) on float32: rint, except exact
    .5 ties (v - trunc(v) is exact in float32), which go away from zero."""
    v = np.asarray(v, dtype=np.float32)
    t = np.trunc(v)
    r = np.rint(v)
    tie = np.abs(v - t) == np.float32(0.5)
    return np.where(tie, t + np.sign(v), r)


def _inv(d: np.ndarray, pos_only: bool) -> np.ndarray:
    ok = d > 0 if pos_only else d != 0
    with np.errstate(divide="ignore"):
        return np.where(ok, np.float32(1.0) / np.where(ok, d, np.float32(1.0)), np.float32(0.0)).astype(np.float32)


def _pack_nibbles(q: np.ndarray) -> np.ndarray:
    q = q.astype(np.uint8)
    return (q[:, :16] & 0x0F) | ((q[:, 16:] & 0x0F) << 4)


def _high_bits(q: np.ndarray) -> np.ndarray:
    bits = ((q.astype(np.uint32) >> 4) & 1) << np.arange(32, dtype=np.uint32)
    return np.bitwise_or.reduce(bits, axis=1).astype(np.uint32)


def _signed_extreme(b: np.ndarray) -> np.ndarray:
    idx = np.argmax(np.abs(b), axis=1)
    return b[np.arange(b.shape[0]), idx]


CHUNK_BLOCKS = 8192  # keeps every temporary ~1 MB, so the allocator reuses it


def quantize(dtype: int, x: np.ndarray) -> np.ndarray:
    """f32 values (length a multiple of 32) -> ggml block bytes of `dtype`."""
    b = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, QK)
    if dtype not in BLOCK_BYTES:
        raise ValueError(f"unsupported dtype {dtype}")
    out = np.empty((b.shape[0], BLOCK_BYTES[dtype]), np.uint8)
    for s in range(0, b.shape[0], CHUNK_BLOCKS):
        out[s:s + CHUNK_BLOCKS] = _quantize_blocks(dtype, b[s:s + CHUNK_BLOCKS])
    return out.reshape(-1)


def _quantize_blocks(dtype: int, b: np.ndarray) -> np.ndarray:
    nblk = b.shape[0]
    out = np.zeros((nblk, BLOCK_BYTES[dtype]), np.uint8)

    def put16(col, vals):
        out[:, col:col + 2] = f32_to_f16_bits(vals).reshape(nblk, 1).view(np.uint8)

    if dtype == 8:  # src/quant.rs:1071-1083
        amax = np.abs(b).max(axis=1)
        d = (amax / np.float32(127.0)).astype(np.float32)
        q = np.clip(_round_away((b * _inv(d, True)[:, None]).astype(np.float32)), -127, 127)
        put16(0, d)
        out[:, 2:] = q.astype(np.int8).view(np.uint8)
    elif dtype in (7, 3):  # src/quant.rs:1088-1113 (and its 4-bit analogue)
        levels = np.float32(31.0 if dtype == 7 else 15.0)
        mn = b.min(axis=1)
        mx = b.max(axis=1)
        d = ((mx - mn) / levels).astype(np.float32)
        q = np.clip(_round_away(((b - mn[:, None]) * _inv(d, True)[:, None]).astype(np.float32)), 0, levels)
        put16(0, d)
        put16(2, mn)
        if dtype == 7:
            out[:, 4:8] = _high_bits(q).reshape(nblk, 1).view(np.uint8)
            out[:, 8:] = _pack_nibbles(q)
        else:
            out[:, 4:] = _pack_nibbles(q)
    elif dtype in (2, 6):
        half = np.float32(8.0 if dtype == 2 else 16.0)
        d = (_signed_extreme(b) / -half).astype(np.float32)
        v = ((b * _inv(d, False)[:, None]).astype(np.float32) + half).astype(np.float32)
        q = np.clip(_round_away(v), 0, 2 * half - 1)
        put16(0, d)
        if dtype == 6:
            out[:, 2:6] = _high_bits(q).reshape(nblk, 1).view(np.uint8)
            out[:, 6:] = _pack_nibbles(q)
        else:
            out[:, 2:] = _pack_nibbles(q)
    return out


def normal_weights(dtype: int, n: int, k: int, seed: int, std: float = 0.02, spread: bool = False) -> np.ndarray:
    """Seeded N(0, std) [n, k] weights quantized to `dtype`; `spread` scales
    each 32-block by 10**U(-1, 1) first."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, k), dtype=np.float32)
    x *= np.float32(std)
    if spread:
        s = (10.0 ** rng.uniform(-1.0, 1.0, size=(n, k // QK, 1))).astype(np.float32)
        x = (x.reshape(n, k // QK, QK) * s).reshape(n, k)
    return quantize(dtype, x)


def normal_weights_many(specs, workers: int = 8):
    """[(dtype, n, k, seed), ...] -> list of ggml byte arrays, built on a
    thread pool (numpy releases the GIL in the heavy loops)."""
    from concurrent.futures import ThreadPoolExecutor

    with ThreadPoolExecutor(max_workers=max(1, workers)) as ex:
        return list(ex.map(lambda s: normal_weights(*s), specs))


# Whisper linear shapes [out, in] per layer (src/encoder.rs:130-171,
# src/decoder.rs:44-53, 148-196, 315-321)
def encoder_layer_shapes(d: int, fc: int):
    return [("q", d, d), ("k", d, d), ("v", d, d), ("out", d, d), ("fc1", fc, d), ("fc2", d, fc)]


def decoder_layer_shapes(d: int, fc: int):
    """The 10 per-layer linears counted by the decode-GEMV workload: self
    Q/K/V/out, cross Q/K/V/out, fc1, fc2."""
    att = [(f"{p}.{x}", d, d) for p in ("self", "cross") for x in ("q", "k", "v", "out")]
    return att + [("fc1", fc, d), ("fc2", d, fc)]


LARGE_V3 = dict(d=1280, fc=5120, layers=32, n_vocab=51866)
SMALL = dict(d=768, fc=3072, layers=12)
TINY = dict(d=384, fc=1536, layers=4)
