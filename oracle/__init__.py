"""ctypes view of oracle/liboracle.so -- TEST INFRASTRUCTURE ONLY.

The oracle is the CPU restatement of rusty_whisper's quantized matmul
(src/quant.rs, the f16 codec of src/model.rs and the f32 dot of src/tensor.rs).
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only as the parity reference or the timed CPU baseline; the product
package (rusty_whisper_amd) never imports it.

See oracle.h for which reference lines each function restates and what pins
each of them.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")

QK = 32
BLOCK_BYTES = {2: 18, 3: 20, 6: 22, 7: 24, 8: 34}
DTYPE_NAMES = {2: "Q4_0", 3: "Q4_1", 6: "Q5_0", 7: "Q5_1", 8: "Q8_0"}
TIER_VNNI, TIER_AVX2, TIER_F32 = 0, 1, 2

_lib = None


def build() -> None:
    """Compile liboracle.so from oracle.c + cpu_baseline.c (gcc via make)."""
    import subprocess

    subprocess.run(["make", "-s", "-B", "-C", _HERE, "liboracle.so"], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run oracle.build()")
        L = C.CDLL(LIB_PATH)
        vp, sz, i32, u32 = C.c_void_p, C.c_size_t, C.c_int, C.c_uint32
        sig = {
            "or_f16_to_f32": (C.c_float, [C.c_uint16]),
            "or_f16_to_f32_array": (None, [vp, sz, vp]),
            "or_f32_to_f16": (C.c_uint16, [C.c_float]),
            "or_block_bytes": (i32, [i32]),
            "or_unpack_block": (i32, [i32, vp, vp, vp, vp]),
            "or_dequant_row": (i32, [i32, vp, sz, vp]),
            "or_quantize_acts": (None, [vp, sz, sz, vp, vp, vp]),
            "or_unpack_row_i8": (i32, [i32, vp, sz, vp, vp, vp, vp]),
            "or_block_dots": (i32, [i32, vp, sz, sz, vp, sz, vp]),
            "or_matmul_emul": (i32, [i32, vp, sz, sz, i32, vp, sz, vp, vp]),
            "or_matmul_exact": (i32, [vp, sz, sz, i32, vp, sz, vp, vp]),
            "or_matmul_t_dense": (None, [vp, sz, sz, vp, sz, vp]),
            "or_test_matrix": (None, [sz, u32, vp]),
            "or_quantize": (sz, [i32, vp, sz, vp]),
            "cb_detect_tier": (i32, []),
            "cb_hw_threads": (i32, []),
            "cb_qtensor_new": (vp, [i32, sz, sz, vp]),
            "cb_qtensor_free": (None, [vp]),
            "cb_matmul_t_q": (i32, [vp, sz, vp, vp, vp, i32, i32, C.POINTER(i32)]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _p(arr: np.ndarray | None):
    return None if arr is None else arr.ctypes.data


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ------------------------------------------------------------- codecs

def f16_to_f32(h: int) -> float:
    """model.rs:68-86"""
    return lib().or_f16_to_f32(h)


def f16_to_f32_bits(codes: np.ndarray) -> np.ndarray:
    """Vector form of f16_to_f32 returning the f32 bit patterns (uint32)."""
    codes = np.ascontiguousarray(codes, dtype=np.uint16)
    out = np.empty(codes.shape, dtype=np.float32)
    lib().or_f16_to_f32_array(_p(codes), codes.size, _p(out))
    return out.view(np.uint32)


def f32_to_f16(x: float) -> int:
    """model.rs:90-115"""
    return lib().or_f32_to_f16(x)


def block_bytes(dtype: int) -> int:
    """quant.rs:43-52 (-1 when unsupported)"""
    return lib().or_block_bytes(dtype)


def unpack_block(dtype: int, block: bytes):
    """quant.rs:98-131 -> (q[32] int8, d, m)"""
    blk = np.frombuffer(bytes(block), dtype=np.uint8).copy()
    q = np.zeros(QK, dtype=np.int8)
    d = np.zeros(1, dtype=np.float32)
    m = np.zeros(1, dtype=np.float32)
    if lib().or_unpack_block(dtype, _p(blk), _p(q), _p(d), _p(m)) != 0:
        raise ValueError(f"unpack of unsupported dtype {dtype}")
    return q, float(d[0]), float(m[0])


def dequant(dtype: int, raw: np.ndarray, n: int, k: int) -> np.ndarray:
    """quant.rs:528-537 over a whole [n,k] matrix (QTensor::to_dense)."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty((n, k), dtype=np.float32)
    if lib().or_dequant_row(dtype, _p(raw), n * k // QK, _p(out)) != 0:
        raise ValueError(f"dequant of unsupported dtype {dtype}")
    return out


def quantize_acts(a: np.ndarray):
    """quant.rs:691-716 -> (q int8 [m,k], d f32 [m,nb], sum i32 [m,nb])"""
    a = _f32(a)
    m, k = a.shape
    nb = k // QK
    q = np.empty((m, k), dtype=np.int8)
    d = np.empty((m, nb), dtype=np.float32)
    s = np.empty((m, nb), dtype=np.int32)
    lib().or_quantize_acts(_p(a), m, k, _p(q), _p(d), _p(s))
    return q, d, s


def unpack_rows(dtype: int, raw: np.ndarray, n: int, k: int):
    """quant.rs:256-320 + 403-418 -> (qb [n,k], db [n,nb], mb [n,nb], sumb [n,nb])"""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    nb = k // QK
    bb = BLOCK_BYTES[dtype]
    qb = np.empty((n, k), dtype=np.int8)
    db = np.empty((n, nb), dtype=np.float32)
    mb = np.empty((n, nb), dtype=np.float32)
    sb = np.empty((n, nb), dtype=np.int32)
    for j in range(n):
        row = raw[j * nb * bb:(j + 1) * nb * bb]
        lib().or_unpack_row_i8(dtype, _p(row), nb, qb[j].ctypes.data, db[j].ctypes.data,
                               mb[j].ctypes.data, sb[j].ctypes.data)
    return qb, db, mb, sb


def block_dots(dtype: int, raw: np.ndarray, n: int, k: int, qa: np.ndarray) -> np.ndarray:
    """Exact per-block integer sums S[i,j,bl] (int32 [m,n,nb])."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    qa = np.ascontiguousarray(qa, dtype=np.int8)
    m = qa.shape[0]
    S = np.empty((m, n, k // QK), dtype=np.int32)
    if lib().or_block_dots(dtype, _p(raw), n, k, _p(qa), m, _p(S)) != 0:
        raise ValueError("bad dtype or k")
    return S


def matmul_emul(a: np.ndarray, dtype: int, raw: np.ndarray, n: int, bias=None,
                tier: int = TIER_VNNI) -> np.ndarray:
    """Bitwise emulation of the reference's int8 tier (VNNI or AVX2)."""
    a = _f32(a)
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    m, k = a.shape
    out = np.empty((m, n), dtype=np.float32)
    b = None if bias is None else _f32(bias)
    if lib().or_matmul_emul(tier, _p(a), m, k, dtype, _p(raw), n, _p(b), _p(out)) != 0:
        raise ValueError("bad tier, dtype or k")
    return out


def matmul_exact(a: np.ndarray, dtype: int, raw: np.ndarray, n: int, bias=None) -> np.ndarray:
    """Exact integer sums combined in float64 (float64 [m,n])."""
    a = _f32(a)
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    m, k = a.shape
    out = np.empty((m, n), dtype=np.float64)
    b = None if bias is None else _f32(bias)
    if lib().or_matmul_exact(_p(a), m, k, dtype, _p(raw), n, _p(b), _p(out)) != 0:
        raise ValueError("bad dtype or k")
    return out


def matmul_t_dense(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """tensor.rs:194-238 (f32, 8-lane dot)."""
    a, b = _f32(a), _f32(b)
    m, k = a.shape
    n = b.shape[0]
    out = np.empty((m, n), dtype=np.float32)
    lib().or_matmul_t_dense(_p(a), m, k, _p(b), n, _p(out))
    return out


def test_matrix(n: int, k: int, seed: int) -> np.ndarray:
    """quant.rs:1115-1123 (flat, n*k values)."""
    out = np.empty(n * k, dtype=np.float32)
    lib().or_test_matrix(n * k, seed, _p(out))
    return out


def quantize(dtype: int, x: np.ndarray) -> np.ndarray:
    """Encode f32 values into ggml blocks of `dtype` (uint8 bytes)."""
    x = _f32(x).reshape(-1)
    if x.size % QK:
        raise ValueError("length must be a multiple of 32")
    raw = np.empty(x.size // QK * BLOCK_BYTES[dtype], dtype=np.uint8)
    lib().or_quantize(dtype, _p(x), x.size, _p(raw))
    return raw


# ------------------------------------------------- CPU baseline (timed)

def cpu_tier() -> int:
    return lib().cb_detect_tier()


def cpu_threads() -> int:
    return lib().cb_hw_threads()


class CpuQTensor:
    """The reference's QTensor + matmul_t_q restated with AVX2 / VNNI
    intrinsics and threads (oracle/cpu_baseline.c): first call cold path,
    packed int8 cache from the second call on."""

    def __init__(self, dtype: int, n: int, k: int, raw: np.ndarray):
        self._raw = np.ascontiguousarray(raw, dtype=np.uint8)
        self.n, self.k, self.dtype = n, k, dtype
        self._h = lib().cb_qtensor_new(dtype, n, k, _p(self._raw))
        if not self._h:
            raise ValueError("bad dtype or k")

    def matmul(self, a: np.ndarray, bias=None, tier: int = -1, threads: int = 0) -> np.ndarray:
        a = _f32(a)
        m = a.shape[0]
        out = np.empty((m, self.n), dtype=np.float32)
        used = C.c_int(-1)
        b = None if bias is None else _f32(bias)
        rc = lib().cb_matmul_t_q(_p(a), m, self._h, _p(b), _p(out), tier, threads, C.byref(used))
        if rc != 0:
            raise RuntimeError(f"cb_matmul_t_q failed ({rc})")
        self.tier_used = used.value
        return out

    def close(self):
        if self._h:
            lib().cb_qtensor_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
