"""ctypes binding of librw_rocm.so (the C ABI declared in include/rw_rocm.h).

This is the thin, typed layer every Python caller goes through.  A non-zero
status becomes RwError carrying the library's error text; the reference
panics on the same conditions (src/quant.rs:757-758, 129).  There is no CPU
fallback: if the library or a gfx950 device is missing, calls raise.
"""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "librw_rocm.so")
HEADER_PATH = os.path.join(os.path.dirname(HERE), "include", "rw_rocm.h")

RW_OK, RW_EINVAL, RW_ENODEV, RW_EHIP, RW_ENOMEM, RW_EIO = 0, -1, -2, -3, -4, -5
CODE_NAMES = {RW_EINVAL: "RW_EINVAL", RW_ENODEV: "RW_ENODEV", RW_EHIP: "RW_EHIP", RW_ENOMEM: "RW_ENOMEM",
              RW_EIO: "RW_EIO"}
Q4_0, Q4_1, Q5_0, Q5_1, Q8_0 = 2, 3, 6, 7, 8
DTYPES = (Q4_0, Q4_1, Q5_0, Q5_1, Q8_0)
QK = 32
GEMV_MAX_M = 8


class RwError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"{CODE_NAMES.get(code, code)}: {message}")
        self.code = code
        self.message = message


class rw_linear(C.Structure):
    _fields_ = [
        ("w", C.c_void_p),
        ("a", C.c_void_p),
        ("bias", C.c_void_p),
        ("out", C.c_void_p),
        ("m", C.c_size_t),
    ]


_SIGNATURES = {
    "rw_rocm_version": (C.c_int, []),
    "rw_rocm_device_count": (C.c_int, []),
    "rw_rocm_init": (C.c_int, [C.c_int]),
    "rw_rocm_block_bytes": (C.c_int, [C.c_int]),
    "rw_rocm_weight_upload": (C.c_int, [C.c_int, C.c_size_t, C.c_size_t, C.c_void_p, C.c_size_t,
                                        C.POINTER(C.c_void_p)]),
    "rw_rocm_weight_free": (C.c_int, [C.c_void_p]),
    "rw_rocm_weight_info": (C.c_int, [C.c_void_p, C.POINTER(C.c_int), C.POINTER(C.c_size_t),
                                      C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]),
    "rw_rocm_gelu_quantize_workspace_size": (C.c_size_t, [C.c_size_t, C.c_size_t]),
    "rw_rocm_matmul_prequant_gelu_quantize_dev": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p,
                                                            C.c_void_p, C.c_size_t, C.c_void_p]),
    "rw_rocm_matmul_t_q": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p,
                                     C.c_void_p]),
    "rw_rocm_matmul_t_q_dev": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p,
                                         C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    "rw_rocm_matmul_t_f32": (C.c_int, [C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p, C.c_size_t, C.c_void_p,
                                       C.c_void_p]),
    "rw_rocm_matmul_t_f32_dev": (C.c_int, [C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p, C.c_size_t, C.c_void_p,
                                           C.c_void_p, C.c_void_p]),
    "rw_rocm_matmul_workspace_size": (C.c_size_t, [C.c_size_t, C.c_size_t]),
    "rw_rocm_matmul_t_q_dev_noalloc": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p,
                                                 C.c_void_p, C.c_void_p]),
    "rw_rocm_quantize_dev": (C.c_int, [C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p, C.c_size_t,
                                       C.c_void_p]),
    "rw_rocm_matmul_prequant_dev": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p, C.c_void_p,
                                              C.c_void_p]),
    "rw_rocm_matmul_prequant_multi_dev": (C.c_int, [C.POINTER(C.c_void_p), C.c_size_t, C.c_void_p, C.c_size_t,
                                                    C.POINTER(C.c_void_p), C.POINTER(C.c_void_p), C.c_void_p]),
    "rw_rocm_matmul_grouped_dev": (C.c_int, [C.POINTER(rw_linear), C.c_size_t, C.c_void_p, C.c_size_t,
                                             C.c_void_p]),
    "rw_rocm_grouped_workspace_size": (C.c_size_t, [C.POINTER(rw_linear), C.c_size_t]),
    "rw_rocm_group_create": (C.c_int, [C.POINTER(rw_linear), C.c_size_t, C.POINTER(C.c_void_p)]),
    "rw_rocm_group_run": (C.c_int, [C.c_void_p, C.c_void_p]),
    "rw_rocm_group_free": (None, [C.c_void_p]),
    "rw_rocm_dequant_rows": (C.c_int, [C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p]),
    "rw_rocm_quantize_acts": (C.c_int, [C.c_void_p, C.c_size_t, C.c_size_t, C.c_void_p, C.c_void_p,
                                        C.c_void_p]),
    "rw_rocm_block_dots": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    "rw_rocm_last_error": (C.c_int, [C.c_char_p, C.c_size_t]),
    "rw_rocm_attention_workspace_size": (C.c_size_t, [C.c_size_t, C.c_size_t, C.c_size_t]),
    "rw_rocm_attention_dev": (C.c_int, [C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t,
                                        C.c_size_t, C.c_size_t, C.c_size_t, C.c_int, C.c_int, C.c_void_p,
                                        C.c_size_t, C.c_void_p, C.c_size_t, C.c_void_p]),
    "rw_rocm_attention": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_size_t,
                                    C.c_int, C.c_int, C.c_void_p]),
    "rw_rocm_encoder_layer_workspace_size": (C.c_size_t, [C.c_void_p, C.c_size_t]),
    "rw_rocm_encoder_layer_dev": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p, C.c_size_t,
                                            C.c_void_p]),
    "rw_rocm_decoder_create": (C.c_int, [C.c_void_p, C.c_size_t, C.POINTER(C.c_void_p)]),
    "rw_rocm_decoder_free": (None, [C.c_void_p]),
    "rw_rocm_decoder_set_audio_dev": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p]),
    "rw_rocm_decoder_reset": (C.c_int, [C.c_void_p]),
    "rw_rocm_decoder_n_past": (C.c_int, [C.c_void_p, C.POINTER(C.c_size_t)]),
    "rw_rocm_decoder_fork": (C.c_int, [C.c_void_p, C.c_void_p, C.POINTER(C.c_void_p)]),
    "rw_rocm_decoder_forward_hidden_dev": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p,
                                                     C.c_void_p]),
    "rw_rocm_decoder_forward_beams_dev": (C.c_int, [C.POINTER(C.c_void_p), C.c_size_t, C.c_void_p, C.c_void_p,
                                                    C.c_void_p]),
    "rw_rocm_logits_topk_dev": (C.c_int, [C.c_void_p, C.c_size_t, C.c_size_t, C.c_size_t, C.c_void_p, C.c_void_p,
                                          C.c_void_p, C.c_size_t, C.c_void_p]),
    "rw_rocm_logits_topk_workspace_size": (C.c_size_t, [C.c_size_t, C.c_size_t, C.c_size_t]),
    "rw_rocm_model_load": (C.c_int, [C.c_char_p, C.c_int, C.POINTER(C.c_void_p)]),
    "rw_rocm_model_free": (None, [C.c_void_p]),
    "rw_rocm_model_hparams": (C.c_int, [C.c_void_p, C.POINTER(C.c_int32)]),
    "rw_rocm_model_mel_filters": (C.c_int, [C.c_void_p, C.POINTER(C.POINTER(C.c_float)),
                                            C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]),
    "rw_rocm_model_vocab_size": (C.c_int, [C.c_void_p, C.POINTER(C.c_size_t)]),
    "rw_rocm_model_token": (C.c_int, [C.c_void_p, C.c_size_t, C.POINTER(C.c_void_p), C.POINTER(C.c_size_t)]),
    "rw_rocm_model_tensor_count": (C.c_int, [C.c_void_p, C.POINTER(C.c_size_t)]),
    "rw_rocm_model_tensor_name": (C.c_int, [C.c_void_p, C.c_size_t, C.POINTER(C.c_char_p)]),
    "rw_rocm_model_tensor": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_int), C.POINTER(C.c_int),
                                       C.POINTER(C.c_size_t)]),
    "rw_rocm_model_weight": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_void_p)]),
    "rw_rocm_model_dense": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.POINTER(C.c_float)),
                                      C.POINTER(C.c_size_t)]),
    "rw_rocm_model_raw": (C.c_int, [C.c_void_p, C.c_char_p, C.POINTER(C.c_void_p), C.POINTER(C.c_size_t)]),
}

_lib = None


def header_symbols() -> list[str]:
    """Every function include/rw_rocm.h declares."""
    text = open(HEADER_PATH).read()
    return sorted(set(re.findall(r"\b(rw_rocm_\w+)\s*\(", text)))


def lib() -> C.CDLL:
    """Load librw_rocm.so (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RwError(RW_ENODEV, f"{LIB_PATH} is not built (run __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    buf = C.create_string_buffer(1024)
    lib().rw_rocm_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def check(rc: int) -> int:
    if rc < 0:
        raise RwError(rc, last_error())
    return rc


def _ptr(a) -> int | None:
    if a is None:
        return None
    if isinstance(a, np.ndarray):
        return a.ctypes.data
    if hasattr(a, "data_ptr"):  # torch.Tensor on the device
        return a.data_ptr()
    return int(a)


def init(device: int = 0) -> None:
    check(lib().rw_rocm_init(device))


def device_count() -> int:
    return lib().rw_rocm_device_count()


def block_bytes(dtype: int) -> int:
    return check(lib().rw_rocm_block_bytes(dtype))


class DeviceWeight:
    """A quantized [n, k] matrix resident in HBM (rw_weight*)."""

    def __init__(self, dtype: int, n: int, k: int, raw: np.ndarray):
        raw = np.ascontiguousarray(raw, dtype=np.uint8)
        h = C.c_void_p()
        check(lib().rw_rocm_weight_upload(dtype, n, k, raw.ctypes.data, raw.nbytes, C.byref(h)))
        self.handle = h.value
        self.dtype, self.n, self.k = dtype, n, k

    def info(self):
        dt, n, k, nbytes = C.c_int(), C.c_size_t(), C.c_size_t(), C.c_size_t()
        check(lib().rw_rocm_weight_info(self.handle, C.byref(dt), C.byref(n), C.byref(k), C.byref(nbytes)))
        return dt.value, n.value, k.value, nbytes.value

    def matmul(self, a: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
        """Host arrays in, host array out (rw_rocm_matmul_t_q)."""
        a = np.ascontiguousarray(a, dtype=np.float32)
        if a.ndim != 2:
            raise ValueError("activations must be 2-D [m, k]")
        m, k = a.shape
        out = np.empty((m, self.n), dtype=np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        if b is not None and b.shape != (self.n,):
            raise ValueError(f"bias must have shape ({self.n},)")
        check(lib().rw_rocm_matmul_t_q(self.handle, a.ctypes.data, m, k, _ptr(b), out.ctypes.data))
        return out

    def matmul_dev(self, a, m: int, out, bias=None, workspace=None, workspace_len: int = 0,
                   stream: int | None = None) -> None:
        """Device pointers (ints or torch tensors), queued on `stream`."""
        check(lib().rw_rocm_matmul_t_q_dev(self.handle, _ptr(a), m, self.k, _ptr(bias), _ptr(out),
                                           _ptr(workspace), workspace_len, stream))

    def matmul_dev_noalloc(self, a, m: int, out, bias=None, stream: int | None = None) -> None:
        """matmul_dev with the library's fixed device scratch (no allocation)."""
        check(lib().rw_rocm_matmul_t_q_dev_noalloc(self.handle, _ptr(a), m, self.k, _ptr(bias), _ptr(out), stream))

    def matmul_prequant_dev(self, workspace, m: int, out, bias=None, stream: int | None = None) -> None:
        """out = (activations quantized into `workspace`) W^T (+ bias)."""
        check(lib().rw_rocm_matmul_prequant_dev(self.handle, _ptr(workspace), m, _ptr(bias), _ptr(out),
                                                stream))

    def dequant_rows(self, row0: int = 0, nrows: int | None = None) -> np.ndarray:
        nrows = self.n - row0 if nrows is None else nrows
        out = np.empty((nrows, self.k), dtype=np.float32)
        check(lib().rw_rocm_dequant_rows(self.handle, row0, nrows, out.ctypes.data))
        return out

    def block_dots(self, qa: np.ndarray) -> np.ndarray:
        qa = np.ascontiguousarray(qa, dtype=np.int8)
        m = qa.shape[0]
        S = np.empty((m, self.n, self.k // QK), dtype=np.int32)
        check(lib().rw_rocm_block_dots(self.handle, qa.ctypes.data, m, S.ctypes.data))
        return S

    def free(self) -> None:
        if getattr(self, "handle", None):
            check(lib().rw_rocm_weight_free(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def matmul_prequant_multi_dev(weights, workspace, m: int, outs, biases=None, stream: int | None = None) -> None:
    """out[i] = (activations quantized into `workspace`) W_i^T (+ biases[i]) for
    up to 4 weights of one dtype and k, in one launch for m > 8."""
    cnt = len(weights)
    warr = (C.c_void_p * max(cnt, 1))(*[w.handle for w in weights])
    oarr = (C.c_void_p * max(cnt, 1))(*[_ptr(o) for o in outs])
    barr = None if biases is None else (C.c_void_p * max(cnt, 1))(*[_ptr(b) for b in biases])
    check(lib().rw_rocm_matmul_prequant_multi_dev(warr, cnt, _ptr(workspace), m, barr, oarr, stream))


def gelu_quantize_workspace_size(m: int, n: int) -> int:
    return lib().rw_rocm_gelu_quantize_workspace_size(m, n)


def matmul_prequant_gelu_quantize_dev(w, workspace, m: int, bias, next_workspace, next_len: int,
                                      stream: int | None = None) -> None:
    """gelu(a W^T + bias) from a quantized `workspace`, quantized into
    `next_workspace` for the next product (rw_rocm_matmul_prequant_gelu_quantize_dev)."""
    check(lib().rw_rocm_matmul_prequant_gelu_quantize_dev(w.handle, _ptr(workspace), m, _ptr(bias),
                                                          _ptr(next_workspace), next_len, stream))


def matmul_t_f32(a: np.ndarray, b: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
    """The dense f32 tier on the device: a[m, k] b[n, k]^T (+ bias), host arrays."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    m, k = a.shape
    n = b.shape[0]
    if b.shape[1] != k:
        raise ValueError(f"inner dims: {k} vs {b.shape[1]}")
    bb = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    out = np.empty((m, n), np.float32)
    check(lib().rw_rocm_matmul_t_f32(a.ctypes.data, m, k, b.ctypes.data, n, None if bb is None else bb.ctypes.data,
                                     out.ctypes.data))
    return out


def matmul_t_f32_dev(a, m: int, k: int, b, n: int, out, bias=None, stream: int | None = None) -> None:
    """Device pointers (ints or torch tensors), queued on `stream`."""
    check(lib().rw_rocm_matmul_t_f32_dev(_ptr(a), m, k, _ptr(b), n, _ptr(bias), _ptr(out), stream))


def workspace_size(m: int, k: int) -> int:
    return lib().rw_rocm_matmul_workspace_size(m, k)


def quantize_dev(a, m: int, k: int, workspace, workspace_len: int, stream: int | None = None) -> None:
    """Quantize device activations a[m, k] into `workspace` (queued on `stream`)."""
    check(lib().rw_rocm_quantize_dev(_ptr(a), m, k, _ptr(workspace), workspace_len, stream))


def quantize_acts(a: np.ndarray):
    """Device quantize_acts_i8 -> (q int8 [m,k], d f32 [m,nb], sum i32 [m,nb])."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    m, k = a.shape
    nb = k // QK
    q = np.empty((m, k), dtype=np.int8)
    d = np.empty((m, nb), dtype=np.float32)
    s = np.empty((m, nb), dtype=np.int32)
    check(lib().rw_rocm_quantize_acts(a.ctypes.data, m, k, q.ctypes.data, d.ctypes.data, s.ctypes.data))
    return q, d, s


def make_linears(items) -> "C.Array":
    """items: iterable of (DeviceWeight, a_ptr, bias_ptr_or_None, out_ptr, m)."""
    items = list(items)
    arr = (rw_linear * len(items))()
    for i, (w, a, b, o, m) in enumerate(items):
        arr[i] = rw_linear(w.handle, _ptr(a), _ptr(b), _ptr(o), m)
    return arr


def grouped_workspace_size(arr) -> int:
    return lib().rw_rocm_grouped_workspace_size(arr, len(arr))


def matmul_grouped_dev(arr, workspace=None, workspace_len: int = 0, stream: int | None = None) -> None:
    check(lib().rw_rocm_matmul_grouped_dev(arr, len(arr), _ptr(workspace), workspace_len, stream))


class Group:
    """A prepared group of decode-shape linears (rw_rocm_group_create): the
    launch tables stay on the device and run() only launches."""

    def __init__(self, arr):
        h = C.c_void_p()
        check(lib().rw_rocm_group_create(arr, len(arr), C.byref(h)))
        self.handle = h.value
        self._arr = arr  # the items' buffers must outlive the group

    def run(self, stream: int | None = None) -> None:
        check(lib().rw_rocm_group_run(self.handle, stream))

    def free(self) -> None:
        if self.handle:
            lib().rw_rocm_group_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ------------------------------------------------------------ attention

def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, n_head: int, causal: bool = False) -> np.ndarray:
    """Host arrays in, host array out (rw_rocm_attention): the reference's
    multi_head_attention (src/encoder.rs:109-119)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    if q.ndim != 2 or k.ndim != 2 or v.shape != k.shape or (k.size and k.shape[1] != q.shape[1]):
        raise ValueError("q [t_q, n_state], k and v [t_kv, n_state]")
    t_q, n_state = q.shape
    out = np.empty((t_q, n_state), dtype=np.float32)
    check(lib().rw_rocm_attention(q.ctypes.data, k.ctypes.data, v.ctypes.data, t_q, k.shape[0], n_state, n_head,
                                  1 if causal else 0, out.ctypes.data))
    return out


def attention_workspace_size(t_q: int, t_kv: int, n_state: int) -> int:
    return lib().rw_rocm_attention_workspace_size(t_q, t_kv, n_state)


def attention_dev(q, k, v, t_q: int, t_kv: int, n_state: int, n_head: int, causal: bool, out,
                  ldq: int | None = None, ldk: int | None = None, ldv: int | None = None, ldo: int | None = None,
                  workspace=None, workspace_len: int = 0, stream: int | None = None) -> None:
    """Device pointers (ints or torch tensors) with row strides in floats."""
    check(lib().rw_rocm_attention_dev(_ptr(q), ldq or n_state, _ptr(k), ldk or n_state, _ptr(v), ldv or n_state,
                                      t_q, t_kv, n_state, n_head, 1 if causal else 0, _ptr(out), ldo or n_state,
                                      _ptr(workspace), workspace_len, stream))


# ------------------------------------------------------- encoder layer

class RwEncoderLayer(C.Structure):
    """struct rw_encoder_layer (include/rw_rocm.h)."""
    _fields_ = [("attn_ln_w", C.c_void_p), ("attn_ln_b", C.c_void_p),
                ("q", C.c_void_p), ("k", C.c_void_p), ("v", C.c_void_p), ("out", C.c_void_p),
                ("q_b", C.c_void_p), ("k_b", C.c_void_p), ("v_b", C.c_void_p), ("out_b", C.c_void_p),
                ("mlp_ln_w", C.c_void_p), ("mlp_ln_b", C.c_void_p),
                ("fc1", C.c_void_p), ("fc2", C.c_void_p), ("fc1_b", C.c_void_p), ("fc2_b", C.c_void_p),
                ("n_head", C.c_int)]


class EncoderLayer:
    """One encoder layer's resident parameters: DeviceWeight matrices and
    device vectors (torch tensors or device pointers), run by
    rw_rocm_encoder_layer_dev (src/encoder.rs:121-175)."""

    VECS = ("attn_ln_w", "attn_ln_b", "q_b", "k_b", "v_b", "out_b", "mlp_ln_w", "mlp_ln_b", "fc1_b", "fc2_b")
    MATS = ("q", "k", "v", "out", "fc1", "fc2")

    def __init__(self, n_head: int, **params):
        self.params = params  # keeps the tensors alive
        fields = {k: _ptr(params.get(k)) for k in self.VECS}
        fields.update({k: params[k].handle for k in self.MATS})
        self.st = RwEncoderLayer(n_head=n_head, **fields)

    def workspace_size(self, t: int) -> int:
        return lib().rw_rocm_encoder_layer_workspace_size(C.byref(self.st), t)

    def run(self, x, t: int, workspace=None, workspace_len: int = 0, stream: int | None = None) -> None:
        """x [t, n_state] on the device, updated in place."""
        check(lib().rw_rocm_encoder_layer_dev(C.byref(self.st), _ptr(x), t, _ptr(workspace), workspace_len,
                                              stream))


# ------------------------------------------------------------- decoder

_DEC_LAYER_VECS = ("attn_ln_w", "attn_ln_b", "q_b", "v_b", "out_b", "cross_ln_w", "cross_ln_b", "cq_b", "cv_b",
                   "cout_b", "mlp_ln_w", "mlp_ln_b", "fc1_b", "fc2_b")
_DEC_LAYER_MATS = ("q", "k", "v", "out", "cq", "ck", "cv", "cout", "fc1", "fc2")


class RwDecoderLayer(C.Structure):
    """struct rw_decoder_layer (include/rw_rocm.h)."""
    _fields_ = [(name, C.c_void_p) for name in (
        "attn_ln_w", "attn_ln_b", "q", "k", "v", "out", "q_b", "v_b", "out_b", "cross_ln_w", "cross_ln_b",
        "cq", "ck", "cv", "cout", "cq_b", "cv_b", "cout_b", "mlp_ln_w", "mlp_ln_b", "fc1", "fc2", "fc1_b",
        "fc2_b")]


class RwDecoderParams(C.Structure):
    _fields_ = [("n_layer", C.c_int), ("n_head", C.c_int), ("n_ctx", C.c_int), ("layers", C.c_void_p),
                ("token_embedding", C.c_void_p), ("positional", C.c_void_p), ("ln_w", C.c_void_p),
                ("ln_b", C.c_void_p)]


class Decoder:
    """rw_decoder: the reference's Decoder (src/decoder.rs:26-213) with its
    caches resident.  layers: list of dicts of DeviceWeight matrices and
    device vectors; token_embedding a DeviceWeight; positional, ln_w, ln_b
    device vectors."""

    def __init__(self, n_head: int, n_ctx: int, n_audio_ctx: int, layers, token_embedding, positional, ln_w, ln_b,
                 _handle=None, _keep=None):
        self._keep = _keep or (layers, token_embedding, positional, ln_w, ln_b)
        if _handle is not None:
            self.handle = _handle
            return
        arr = (RwDecoderLayer * len(layers))()
        for i, L in enumerate(layers):
            for k in _DEC_LAYER_VECS:
                setattr(arr[i], k, _ptr(L.get(k)))
            for k in _DEC_LAYER_MATS:
                setattr(arr[i], k, L[k].handle)
        prm = RwDecoderParams(len(layers), n_head, n_ctx, C.cast(arr, C.c_void_p), token_embedding.handle,
                              _ptr(positional), _ptr(ln_w), _ptr(ln_b))
        h = C.c_void_p()
        check(lib().rw_rocm_decoder_create(C.byref(prm), n_audio_ctx, C.byref(h)))
        self.handle = h.value

    @property
    def token_embedding(self) -> DeviceWeight:
        """The tied embedding, whose product with the hidden rows is the
        logits (src/decoder.rs:315-321)."""
        return self._keep[1]

    def set_audio(self, enc_out, stream: int | None = None) -> None:
        check(lib().rw_rocm_decoder_set_audio_dev(self.handle, _ptr(enc_out), stream))

    def reset(self) -> None:
        check(lib().rw_rocm_decoder_reset(self.handle))

    @property
    def n_past(self) -> int:
        n = C.c_size_t()
        check(lib().rw_rocm_decoder_n_past(self.handle, C.byref(n)))
        return n.value

    def fork(self, stream: int | None = None) -> "Decoder":
        h = C.c_void_p()
        check(lib().rw_rocm_decoder_fork(self.handle, stream, C.byref(h)))
        return Decoder(0, 0, 0, None, None, None, None, None, _handle=h.value, _keep=self._keep)

    def forward_hidden(self, tokens, hidden, stream: int | None = None) -> None:
        """tokens: host ids; hidden: device [len(tokens), n_state]."""
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        check(lib().rw_rocm_decoder_forward_hidden_dev(self.handle, t.ctypes.data, t.size, _ptr(hidden), stream))

    def free(self) -> None:
        if getattr(self, "handle", None):
            lib().rw_rocm_decoder_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def decoder_forward_beams(beams, tokens, hidden, stream: int | None = None) -> None:
    """One beam-search step: beam i (a Decoder forked from one decoder)
    forwards tokens[i]; hidden: device [len(beams), n_state]."""
    t = np.ascontiguousarray(tokens, dtype=np.uint32)
    arr = (C.c_void_p * max(len(beams), 1))(*[b.handle for b in beams])
    check(lib().rw_rocm_decoder_forward_beams_dev(arr, len(beams), t.ctypes.data, _ptr(hidden), stream))


def logits_topk_dev(logits, rows: int, n_vocab: int, k: int, ids, logprobs, stream: int | None = None,
                    workspace=None, workspace_len: int = 0) -> None:
    """log_softmax + top_k of each row of device logits into device ids
    (uint32 [rows, k]) and logprobs (f32 [rows, k])."""
    check(lib().rw_rocm_logits_topk_dev(_ptr(logits), rows, n_vocab, k, _ptr(ids), _ptr(logprobs),
                                        _ptr(workspace), workspace_len, stream))


def logits_topk_workspace_size(rows: int, n_vocab: int, k: int) -> int:
    return lib().rw_rocm_logits_topk_workspace_size(rows, n_vocab, k)


MODEL_PARSE_ONLY = 1
HPARAM_NAMES = ("n_vocab", "n_audio_ctx", "n_audio_state", "n_audio_head", "n_audio_layer", "n_text_ctx",
                "n_text_state", "n_text_head", "n_text_layer", "n_mels", "ftype")


class _ModelWeight(DeviceWeight):
    """A quantized matrix owned by a Model (freed with it)."""

    def __init__(self, handle: int, dtype: int, n: int, k: int, owner: "Model"):
        self.handle, self.dtype, self.n, self.k = handle, dtype, n, k
        self._owner = owner

    def free(self) -> None:
        self.handle = None

    def __del__(self):
        pass


class Model:
    """A whisper model file (ggml .bin or GGUF) loaded by rw_rocm_model_load:
    hparams, mel filters, vocab, and named tensors -- quantized matrices as
    resident device weights, the rest as host f32 arrays."""

    def __init__(self, path: str, parse_only: bool = False):
        h = C.c_void_p()
        check(lib().rw_rocm_model_load(os.fsencode(path), MODEL_PARSE_ONLY if parse_only else 0, C.byref(h)))
        self.handle = h.value
        hp = (C.c_int32 * 11)()
        check(lib().rw_rocm_model_hparams(self.handle, hp))
        self.hparams = dict(zip(HPARAM_NAMES, list(hp)))

    def mel_filters(self) -> np.ndarray:
        p, nm, nf = C.POINTER(C.c_float)(), C.c_size_t(), C.c_size_t()
        check(lib().rw_rocm_model_mel_filters(self.handle, C.byref(p), C.byref(nm), C.byref(nf)))
        n = nm.value * nf.value
        if n == 0:
            return np.zeros((nm.value, nf.value), dtype=np.float32)
        return np.ctypeslib.as_array(p, shape=(n,)).copy().reshape(nm.value, nf.value)

    def vocab(self) -> list[bytes]:
        n = C.c_size_t()
        check(lib().rw_rocm_model_vocab_size(self.handle, C.byref(n)))
        out = []
        for i in range(n.value):
            p, ln = C.c_void_p(), C.c_size_t()
            check(lib().rw_rocm_model_token(self.handle, i, C.byref(p), C.byref(ln)))
            out.append(C.string_at(p.value, ln.value) if ln.value else b"")
        return out

    def names(self) -> list[str]:
        n = C.c_size_t()
        check(lib().rw_rocm_model_tensor_count(self.handle, C.byref(n)))
        out = []
        for i in range(n.value):
            nm = C.c_char_p()
            check(lib().rw_rocm_model_tensor_name(self.handle, i, C.byref(nm)))
            out.append(nm.value.decode(errors="replace"))
        return out

    def tensor(self, name: str):
        """(dtype, row-major shape, is_quantized_matrix)."""
        dt, nd = C.c_int(), C.c_int()
        sh = (C.c_size_t * 3)()
        q = check(lib().rw_rocm_model_tensor(self.handle, name.encode(), C.byref(dt), C.byref(nd), sh))
        return dt.value, tuple(sh[: nd.value]), bool(q)

    def weight(self, name: str) -> DeviceWeight:
        h = C.c_void_p()
        check(lib().rw_rocm_model_weight(self.handle, name.encode(), C.byref(h)))
        dt, shape, _ = self.tensor(name)
        return _ModelWeight(h.value, dt, shape[0], shape[1], self)

    def dense(self, name: str) -> np.ndarray:
        p, n = C.POINTER(C.c_float)(), C.c_size_t()
        check(lib().rw_rocm_model_dense(self.handle, name.encode(), C.byref(p), C.byref(n)))
        _, shape, _ = self.tensor(name)
        if n.value == 0:
            return np.zeros(shape, dtype=np.float32)
        return np.ctypeslib.as_array(p, shape=(n.value,)).copy().reshape(shape)

    def raw(self, name: str) -> bytes:
        p, n = C.c_void_p(), C.c_size_t()
        check(lib().rw_rocm_model_raw(self.handle, name.encode(), C.byref(p), C.byref(n)))
        return C.string_at(p.value, n.value) if n.value else b""

    def free(self) -> None:
        if getattr(self, "handle", None):
            lib().rw_rocm_model_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
