"""Multi-head attention, restated in numpy -- TEST INFRASTRUCTURE ONLY.

The CPU restatement of rusty_whisper's attention (src/encoder.rs:48-80
mha_split_kv, :109-119 multi_head_attention, src/encoder.rs:28-41
split_heads, src/tensor.rs:309-330 softmax), used by tests/ to check the
device kernel.  The product package never imports it.

Pinned by tests/test_attention_oracle.py: the reference's own attention
tests (src/encoder.rs:328-375), brute force over tiny inputs, SciPy's
softmax in float64, and invariants (kv permutation, head independence,
softmax shift invariance).
"""
from __future__ import annotations

import numpy as np


def split_heads(x: np.ndarray, n_head: int) -> np.ndarray:
    """[t, n_state] -> [n_head, t, n_state / n_head] (src/encoder.rs:28-41)."""
    t, n_state = x.shape
    if n_state % n_head:
        raise ValueError("n_state must be a multiple of n_head")
    return np.ascontiguousarray(x.reshape(t, n_head, n_state // n_head).transpose(1, 0, 2))


def softmax_rows(s: np.ndarray) -> np.ndarray:
    """Row-wise softmax as src/tensor.rs:309-330: subtract the row maximum,
    exponentiate, divide by the sum (float32 throughout)."""
    s = np.asarray(s, dtype=np.float32)
    mx = np.max(s, axis=-1, keepdims=True)
    e = np.exp(s - mx, dtype=np.float32)
    return (e / np.sum(e, axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)


def mha(q: np.ndarray, k: np.ndarray, v: np.ndarray, n_head: int, causal: bool,
        dtype=np.float32) -> np.ndarray:
    """out[t_q, n_state] = concat_h softmax(q_h k_h^T / sqrt(dh) + mask) v_h
    (src/encoder.rs:48-80).  Query row i sits at absolute position
    t_kv - t_q + i; with `causal` it sees kv rows 0 .. t_kv - t_q + i.
    dtype float64 gives the same steps in double precision."""
    q = np.asarray(q, dtype=dtype)
    k = np.asarray(k, dtype=dtype)
    v = np.asarray(v, dtype=dtype)
    t_q, n_state = q.shape
    t_kv = k.shape[0]
    if k.shape[1] != n_state or v.shape != k.shape:
        raise ValueError("k and v must be [t_kv, n_state] like q's columns")
    if causal and t_q > t_kv:
        raise ValueError("causal attention needs t_q <= t_kv")
    dh = n_state // n_head
    scale = dtype(1.0) / np.sqrt(dtype(dh))
    qh, kh, vh = split_heads(q, n_head), split_heads(k, n_head), split_heads(v, n_head)
    out = np.empty((t_q, n_state), dtype=dtype)
    for h in range(n_head):
        s = (qh[h] @ kh[h].T).astype(dtype) * scale
        if causal:
            off = t_kv - t_q
            j = np.arange(t_kv)[None, :]
            i = np.arange(t_q)[:, None]
            s = np.where(j > off + i, dtype(-np.inf), s)
        mx = np.max(s, axis=-1, keepdims=True)
        e = np.exp(s - mx)
        p = e / np.sum(e, axis=-1, keepdims=True)
        out[:, h * dh:(h + 1) * dh] = p @ vh[h]
    return out
