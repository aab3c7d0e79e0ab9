"""One whisper encoder layer, restated on the CPU -- TEST INFRASTRUCTURE ONLY.

self_attention_block + mlp_block of src/encoder.rs:121-175 (non-causal), with
layernorm (src/tensor.rs:274-287), GELU (src/tensor.rs:289-305), the
quantized linears of src/quant.rs (the oracle's bitwise emulation of the
reference's int8 tier, oracle.matmul_emul) and attention (oracle/attention.py).
Used by tests/ to check the device encoder layer; the product package never
imports it.

Pinned by tests/test_encoder_oracle.py: layernorm's closed form (zero mean,
unit variance before the affine part) and a float64 restatement, GELU's
known values and its relation to the exact erf form, and the layer against a
float64 composition of the same steps with dense dequantized weights.
"""
from __future__ import annotations

import numpy as np

import oracle as O
from oracle.attention import mha

EPS = np.float32(1e-5)


def layernorm(x: np.ndarray, w: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Row-wise (x - mean) * inv * w + b in float32, inv = 1 / sqrt(var + 1e-5)."""
    x = np.asarray(x, np.float32)
    cols = np.float32(x.shape[1])
    mean = (x.sum(axis=1, dtype=np.float32) / cols).astype(np.float32)[:, None]
    d = (x - mean).astype(np.float32)
    var = ((d * d).sum(axis=1, dtype=np.float32) / cols).astype(np.float32)[:, None]
    inv = (np.float32(1.0) / np.sqrt(var + EPS)).astype(np.float32)
    return (d * inv * np.asarray(w, np.float32) + np.asarray(b, np.float32)).astype(np.float32)


def gelu(x: np.ndarray) -> np.ndarray:
    """0.5 t (1 + tanh(sqrt(2/pi) (t + 0.044715 t^3))) in float32."""
    t = np.asarray(x, np.float32)
    inner = np.float32(0.7978846) * (t + np.float32(0.044715) * t * t * t)
    return (np.float32(0.5) * t * (np.float32(1.0) + np.tanh(inner))).astype(np.float32)


def linear(a: np.ndarray, w: dict, bias=None) -> np.ndarray:
    """linear_w for a quantized weight w = {"dtype", "raw", "n"} (src/quant.rs:1054-1063)."""
    return O.matmul_emul(a, w["dtype"], w["raw"], w["n"], bias=bias, tier=O.TIER_VNNI)


def encoder_layer(x: np.ndarray, p: dict, n_head: int) -> np.ndarray:
    """x [t, n_state] -> x after the attention and MLP sub-blocks.  p holds
    attn_ln_w/b, q/k/v/out (quantized weights), q_b, v_b, out_b, mlp_ln_w/b,
    fc1, fc1_b, fc2, fc2_b."""
    x = np.array(x, np.float32)
    cur = layernorm(x, p["attn_ln_w"], p["attn_ln_b"])
    q = linear(cur, p["q"], p["q_b"])
    k = linear(cur, p["k"], None)  # whisper's key projection has no bias
    v = linear(cur, p["v"], p["v_b"])
    attn = mha(q, k, v, n_head, False)
    x = (x + linear(attn, p["out"], p["out_b"])).astype(np.float32)
    cur = layernorm(x, p["mlp_ln_w"], p["mlp_ln_b"])
    h = gelu(linear(cur, p["fc1"], p["fc1_b"]))
    return (x + linear(h, p["fc2"], p["fc2_b"])).astype(np.float32)


def encoder_layer_f64(x: np.ndarray, p: dict, n_head: int) -> np.ndarray:
    """The same steps in float64 with the weights dequantized (no activation
    quantization): what the quantized layer approximates."""
    def dense(w):
        return O.dequant(w["dtype"], w["raw"], w["n"], w["raw"].size // O.BLOCK_BYTES[w["dtype"]] * 32 // w["n"])

    def ln(x, w, b):
        m = x.mean(axis=1, keepdims=True)
        v = ((x - m) ** 2).mean(axis=1, keepdims=True)
        return (x - m) / np.sqrt(v + 1e-5) * w + b

    def lin(a, w, b):
        y = a @ dense(w).astype(np.float64).T
        return y if b is None else y + b

    x = np.asarray(x, np.float64)
    cur = ln(x, p["attn_ln_w"], p["attn_ln_b"])
    q, k, v = lin(cur, p["q"], p["q_b"]), lin(cur, p["k"], None), lin(cur, p["v"], p["v_b"])
    x = x + lin(mha(q, k, v, n_head, False, dtype=np.float64), p["out"], p["out_b"])
    cur = ln(x, p["mlp_ln_w"], p["mlp_ln_b"])
    t = lin(cur, p["fc1"], p["fc1_b"])
    h = 0.5 * t * (1 + np.tanh(np.sqrt(2 / np.pi) * (t + 0.044715 * t ** 3)))
    return x + lin(h, p["fc2"], p["fc2_b"])
