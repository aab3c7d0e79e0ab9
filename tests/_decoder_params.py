"""Random decoder parameters (quantized weights + vectors) shared by the
decoder tests."""
import numpy as np

import oracle as O


def decoder_params(n, f, n_layer, n_vocab, n_ctx, dtype, seed, wscale=0.05, dtypes=None):
    """`dtypes` maps a layer weight's name ("q", "k", ..., "fc2") to a dtype
    other than `dtype`."""
    rng = np.random.default_rng(seed)
    dtypes = dtypes or {}

    def w(rows, cols, name=""):
        dt = dtypes.get(name, dtype)
        raw = O.quantize(dt, (rng.standard_normal((rows, cols)) * wscale).astype(np.float32))
        return {"dtype": dt, "raw": raw, "n": rows, "k": cols}

    def vec(k, s=0.1, c=0.0):
        return (rng.standard_normal(k) * s + c).astype(np.float32)

    layers = []
    for _ in range(n_layer):
        L = {}
        for name in ("q", "k", "v", "out", "cq", "ck", "cv", "cout"):
            L[name] = w(n, n, name)
        L["fc1"], L["fc2"] = w(f, n, "fc1"), w(n, f, "fc2")
        for name in ("attn_ln", "cross_ln", "mlp_ln"):
            L[name + "_w"], L[name + "_b"] = vec(n, 0.1, 1.0), vec(n)
        for name in ("q_b", "v_b", "out_b", "cq_b", "cv_b", "cout_b", "fc2_b"):
            L[name] = vec(n)
        L["fc1_b"] = vec(f)
        layers.append(L)
    tok = O.quantize(dtype, (rng.standard_normal((n_vocab, n)) * 0.5).astype(np.float32))
    return {"layers": layers, "tok": {"dtype": dtype, "raw": tok, "n": n_vocab, "k": n},
            "pos": vec(n_ctx * n, 0.3).reshape(n_ctx, n), "ln_w": vec(n, 0.1, 1.0), "ln_b": vec(n)}
