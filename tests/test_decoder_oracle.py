"""The decoder oracle (oracle/decoder.py) pinned without a GPU: the
kv-cache invariant the reference's decoding relies on (a prompt in one pass
equals the same tokens fed one at a time, up to int8 activation-quantization
noise), fork independence, and the
first step against a float64 composition on dequantized weights."""
import numpy as np

import oracle as O
from oracle.attention import mha
from oracle.decoder import Decoder
from _decoder_params import decoder_params


def _setup(seed=1):
    p = decoder_params(n=128, f=512, n_layer=2, n_vocab=300, n_ctx=32, dtype=8, seed=seed)
    enc = np.random.default_rng(seed + 1).standard_normal((50, 128)).astype(np.float32)
    return p, enc


def test_prompt_at_once_equals_token_by_token():
    p, enc = _setup()
    toks = [5, 17, 250, 3, 99]
    a = Decoder(p, 2, enc).forward_hidden(toks)
    d = Decoder(p, 2, enc)
    b = np.concatenate([d.forward_hidden([t]) for t in toks])
    # the same products row by row; float32 sums of differently shaped
    # products may flip an int8 activation rounding downstream, so the rows
    # agree to the quantization noise (the max error over the row's L2 norm)
    err = np.max(np.abs(a - b), axis=1) / np.linalg.norm(a, axis=1)
    assert err.max() < 5e-3, err
    assert d.n_past == 5


def test_fork_is_independent():
    p, enc = _setup(2)
    d = Decoder(p, 2, enc)
    d.forward_hidden([1, 2, 3])
    f = d.fork()
    x1 = d.forward_hidden([7])
    f.forward_hidden([8])
    x2 = f.fork().forward_hidden([7])  # f's history differs (8), so its next step differs
    d2 = Decoder(p, 2, enc)
    d2.forward_hidden([1, 2, 3])
    np.testing.assert_array_equal(d2.forward_hidden([7]), x1)
    assert np.abs(x2 - x1).max() > 1e-3


def test_first_step_close_to_float64():
    p, enc = _setup(3)
    got = Decoder(p, 2, enc).forward_hidden([11, 12])

    def dense(w):
        return O.dequant(w["dtype"], w["raw"], w["n"], w["k"]).astype(np.float64)

    def ln(x, w, b):
        m = x.mean(1, keepdims=True)
        return (x - m) / np.sqrt(((x - m) ** 2).mean(1, keepdims=True) + 1e-5) * w + b

    def lin(a, w, b):
        y = a @ dense(w).T
        return y if b is None else y + b

    e64 = enc.astype(np.float64)
    x = dense(p["tok"])[[11, 12]] + p["pos"][:2]
    for L in p["layers"]:
        cur = ln(x, L["attn_ln_w"], L["attn_ln_b"])
        q, k, v = lin(cur, L["q"], L["q_b"]), lin(cur, L["k"], None), lin(cur, L["v"], L["v_b"])
        x = x + lin(mha(q, k, v, 2, True, dtype=np.float64), L["out"], L["out_b"])
        cur = ln(x, L["cross_ln_w"], L["cross_ln_b"])
        q = lin(cur, L["cq"], L["cq_b"])
        ck, cv = lin(e64, L["ck"], None), lin(e64, L["cv"], L["cv_b"])
        x = x + lin(mha(q, ck, cv, 2, False, dtype=np.float64), L["cout"], L["cout_b"])
        cur = ln(x, L["mlp_ln_w"], L["mlp_ln_b"])
        t = lin(cur, L["fc1"], L["fc1_b"])
        x = x + lin(0.5 * t * (1 + np.tanh(np.sqrt(2 / np.pi) * (t + 0.044715 * t ** 3))), L["fc2"], L["fc2_b"])
    ref = ln(x, p["ln_w"], p["ln_b"])
    err = np.max(np.abs(got - ref), axis=1) / np.linalg.norm(ref, axis=1)
    assert err.max() < 1e-2
