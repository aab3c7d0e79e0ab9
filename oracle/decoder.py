"""The whisper text decoder's forward_hidden, restated on the CPU -- TEST
INFRASTRUCTURE ONLY.

Decoder::new / fork / reset / forward_hidden of src/decoder.rs:36-213: the
token embedding row (dequantized, src/quant.rs row_f32) plus the learned
position, then per layer causal self-attention over the cache and the new
rows, cross-attention to K/V projected once from the encoder output, and the
MLP; the final layernorm.  Built from the pinned pieces: oracle.matmul_emul
(the reference's int8 linears), oracle/attention.py, oracle/encoder.py's
layernorm and GELU.  The product package never imports it.

Pinned by tests/test_decoder_oracle.py: the reference's kv-cache invariant
(one prompt pass equals the same tokens fed one by one), fork independence,
and a float64 composition of the same steps on dequantized weights.
"""
from __future__ import annotations

import numpy as np

import oracle as O
from oracle.attention import mha
from oracle.encoder import gelu, layernorm, linear


class Decoder:
    def __init__(self, p: dict, n_head: int, enc_out: np.ndarray):
        """p: "layers" (list of dicts with attn_ln_w/b, q, k, v, out, q_b, v_b,
        out_b, cross_ln_w/b, cq, ck, cv, cout, cq_b, cv_b, cout_b, mlp_ln_w/b,
        fc1, fc1_b, fc2, fc2_b), "tok" (quantized [n_vocab, n]), "pos"
        ([n_ctx, n]), "ln_w", "ln_b"."""
        self.p, self.n_head = p, n_head
        self.cross = [(linear(enc_out, L["ck"], None), linear(enc_out, L["cv"], L["cv_b"])) for L in p["layers"]]
        self.k = [np.zeros((0, p["pos"].shape[1]), np.float32) for _ in p["layers"]]
        self.v = [np.zeros((0, p["pos"].shape[1]), np.float32) for _ in p["layers"]]
        self.n_past = 0

    def fork(self) -> "Decoder":
        c = Decoder.__new__(Decoder)
        c.p, c.n_head, c.cross, c.n_past = self.p, self.n_head, self.cross, self.n_past
        c.k, c.v = [k.copy() for k in self.k], [v.copy() for v in self.v]
        return c

    def embed(self, tokens) -> np.ndarray:
        tok = self.p["tok"]
        n = self.p["pos"].shape[1]
        bb = O.BLOCK_BYTES[tok["dtype"]] * (n // 32)
        rows = [O.dequant(tok["dtype"], tok["raw"][t * bb:(t + 1) * bb], 1, n)[0] for t in tokens]
        return (np.stack(rows) + self.p["pos"][self.n_past:self.n_past + len(tokens)]).astype(np.float32)

    def forward_hidden(self, tokens) -> np.ndarray:
        x = self.embed(tokens)
        h = self.n_head
        for l, L in enumerate(self.p["layers"]):
            cur = layernorm(x, L["attn_ln_w"], L["attn_ln_b"])
            q = linear(cur, L["q"], L["q_b"])
            self.k[l] = np.concatenate([self.k[l], linear(cur, L["k"], None)])
            self.v[l] = np.concatenate([self.v[l], linear(cur, L["v"], L["v_b"])])
            x = (x + linear(mha(q, self.k[l], self.v[l], h, True), L["out"], L["out_b"])).astype(np.float32)
            cur = layernorm(x, L["cross_ln_w"], L["cross_ln_b"])
            q = linear(cur, L["cq"], L["cq_b"])
            ck, cv = self.cross[l]
            x = (x + linear(mha(q, ck, cv, h, False), L["cout"], L["cout_b"])).astype(np.float32)
            cur = layernorm(x, L["mlp_ln_w"], L["mlp_ln_b"])
            x = (x + linear(gelu(linear(cur, L["fc1"], L["fc1_b"])), L["fc2"], L["fc2_b"])).astype(np.float32)
        self.n_past += len(tokens)
        return layernorm(x, self.p["ln_w"], self.p["ln_b"])


def log_softmax(row: np.ndarray) -> np.ndarray:
    """src/transcribe.rs:482-486 in float32: the maximum (a fold from -inf),
    lse = max + ln(sum of exp(v - max)) summed in index order, lp = v - lse."""
    row = np.asarray(row, dtype=np.float32)
    mx = np.float32(-np.inf)
    for v in row[~np.isnan(row)]:
        mx = max(mx, v)
    terms = np.exp((row - mx).astype(np.float32)).astype(np.float32)
    s = np.cumsum(terms, dtype=np.float32)[-1] if len(terms) else np.float32(0.0)
    lse = np.float32(mx + np.float32(np.log(s)))
    return (row - lse).astype(np.float32)


def top_k(lps: np.ndarray, k: int):
    """src/transcribe.rs:672-685: scan the log-probs in id order, skip
    exactly -inf, insert (lp, id) at partition_point(b > lp) of the list kept
    sorted by lp while it has fewer than k entries or lp beats its last."""
    best = []
    for i, lp in enumerate(np.asarray(lps, dtype=np.float32).tolist()):
        if lp == float("-inf"):
            continue
        if len(best) < k or lp > best[-1][0]:
            pos = 0
            while pos < len(best) and best[pos][0] > lp:
                pos += 1
            best.insert(pos, (lp, i))
            del best[k:]
    return best
