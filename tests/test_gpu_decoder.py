"""GPU parity of the device decoder (rw_decoder: create, set_audio,
forward_hidden, fork, reset) against the oracle's restatement of the
reference's Decoder (oracle/decoder.py, src/decoder.rs:36-213).

Bar: every step's hidden rows within 4e-3 of the oracle's, max error over
the oracle row's L2 norm -- a chain of per-product 1e-3 bars and
attention, through every layer -- over a prompt (GEMV regime at <= 8 rows,
GEMM regime above) and single-token steps (measured 0.8-2.6e-3); a layer
whose q, k and v differ in dtype within 5e-3 (measured 3.2e-3); forks
match independently decoded branches bit for bit.  Each test prints its
errors."""
import numpy as np
import pytest

from oracle.decoder import Decoder as OD
from rusty_whisper_amd import _abi as A
from _decoder_params import decoder_params

pytestmark = pytest.mark.gpu
TOL = 4e-3
TOL_MIXED = 5e-3


@pytest.fixture(scope="module")
def torch():
    import torch as T

    A.init(0)
    return T


def device_decoder(torch, p, n_head, n_audio):
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")  # noqa: E731
    layers = []
    for L in p["layers"]:
        d = {}
        for k, v in L.items():
            d[k] = A.DeviceWeight(v["dtype"], v["n"], v["k"], v["raw"]) if isinstance(v, dict) else dev(v)
        layers.append(d)
    tok = p["tok"]
    return A.Decoder(n_head, p["pos"].shape[0], n_audio, layers, A.DeviceWeight(tok["dtype"], tok["n"], tok["k"],
                                                                                 tok["raw"]),
                     dev(p["pos"]), dev(p["ln_w"]), dev(p["ln_b"]))


def rel(got, ref):
    return float(np.max(np.max(np.abs(got - ref), axis=1) / np.linalg.norm(ref, axis=1)))


def step(torch, d, toks, n):
    h = torch.empty(len(toks), n, device="cuda:0")
    d.forward_hidden(toks, h)
    torch.cuda.synchronize()
    return h.cpu().numpy()


@pytest.mark.parametrize("n,n_layer,dtype,prompt", [(128, 2, 8, [50257 % 300, 3, 7]), (256, 2, 7, list(range(12))),
                                                    (384, 1, 6, [1, 2, 3, 4, 5, 6, 7, 8, 9])],
                         ids=lambda x: str(x))
def test_decoder_parity(torch, n, n_layer, dtype, prompt):
    heads, n_audio = n // 64, 120
    p = decoder_params(n=n, f=4 * n, n_layer=n_layer, n_vocab=300, n_ctx=40, dtype=dtype, seed=n + n_layer)
    enc = np.random.default_rng(n).standard_normal((n_audio, n)).astype(np.float32)
    print(f"decoder n={n} layers={n_layer} dtype={dtype} prompt={len(prompt)}", flush=True)
    d = device_decoder(torch, p, heads, n_audio)
    d.set_audio(torch.from_numpy(enc).to("cuda:0"))
    o = OD(p, heads, enc)
    errs = [rel(step(torch, d, prompt, n), o.forward_hidden(prompt))]
    for t in (17, 250, 4, 99):
        errs.append(rel(step(torch, d, [t], n), o.forward_hidden([t])))
    print("  errors", ["%.2g" % e for e in errs], flush=True)
    assert d.n_past == len(prompt) + 4
    assert max(errs) <= TOL, errs


def test_decoder_wide_rows(torch):
    """n = 2560 (40 heads), fc 10240: rows of 80 blocks (layernorm statistics
    over more than 64 blocks, the one-row form's records from its
    registers after them) and fc2 over 320 blocks (longer than the one-row
    form's registers hold: its fill), in a 3-row prompt and single-token
    steps, against the oracle."""
    n, heads, n_audio = 2560, 40, 64
    p = decoder_params(n=n, f=4 * n, n_layer=1, n_vocab=300, n_ctx=16, dtype=6, seed=2560)
    enc = np.random.default_rng(2560).standard_normal((n_audio, n)).astype(np.float32)
    print("decoder n=2560 fc=10240: 1 layer, Q5_0", flush=True)
    d = device_decoder(torch, p, heads, n_audio)
    d.set_audio(torch.from_numpy(enc).to("cuda:0"))
    o = OD(p, heads, enc)
    errs = [rel(step(torch, d, [5, 6, 7], n), o.forward_hidden([5, 6, 7]))]
    for t in (17, 250, 4):
        errs.append(rel(step(torch, d, [t], n), o.forward_hidden([t])))
    print("  errors", ["%.2g" % e for e in errs], flush=True)
    assert max(errs) <= TOL, errs


def test_fork_and_reset(torch):
    n, heads = 128, 2
    p = decoder_params(n=n, f=512, n_layer=2, n_vocab=300, n_ctx=16, dtype=8, seed=4)
    enc = np.random.default_rng(4).standard_normal((64, n)).astype(np.float32)
    d = device_decoder(torch, p, heads, 64)
    d.set_audio(torch.from_numpy(enc).to("cuda:0"))
    step(torch, d, [1, 2, 3], n)
    f = d.fork()
    a = step(torch, d, [7], n)
    b = step(torch, f, [7], n)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))  # same history, same step
    step(torch, f, [9], n)
    assert f.n_past == 5 and d.n_past == 4
    d.reset()
    again = step(torch, d, [1, 2, 3], n)
    d2 = device_decoder(torch, p, heads, 64)
    d2.set_audio(torch.from_numpy(enc).to("cuda:0"))
    assert np.array_equal(again.view(np.uint32), step(torch, d2, [1, 2, 3], n).view(np.uint32))
    with pytest.raises(A.RwError, match="context overflow"):
        step(torch, d, list(range(14)), n)
    with pytest.raises(A.RwError, match="out of range"):
        step(torch, d, [300], n)


def test_decoder_long_cache(torch):
    """A 300-token prompt and steps past it: causal self-attention over the
    prompt and over a 301-303 row cache both split their kv blocks over two
    workgroups (some prompt query blocks' runs see no key) and merge them."""
    n, heads, n_audio = 128, 2, 120
    p = decoder_params(n=n, f=4 * n, n_layer=1, n_vocab=300, n_ctx=448, dtype=6, seed=7)
    enc = np.random.default_rng(3).standard_normal((n_audio, n)).astype(np.float32)
    prompt = [int(t) for t in np.random.default_rng(5).integers(0, 300, 300)]
    print("decoder long cache: prompt 300, n_ctx 448", flush=True)
    d = device_decoder(torch, p, heads, n_audio)
    d.set_audio(torch.from_numpy(enc).to("cuda:0"))
    o = OD(p, heads, enc)
    errs = [rel(step(torch, d, prompt, n), o.forward_hidden(prompt))]
    for t in (17, 250, 4):
        errs.append(rel(step(torch, d, [t], n), o.forward_hidden([t])))
    print("  errors", ["%.2g" % e for e in errs], flush=True)
    assert d.n_past == 303
    assert max(errs) <= TOL, errs


def test_decoder_mixed_qkv_dtypes(torch):
    """q, k and v of different dtypes (Q5_0 / Q8_0 / Q5_0): the step's
    layernorm runs alone and the three products go one by one, in both
    product regimes (a 12-token prompt, then single tokens)."""
    n, heads, n_audio = 256, 4, 120
    p = decoder_params(n=n, f=4 * n, n_layer=2, n_vocab=300, n_ctx=40, dtype=6, seed=17, dtypes={"k": 8})
    enc = np.random.default_rng(17).standard_normal((n_audio, n)).astype(np.float32)
    d = device_decoder(torch, p, heads, n_audio)
    d.set_audio(torch.from_numpy(enc).to("cuda:0"))
    o = OD(p, heads, enc)
    prompt = list(range(3, 15))
    errs = [rel(step(torch, d, prompt, n), o.forward_hidden(prompt))]
    for t in (17, 250, 4):
        errs.append(rel(step(torch, d, [t], n), o.forward_hidden([t])))
    print("  errors", ["%.2g" % e for e in errs], flush=True)
    assert max(errs) <= TOL_MIXED, errs


def test_large_v3_decoder_slice_with_logits(torch):
    """The large-v3 decoder's shapes (n = 1280, 20 heads, fc 5120, vocabulary
    51866, 1500 audio rows, 448 context rows) on two of its 32 layers, Q5_0:
    a 3-token prompt and three single-token steps against the oracle, and the
    tied-embedding logits [51866 x 1280] (src/decoder.rs:315-321) of every
    step against the oracle's product of the same hidden rows."""
    import oracle as O
    from _data import rel_row_l2

    n, heads, n_audio, n_vocab = 1280, 20, 1500, 51866
    p = decoder_params(n=n, f=4 * n, n_layer=2, n_vocab=n_vocab, n_ctx=448, dtype=6, seed=1280)
    enc = np.random.default_rng(1280).standard_normal((n_audio, n)).astype(np.float32)
    print("large-v3 decoder slice: 2 layers, vocab 51866, 1500 audio rows", flush=True)
    d = device_decoder(torch, p, heads, n_audio)
    d.set_audio(torch.from_numpy(enc).to("cuda:0"))
    o = OD(p, heads, enc)
    tok = d.token_embedding
    errs, lerrs = [], []
    for toks in ([50258, 50259, 50359], [440], [3111], [50257]):
        h = step(torch, d, toks, n)
        errs.append(rel(h, o.forward_hidden(toks)))
        hd = torch.from_numpy(h).to("cuda:0")
        logits = torch.empty(len(toks), n_vocab, device="cuda:0")
        tok.matmul_dev(hd, len(toks), logits)
        torch.cuda.synchronize()
        ref = O.matmul_emul(h, 6, p["tok"]["raw"], n_vocab)
        lerrs.append(rel_row_l2(logits.cpu().numpy(), ref))
    print("  hidden errors", ["%.2g" % e for e in errs], "logits errors", ["%.2g" % e for e in lerrs], flush=True)
    assert max(errs) <= TOL, errs
    assert max(lerrs) <= 1e-3, lerrs
