"""GPU parity of the beam-search pieces against the oracle:

* rw_rocm_logits_topk_dev: log_softmax + top_k of each logits row
  (src/transcribe.rs:482-486, 672-685) against oracle/decoder.py's
  restatement.  Bars: the ids equal (random logits have no ties; rows built
  from repeated values test the tie rules exactly, since equal logits give
  equal log-probs whatever the log-sum-exp), log-probs within the reference's
  own log-sum-exp error (its sequential f32 sum: n 2^-24 of the sum) plus one
  rounding; rows whose log-sum-exp is NaN give NaN log-probs.
* rw_rocm_decoder_forward_beams_dev: one step of several forked beams at once
  against each beam stepped alone through rw_rocm_decoder_forward_hidden_dev
  (within 1e-5 of the row's norm: the products see more rows and the
  attention's kv split is chosen for all beams together) and against the
  oracle decoder (the decoder tests' 4e-3 bar); the beams' caches then hold
  the same rows (a second step agrees too).
"""
import numpy as np
import pytest

from oracle.decoder import Decoder as OD
from oracle.decoder import log_softmax, top_k
from rusty_whisper_amd import _abi as A
from _decoder_params import decoder_params

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch as T

    A.init(0)
    return T


def device_topk(torch, logits: np.ndarray, k: int):
    rows, n = logits.shape
    ld = torch.from_numpy(np.ascontiguousarray(logits)).to("cuda:0")
    ids = torch.empty(rows, k, dtype=torch.int32, device="cuda:0")
    lps = torch.empty(rows, k, device="cuda:0")
    A.logits_topk_dev(ld, rows, n, k, ids, lps)
    torch.cuda.synchronize()
    return ids.cpu().numpy().view(np.uint32), lps.cpu().numpy()


def check_rows(logits, k, ids, lps, exact_lp=False):
    for r in range(logits.shape[0]):
        ref_lp = log_softmax(logits[r])
        want = top_k(ref_lp, k)
        got_ids = [int(i) for i in ids[r] if i != 0xFFFFFFFF]
        assert got_ids == [i for _, i in want], (r, got_ids[:8], want[:8])
        assert np.all(ids[r][len(want):] == 0xFFFFFFFF) and np.all(lps[r][len(want):] == -np.inf)
        if want and np.isnan(want[0][0]):  # a NaN log-sum-exp: every log-prob NaN
            assert np.all(np.isnan(lps[r][:len(want)]))
        elif want:
            wl = np.array([v for v, _ in want], np.float64)
            n = np.isfinite(logits[r]).sum()
            tol = n * 2.0 ** -24 * 1.0 + 2 * np.spacing(np.abs(wl).max())
            assert np.max(np.abs(lps[r][:len(want)] - wl)) <= tol


@pytest.mark.parametrize("k", [1, 5, 16])
def test_topk_random_vocab_rows(torch, k):
    rng = np.random.default_rng(k)
    logits = (rng.standard_normal((5, 51866)) * 3).astype(np.float32)
    logits[:, rng.choice(51866, 3000, replace=False)] = -np.inf  # suppressed tokens
    ids, lps = device_topk(torch, logits, k)
    check_rows(logits, k, ids, lps)


def test_topk_reference_known_answer(torch):
    # src/transcribe.rs:1895-1901, as logits (log_softmax keeps the order)
    logits = np.array([[-5.0, -1.0, -np.inf, -0.5, -3.0]], np.float32)
    ids, lps = device_topk(torch, logits, 3)
    assert ids[0].tolist() == [3, 1, 4]
    ids, lps = device_topk(torch, logits, 10)
    assert ids[0][:4].tolist() == [3, 1, 4, 0] and np.all(ids[0][4:] == 0xFFFFFFFF)
    check_rows(logits, 10, ids, lps)


def test_topk_ties_and_short_rows(torch):
    rng = np.random.default_rng(7)
    logits = rng.integers(-4, 3, size=(4, 3000)).astype(np.float32)  # many exact ties
    logits[1, :] = -np.inf
    logits[1, [17, 2000]] = [1.0, 1.0]  # two candidates only
    logits[2, :] = 5.0  # all tied
    for k in (4, 16):
        ids, lps = device_topk(torch, logits, k)
        check_rows(logits, k, ids, lps)


def test_topk_tied_entries_pushed_out_by_larger_ones(torch):
    """The reference's scan inserts ahead of equal entries and cuts the list
    at k, so a later, larger log-prob pushes out the earliest id of a tied
    group at the cut-off (src/transcribe.rs:672-685)."""
    ids, lps = device_topk(torch, np.array([[0.0, 0.0, 0.5]], np.float32), 2)
    assert ids[0].tolist() == [2, 1]
    # across chunks: five entries tied at the cut-off, three larger ones
    # arriving between them; the scan admits ids 5, 100, 3000 and 9000 and
    # keeps the last two of them
    row = np.full((1, 51866), -20.0, np.float32)
    row[0, [5, 100, 3000, 9000, 20000]] = 1.0
    row[0, [2100, 40000, 51000]] = 2.0
    ids, lps = device_topk(torch, row, 5)
    assert ids[0].tolist() == [51000, 40000, 2100, 9000, 3000]
    check_rows(row, 5, ids, lps)
    # random sparse rows of a few tied values over many chunks
    rng = np.random.default_rng(13)
    for k in (2, 5, 16):
        rows = np.full((6, 51866), -np.inf, np.float32)
        rows[:3] = -30.0
        for r in range(6):
            at = rng.choice(51866, 60, replace=False)
            rows[r, at] = rng.integers(0, 6, 60).astype(np.float32)
        ids, lps = device_topk(torch, rows, k)
        check_rows(rows, k, ids, lps)


def test_topk_nan_log_sum_exp_rows(torch):
    """A NaN or +inf logit, or a row of -inf only, makes the reference's
    log-sum-exp NaN and so every log-prob; its scan then keeps ids
    min(k, n) - 1 .. 0."""
    rows = np.random.default_rng(17).standard_normal((4, 5000)).astype(np.float32)
    rows[0, 4321] = np.nan
    rows[1, 77] = np.inf
    rows[2, :] = -np.inf
    rows[3, 2049] = np.nan  # in the second chunk only
    for k in (1, 5):
        ids, lps = device_topk(torch, rows, k)
        assert all(ids[r].tolist() == list(range(k - 1, -1, -1)) for r in range(4))
        check_rows(rows, k, ids, lps)
    ids, lps = device_topk(torch, np.array([[0.0, np.nan, 1.0]], np.float32), 5)
    assert ids[0].tolist() == [2, 1, 0, 0xFFFFFFFF, 0xFFFFFFFF]
    assert np.all(np.isnan(lps[0][:3])) and np.all(lps[0][3:] == -np.inf)


def test_topk_masked_chunks_and_caller_workspace(torch):
    """Whole 2048-logit chunks suppressed (their partial sums are empty), the
    answer in the last, partial chunk, and a caller workspace."""
    rng = np.random.default_rng(11)
    logits = (rng.standard_normal((3, 51866)) * 2).astype(np.float32)
    logits[0, :49000] = -np.inf
    logits[1, 2048:8192] = -np.inf
    logits[2, 51860:] = 40.0
    k = 8
    wsz = A.logits_topk_workspace_size(3, 51866, k)
    ws = torch.empty(wsz, dtype=torch.uint8, device="cuda:0")
    ld = torch.from_numpy(logits).to("cuda:0")
    ids = torch.empty(3, k, dtype=torch.int32, device="cuda:0")
    lps = torch.empty(3, k, device="cuda:0")
    A.logits_topk_dev(ld, 3, 51866, k, ids, lps, workspace=ws, workspace_len=wsz)
    torch.cuda.synchronize()
    check_rows(logits, k, ids.cpu().numpy().view(np.uint32), lps.cpu().numpy())


def test_topk_rejects_bad_arguments(torch):
    x = torch.zeros(1, 10, device="cuda:0")
    ids = torch.empty(1, 17, dtype=torch.int32, device="cuda:0")
    lps = torch.empty(1, 17, device="cuda:0")
    with pytest.raises(A.RwError, match="between 1 and 16"):
        A.logits_topk_dev(x, 1, 10, 17, ids, lps)
    with pytest.raises(A.RwError, match="n_vocab"):
        A.logits_topk_dev(x, 1, 131073, 5, ids, lps)


def _device_decoder(torch, p, n_head, n_audio):
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")  # noqa: E731
    layers = []
    for L in p["layers"]:
        layers.append({k: A.DeviceWeight(v["dtype"], v["n"], v["k"], v["raw"]) if isinstance(v, dict) else dev(v)
                       for k, v in L.items()})
    tok = p["tok"]
    return A.Decoder(n_head, p["pos"].shape[0], n_audio, layers,
                     A.DeviceWeight(tok["dtype"], tok["n"], tok["k"], tok["raw"]), dev(p["pos"]), dev(p["ln_w"]),
                     dev(p["ln_b"]))


def _rel(got, ref):
    return float(np.max(np.max(np.abs(got - ref), axis=1) / np.linalg.norm(ref, axis=1)))


@pytest.mark.parametrize("n,n_layer,dtype,nb", [(256, 2, 6, 5), (128, 1, 8, 8), (1280, 2, 6, 5)],
                         ids=lambda x: str(x))
def test_beams_match_separate_steps(torch, n, n_layer, dtype, nb):
    heads, n_audio = n // 64, 120 if n < 1280 else 1500
    p = decoder_params(n=n, f=4 * n, n_layer=n_layer, n_vocab=300, n_ctx=40, dtype=dtype, seed=n + nb)
    enc = np.random.default_rng(n).standard_normal((n_audio, n)).astype(np.float32)
    print(f"beams n={n} layers={n_layer} dtype={dtype} beams={nb}", flush=True)
    d = _device_decoder(torch, p, heads, n_audio)
    d.set_audio(torch.from_numpy(enc).to("cuda:0"))
    hid = torch.empty(8, n, device="cuda:0")
    d.forward_hidden([1, 2, 3], hid[:3])
    beams = [d] + [d.fork() for _ in range(nb - 1)]
    alone = [d.fork() for _ in range(nb)]  # the same history, stepped one by one
    for step, toks in enumerate(([7, 11, 250, 4, 99, 5, 6, 42][:nb], [3, 3, 17, 299, 0, 8, 9, 10][:nb])):
        hb = torch.empty(nb, n, device="cuda:0")
        A.decoder_forward_beams(beams, toks, hb)
        torch.cuda.synchronize()
        got = hb.cpu().numpy()
        ref = np.concatenate([_step(torch, alone[i], [t], n) for i, t in enumerate(toks)])
        err = _rel(got, ref)
        print(f"  step {step}: vs separate steps {err:.3g}", flush=True)
        assert err <= 1e-5, err
        assert all(b.n_past == 4 + step for b in beams)
    # the oracle for beam 0's history (tokens 7 then 3)
    ob = OD(p, heads, enc)
    ob.forward_hidden([1, 2, 3])
    ob.forward_hidden([7])
    want = ob.forward_hidden([3])
    err = _rel(got[0:1], want)
    print(f"  beam 0 vs the oracle decoder {err:.3g}", flush=True)
    assert err <= 4e-3, err


def _step(torch, dec, toks, n):
    h = torch.empty(len(toks), n, device="cuda:0")
    dec.forward_hidden(toks, h)
    torch.cuda.synchronize()
    return h.cpu().numpy()


def test_beams_reject_bad_sets(torch):
    n, heads = 128, 2
    p = decoder_params(n=n, f=512, n_layer=1, n_vocab=300, n_ctx=16, dtype=8, seed=3)
    enc = np.random.default_rng(3).standard_normal((64, n)).astype(np.float32)
    d = _device_decoder(torch, p, heads, 64)
    d.set_audio(torch.from_numpy(enc).to("cuda:0"))
    hb = torch.empty(4, n, device="cuda:0")
    f = d.fork()
    with pytest.raises(A.RwError, match="listed twice"):
        A.decoder_forward_beams([d, d], [1, 2], hb)
    _step(torch, f, [5], n)
    with pytest.raises(A.RwError, match="cached tokens"):
        A.decoder_forward_beams([d, f], [1, 2], hb)
    other = _device_decoder(torch, p, heads, 64)
    other.set_audio(torch.from_numpy(enc).to("cuda:0"))
    with pytest.raises(A.RwError, match="not a fork"):
        A.decoder_forward_beams([d, other], [1, 2], hb)
    with pytest.raises(A.RwError, match="out of range"):
        A.decoder_forward_beams([d, d.fork()], [1, 300], hb)
    with pytest.raises(A.RwError, match="between 1 and 8"):
        A.decoder_forward_beams([], [], hb)
