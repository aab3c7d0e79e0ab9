"""The oracle's log_softmax and top_k (oracle/decoder.py, restating
src/transcribe.rs:482-486 and 672-685), pinned by the reference's own top_k
test, a float64 log-sum-exp and a brute-force selection."""
import numpy as np
from scipy.special import logsumexp

from oracle.decoder import log_softmax, top_k


def test_top_k_reference_known_answer():
    # src/transcribe.rs:1895-1901
    lps = np.array([-5.0, -1.0, -np.inf, -0.5, -3.0], np.float32)
    assert top_k(lps, 3) == [(-0.5, 3), (-1.0, 1), (-3.0, 4)]
    assert len(top_k(lps, 10)) == 4  # masked entries never appear


def test_top_k_ties_keep_earlier_ids_listed_later_first():
    lps = np.array([1.0, 3.0, 3.0, 3.0, 2.0], np.float32)
    assert top_k(lps, 2) == [(3.0, 2), (3.0, 1)]
    assert top_k(lps, 4) == [(3.0, 3), (3.0, 2), (3.0, 1), (2.0, 4)]


def test_top_k_is_the_k_largest():
    rng = np.random.default_rng(3)
    for _ in range(20):
        lps = rng.standard_normal(300).astype(np.float32)
        lps[rng.choice(300, 30, replace=False)] = -np.inf
        got = top_k(lps, 7)
        order = sorted((v, i) for i, v in enumerate(lps.tolist()) if v != -np.inf)
        want = [(v, i) for v, i in reversed(order[-7:])]
        assert got == want


def test_log_softmax_against_float64():
    rng = np.random.default_rng(4)
    row = (rng.standard_normal(51866) * 4).astype(np.float32)
    row[::97] = -np.inf
    got = log_softmax(row)
    want = row.astype(np.float64) - logsumexp(row[np.isfinite(row)].astype(np.float64))
    fin = np.isfinite(row)
    diff = got[fin].astype(np.float64) - want[fin]
    # the reference sums 51866 positive f32 terms in index order: its lse
    # carries up to n 2^-24 relative error of the sum, the same shift for
    # every entry, and each lp one more rounding of its own
    assert np.max(np.abs(diff)) < fin.sum() * 2.0 ** -24
    assert np.max(diff) - np.min(diff) <= 2 * np.max(np.spacing(np.abs(got[fin])))
    assert np.all(got[~fin] == -np.inf)
    assert abs(np.exp(got[fin].astype(np.float64)).sum() - 1.0) < fin.sum() * 2.0 ** -24
