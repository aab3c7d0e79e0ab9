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


def _top_k_by_rank(lps, k):
    """The kept list described by ranks instead of the scan: v* is the k-th
    largest log-prob and g the count above it; every entry above v* stays,
    and of the entries equal to v* those with fewer than k entries >= v*
    before them in id order are admitted, the last k - g of them kept.
    Listed by log-prob, equal ones later id first."""
    fin = [(v, i) for i, v in enumerate(lps.tolist()) if v != -np.inf]
    if len(fin) <= k:
        kept = fin
    else:
        vs = sorted((v for v, _ in fin), reverse=True)[k - 1]
        above = [(v, i) for v, i in fin if v > vs]
        adm, seen = [], 0
        for v, i in fin:
            if v == vs and seen < k:
                adm.append((v, i))
            seen += v >= vs
        kept = above + adm[len(adm) - (k - len(above)):]
    return sorted(kept, key=lambda e: (-e[0], -e[1]))


def test_top_k_tied_entries_pushed_out_by_larger_ones():
    assert top_k(np.array([-1.0, -1.0, -0.5], np.float32), 2) == [(-0.5, 2), (-1.0, 1)]
    rng = np.random.default_rng(8)
    for _ in range(300):
        lps = rng.integers(-4, 1, 40).astype(np.float32)
        lps[rng.random(40) < 0.2] = -np.inf
        for k in (1, 2, 3, 5, 8):
            assert top_k(lps, k) == _top_k_by_rank(lps, k)


def test_top_k_of_nan_log_probs():
    # a NaN or +inf logit, or -inf only, gives NaN log-probs throughout
    for row in ([0.0, np.nan, 1.0, 2.0], [np.inf, 0.0, 1.0, 2.0], [-np.inf] * 4):
        lp = log_softmax(np.array(row, np.float32))
        assert np.all(np.isnan(lp))
        assert [i for _, i in top_k(lp, 3)] == [2, 1, 0]
