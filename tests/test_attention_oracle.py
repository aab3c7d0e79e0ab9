"""The attention oracle (oracle/attention.py) pinned without a GPU.

* The reference's own attention tests, restated (src/encoder.rs:328-375).
* Brute force: a plain triple loop over tiny inputs in float64.
* SciPy's softmax in float64 on the same scores.
* Invariants a wrong index or a dropped term breaks: permuting kv rows
  (with k and v together) leaves a non-causal output unchanged; each head's
  output columns depend on that head's columns only; adding a constant to
  every score of a row changes nothing; causal row i ignores kv rows past
  t_kv - t_q + i.
"""
import math

import numpy as np
import pytest
from scipy.special import softmax as sp_softmax

from oracle.attention import mha, softmax_rows, split_heads


def fill(shape, seed):
    """A deterministic fill like the reference tests' helper (values in [-1, 1))."""
    rng = np.random.default_rng(seed)
    return rng.uniform(-1, 1, size=shape).astype(np.float32)


def test_mha_single_head_hand_computed():
    """src/encoder.rs:328-345"""
    k = np.array([[1.0], [-1.0]], np.float32)
    v = np.array([[10.0], [20.0]], np.float32)
    assert abs(mha(np.zeros((1, 1), np.float32), k, v, 1, False)[0, 0] - 15.0) < 1e-4
    assert abs(mha(np.array([[50.0]], np.float32), k, v, 1, False)[0, 0] - 10.0) < 1e-3


def test_mha_causal_mask_blocks_future():
    """src/encoder.rs:347-358"""
    k = np.array([[0.0], [100.0], [100.0]], np.float32)
    v = np.array([[7.0], [8.0], [9.0]], np.float32)
    q = np.ones((3, 1), np.float32)
    out = mha(q, k, v, 1, True)
    assert abs(out[0, 0] - 7.0) < 1e-5
    assert out[2, 0] > 7.5


def test_mha_incremental_query_aligns_to_end():
    """src/encoder.rs:360-374"""
    k, v, q_full = fill((3, 4), 31), fill((3, 4), 32), fill((3, 4), 33)
    full = mha(q_full, k, v, 2, True)
    inc = mha(q_full[2:3], k, v, 2, True)
    assert np.all(np.abs(inc[0] - full[2]) < 1e-5)


def brute(q, k, v, n_head, causal):
    t_q, n = q.shape
    t_kv = k.shape[0]
    dh = n // n_head
    out = np.zeros((t_q, n))
    for h in range(n_head):
        c = slice(h * dh, (h + 1) * dh)
        for i in range(t_q):
            lim = t_kv - t_q + i if causal else t_kv - 1
            s = [sum(float(q[i, c][d]) * float(k[j, c][d]) for d in range(dh)) / math.sqrt(dh)
                 for j in range(lim + 1)]
            mx = max(s)
            e = [math.exp(x - mx) for x in s]
            z = sum(e)
            for d in range(dh):
                out[i, h * dh + d] = sum(e[j] / z * float(v[j, c][d]) for j in range(lim + 1))
    return out


@pytest.mark.parametrize("t_q,t_kv,n,heads,causal", [(3, 3, 4, 2, False), (2, 5, 6, 3, True), (4, 4, 8, 1, True),
                                                     (1, 6, 6, 2, False), (5, 7, 4, 4, False)])
def test_brute_force_tiny(t_q, t_kv, n, heads, causal):
    q, k, v = fill((t_q, n), 1), fill((t_kv, n), 2) * 3, fill((t_kv, n), 3)
    want = brute(q, k, v, heads, causal)
    np.testing.assert_allclose(mha(q, k, v, heads, causal, dtype=np.float64), want, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(mha(q, k, v, heads, causal), want, rtol=2e-5, atol=2e-6)


def test_against_scipy_softmax_float64():
    q, k, v = fill((37, 64), 4) * 4, fill((50, 64), 5) * 4, fill((50, 64), 6)
    s = (q.astype(np.float64) @ k.astype(np.float64).T) / 8.0
    want = sp_softmax(s, axis=1) @ v.astype(np.float64)
    np.testing.assert_allclose(mha(q, k, v, 1, False, dtype=np.float64), want, rtol=1e-12, atol=1e-13)
    got32 = mha(q, k, v, 1, False)
    assert np.max(np.abs(got32 - want)) < 1e-5


def test_softmax_rows_shift_invariant_and_normalized():
    s = fill((6, 40), 7) * 30
    p = softmax_rows(s)
    np.testing.assert_allclose(p.sum(axis=1), 1.0, rtol=1e-6)
    np.testing.assert_allclose(softmax_rows(s + 17.0), p, rtol=2e-5, atol=1e-7)
    np.testing.assert_allclose(p, sp_softmax(s.astype(np.float64), axis=1), rtol=2e-5, atol=1e-8)


def test_kv_permutation_and_head_independence():
    q, k, v = fill((20, 24), 8), fill((30, 24), 9), fill((30, 24), 10)
    base = mha(q, k, v, 3, False)
    perm = np.random.default_rng(0).permutation(30)
    np.testing.assert_allclose(mha(q, k[perm], v[perm], 3, False), base, rtol=1e-5, atol=1e-6)
    # changing head 1's columns of k changes head 1's output only
    k2 = k.copy()
    k2[:, 8:16] *= -2
    out2 = mha(q, k2, v, 3, False)
    np.testing.assert_array_equal(out2[:, :8], base[:, :8])
    np.testing.assert_array_equal(out2[:, 16:], base[:, 16:])
    assert np.abs(out2[:, 8:16] - base[:, 8:16]).max() > 1e-3


def test_causal_rows_ignore_future_kv():
    q, k, v = fill((4, 8), 11), fill((9, 8), 12), fill((9, 8), 13)
    out = mha(q, k, v, 2, True)
    k2, v2 = k.copy(), v.copy()
    k2[6:] = 99.0  # rows past position 5 + 0 for query 0 (t_kv - t_q = 5)
    v2[6:] = -99.0
    out2 = mha(q, k2, v2, 2, True)
    np.testing.assert_array_equal(out2[0], out[0])
    assert np.abs(out2[3] - out[3]).max() > 1.0  # the last query sees them


def test_split_heads_layout():
    x = np.arange(12, dtype=np.float32).reshape(2, 6)
    h = split_heads(x, 3)
    assert h.shape == (3, 2, 2)
    np.testing.assert_array_equal(h[1], [[2, 3], [8, 9]])
