"""GPU parity of rw_rocm_attention against the oracle (oracle/attention.py,
the reference's mha_split_kv, src/encoder.rs:48-80).

Bar (written in each test): outputs within 1e-3 of the float32 oracle,
max error scaled by the oracle row's L2 norm (the matmul path's tolerance),
and within 1e-5 of the float64 oracle on the same scale (measured: at most
9e-7 for unit-scale inputs, 4e-6 for inputs of magnitude 1e-3 whose f16
residuals are subnormal; the float32 oracle itself is at 3e-7)."""
import numpy as np
import pytest

from oracle.attention import mha
from rusty_whisper_amd import _abi as A

pytestmark = pytest.mark.gpu

TOL = 1e-3
TIGHT = 1e-5


@pytest.fixture(scope="module", autouse=True)
def _device():
    A.init(0)


@pytest.fixture(scope="module")
def torch():
    import torch as T

    T.cuda.init()
    return T


def rel_row_l2(got, ref):
    den = np.maximum(np.linalg.norm(ref.astype(np.float64), axis=1), 1e-30)
    return float(np.max(np.max(np.abs(got.astype(np.float64) - ref), axis=1) / den))


def inputs(t_q, t_kv, n, seed, scale=1.0):
    """N(0, scale) queries and keys (scale 3 peaks the softmax); values N(0,
    1), or N(0, scale) when scale < 1."""
    rng = np.random.default_rng(seed)
    q = (rng.standard_normal((t_q, n)) * scale).astype(np.float32)
    k = (rng.standard_normal((t_kv, n)) * scale).astype(np.float32)
    v = (rng.standard_normal((t_kv, n)) * min(scale, 1.0)).astype(np.float32)
    return q, k, v


def check(got, q, k, v, heads, causal):
    ref32 = mha(q, k, v, heads, causal)
    ref64 = mha(q, k, v, heads, causal, dtype=np.float64)
    assert np.all(np.isfinite(got))
    e32, e64 = rel_row_l2(got, ref32), rel_row_l2(got, ref64)
    print(f"  error vs float32 oracle {e32:.3g}, vs float64 {e64:.3g}", flush=True)
    assert e32 <= TOL, e32
    assert e64 <= TIGHT, e64
    return e64


SHAPES = [
    (1500, 1500, 1280, 20, False, 1.0),  # large-v3 encoder self-attention
    (1500, 1500, 384, 6, False, 1.0),    # tiny encoder
    (1500, 1500, 384, 6, False, 3.0),    # peaked scores
    (37, 37, 128, 2, False, 1.0),
    (64, 200, 256, 4, False, 1.0),
    (33, 1, 64, 1, False, 1.0),
    (100, 100, 64, 1, True, 1.0),
    (5, 40, 128, 2, True, 1.0),          # decoder prompt against a cache
    (1, 77, 384, 6, True, 1.0),          # one decode step
    (1, 1500, 1280, 20, False, 1.0),     # cross-attention, one token
    (130, 130, 192, 3, True, 2.0),
    (200, 300, 128, 2, False, 1e-3),     # small values: f16 residuals would be subnormal
    (5, 448, 384, 6, True, 1.0),         # split kv (few query blocks), causal
    (2, 1500, 384, 6, False, 2.0),       # split kv over 11 runs
]


@pytest.mark.parametrize("t_q,t_kv,n,heads,causal,scale", SHAPES, ids=lambda x: str(x))
def test_attention_parity(t_q, t_kv, n, heads, causal, scale):
    q, k, v = inputs(t_q, t_kv, n, seed=t_q * 7 + t_kv + n, scale=scale)
    print(f"attention t_q={t_q} t_kv={t_kv} n={n} heads={heads} causal={causal}", flush=True)
    check(A.attention(q, k, v, heads, causal), q, k, v, heads, causal)


def test_reference_hand_computed_at_head_size_64():
    """src/encoder.rs:328-345 lifted to 64-value heads: a zero query attends
    uniformly; a huge one picks the best-matching key."""
    k = np.zeros((2, 64), np.float32)
    k[0, 0], k[1, 0] = 1.0, -1.0
    v = np.zeros((2, 64), np.float32)
    v[0, :], v[1, :] = 10.0, 20.0
    out = A.attention(np.zeros((1, 64), np.float32), k, v, 1, False)
    assert np.all(np.abs(out - 15.0) < 1e-4)
    qb = np.zeros((1, 64), np.float32)
    qb[0, 0] = 400.0  # score 50 after the 1/8 scale, as the reference's q=50 with d=1
    out = A.attention(qb, k, v, 1, False)
    assert np.all(np.abs(out - 10.0) < 1e-3)


def test_reference_causal_mask_blocks_future():
    """src/encoder.rs:347-358 at 64-value heads."""
    k = np.zeros((3, 64), np.float32)
    k[1:, 0] = 100.0
    v = np.stack([np.full(64, 7.0), np.full(64, 8.0), np.full(64, 9.0)]).astype(np.float32)
    q = np.zeros((3, 64), np.float32)
    q[:, 0] = 8.0
    out = A.attention(q, k, v, 1, True)
    assert np.all(np.abs(out[0] - 7.0) < 1e-5)
    assert np.all(out[2] > 7.5)


@pytest.mark.parametrize("t_kv", [3, 40, 448])
def test_incremental_query_aligns_to_end(t_kv):
    """src/encoder.rs:360-374: one query row against t_kv keys equals the
    last row of the full causal pass (the kv-cache invariant)."""
    q, k, v = inputs(t_kv, t_kv, 128, seed=t_kv)
    full = A.attention(q, k, v, 2, True)
    inc = A.attention(q[-1:], k, v, 2, True)
    assert np.max(np.abs(inc[0] - full[-1])) <= 1e-5 * max(1.0, np.abs(full[-1]).max())


def test_no_keys_gives_zeros():
    q = np.ones((3, 64), np.float32)
    e = np.zeros((0, 64), np.float32)
    assert not A.attention(q, e, e, 1, False).any()


def test_device_entry_with_strided_rows(torch):
    """q, k and v as column blocks of one fused [t, 3 n] projection, output
    into a wider buffer: the row strides are honoured."""
    t, n, heads = 300, 256, 4
    rng = np.random.default_rng(5)
    qkv = rng.standard_normal((t, 3 * n)).astype(np.float32)
    dev = torch.from_numpy(qkv).to("cuda:0")
    out = torch.full((t, n + 64), 7.0, device="cuda:0")
    A.attention_dev(dev[:, :n], dev[:, n:2 * n], dev[:, 2 * n:], t, t, n, heads, False, out,
                    ldq=3 * n, ldk=3 * n, ldv=3 * n, ldo=n + 64)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.all(got[:, n:] == 7.0)
    check(got[:, :n], qkv[:, :n], qkv[:, n:2 * n], qkv[:, 2 * n:], heads, False)


def test_repeated_calls_are_bitwise_stable():
    q, k, v = inputs(200, 200, 128, seed=9)
    a = A.attention(q, k, v, 2, False)
    b = A.attention(q, k, v, 2, False)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_query_rows_do_not_depend_on_the_call_shape():
    """The same query rows against the same keys, in three call shapes: 100
    query rows (K and V split into planes first, two 32-query tiles per
    workgroup), 40 rows (one query block: K and V read as f32 rows and split
    in the kernel, two tiles) and 20 rows (f32 rows, one tile).  A query
    row's result is the same bits in all three, and matches the oracle."""
    q, k, v = inputs(100, 300, 256, seed=21)
    full = A.attention(q, k, v, 4, False)
    for t in (40, 20):
        part = A.attention(q[:t], k, v, 4, False)
        assert np.array_equal(part.view(np.uint32), full[:t].view(np.uint32)), t
    check(full, q, k, v, 4, False)


@pytest.mark.parametrize("t_q", [1, 5, 33])
def test_decoding_shapes_with_strided_rows(torch, t_q):
    """Decoding-step shapes (a few query rows, causal, aligned to the end of
    the keys) read through row strides wider than n: K and V are loaded as
    f32 rows by the attention kernel itself."""
    t_kv, n, heads = 77, 256, 4
    rng = np.random.default_rng(t_q)
    kv = rng.standard_normal((t_kv, 3 * n)).astype(np.float32)
    qf = rng.standard_normal((t_q, 2 * n)).astype(np.float32)
    dk = torch.from_numpy(kv).to("cuda:0")
    dq = torch.from_numpy(qf).to("cuda:0")
    out = torch.full((t_q, n + 64), 7.0, device="cuda:0")
    A.attention_dev(dq[:, :n], dk[:, :n], dk[:, 2 * n:], t_q, t_kv, n, heads, True, out,
                    ldq=2 * n, ldk=3 * n, ldv=3 * n, ldo=n + 64)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.all(got[:, n:] == 7.0)
    check(got[:, :n], qf[:, :n], kv[:, :n], kv[:, 2 * n:], heads, True)
