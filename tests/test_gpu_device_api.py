"""Device-pointer entry points on the GPU, through the C ABI.

Bars (written in each test):
  * the encoder GEMM's activation plane (m > 8) holds, bit for bit, the f16
    values f16(q_a * f32(d_a * 2^(15-e))) of quantize_acts_i8's q_a and d_a,
    with 2^(e-1) <= the row's largest |x| < 2^e (e >= -110; 15 for zero or
    non-finite rows), the row scales 2^(e-15), and the row sums
    ps = sum over blocks of d_a * sum(q_a) within nb * 2^-23 of their
    float64 value (relative to the sum of the terms' magnitudes);
  * one launch for several weights on one quantized input matches the
    oracle (1e-3 row-L2, and the regime's bound against the exact float64
    combination), its rows do not depend on m, and in the decode shape it
    is bitwise the single-weight call;
  * quantizing inside the decode launch and quantizing separately
    (rw_rocm_quantize_dev + rw_rocm_matmul_prequant_dev) give bitwise the
    same outputs, in both regimes;
  * a prepared group gives bitwise what a grouped launch gives; both give,
    per item, what the same linear gives alone up to the f32 reassociation
    of the k-split parts (a single linear splits k over more wavefronts):
    within 1e-6 of the row's L2 norm;
  * device and host entry points agree bitwise;
  * outputs stay within 1e-3 of the reference CPU path (max error over the
    reference row's L2 norm), also when the activations go through LDS in
    several chunks.
"""
import numpy as np
import pytest

import oracle as O
from rusty_whisper_amd import _abi as A

from _data import DTYPES, NAMES, activations, check_combine, edge_activation_rows, rel_row_l2, weights

pytestmark = pytest.mark.gpu

ROW_L2_TOL = 1e-3


@pytest.fixture(scope="module")
def torch():
    import torch as t
    A.init(0)
    return t


def _dev(torch, x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0")


def _bits(x):
    return np.ascontiguousarray(x).view(np.uint32)


def _single(torch, w, a, bias=None):
    m = a.shape[0]
    out = torch.empty(m, w.n, device="cuda:0")
    w.matmul_dev(_dev(torch, a), m, out, None if bias is None else _dev(torch, bias))
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: NAMES[d])
@pytest.mark.parametrize("m", [1, 5, 8, 9, 40])
def test_device_matches_host_bitwise(torch, dtype, m):
    k, n = 416, 75
    raw = weights(dtype, n, k, seed=5 + m)
    w = A.DeviceWeight(dtype, n, k, raw)
    a = activations(m, k, seed=7 * m + dtype)
    bias = np.random.default_rng(m).standard_normal(n).astype(np.float32)
    assert np.array_equal(_bits(_single(torch, w, a, bias)), _bits(w.matmul(a, bias)))


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: NAMES[d])
@pytest.mark.parametrize("m", [1, 3, 8, 9, 70])
def test_prequant_matches_fused_bitwise(torch, dtype, m):
    k, n = 1280, 96
    raw = weights(dtype, n, k, seed=31 + m)
    w = A.DeviceWeight(dtype, n, k, raw)
    a = activations(m, k, seed=m + 100 * dtype, outliers=0.01)
    fused = _single(torch, w, a)
    wsz = A.workspace_size(m, k)
    ws = torch.empty(wsz, dtype=torch.uint8, device="cuda:0")
    out = torch.empty(m, n, device="cuda:0")
    A.quantize_dev(_dev(torch, a), m, k, ws, wsz)
    w.matmul_prequant_dev(ws, m, out)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(out.cpu().numpy()), _bits(fused))
    assert rel_row_l2(fused, O.matmul_emul(a, dtype, raw, n)) <= ROW_L2_TOL


# (dtype, m, n, k, bias): every k split of a grouped launch (k up to 2816
# -> 1 wavefront set, 5120 -> 2, 16384 -> 4), ragged n, an m = 0 entry, two
# entries that share a launch, and one large enough in k (m = 8) that its
# activations pass through LDS in several chunks
GROUP = [
    (7, 5, 1280, 1280, True),
    (6, 5, 96, 5120, False),
    (2, 1, 41, 384, True),
    (3, 8, 70, 768, True),
    (8, 3, 33, 96, False),
    (7, 5, 200, 1280, False),
    (6, 0, 10, 64, False),
    (8, 8, 64, 16384, True),
    (3, 2, 1, 32, True),
]


def _group_items(torch, specs, seed):
    rng = np.random.default_rng(seed)
    items, host = [], []
    for j, (dt, m, n, k, has_b) in enumerate(specs):
        raw = weights(dt, n, k, seed=seed + 13 * j)
        w = A.DeviceWeight(dt, n, k, raw)
        a = activations(m, k, seed=seed + 7 * j) if m else np.zeros((0, k), np.float32)
        b = rng.standard_normal(n).astype(np.float32) if has_b else None
        da = _dev(torch, a) if m else torch.empty(1, device="cuda:0")
        db = None if b is None else _dev(torch, b)
        out = torch.full((max(m, 1), n), float("nan"), device="cuda:0")
        items.append((w, da, db, out, m))
        host.append((w, a, b, raw))
    return items, host


def test_grouped_matches_single(torch):
    items, host = _group_items(torch, GROUP, seed=900)
    arr = A.make_linears(items)
    wsz = A.grouped_workspace_size(arr)
    ws = torch.empty(wsz, dtype=torch.uint8, device="cuda:0")
    A.matmul_grouped_dev(arr, ws, wsz)
    torch.cuda.synchronize()
    for (w, _, _, out, m), (_, a, b, raw) in zip(items, host):
        if m == 0:
            assert torch.isnan(out).all(), "an m = 0 entry must write nothing"
            continue
        got = out.cpu().numpy()
        assert rel_row_l2(got, _single(torch, w, a, b)) <= 1e-6, (w.dtype, m, w.n, w.k)
        ref = O.matmul_emul(a, w.dtype, raw, w.n, bias=b)
        assert rel_row_l2(got, ref) <= ROW_L2_TOL, (w.dtype, m, w.n, w.k)


def test_prepared_group_matches_grouped_bitwise(torch):
    items, _ = _group_items(torch, GROUP, seed=901)
    arr = A.make_linears(items)
    A.matmul_grouped_dev(arr)  # the library's own workspace for this stream
    torch.cuda.synchronize()
    first = [o.cpu().numpy().copy() for (_, _, _, o, m) in items]
    g = A.Group(arr)
    for _ in range(3):  # repeated runs of one prepared group
        for (_, _, _, o, m) in items:
            if m:
                o.fill_(float("nan"))
        g.run()
        torch.cuda.synchronize()
        for (_, _, _, o, m), f in zip(items, first):
            assert np.array_equal(_bits(o.cpu().numpy()), _bits(f))
    g.free()


def test_grouped_back_to_back_calls_keep_their_tables(torch):
    # two different groups queued on one stream with no host wait between:
    # the second call's tables must not overwrite what the first launch reads
    items1, host1 = _group_items(torch, GROUP[:4], seed=902)
    items2, host2 = _group_items(torch, GROUP[4:], seed=903)
    arr1, arr2 = A.make_linears(items1), A.make_linears(items2)
    for _ in range(2):
        A.matmul_grouped_dev(arr1)
        A.matmul_grouped_dev(arr2)
    torch.cuda.synchronize()
    for items, host in ((items1, host1), (items2, host2)):
        for (w, _, _, out, m), (_, a, b, _) in zip(items, host):
            if m:
                assert rel_row_l2(out.cpu().numpy(), _single(torch, w, a, b)) <= 1e-6


@pytest.mark.parametrize("dtype", [2, 7], ids=["Q4_0", "Q5_1"])
def test_gemv_chunked_k_rows_independent_of_m(torch, dtype):
    # k = 16384: at m = 8 the activations go through LDS in several chunks, at
    # m = 1 in one; a row's result must not depend on that
    k, n = 16384, 40
    raw = weights(dtype, n, k, seed=77)
    w = A.DeviceWeight(dtype, n, k, raw)
    a = activations(8, k, seed=78, outliers=0.01)
    got8 = _single(torch, w, a)
    got1 = _single(torch, w, a[:1])
    assert np.array_equal(_bits(got8[:1]), _bits(got1))
    assert rel_row_l2(got8, O.matmul_emul(a, dtype, raw, n)) <= ROW_L2_TOL


def test_grouped_rejects_bad_items(torch):
    w = A.DeviceWeight(8, 32, 64, weights(8, 32, 64, seed=1))
    a = torch.zeros(9, 64, device="cuda:0")
    o = torch.zeros(9, 32, device="cuda:0")
    with pytest.raises(A.RwError, match="m = 9"):
        A.matmul_grouped_dev(A.make_linears([(w, a, None, o, 9)]))
    arr = A.make_linears([(w, a, None, o, 5)])
    wsz = A.grouped_workspace_size(arr)
    assert wsz > 0
    ws = torch.empty(wsz, dtype=torch.uint8, device="cuda:0")
    with pytest.raises(A.RwError, match="workspace"):
        A.matmul_grouped_dev(arr, ws, wsz - 1)
    with pytest.raises(A.RwError, match="m = 0"):
        A.Group(A.make_linears([(w, a, None, o, 0)]))


@pytest.mark.parametrize("dtype,n,m", [(7, 96, 5), (7, 160, 70), (2, 64, 9), (8, 33, 1)])
def test_graph_replay_matches_eager(torch, dtype, n, m):
    # the library's launches (separate quantize + product, and the fused
    # decode call) captured in a HIP graph and replayed three times with eager
    # work in between: every replay bitwise equal to the eager result
    k = 1280
    raw = weights(dtype, n, k, seed=60 + m)
    w = A.DeviceWeight(dtype, n, k, raw)
    a = _dev(torch, activations(m, k, seed=61 + m))
    bias = _dev(torch, np.random.default_rng(m).standard_normal(n).astype(np.float32))
    wsz = A.workspace_size(m, k)
    ws = torch.empty(wsz, dtype=torch.uint8, device="cuda:0")
    out1 = torch.empty(m, n, device="cuda:0")
    out2 = torch.empty(m, n, device="cuda:0")

    def calls(stream):
        A.quantize_dev(a, m, k, ws, wsz, stream)
        w.matmul_prequant_dev(ws, m, out1, bias, stream)
        w.matmul_dev(a, m, out2, None, ws, wsz, stream)

    calls(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    ref1, ref2 = out1.cpu().numpy().copy(), out2.cpu().numpy().copy()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        calls(torch.cuda.current_stream().cuda_stream)
    for rep in range(3):
        out1.fill_(float("nan"))
        out2.fill_(float("nan"))
        junk = torch.randn(1 << 16, device="cuda:0").sum()  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(_bits(out1.cpu().numpy()), _bits(ref1)), rep
        assert np.array_equal(_bits(out2.cpu().numpy()), _bits(ref2)), rep
        del junk
    del graph


def _scale_rows(k):
    """Rows for the per-row power-of-two scale of the f16 plane."""
    rows = []
    big = np.full(k, 1e-20, np.float32)
    big[:32] = np.linspace(-1e30, 1e30, 32, dtype=np.float32)  # a huge block beside tiny ones
    rows.append(big)
    p2 = np.zeros(k, np.float32)
    p2[:4] = [2.0, -1.0, 0.25, -2.0]  # amax exactly a power of two
    rows.append(p2)
    rows.append(np.full(k, -0.0, np.float32))  # -0 inputs quantize to +0
    tiny = np.full(k, 1e-40, np.float32)  # subnormal row maximum: e clamps at -110
    tiny[::3] = -3e-41
    rows.append(tiny)
    late = np.full(k, 3e-3, np.float32)  # the row maximum in the last block (the last pass's wavefront)
    late[-1] = -7e4
    rows.append(late)
    return np.stack(rows)


def _a16_expected(a):
    """The f16 plane's values and row scales, from the oracle's q_a and d_a."""
    m, k = a.shape
    with np.errstate(all="ignore"):
        q, d, _ = O.quantize_acts(a)
    amax = np.fmax.reduce(np.abs(a), axis=1, initial=np.float32(0))  # NaN skipped, as the Rust fold
    e = np.full(m, 15, np.int64)
    ok = (amax > 0) & np.isfinite(amax)
    e[ok] = np.maximum(np.frexp(amax[ok])[1], -110)
    down = np.ldexp(np.float32(1), (15 - e)).astype(np.float32)
    dd = (d * down[:, None]).astype(np.float32)
    with np.errstate(all="ignore"):
        vals = (q.astype(np.float32) * np.repeat(dd, 32, axis=1)).astype(np.float16)
    return vals, np.ldexp(np.float32(1), (e - 15)).astype(np.float32)


def _a16_index(m, k):
    rows = (m + 31) // 32 * 32
    nb = k // 32
    i = np.arange(rows)[:, None]
    kk = np.arange(k)[None, :]
    g, r, bl, e = i // 32, i % 32, kk // 32, kk % 32
    return (g * nb + bl) * 1024 + (e >> 4) * 512 + (32 * ((e >> 3) & 1) + r) * 8 + (e & 7)


@pytest.mark.parametrize("k", [32, 96, 416, 1024, 1056, 1280, 1568, 2048, 2080, 4128, 5120, 8224, 16384])
def test_gemm_activation_plane_bit_exact(torch, k):
    # one, two and four wavefronts per row (416: two of one pass; 1024: four);
    # rows of 5-20 passes store in row runs (1280: 8 rows per wavefront, two
    # parts of three passes; 2048 and 5120: 4 rows, four parts), including
    # ragged block counts whose last pass is partly past the row (1056, 1568,
    # 2080, 4128: 33, 49, 65, 129 blocks); 8224 and 16384 take the long-row
    # path (the row is read twice)
    a = np.concatenate([activations(21, k, seed=k, outliers=0.01), edge_activation_rows(k), _scale_rows(k)])
    m = a.shape[0]
    assert m > 8  # the encoder (f16) layout
    wsz = A.workspace_size(m, k)
    ws = torch.zeros(wsz, dtype=torch.uint8, device="cuda:0")
    A.quantize_dev(_dev(torch, a), m, k, ws, wsz)
    torch.cuda.synchronize()
    raw = ws.cpu().numpy()
    rows = (m + 31) // 32 * 32
    plane = raw[:rows * k * 2].view(np.uint16)[_a16_index(m, k)]
    off_rs = (rows * k * 2 + 255) // 256 * 256
    rs = raw[off_rs:off_rs + rows * 4].view(np.float32)
    want, want_rs = _a16_expected(a)
    assert np.array_equal(plane[:m], want.view(np.uint16)), np.argwhere(plane[:m] != want.view(np.uint16))[:5]
    assert np.array_equal(rs[:m].view(np.uint32), want_rs.view(np.uint32))
    assert not plane[m:].any() and not rs[m:].any()  # padding rows of the last row group
    # ps: the row's sum over blocks of d_a * sum(q_a) (the min term's
    # activation factor), each product rounded once and summed in f32
    off_ps = (off_rs + rows * 4 + 255) // 256 * 256
    ps = raw[off_ps:off_ps + rows * 4].view(np.float32)
    with np.errstate(all="ignore"):
        q, d, s = O.quantize_acts(a)
        terms = (d * s.astype(np.float32)).astype(np.float64)
    fin = np.all(np.isfinite(terms), axis=1)
    want_ps = terms.sum(axis=1)
    tol = terms.shape[1] * 2.0 ** -23 * np.abs(terms).sum(axis=1)
    assert np.all(np.abs(ps[:m][fin] - want_ps[fin]) <= tol[fin]), np.argwhere(np.abs(ps[:m] - want_ps) > tol)[:5]
    assert not ps[m:].any()


# (dtype, m, [n_i], k, [has bias]): q/k/v of the large-v3 encoder, ragged
# widths, a single weight, four weights with a long row, and the decode shape
MULTI = [
    (7, 40, [1280, 1280, 1280], 1280, [True, False, True]),
    (2, 70, [96, 33, 200], 416, [False, True, True]),
    (8, 9, [64], 96, [True]),
    (6, 33, [64, 64, 64, 64], 5120, [True, True, False, True]),
    (3, 5, [70, 40], 256, [True, False]),
]


@pytest.mark.parametrize("dtype,m,ns,k,hasb", MULTI, ids=lambda x: str(x))
def test_prequant_multi(torch, dtype, m, ns, k, hasb):
    rng = np.random.default_rng(m + k)
    raws = [weights(dtype, n, k, seed=17 * i + n) for i, n in enumerate(ns)]
    ws_ = [A.DeviceWeight(dtype, n, k, raw) for n, raw in zip(ns, raws)]
    biases = [rng.standard_normal(n).astype(np.float32) if hb else None for n, hb in zip(ns, hasb)]
    a = activations(m, k, seed=m * 3 + k, outliers=0.01)
    wsz = A.workspace_size(m, k)
    ws = torch.empty(wsz, dtype=torch.uint8, device="cuda:0")
    A.quantize_dev(_dev(torch, a), m, k, ws, wsz)

    def run(mm):
        outs = [torch.full((mm, n), float("nan"), device="cuda:0") for n in ns]
        A.matmul_prequant_multi_dev(ws_, ws, mm, outs, [None if b is None else _dev(torch, b) for b in biases])
        torch.cuda.synchronize()
        return [o.cpu().numpy() for o in outs]

    got = run(m)
    for w, raw, b, y in zip(ws_, raws, biases, got):
        ref = O.matmul_emul(a, dtype, raw, w.n, bias=b)
        assert rel_row_l2(y, ref) <= ROW_L2_TOL
        check_combine(y, a, dtype, raw, w.n, b)
        if m <= A.GEMV_MAX_M:  # decode shape: bitwise the single-weight call
            single = torch.empty(m, w.n, device="cuda:0")
            w.matmul_prequant_dev(ws, m, single, None if b is None else _dev(torch, b))
            torch.cuda.synchronize()
            assert np.array_equal(_bits(single.cpu().numpy()), _bits(y))
    if m > 9:  # rows do not depend on m: quantize the first 9 rows alone
        A.quantize_dev(_dev(torch, a[:9]), 9, k, ws, wsz)
        for y9, y in zip(run(9), got):
            assert np.array_equal(_bits(y9), _bits(y[:9]))


def test_prequant_multi_rejects_bad_sets(torch):
    w1 = A.DeviceWeight(7, 64, 128, weights(7, 64, 128, seed=1))
    w2 = A.DeviceWeight(7, 64, 96, weights(7, 64, 96, seed=2))
    w3 = A.DeviceWeight(8, 64, 128, weights(8, 64, 128, seed=3))
    ws = torch.zeros(A.workspace_size(20, 128), dtype=torch.uint8, device="cuda:0")
    o = [torch.zeros(20, 64, device="cuda:0") for _ in range(5)]
    with pytest.raises(A.RwError, match="differs"):
        A.matmul_prequant_multi_dev([w1, w2], ws, 20, o[:2])
    with pytest.raises(A.RwError, match="differs"):
        A.matmul_prequant_multi_dev([w1, w3], ws, 20, o[:2])
    with pytest.raises(A.RwError, match="count"):
        A.matmul_prequant_multi_dev([w1] * 5, ws, 20, o)
    with pytest.raises(A.RwError, match="count"):
        A.matmul_prequant_multi_dev([], ws, 20, [])
