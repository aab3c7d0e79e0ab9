"""GPU parity at the workloads of the benchmark configurations, through the
C ABI, against the oracle.

  * tiny.en fc1, Q5_1, M = 1500 (the whole matrix against the oracle);
  * small.en encoder linears, Q8_0, d = 768, fc 3072, M = 1500, with 1% of
    the activation channels scaled x20;
  * large-v3 encoder linears in Q4_0 and Q4_1, M = 1500, each weight block
    scaled by 10**U(-1, 1) (two decades);
  * large-v3 decoder linears in Q5_0 at M = 1 and M = 5, the [51866 x 1280]
    logits projection included, single launches and one grouped launch;
  * large-v3-turbo batch: M = 12000 (8 stacked windows) through the encoder
    shapes and the cross K/V projection, M = 40 (8 x 5 beam rows) through the
    decoder shapes and the logits.

Bars: 1e-3 of the reference CPU path (max error over the reference row's L2
norm), and the regime's analytic bound against the exact combination
(tests/_data.py).  Where the oracle would take minutes at full size, a seeded
sample of rows (both ends, row-group and tile boundaries, random rows) is
compared with it.  That is sound because a row's result depends on its own
activations only: the reference's rows are independent of M
(src/quant.rs:1372-1384), and so are this library's within a regime, which
each full-size test checks bit for bit by running the sampled rows alone.
Every output of every full-size run is also checked finite.
"""
import numpy as np
import pytest

import oracle as O
from rusty_whisper_amd import _abi as A
from rusty_whisper_amd import synth

from _data import activations, check_combine, rel_row_l2, weights

pytestmark = pytest.mark.gpu

TOL = 1e-3
LV3_SHAPES = [(1280, 1280), (5120, 1280), (1280, 5120)]  # q/k/v/out, fc1, fc2 as [n, k]


@pytest.fixture(scope="module")
def torch():
    import torch as T

    A.init(0)
    return T


def sample_rows(m: int, seed: int, extra: int = 40) -> np.ndarray:
    rng = np.random.default_rng(seed)
    fixed = {0, 1, 31, 32, 95, 127, 128, 1499, 1500, m // 2, m - 33, m - 32, m - 2, m - 1}
    rnd = set(rng.choice(m, size=min(extra, m), replace=False).tolist())
    return np.array(sorted(x for x in fixed | rnd if 0 <= x < m))


def run_dev(torch, w, a, bias=None):
    ad = torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")
    out = torch.empty(a.shape[0], w.n, device="cuda:0")
    bd = None if bias is None else torch.from_numpy(bias).to("cuda:0")
    w.matmul_dev(ad, a.shape[0], out, bd)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def bias_for(n: int, seed: int) -> np.ndarray:
    return (np.random.default_rng(seed).standard_normal(n) * 0.1).astype(np.float32)


def check_sampled(torch, dtype, n, k, m, seed, *, spread=False, outliers=0.0, with_bias=True):
    print(f"{synth.NAMES[dtype]} [{n}x{k}] m={m} spread={spread} outliers={outliers}", flush=True)
    raw = weights(dtype, n, k, seed, spread=spread)
    a = activations(m, k, seed + 1, outliers)
    b = bias_for(n, seed + 2) if with_bias else None
    w = A.DeviceWeight(dtype, n, k, raw)
    full = run_dev(torch, w, a, b)
    assert np.all(np.isfinite(full))
    rows = sample_rows(m, seed)
    assert len(rows) > A.GEMV_MAX_M  # the sample runs in the full run's regime
    alone = run_dev(torch, w, a[rows], b)
    assert np.array_equal(full[rows].view(np.uint32), alone.view(np.uint32)), "a row depends on m"
    ref = O.matmul_emul(a[rows], dtype, raw, n, bias=b)
    err = rel_row_l2(full[rows], ref)
    print(f"  sampled {len(rows)} rows: error {err:.3g}", flush=True)
    assert err <= TOL
    check_combine(full[rows], a[rows], dtype, raw, n, b)
    w.free()


def check_whole(torch, dtype, n, k, m, seed, *, with_bias=True):
    print(f"{synth.NAMES[dtype]} [{n}x{k}] m={m} (whole output)", flush=True)
    raw = weights(dtype, n, k, seed)
    a = activations(m, k, seed + 1)
    b = bias_for(n, seed + 2) if with_bias else None
    w = A.DeviceWeight(dtype, n, k, raw)
    got = run_dev(torch, w, a, b)
    ref = O.matmul_emul(a, dtype, raw, n, bias=b)
    err = rel_row_l2(got, ref)
    print(f"  error {err:.3g}", flush=True)
    assert np.all(np.isfinite(got))
    assert err <= TOL
    check_combine(got, a, dtype, raw, n, b)
    w.free()
    return got


# ------------------------------------------------------------ config 1


def test_tiny_fc1_q5_1_whole(torch):
    check_whole(torch, A.Q5_1, 1536, 384, 1500, seed=11)


# ------------------------------------------------------------ config 2


@pytest.mark.parametrize("n,k", [(768, 768), (3072, 768), (768, 3072)], ids=lambda x: str(x))
def test_small_q8_0_outliers_m1500(torch, n, k):
    check_sampled(torch, A.Q8_0, n, k, 1500, seed=20 + n // 256 + k // 256, outliers=0.01)


def test_small_q8_0_qkv_one_launch(torch):
    """q, k and v of a small.en layer on one quantized input (one GEMM launch
    for three weights), k without bias, each against the oracle."""
    m, d = 1500, 768
    a = activations(m, d, 31, outliers=0.01)
    raws = [weights(A.Q8_0, d, d, 32 + i) for i in range(3)]
    biases = [bias_for(d, 40), None, bias_for(d, 41)]
    ws_len = A.workspace_size(m, d)
    ws = torch.empty(ws_len, dtype=torch.uint8, device="cuda:0")
    ad = torch.from_numpy(a).to("cuda:0")
    A.quantize_dev(ad, m, d, ws, ws_len)
    ws_w = [A.DeviceWeight(A.Q8_0, d, d, r) for r in raws]
    outs = [torch.empty(m, d, device="cuda:0") for _ in range(3)]
    bd = [None if b is None else torch.from_numpy(b).to("cuda:0") for b in biases]
    A.matmul_prequant_multi_dev(ws_w, ws, m, outs, bd)
    torch.cuda.synchronize()
    rows = sample_rows(m, 33)
    for raw, b, o in zip(raws, biases, outs):
        got = o.cpu().numpy()
        assert np.all(np.isfinite(got))
        ref = O.matmul_emul(a[rows], A.Q8_0, raw, d, bias=b)
        assert rel_row_l2(got[rows], ref) <= TOL
        check_combine(got[rows], a[rows], A.Q8_0, raw, d, b)


# ------------------------------------------------------------ config 4


@pytest.mark.parametrize("dtype", [A.Q4_0, A.Q4_1], ids=["Q4_0", "Q4_1"])
@pytest.mark.parametrize("n,k", LV3_SHAPES, ids=lambda x: str(x))
def test_large_v3_q4_spread_m1500(torch, dtype, n, k):
    check_sampled(torch, dtype, n, k, 1500, seed=50 + dtype + n // 640, spread=True)


# ------------------------------------------------------------ config 3


@pytest.mark.parametrize("m", [1, 5])
@pytest.mark.parametrize("n,k", LV3_SHAPES + [(51866, 1280)], ids=lambda x: str(x))
def test_large_v3_decoder_q5_0(torch, m, n, k):
    check_whole(torch, A.Q5_0, n, k, m, seed=70 + n // 640 + k // 640, with_bias=n != 51866)


def test_large_v3_decoder_layer_grouped_q5_0(torch):
    """One decoder layer's ten linears plus the logits at M = 5 in one
    grouped launch, each against the oracle."""
    m, d, fc = 5, 1280, 5120
    shapes = [(name, n, k) for name, n, k in synth.decoder_layer_shapes(d, fc)] + [("logits", 51866, d)]
    items, refs, keep = [], [], []
    for i, (name, n, k) in enumerate(shapes):
        raw = weights(A.Q5_0, n, k, 90 + i)
        a = activations(m, k, 120 + i)
        b = None if name in ("self.k", "cross.k", "logits") else bias_for(n, 150 + i)
        w = A.DeviceWeight(A.Q5_0, n, k, raw)
        ad = torch.from_numpy(a).to("cuda:0")
        bd = None if b is None else torch.from_numpy(b).to("cuda:0")
        out = torch.empty(m, n, device="cuda:0")
        items.append((w, ad, bd, out, m))
        refs.append((name, a, raw, n, b))
        keep.append((w, ad, bd, out))
    arr = A.make_linears(items)
    A.matmul_grouped_dev(arr)
    torch.cuda.synchronize()
    for (name, a, raw, n, b), (_, _, _, out) in zip(refs, keep):
        got = out.cpu().numpy()
        ref = O.matmul_emul(a, A.Q5_0, raw, n, bias=b)
        err = rel_row_l2(got, ref)
        assert err <= TOL, (name, err)
        check_combine(got, a, A.Q5_0, raw, n, b)


# ------------------------------------------------------------ config 5


@pytest.mark.parametrize("n,k", LV3_SHAPES, ids=lambda x: str(x))
def test_turbo_q5_1_m12000(torch, n, k):
    """8 stacked windows through the encoder shapes; (1280, 1280) without a
    bias is also the decoder's cross K projection of the stacked windows."""
    check_sampled(torch, A.Q5_1, n, k, 12000, seed=200 + n // 640 + k // 640, with_bias=n != k)


@pytest.mark.parametrize("n,k", LV3_SHAPES + [(51866, 1280)], ids=lambda x: str(x))
def test_turbo_q5_1_m40(torch, n, k):
    """8 windows x 5 beam rows through the decoder shapes and the logits."""
    if n == 51866:
        check_sampled(torch, A.Q5_1, n, k, 40, seed=300, with_bias=False)
    else:
        check_whole(torch, A.Q5_1, n, k, 40, seed=310 + n // 640 + k // 640)


@pytest.mark.parametrize("m", [1500, 12000])
def test_large_v3_qkv_one_launch_rows_independent_of_m(torch, m):
    """q, k and v of a large-v3 layer in one launch (96-row tiles at
    M = 1500, 128-row tiles at M = 12000): the sampled rows run alone (64-row
    tiles) give the same bits, and match the oracle."""
    d = 1280
    a = activations(m, d, 61)
    raws = [weights(A.Q5_1, d, d, 62 + i) for i in range(3)]
    ws_w = [A.DeviceWeight(A.Q5_1, d, d, r) for r in raws]
    rows = sample_rows(m, 63)

    def run(x):
        mm = x.shape[0]
        ws_len = A.workspace_size(mm, d)
        ws = torch.empty(ws_len, dtype=torch.uint8, device="cuda:0")
        A.quantize_dev(torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0"), mm, d, ws, ws_len)
        outs = [torch.empty(mm, d, device="cuda:0") for _ in range(3)]
        A.matmul_prequant_multi_dev(ws_w, ws, mm, outs)
        torch.cuda.synchronize()
        return [o.cpu().numpy() for o in outs]

    full, alone = run(a), run(a[rows])
    for raw, f, s in zip(raws, full, alone):
        assert np.all(np.isfinite(f))
        assert np.array_equal(f[rows].view(np.uint32), s.view(np.uint32)), "a row depends on m"
        assert rel_row_l2(s, O.matmul_emul(a[rows], A.Q5_1, raw, d)) <= TOL
