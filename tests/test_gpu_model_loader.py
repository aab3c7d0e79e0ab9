"""Model files to resident weights on the device: rw_rocm_model_load without
RW_MODEL_PARSE_ONLY uploads every 2-D quantized tensor, and the uploaded
weights answer like weights uploaded from the same bytes directly.

Bars: dequantized rows bit-exact with the oracle (quant.rs:528-537); matmul
outputs bit-identical to a DeviceWeight built from the same blocks, and
within 1e-3 row-L2 of the reference CPU path."""
import numpy as np
import pytest

import oracle as O
from rusty_whisper_amd import _abi as A

from _data import DTYPES, NAMES, activations, rel_row_l2, weights
import _modelfile as MF

pytestmark = pytest.mark.gpu

ROW_L2_TOL = 1e-3
HP = [51865, 1500, 384, 6, 4, 448, 384, 6, 4, 80, 1]


@pytest.fixture(scope="module", autouse=True)
def _device():
    A.init(0)


def _tensors():
    out = []
    for i, dt in enumerate(DTYPES):
        n, k = 96 + 32 * i, 256 + 64 * i
        out.append((f"blocks.{i}.attn.query.weight", dt, n, k, weights(dt, n, k, seed=70 + i)))
    return out


@pytest.mark.parametrize("container", ["ggml", "gguf"])
def test_loaded_weights_match_direct_upload(tmp_path, container):
    ts = _tensors()
    bias = np.linspace(-1, 1, 7, dtype=np.float32)
    if container == "ggml":
        data = MF.ggml_bytes(HP, tokens=[b"a"], tensors=[(nm, dt, [k, n], raw.tobytes()) for nm, dt, n, k, raw in ts]
                             + [("bias", 0, [7], bias.astype("<f4").tobytes())])
    else:
        data = MF.gguf_bytes(HP, tokens=[b"a"], tensors=[(nm, dt, [n, k], raw.tobytes()) for nm, dt, n, k, raw in ts]
                             + [("bias", 0, [7], bias.astype("<f4").tobytes())])
    p = tmp_path / f"m.{container}"
    p.write_bytes(data)
    print(f"model {container}: {len(ts)} quantized matrices", flush=True)
    m = A.Model(str(p))
    np.testing.assert_array_equal(m.dense("bias"), bias)
    with pytest.raises(A.RwError, match="dense"):
        m.weight("bias")
    for nm, dt, n, k, raw in ts:
        w = m.weight(nm)
        assert w.info()[:3] == (dt, n, k), NAMES[dt]
        got = w.dequant_rows()
        assert np.array_equal(got.view(np.uint32), O.dequant(dt, raw, n, k).view(np.uint32)), NAMES[dt]
        direct = A.DeviceWeight(dt, n, k, raw)
        for mrows in (1, 5, 40):
            a = activations(mrows, k, seed=mrows + k)
            y = w.matmul(a)
            assert np.array_equal(y.view(np.uint32), direct.matmul(a).view(np.uint32)), (NAMES[dt], mrows)
            ref = O.matmul_emul(a, dt, raw, n, tier=O.TIER_VNNI)
            assert rel_row_l2(y, ref) <= ROW_L2_TOL, (NAMES[dt], mrows)
        direct.free()
    m.free()
