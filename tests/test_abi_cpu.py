"""The C ABI without compute: the library loads, exports every symbol
include/rw_rocm.h declares, and turns the reference's panic conditions
(src/quant.rs:757-758, 129) into status codes + error text.  No GPU needed."""
import ctypes as C

import numpy as np
import pytest

from rusty_whisper_amd import _abi as A


def test_library_loads_and_exports_every_declared_symbol():
    L = A.lib()
    declared = A.header_symbols()
    assert len(declared) >= 16
    missing = [s for s in declared if not hasattr(L, s)]
    assert not missing, missing
    # and the binding declares a signature for each of them
    assert sorted(A._SIGNATURES) == declared


def test_version():
    assert A.lib().rw_rocm_version() == 0x000100


def test_block_bytes_matches_reference_table():
    assert [A.block_bytes(d) for d in A.DTYPES] == [18, 20, 22, 24, 34]
    for bad in (0, 1, 4, 5, 9, -1):
        with pytest.raises(A.RwError) as e:
            A.block_bytes(bad)
        assert e.value.code == A.RW_EINVAL and "unsupported dtype" in e.value.message


def _upload(dtype, n, k, raw_len=None, raw="auto", out=True):
    bb = {2: 18, 3: 20, 6: 22, 7: 24, 8: 34}.get(dtype, 18)
    nbytes = raw_len if raw_len is not None else n * (k // 32) * bb
    buf = np.zeros(max(nbytes, 1), np.uint8)
    h = C.c_void_p()
    ptr = buf.ctypes.data if raw == "auto" else raw
    return A.lib().rw_rocm_weight_upload(dtype, n, k, ptr, nbytes, C.byref(h) if out else None)


@pytest.mark.parametrize("args,needle", [
    ((5, 4, 32), "unsupported dtype"),     # quant.rs:129 panic
    ((8, 4, 48), "multiple of 32"),        # quant.rs:758 assert
    ((8, 4, 0), "multiple of 32"),
    ((8, 0, 32), "n must be positive"),
])
def test_upload_rejects_bad_shapes(args, needle):
    assert _upload(*args) == A.RW_EINVAL
    assert needle in A.last_error()


def test_upload_rejects_wrong_length_and_nulls():
    assert _upload(8, 4, 32, raw_len=4 * 34 - 1) == A.RW_EINVAL
    assert "raw length" in A.last_error()
    assert _upload(8, 4, 32, raw=None) == A.RW_EINVAL
    assert _upload(8, 4, 32, out=False) == A.RW_EINVAL


def test_matmul_rejects_null_weight():
    a = np.zeros((2, 32), np.float32)
    out = np.zeros((2, 4), np.float32)
    rc = A.lib().rw_rocm_matmul_t_q(None, a.ctypes.data, 2, 32, None, out.ctypes.data)
    assert rc == A.RW_EINVAL and "weight is NULL" in A.last_error()
    rc = A.lib().rw_rocm_matmul_t_q_dev(None, None, 0, 32, None, None, None, 0, None)
    assert rc == A.RW_EINVAL


def test_workspace_sizes():
    assert A.workspace_size(0, 64) == 0
    assert A.workspace_size(4, 33) == 0
    small = A.workspace_size(1, 1280)
    assert small >= 32 * 1280  # one row group of int8 quants
    assert A.workspace_size(33, 1280) >= 2 * 32 * 1280


def test_quantize_entry_rejects_bad_k():
    a = np.zeros((1, 48), np.float32)
    rc = A.lib().rw_rocm_quantize_acts(a.ctypes.data, 1, 48, None, None, None)
    assert rc == A.RW_EINVAL


def test_no_device_is_an_error_not_a_fallback():
    if A.device_count() > 0:
        pytest.skip("a device is present: covered by the gpu tests")
    assert _upload(8, 4, 32) == A.RW_ENODEV
    with pytest.raises(A.RwError) as e:
        A.init(0)
    assert e.value.code == A.RW_ENODEV


def test_last_error_truncates_safely():
    _upload(5, 4, 32)
    buf = C.create_string_buffer(8)
    n = A.lib().rw_rocm_last_error(buf, 8)
    assert n > 7 and len(buf.value) == 7


def test_owning_classes_free_on_collection():
    """Every binding class that owns device memory (has free()) releases it
    when collected: __del__ is a method of the class itself, not a function
    nested elsewhere in the module."""
    import ast
    import inspect

    tree = ast.parse(inspect.getsource(A))
    for node in ast.walk(tree):
        if isinstance(node, ast.FunctionDef) and node.name != "__del__":
            nested = [n.name for n in ast.walk(node) if isinstance(n, ast.FunctionDef) and n.name == "__del__"]
            assert not nested, f"__del__ nested in function {node.name}"
    for cls in (A.DeviceWeight, A.Decoder, A.Group, A.Model):
        assert "free" in vars(cls) and "__del__" in vars(cls), cls.__name__
