"""rw_rocm_attention's argument checks, without a device (they run before any
HIP call): the reference's conditions (src/encoder.rs:48-58, 109-119) and
the kernel's own limits come back as RW_EINVAL with a message."""
import ctypes as C

import numpy as np
import pytest

from rusty_whisper_amd import _abi as A


def _call(t_q, t_kv, n_state, n_head, causal, ldq=None, q_off=0, ldv=None, v_off=0):
    q = np.zeros(max(t_q * (ldq or n_state) + 16, 1), np.float32)
    k = np.zeros(max(t_kv * n_state, 1), np.float32)
    v = np.zeros(max(t_kv * (ldv or n_state) + 16, 1), np.float32)
    out = np.zeros(max(t_q * n_state, 1), np.float32)
    return A.lib().rw_rocm_attention_dev(q.ctypes.data + q_off, ldq or n_state, k.ctypes.data, n_state,
                                         v.ctypes.data + v_off, ldv or n_state, t_q, t_kv, n_state, n_head, causal,
                                         out.ctypes.data, n_state, None, 0, None)


@pytest.mark.parametrize("args,msg", [
    ((4, 4, 96, 2, 0), "head size 48 unsupported"),
    ((4, 4, 131, 2, 0), "not a positive multiple of n_head"),
    ((4, 4, 128, 0, 0), "not a positive multiple of n_head"),
    ((5, 4, 128, 2, 1), "causal attention needs t_q <= t_kv"),
])
def test_rejected_shapes(args, msg):
    assert _call(*args) == A.RW_EINVAL
    assert msg in A.last_error()


def test_rejects_short_or_misaligned_rows():
    assert _call(4, 4, 128, 2, 0, ldq=100) == A.RW_EINVAL
    assert "row stride is smaller" in A.last_error()
    assert _call(4, 4, 128, 2, 0, ldq=130) == A.RW_EINVAL
    assert "16-byte aligned" in A.last_error()
    assert _call(4, 4, 128, 2, 0, q_off=4) == A.RW_EINVAL
    assert "16-byte aligned" in A.last_error()
    # v is read with 16-byte loads too
    assert _call(4, 4, 128, 2, 0, ldv=130) == A.RW_EINVAL
    assert "16-byte aligned" in A.last_error()
    assert _call(4, 4, 128, 2, 0, v_off=8) == A.RW_EINVAL
    assert "16-byte aligned" in A.last_error()


def test_rejects_head_counts_past_the_packed_grid():
    # k_attn carries its grid's head extent (times up to 8 beams) above 8 bits
    # of one int argument
    assert _call(0, 0, (1 << 19) * 64, 1 << 19, 0) == A.RW_EINVAL
    assert "too large" in A.last_error()
    assert _call(0, 0, ((1 << 19) - 1) * 64, (1 << 19) - 1, 0) == A.RW_OK  # an empty call within the bound


def test_empty_query_is_a_noop():
    assert _call(0, 4, 128, 2, 0) == A.RW_OK


def test_workspace_size_covers_the_planes():
    # q pairs over 64-row padding, k and v^T pairs over 32-row padding
    n = A.attention_workspace_size(1500, 1500, 1280)
    assert n >= 20 * 1536 * 64 * 4 + 2 * 20 * 1504 * 64 * 4
