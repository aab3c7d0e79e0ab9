"""rw_rocm_model_load on synthetic ggml .bin and GGUF files, parse-only (no
device).  The first tests restate the reference's own loader tests
(src/model.rs:282-428, src/gguf.rs:469-560) through the C ABI; the rest cover
its error paths and the container details it reads (widened metadata
integers, alignment, trailing bytes, repeated names).  Non-2-D quantized
tensors are densified by the loader and checked against the oracle's
dequantization; 2-D ones keep their bytes verbatim."""
from __future__ import annotations

import struct

import numpy as np
import pytest

import oracle as O
from rusty_whisper_amd import _abi as A
from tests import _modelfile as MF

TINY_HP = [3, 1500, 8, 2, 4, 448, 8, 2, 4, 2, 1]


def load(tmp_path, data: bytes, name="m.bin") -> A.Model:
    p = tmp_path / name
    p.write_bytes(data)
    return A.Model(str(p), parse_only=True)


def load_err(tmp_path, data: bytes) -> A.RwError:
    with pytest.raises(A.RwError) as e:
        load(tmp_path, data)
    return e.value


def f32b(vals) -> bytes:
    return np.asarray(vals, "<f4").tobytes()


# --------------------------------------------------- reference tests, restated

def test_loads_synthetic_model(tmp_path):
    """src/model.rs:294-346"""
    data = MF.ggml_bytes(
        TINY_HP, mel=np.array([[0.1, 0.2, 0.3], [0.4, 0.5, 0.6]], np.float32), tokens=[b"hi", b"yo"],
        tensors=[("w", 0, [2, 3], f32b([1, 2, 3, 4, 5, 6])),
                 ("b", 1, [2], struct.pack("<HH", 0x3C00, 0xC000))])
    m = load(tmp_path, data)
    assert m.hparams["n_vocab"] == 3 and m.hparams["n_audio_layer"] == 4  # model_type "tiny"
    np.testing.assert_array_equal(m.mel_filters().reshape(-1), np.float32([0.1, 0.2, 0.3, 0.4, 0.5, 0.6]))
    assert m.mel_filters().shape == (2, 3)
    v = m.vocab()
    assert len(v) == 3 and v[1] == b"yo" and v[2] == b"[_extra_token_2]"
    assert m.tensor("w") == (0, (3, 2), False)  # dims flipped to row-major
    np.testing.assert_array_equal(m.dense("w"), np.float32([[1, 2], [3, 4], [5, 6]]))
    np.testing.assert_array_equal(m.dense("b"), np.float32([1.0, -2.0]))
    assert sorted(m.names()) == ["b", "w"]
    m.free()


def test_loads_quantized_tensor_from_synthetic_file(tmp_path):
    """src/model.rs:392-421: a 2-D q8_0 tensor stays quantized."""
    blk = struct.pack("<H", 0x3C00) + bytes([2] * 32)
    data = MF.ggml_bytes([3, 1500, 8, 2, 4, 448, 8, 2, 4, 2, 8], tensors=[("q", 8, [32, 1], blk)])
    m = load(tmp_path, data)
    assert m.tensor("q") == (8, (1, 32), True)
    assert m.raw("q") == blk
    np.testing.assert_array_equal(O.dequant(8, np.frombuffer(m.raw("q"), np.uint8), 1, 32), np.full((1, 32), 2.0))
    assert m.vocab() == [b"[_extra_token_0]", b"[_extra_token_1]", b"[_extra_token_2]"]
    assert m.mel_filters().shape == (0, 0)
    with pytest.raises(A.RwError, match="parse-only"):
        m.weight("q")
    with pytest.raises(A.RwError, match="not dense"):
        m.dense("q")


def test_rejects_bad_magic(tmp_path):
    """src/model.rs:423-427"""
    e = load_err(tmp_path, struct.pack("<I", 0xDEADBEEF))
    assert e.code == A.RW_EINVAL and "bad magic 0xdeadbeef" in e.message


def test_f16_tensor_uses_the_exact_conversion(tmp_path):
    """src/model.rs:282-291 values through an f16 tensor (dtype 1)."""
    codes = [0x0000, 0x3C00, 0xC000, 0x3555, 0x0001, 0x7C00, 0x7E00, 0x8000, 0x7BFF, 0x03FF]
    data = MF.ggml_bytes(TINY_HP, tensors=[("h", 1, [len(codes)], struct.pack(f"<{len(codes)}H", *codes))])
    d = load(tmp_path, data).dense("h")
    assert d[0] == 0.0 and d[1] == 1.0 and d[2] == -2.0 and d[3] == np.float32(0.33325195)
    assert abs(d[4] - 5.9604645e-8) < 1e-12 and np.isinf(d[5]) and np.isnan(d[6])
    assert np.signbit(d[7]) and d[8] == 65504.0 and d[9] == np.float32(6.0975552e-05)
    # every code, against the oracle's f16_to_f32
    allc = np.arange(65536, dtype=np.uint16)
    data = MF.ggml_bytes(TINY_HP, tensors=[("h", 1, [65536], allc.astype("<u2").tobytes())])
    d = load(tmp_path, data).dense("h")
    np.testing.assert_array_equal(d.view(np.uint32), O.f16_to_f32_bits(allc))


def _sample_gguf(**kw) -> bytes:
    """The reference's GGUF sample model (src/gguf.rs:475-515)."""
    raw = b"".join(struct.pack("<H", 0x3C00) + bytes([row + 1] * 32) for row in range(2))
    mel = (np.arange(2 * 201, dtype=np.float32) * 0.5).reshape(2, 201)
    tensors = sorted([("encoder.conv1.bias", 0, [3], f32b([1.0, -2.0, 0.5])),
                      ("decoder.token_embedding.weight", 8, [2, 32], raw)])
    return MF.gguf_bytes([4, 10, 8, 2, 1, 6, 8, 2, 1, 2, 1], mel=mel, tokens=[b"a", b"bc", b"", b"\xff\xfe"],
                         tensors=tensors, **kw)


def test_gguf_round_trip(tmp_path):
    """src/gguf.rs:518-546"""
    data = _sample_gguf()
    assert data[:4] == b"GGUF"
    m = load(tmp_path, data, "m.gguf")
    assert list(m.hparams.values()) == [4, 10, 8, 2, 1, 6, 8, 2, 1, 2, 1]
    assert m.vocab() == [b"a", b"bc", b"", b"\xff\xfe"]
    np.testing.assert_array_equal(m.mel_filters(), (np.arange(402, dtype=np.float32) * 0.5).reshape(2, 201))
    assert sorted(m.names()) == ["decoder.token_embedding.weight", "encoder.conv1.bias"]
    np.testing.assert_array_equal(m.dense("encoder.conv1.bias"), np.float32([1.0, -2.0, 0.5]))
    assert m.tensor("decoder.token_embedding.weight") == (8, (2, 32), True)
    d = O.dequant(8, np.frombuffer(m.raw("decoder.token_embedding.weight"), np.uint8), 2, 32)
    np.testing.assert_array_equal(d, np.float32([[1.0] * 32, [2.0] * 32]))


def test_gguf_rejects_wrong_architecture(tmp_path):
    """src/gguf.rs:548-557"""
    data = bytearray(_sample_gguf())
    pos = data.find(b"whisper")
    data[pos:pos + 7] = b"whooper"
    e = load_err(tmp_path, bytes(data))
    assert 'architecture is not "whisper"' in e.message


# ------------------------------------------------------------ dense densify

@pytest.mark.parametrize("dtype", A.DTYPES)
@pytest.mark.parametrize("dims", [[64], [32, 2, 3]])
def test_non_matrix_quantized_tensors_become_dense(tmp_path, dtype, dims):
    """Quantized tensors of rank != 2 are Weight::Dense(qt.to_dense())
    (src/model.rs:232-239): d*q + m per element, as the oracle dequantizes."""
    n = int(np.prod(dims))
    rng = np.random.default_rng(dtype)
    raw = O.quantize(dtype, rng.standard_normal(n).astype(np.float32))
    data = MF.ggml_bytes(TINY_HP, tensors=[("t", dtype, dims, raw.tobytes())])
    m = load(tmp_path, data)
    assert m.tensor("t") == (dtype, tuple(reversed(dims)), False)
    np.testing.assert_array_equal(m.dense("t").reshape(-1), O.dequant(dtype, raw, 1, n).reshape(-1))


def test_dequant_known_blocks(tmp_path):
    """src/model.rs:348-381's blocks, densified through 1-D tensors."""
    q8 = bytearray(34)
    q8[0:2] = struct.pack("<H", 0x3800)
    q8[2:5] = bytes([0, 1, 0xFE])
    q8[5:34] = bytes([3] * 29)
    q4 = bytearray(18)
    q4[0:2] = struct.pack("<H", 0x3C00)
    q4[2] = 0xF8
    q5 = bytearray(22)
    q5[0:2] = struct.pack("<H", 0x3C00)
    q5[2:6] = struct.pack("<I", 1)
    data = MF.ggml_bytes(TINY_HP, tensors=[("a", 8, [32], bytes(q8)), ("b", 2, [32], bytes(q4)),
                                           ("c", 6, [32], bytes(q5))])
    m = load(tmp_path, data)
    a, b, c = m.dense("a"), m.dense("b"), m.dense("c")
    assert list(a[:3]) == [0.0, 0.5, -1.0] and a[31] == 1.5
    assert b[0] == 0.0 and b[16] == 7.0 and b[1] == -8.0
    assert c[0] == 0.0 and c[16] == -16.0


# ------------------------------------------------------------- ggml details

def test_ggml_trailing_bytes_end_the_tensor_list(tmp_path):
    """Fewer than 4 bytes after the last tensor read as end of file
    (read_i32's UnexpectedEof breaks the loop, src/model.rs:199-203)."""
    base = MF.ggml_bytes(TINY_HP, tensors=[("w", 0, [2], f32b([1, 2]))])
    for extra in (b"", b"\x01", b"\x01\x02\x03"):
        assert load(tmp_path, base + extra).names() == ["w"]
    e = load_err(tmp_path, base + b"\x01\x00\x00\x00")
    assert "failed to fill whole buffer" in e.message


def test_ggml_repeated_name_keeps_last(tmp_path):
    data = MF.ggml_bytes(TINY_HP, tensors=[("w", 0, [2], f32b([1, 2])), ("w", 0, [3], f32b([4, 5, 6]))])
    m = load(tmp_path, data)
    assert m.names() == ["w"]
    np.testing.assert_array_equal(m.dense("w"), np.float32([4, 5, 6]))


def test_ggml_zero_dims_is_a_scalar(tmp_path):
    m = load(tmp_path, MF.ggml_bytes(TINY_HP, tensors=[("s", 0, [], f32b([7]))]))
    assert m.tensor("s") == (0, (1,), False)
    np.testing.assert_array_equal(m.dense("s"), np.float32([7]))


def test_ggml_file_with_more_tokens_than_n_vocab(tmp_path):
    m = load(tmp_path, MF.ggml_bytes(TINY_HP, tokens=[b"a", b"b", b"c", b"d"]))
    assert m.vocab() == [b"a", b"b", b"c", b"d"]


@pytest.mark.parametrize("case,msg", [
    ("short_magic", "failed to fill whole buffer"),
    ("short_hparams", "failed to fill whole buffer"),
    ("short_mel", "failed to fill whole buffer"),
    ("short_token", "failed to fill whole buffer"),
    ("short_tensor_header", "failed to fill whole buffer"),
    ("short_tensor_data", "failed to fill whole buffer"),
    ("unsupported_dtype", "tensor 'x': unsupported dtype 4"),
    ("indivisible", "tensor 'x': 48 elements not divisible by block size"),
    ("huge_dims", "failed to fill whole buffer"),
    ("four_dims", "tensor with 4 dimensions"),
])
def test_ggml_errors(tmp_path, case, msg):
    full = MF.ggml_bytes(TINY_HP, mel=np.ones((2, 3), np.float32), tokens=[b"hi"],
                         tensors=[("w", 0, [4], f32b([1, 2, 3, 4]))])
    hdr = 4 + 11 * 4
    data = {
        "short_magic": full[:3],
        "short_hparams": full[:hdr - 2],
        "short_mel": full[:hdr + 8 + 20],
        "short_token": full[:hdr + 8 + 24 + 4 + 4 + 1],
        "short_tensor_header": full[:hdr + 8 + 24 + 4 + 4 + 2 + 6],
        "short_tensor_data": full[:-1],
        "unsupported_dtype": MF.ggml_bytes(TINY_HP, tensors=[("x", 4, [32], bytes(20))]),
        "indivisible": MF.ggml_bytes(TINY_HP, tensors=[("x", 2, [48], bytes(36))]),
        "huge_dims": MF.ggml_bytes(TINY_HP, tensors=[("x", 0, [0x7FFFFFFF, 0x7FFFFFFF, 0x7FFFFFFF], b"")]),
        "four_dims": MF.ggml_bytes(TINY_HP, tensors=[("x", 0, [1, 1, 1, 1], f32b([1]))]),
    }[case]
    e = load_err(tmp_path, data)
    assert e.code == A.RW_EINVAL and msg in e.message, e.message


def test_missing_file_is_an_io_error(tmp_path):
    with pytest.raises(A.RwError) as e:
        A.Model(str(tmp_path / "nope.bin"), parse_only=True)
    assert e.value.code == A.RW_EIO and "nope.bin" in e.value.message


# ------------------------------------------------------------- gguf details

def test_gguf_integer_widths_and_skipped_values(tmp_path):
    """Every integer metadata type widens to i64 (src/gguf.rs:116-146); f32,
    f64, bool-as-u8 and arrays of numbers are read past."""
    hp = [4, 10, 8, 2, 1, 6, 8, 2, 1, 2, 1]
    fmt = [(MF.T_U8, "<B"), (MF.T_I8, "<b"), (MF.T_U16, "<H"), (MF.T_I16, "<h"), (MF.T_U32, "<I"),
           (MF.T_I32, "<i"), (MF.T_BOOL, "<B"), (MF.T_U64, "<Q"), (MF.T_I64, "<q"), (MF.T_U32, "<I"),
           (MF.T_I16, "<h")]
    hkv = [MF.kv(k, t, struct.pack(f, v)) for k, v, (t, f) in zip(MF.HPARAM_KEYS, hp, fmt)]
    extra = [MF.kv("x.f32", MF.T_F32, struct.pack("<f", 1.5)), MF.kv("x.f64", MF.T_F64, struct.pack("<d", 2.5)),
             MF.kv("x.arr", MF.T_ARRAY, struct.pack("<IQ", MF.T_U16, 3) + struct.pack("<3H", 1, 2, 3)),
             MF.kv("x.nest", MF.T_ARRAY, struct.pack("<IQ", MF.T_ARRAY, 1) + struct.pack("<IQ", MF.T_F32, 2) +
                   struct.pack("<2f", 0, 1)),
             MF.kv("x.str", MF.T_STRING, MF._s(b"whisper-ish"))]
    m = load(tmp_path, MF.gguf_bytes(hp, tokens=[b"a"], extra_kv=extra, hparam_kv=hkv), "m.gguf")
    assert list(m.hparams.values()) == hp
    assert m.vocab() == [b"a", b"[_extra_token_1]", b"[_extra_token_2]", b"[_extra_token_3]"]
    # i16 sign-extends, u8 does not
    hkv[10] = MF.kv(MF.HPARAM_KEYS[10], MF.T_I16, struct.pack("<h", -3))
    hkv[0] = MF.kv(MF.HPARAM_KEYS[0], MF.T_U8, struct.pack("<B", 200))
    m = load(tmp_path, MF.gguf_bytes(hp, hparam_kv=hkv), "m.gguf")
    assert m.hparams["ftype"] == -3 and m.hparams["n_vocab"] == 200


@pytest.mark.parametrize("alignment", [32, 64, 1, 7])
def test_gguf_alignment(tmp_path, alignment):
    w = f32b(np.arange(5))
    raw = O.quantize(2, np.linspace(-1, 1, 64, dtype=np.float32)).tobytes()
    data = MF.gguf_bytes([4, 10, 8, 2, 1, 6, 8, 2, 1, 2, 1], tensors=[("a", 0, [5], w), ("q", 2, [2, 32], raw)],
                         alignment=alignment)
    m = load(tmp_path, data, "m.gguf")
    np.testing.assert_array_equal(m.dense("a"), np.arange(5, dtype=np.float32))
    assert m.raw("q") == raw and m.tensor("q") == (2, (2, 32), True)


@pytest.mark.parametrize("case,msg", [
    ("version1", "gguf: unsupported version 1"),
    ("version4", "gguf: unsupported version 4"),
    ("missing_key", "gguf: missing metadata key whisper.n_text_layer"),
    ("unknown_type", "gguf: unknown metadata type 13"),
    ("unsupported_type", "gguf: tensor 'q': unsupported type 5"),
    ("out_of_bounds", "gguf: tensor 'q' out of bounds"),
    ("truncated_kv", "gguf: truncated file"),
    ("truncated_counts", "gguf: truncated file"),
])
def test_gguf_errors(tmp_path, case, msg):
    hp = [4, 10, 8, 2, 1, 6, 8, 2, 1, 2, 1]
    raw = bytes(36)
    good = MF.gguf_bytes(hp, tensors=[("q", 2, [2, 32], raw)])
    hkv = [MF.kv_i32(k, v) for k, v in zip(MF.HPARAM_KEYS, hp)]
    data = {
        "version1": MF.gguf_bytes(hp, version=1),
        "version4": MF.gguf_bytes(hp, version=4),
        "missing_key": MF.gguf_bytes(hp, hparam_kv=hkv[:8] + hkv[9:]),
        "unknown_type": MF.gguf_bytes(hp, extra_kv=[MF.kv("x", 13, b"\0" * 8)]),
        "unsupported_type": MF.gguf_bytes(hp, tensors=[("q", 5, [2, 32], raw)]),
        "out_of_bounds": good[:-1],
        "truncated_kv": good[:60],
        "truncated_counts": good[:12],
    }[case]
    e = load_err(tmp_path, data)
    assert e.code == A.RW_EINVAL and msg in e.message, e.message


def test_gguf_without_mel_tensor_has_empty_filters(tmp_path):
    m = load(tmp_path, MF.gguf_bytes([4, 10, 8, 2, 1, 6, 8, 2, 1, 2, 1]), "m.gguf")
    assert m.mel_filters().size == 0 and m.names() == []
