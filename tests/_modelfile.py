"""Writers for small whisper model files, used to feed the loader in tests.

ggml_bytes() lays out the legacy container the way the reference reads it
(src/model.rs:145-275): magic, 11 i32 hparams, n_mel/n_fft + f32 filters,
token count + (len, bytes) tokens, then tensors as (n_dims, name_len, dtype,
ggml dims innermost-first, name, data) until the end of the file.

gguf_bytes() writes GGUF v3 with the reference's metadata mapping
(src/gguf.rs:1-22, 306-440): general.architecture, general.alignment, the 11
whisper.* hparams as i32, tokenizer.ggml.tokens; the mel filterbank as an f32
tensor "whisper.mel_filters"; tensor data at aligned offsets.
"""
from __future__ import annotations

import struct

import numpy as np

GGML_MAGIC = 0x67676D6C
GGUF_MAGIC = 0x46554747

HPARAM_KEYS = ("whisper.n_vocab", "whisper.n_audio_ctx", "whisper.n_audio_state", "whisper.n_audio_head",
               "whisper.n_audio_layer", "whisper.n_text_ctx", "whisper.n_text_state", "whisper.n_text_head",
               "whisper.n_text_layer", "whisper.n_mels", "whisper.ftype")

# GGUF metadata value types
T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STRING, T_ARRAY, T_U64, T_I64, T_F64 = range(13)


def i32(v: int) -> bytes:
    return struct.pack("<i", v)


def ggml_tensor(name: str, dtype: int, dims: list[int], data: bytes) -> bytes:
    """One tensor record; dims innermost-first as ggml stores them."""
    nm = name.encode()
    return i32(len(dims)) + i32(len(nm)) + i32(dtype) + b"".join(i32(d) for d in dims) + nm + data


def ggml_bytes(hparams, mel=None, tokens=(), tensors=(), n_tokens=None) -> bytes:
    """mel: 2-D float array (or None for 0 x 0); tensors: (name, dtype, dims, data)."""
    out = [i32(GGML_MAGIC), *(i32(v) for v in hparams)]
    mel = np.zeros((0, 0), np.float32) if mel is None else np.asarray(mel, np.float32)
    out += [i32(mel.shape[0]), i32(mel.shape[1]), mel.astype("<f4").tobytes()]
    out.append(i32(len(tokens) if n_tokens is None else n_tokens))
    for t in tokens:
        out += [i32(len(t)), bytes(t)]
    out += [ggml_tensor(*t) for t in tensors]
    return b"".join(out)


def _s(b: bytes) -> bytes:
    return struct.pack("<Q", len(b)) + b


def kv(key: str, t: int, payload: bytes) -> bytes:
    return _s(key.encode()) + struct.pack("<I", t) + payload


def kv_i32(key: str, v: int) -> bytes:
    return kv(key, T_I32, struct.pack("<i", v))


def gguf_bytes(hparams, mel=None, tokens=(), tensors=(), arch=b"whisper", alignment=32, version=3,
               extra_kv=(), hparam_kv=None) -> bytes:
    """tensors: (name, dtype, row-major shape, data bytes) in file order.

    extra_kv: extra serialized pairs placed before the hparams; hparam_kv
    replaces the i32 hparam pairs (to write other integer widths)."""
    kvs = [kv("general.architecture", T_STRING, _s(arch)),
           kv("general.alignment", T_U32, struct.pack("<I", alignment)), *extra_kv]
    kvs += list(hparam_kv) if hparam_kv is not None else [kv_i32(k, v) for k, v in zip(HPARAM_KEYS, hparams)]
    kvs.append(kv("tokenizer.ggml.tokens", T_ARRAY,
                  struct.pack("<IQ", T_STRING, len(tokens)) + b"".join(_s(bytes(t)) for t in tokens)))
    descs = []
    if mel is not None:
        mel = np.asarray(mel, np.float32)
        descs.append(("whisper.mel_filters", 0, list(mel.shape), mel.astype("<f4").tobytes()))
    descs += list(tensors)
    hdr, blobs, off = [], [], 0
    for name, dtype, shape, data in descs:
        hdr.append(_s(name.encode()) + struct.pack("<I", len(shape)) +
                   b"".join(struct.pack("<Q", d) for d in reversed(shape)) + struct.pack("<IQ", dtype, off))
        blobs.append((off, data))
        off = (off + len(data) + alignment - 1) // alignment * alignment
    head = (struct.pack("<IIQQ", GGUF_MAGIC, version, len(descs), len(kvs)) + b"".join(kvs) + b"".join(hdr))
    head += b"\0" * (-len(head) % alignment)
    body = bytearray(max((o + len(d) for o, d in blobs), default=0))  # no padding after the last tensor
    for o, data in blobs:
        body[o:o + len(data)] = data
    return head + bytes(body)
