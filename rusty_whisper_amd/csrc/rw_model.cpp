// rw_model.cpp -- whisper model files straight to resident weights.
//
// Reads the two containers the reference loads (src/model.rs:145-275, the
// legacy ggml ".bin"; src/gguf.rs:156-300, GGUF) from a read-only memory map
// and uploads every 2-D block-quantized matrix to the device through
// rw_rocm_weight_upload, from the mapped bytes, with no host copy of the
// blocks.  Everything else (biases, layernorms, convolutions, f16/f32
// matrices, quantized tensors of other ranks) becomes host f32 exactly as the
// reference's Weight::Dense: f16 through the exact bit conversion of
// model.rs:68-86, quantized through x = d*q + m (dequant_row_scalar,
// src/quant.rs:528-537).  Shapes are flipped to row-major as the reference
// does.  Failures carry the reference's messages; the reference returns them
// as io::Error, this library as RW_EINVAL (malformed file) or RW_EIO (file
// not readable) with the text in rw_rocm_last_error.
//
// Host code only: parsing needs no device (RW_MODEL_PARSE_ONLY skips the
// uploads and keeps every quantized tensor as its mapped blocks).
#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "rw_rocm.h"

int rw_internal_fail(int code, const char *msg);  // rw_rocm.hip: the thread's error text

namespace {

constexpr uint32_t GGML_MAGIC = 0x67676d6cu;  // src/model.rs:22
constexpr uint32_t GGUF_MAGIC = 0x46554747u;  // src/gguf.rs:33 ("GGUF")
constexpr size_t QK = 32;
constexpr size_t N_HPARAMS = 11;

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  return rw_internal_fail(code, buf);
}

// src/quant.rs:43-52 (the dtypes with a block layout)
long block_bytes(int dtype) {
  switch (dtype) {
    case 2: return 18;
    case 3: return 20;
    case 6: return 22;
    case 7: return 24;
    case 8: return 34;
    default: return -1;
  }
}

// IEEE half -> single, the bit rules of src/model.rs:68-86 (NaN payload
// kept as frac << 13)
float f16_to_f32(uint16_t h) {
  const uint32_t sign = h >> 15, exp = (h >> 10) & 0x1f, frac = h & 0x3ff;
  uint32_t bits;
  if (exp == 0 && frac == 0) {
    bits = sign << 31;
  } else if (exp == 0) {
    const uint32_t p = 31u - (uint32_t)__builtin_clz(frac);
    bits = (sign << 31) | ((p + 103u) << 23) | (((frac << (10u - p)) & 0x3ffu) << 13);
  } else if (exp == 0x1f) {
    bits = (sign << 31) | 0x7f800000u | (frac << 13);
  } else {
    bits = (sign << 31) | ((exp + 112u) << 23) | (frac << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
uint32_t rd32(const uint8_t *p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
uint64_t rd64(const uint8_t *p) { return (uint64_t)rd32(p) | ((uint64_t)rd32(p + 4) << 32); }

// One block of a quantized tensor to f32: x = d*q + m with q the centered
// int (src/quant.rs:98-131, 528-537); two roundings, as the reference.
void dequant_block(int dtype, const uint8_t *b, float *out) {
  const float d = f16_to_f32(rd16(b));
  float m = 0.0f;
  const uint8_t *qs;
  uint32_t qh = 0;
  switch (dtype) {
    case 2: qs = b + 2; break;
    case 3: m = f16_to_f32(rd16(b + 2)); qs = b + 4; break;
    case 6: qh = rd32(b + 2); qs = b + 6; break;
    case 7: m = f16_to_f32(rd16(b + 2)); qh = rd32(b + 4); qs = b + 8; break;
    default: qs = b + 2; break;
  }
  for (size_t j = 0; j < QK; ++j) {
    int q;
    if (dtype == 8) {
      q = (int8_t)qs[j];
    } else {
      q = j < 16 ? (qs[j] & 0xf) : (qs[j - 16] >> 4);
      if (dtype == 6 || dtype == 7) q |= (int)((qh >> j) & 1u) << 4;
      if (dtype == 2) q -= 8;
      if (dtype == 6) q -= 16;
    }
    out[j] = d * (float)q + m;  // two roundings: the library is built without fp contraction
  }
}

}  // namespace

struct rw_model {
  int32_t hp[N_HPARAMS] = {};
  std::vector<float> mel;
  size_t n_mel = 0, n_fft = 0;
  std::vector<std::string> vocab;
  struct Tensor {
    std::string name;
    int dtype = 0;
    int ndims = 0;
    size_t shape[3] = {1, 1, 1};  // row-major, ndims entries
    const uint8_t *raw = nullptr;  // the tensor's bytes in the map
    size_t raw_len = 0;
    rw_weight *w = nullptr;        // 2-D block-quantized, uploaded
    std::vector<float> dense;      // everything else
    bool quant2d = false;
  };
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, size_t> by_name;
  void *map = nullptr;
  size_t map_len = 0;

  ~rw_model() {
    for (Tensor &t : tensors)
      if (t.w) rw_rocm_weight_free(t.w);
    if (map) munmap(map, map_len);
  }
};

namespace {

// A tensor's data -> its Weight: 2-D block-quantized stays in blocks (and is
// uploaded unless parse_only), the rest becomes dense f32.
int finish_tensor(rw_model::Tensor &t, size_t n_elems, bool parse_only) {
  if (t.dtype == 0) {
    t.dense.resize(n_elems);
    memcpy(t.dense.data(), t.raw, n_elems * 4);
  } else if (t.dtype == 1) {
    t.dense.resize(n_elems);
    for (size_t i = 0; i < n_elems; ++i) t.dense[i] = f16_to_f32(rd16(t.raw + 2 * i));
  } else if (t.ndims == 2) {
    t.quant2d = true;
    if (!parse_only) {
      int rc = rw_rocm_weight_upload(t.dtype, t.shape[0], t.shape[1], t.raw, t.raw_len, &t.w);
      if (rc) {
        char inner[384];
        rw_rocm_last_error(inner, sizeof inner);
        return fail(rc, "tensor '%s': %s", t.name.c_str(), inner);
      }
    }
  } else {
    const size_t bb = (size_t)block_bytes(t.dtype);
    const size_t nbk = t.raw_len / bb;
    t.dense.resize(nbk * QK);
    for (size_t b = 0; b < nbk; ++b) dequant_block(t.dtype, t.raw + b * bb, t.dense.data() + b * QK);
  }
  return RW_OK;
}

int add_tensor(rw_model *M, rw_model::Tensor &&t) {
  if (M->by_name.count(t.name)) {
    // the reference's HashMap::insert keeps the last one
    rw_model::Tensor &old = M->tensors[M->by_name[t.name]];
    if (old.w) rw_rocm_weight_free(old.w);
    old = std::move(t);
    return RW_OK;
  }
  M->by_name[t.name] = M->tensors.size();
  M->tensors.push_back(std::move(t));
  return RW_OK;
}

// Legacy ggml container, src/model.rs:145-275.  `p` is past the magic.
int load_ggml(rw_model *M, const uint8_t *buf, size_t len, size_t p, bool parse_only) {
  auto need = [&](size_t n) { return n <= len - p; };  // p <= len always
  auto i32 = [&](int32_t &v) {
    if (!need(4)) return false;
    v = (int32_t)rd32(buf + p);
    p += 4;
    return true;
  };
  for (size_t i = 0; i < N_HPARAMS; ++i)
    if (!i32(M->hp[i])) return fail(RW_EINVAL, "failed to fill whole buffer");
  int32_t n_mel, n_fft;
  if (!i32(n_mel) || !i32(n_fft)) return fail(RW_EINVAL, "failed to fill whole buffer");
  const size_t nf = (size_t)(uint32_t)n_mel * (size_t)(uint32_t)n_fft;
  if (nf > len / 4 || !need(nf * 4)) return fail(RW_EINVAL, "failed to fill whole buffer");
  M->n_mel = (size_t)(uint32_t)n_mel;
  M->n_fft = (size_t)(uint32_t)n_fft;
  M->mel.resize(nf);
  memcpy(M->mel.data(), buf + p, nf * 4);
  p += nf * 4;
  int32_t n_tokens;
  if (!i32(n_tokens)) return fail(RW_EINVAL, "failed to fill whole buffer");
  for (int32_t i = 0; i < n_tokens; ++i) {
    int32_t l;
    if (!i32(l) || !need((size_t)(uint32_t)l)) return fail(RW_EINVAL, "failed to fill whole buffer");
    M->vocab.emplace_back((const char *)buf + p, (size_t)(uint32_t)l);
    p += (size_t)(uint32_t)l;
  }
  for (int32_t i = n_tokens; i < M->hp[0]; ++i) M->vocab.push_back("[_extra_token_" + std::to_string(i) + "]");

  // tensors until the end of the file (fewer than 4 bytes left ends the list)
  while (need(4)) {
    int32_t n_dims, name_len, dtype;
    i32(n_dims);
    if (!i32(name_len) || !i32(dtype)) return fail(RW_EINVAL, "failed to fill whole buffer");
    if (n_dims < 0 || n_dims > 3) return fail(RW_EINVAL, "tensor with %d dimensions (at most 3)", n_dims);
    size_t dims[3] = {1, 1, 1};
    for (int d = 0; d < n_dims; ++d) {
      int32_t v;
      if (!i32(v)) return fail(RW_EINVAL, "failed to fill whole buffer");
      dims[d] = (size_t)(uint32_t)v;
    }
    if (!need((size_t)(uint32_t)name_len)) return fail(RW_EINVAL, "failed to fill whole buffer");
    rw_model::Tensor t;
    t.name.assign((const char *)buf + p, (size_t)(uint32_t)name_len);
    p += (size_t)(uint32_t)name_len;
    t.dtype = dtype;
    t.ndims = n_dims > 0 ? n_dims : 1;
    // ggml dims are innermost-first; row-major flips them
    for (int d = 0; d < t.ndims; ++d) t.shape[d] = dims[t.ndims - 1 - d];
    size_t n_elems, nbytes;
    if (__builtin_mul_overflow(dims[0], dims[1], &n_elems) || __builtin_mul_overflow(n_elems, dims[2], &n_elems) ||
        n_elems > len)
      return fail(RW_EINVAL, "failed to fill whole buffer");
    if (dtype == 0) {
      nbytes = n_elems * 4;
    } else if (dtype == 1) {
      nbytes = n_elems * 2;
    } else {
      const long bb = block_bytes(dtype);
      if (bb < 0) return fail(RW_EINVAL, "tensor '%s': unsupported dtype %d", t.name.c_str(), dtype);
      if (n_elems % QK)
        return fail(RW_EINVAL, "tensor '%s': %zu elements not divisible by block size", t.name.c_str(), n_elems);
      nbytes = n_elems / QK * (size_t)bb;
    }
    if (!need(nbytes)) return fail(RW_EINVAL, "failed to fill whole buffer");
    t.raw = buf + p;
    t.raw_len = nbytes;
    p += nbytes;
    int rc = finish_tensor(t, n_elems, parse_only);
    if (rc) return rc;
    add_tensor(M, std::move(t));
  }
  return RW_OK;
}

// GGUF, src/gguf.rs:156-300 (version 2 or 3; the reference's metadata
// mapping).  `p` is past the magic.
int load_gguf(rw_model *M, const uint8_t *buf, size_t len, size_t p, bool parse_only) {
  bool trunc = false;
  auto take = [&](size_t n) -> const uint8_t * {
    if (trunc || n > len - p) {
      trunc = true;
      return nullptr;
    }
    const uint8_t *r = buf + p;
    p += n;
    return r;
  };
  auto u32 = [&]() -> uint32_t {
    const uint8_t *r = take(4);
    return r ? rd32(r) : 0;
  };
  auto u64 = [&]() -> uint64_t {
    const uint8_t *r = take(8);
    return r ? rd64(r) : 0;
  };
  auto str = [&]() -> std::string {
    const uint64_t l = u64();
    const uint8_t *r = trunc ? nullptr : take((size_t)l);
    return r ? std::string((const char *)r, (size_t)l) : std::string();
  };
  const char *TRUNC = "gguf: truncated file";
  const uint32_t version = u32();
  if (trunc) return fail(RW_EINVAL, "%s", TRUNC);
  if (version < 2 || version > 3) return fail(RW_EINVAL, "gguf: unsupported version %u", version);
  const uint64_t n_tensors = u64(), n_kv = u64();
  if (trunc) return fail(RW_EINVAL, "%s", TRUNC);

  static const char *KEYS[N_HPARAMS] = {"whisper.n_vocab",      "whisper.n_audio_ctx",  "whisper.n_audio_state",
                                        "whisper.n_audio_head", "whisper.n_audio_layer", "whisper.n_text_ctx",
                                        "whisper.n_text_state", "whisper.n_text_head",  "whisper.n_text_layer",
                                        "whisper.n_mels",       "whisper.ftype"};
  std::unordered_map<std::string, int64_t> ints;
  std::vector<std::string> tokens;
  size_t alignment = 32;
  // one metadata value of type t: integers (with the reference's widening
  // rules) or strings kept, the rest skipped
  struct Val {
    int kind = 0;  // 0 other, 1 integer, 2 strings
    int64_t i = 0;
    std::vector<std::string> s;
  };
  int bad_type = -1;
  auto value = [&](auto &&self, uint32_t t) -> Val {
    Val v;
    const uint8_t *r;
    switch (t) {
      case 0:
      case 1:
      case 7:
        if ((r = take(1))) v.kind = 1, v.i = r[0];
        break;
      case 2:
      case 3:
        if ((r = take(2))) v.kind = 1, v.i = (int16_t)rd16(r);
        break;
      case 4:
        if ((r = take(4))) v.kind = 1, v.i = (int64_t)rd32(r);
        break;
      case 5:
        if ((r = take(4))) v.kind = 1, v.i = (int32_t)rd32(r);
        break;
      case 6:
        take(4);
        break;
      case 8:
        v.kind = 2;
        v.s.push_back(str());
        break;
      case 9: {
        const uint32_t et = u32();
        const uint64_t n = u64();
        if (et == 8) {
          v.kind = 2;
          for (uint64_t k = 0; k < n && !trunc; ++k) v.s.push_back(str());
        } else {
          for (uint64_t k = 0; k < n && !trunc && bad_type < 0; ++k) self(self, et);
        }
        break;
      }
      case 10:
      case 11:
        if ((r = take(8))) v.kind = 1, v.i = (int64_t)rd64(r);
        break;
      case 12:
        take(8);
        break;
      default:
        if (bad_type < 0) bad_type = (int)t;
    }
    return v;
  };
  for (uint64_t k = 0; k < n_kv; ++k) {
    const std::string key = str();
    const uint32_t t = u32();
    if (trunc) return fail(RW_EINVAL, "%s", TRUNC);
    Val v = value(value, t);
    if (bad_type >= 0) return fail(RW_EINVAL, "gguf: unknown metadata type %d", bad_type);
    if (trunc) return fail(RW_EINVAL, "%s", TRUNC);
    if (v.kind == 1) {
      if (key == "general.alignment") alignment = (size_t)v.i;
      ints[key] = v.i;
    } else if (v.kind == 2) {
      if (key == "tokenizer.ggml.tokens") {
        tokens = std::move(v.s);
      } else if (key == "general.architecture" && (v.s.empty() || v.s[0] != "whisper")) {
        return fail(RW_EINVAL, "gguf: general.architecture is not \"whisper\"");
      }
    }
  }
  for (size_t i = 0; i < N_HPARAMS; ++i) {
    auto it = ints.find(KEYS[i]);
    if (it == ints.end()) return fail(RW_EINVAL, "gguf: missing metadata key %s", KEYS[i]);
    M->hp[i] = (int32_t)it->second;
  }
  if (alignment == 0) return fail(RW_EINVAL, "gguf: alignment 0");

  struct Info {
    std::string name;
    std::vector<size_t> shape;
    int dtype;
    uint64_t offset;
  };
  std::vector<Info> infos;
  for (uint64_t k = 0; k < n_tensors; ++k) {
    Info in;
    in.name = str();
    const uint32_t nd = u32();
    if (trunc) return fail(RW_EINVAL, "%s", TRUNC);
    if (nd > 3) return fail(RW_EINVAL, "gguf: tensor '%s' has %u dimensions (at most 3)", in.name.c_str(), nd);
    for (uint32_t d = 0; d < nd; ++d) in.shape.push_back((size_t)u64());
    in.dtype = (int)u32();
    in.offset = u64();
    if (trunc) return fail(RW_EINVAL, "%s", TRUNC);
    // dims fastest-varying first; row-major flips them
    std::vector<size_t> rev(in.shape.rbegin(), in.shape.rend());
    in.shape = rev;
    infos.push_back(std::move(in));
  }
  const size_t data_start = (p + alignment - 1) / alignment * alignment;

  M->vocab = std::move(tokens);
  for (int32_t i = (int32_t)M->vocab.size(); i < M->hp[0]; ++i)
    M->vocab.push_back("[_extra_token_" + std::to_string(i) + "]");

  for (Info &in : infos) {
    size_t n_elems = 1;
    for (size_t d : in.shape)
      if (__builtin_mul_overflow(n_elems, d, &n_elems) || n_elems > len)
        return fail(RW_EINVAL, "gguf: tensor '%s' out of bounds", in.name.c_str());
    size_t nbytes;
    if (in.dtype == 0) {
      nbytes = n_elems * 4;
    } else if (in.dtype == 1) {
      nbytes = n_elems * 2;
    } else {
      const long bb = block_bytes(in.dtype);
      if (bb < 0) return fail(RW_EINVAL, "gguf: tensor '%s': unsupported type %d", in.name.c_str(), in.dtype);
      nbytes = n_elems / QK * (size_t)bb;
    }
    if (in.offset > len || data_start > len - in.offset || nbytes > len - data_start - in.offset)
      return fail(RW_EINVAL, "gguf: tensor '%s' out of bounds", in.name.c_str());
    rw_model::Tensor t;
    t.name = in.name;
    t.dtype = in.dtype;
    t.ndims = in.shape.empty() ? 1 : (int)in.shape.size();
    for (size_t d = 0; d < in.shape.size(); ++d) t.shape[d] = in.shape[d];
    t.raw = buf + data_start + in.offset;
    t.raw_len = nbytes;
    int rc = finish_tensor(t, n_elems, parse_only);
    if (rc) return rc;
    if (t.name == "whisper.mel_filters") {
      M->mel = t.dense;
      M->n_mel = t.ndims == 2 ? t.shape[0] : 1;
      M->n_fft = t.ndims == 2 ? t.shape[1] : t.dense.size();
      if (t.w) rw_rocm_weight_free(t.w);
    } else {
      add_tensor(M, std::move(t));
    }
  }
  return RW_OK;
}

const rw_model::Tensor *find(const rw_model *m, const char *name) {
  if (!m || !name) return nullptr;
  auto it = m->by_name.find(name);
  return it == m->by_name.end() ? nullptr : &m->tensors[it->second];
}

}  // namespace

extern "C" {

int rw_rocm_model_load(const char *path, int flags, rw_model **out) {
  if (!out) return fail(RW_EINVAL, "out is NULL");
  *out = nullptr;
  if (!path) return fail(RW_EINVAL, "path is NULL");
  const int fd = open(path, O_RDONLY);
  if (fd < 0) return fail(RW_EIO, "%s: %s", path, strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0) {
    const int e = errno;
    close(fd);
    return fail(RW_EIO, "%s: %s", path, strerror(e));
  }
  const size_t len = (size_t)st.st_size;
  void *map = nullptr;
  if (len > 0) {
    map = mmap(nullptr, len, PROT_READ, MAP_PRIVATE, fd, 0);
    if (map == MAP_FAILED) {
      const int e = errno;
      close(fd);
      return fail(RW_EIO, "%s: mmap: %s", path, strerror(e));
    }
  }
  close(fd);
  rw_model *M = new rw_model();
  M->map = map;
  M->map_len = len;
  const uint8_t *buf = (const uint8_t *)map;
  const bool parse_only = (flags & RW_MODEL_PARSE_ONLY) != 0;
  int rc;
  if (len < 4) {
    rc = fail(RW_EINVAL, "failed to fill whole buffer");
  } else {
    const uint32_t magic = rd32(buf);
    if (magic == GGUF_MAGIC) rc = load_gguf(M, buf, len, 4, parse_only);
    else if (magic == GGML_MAGIC) rc = load_ggml(M, buf, len, 4, parse_only);
    else rc = fail(RW_EINVAL, "bad magic %#x, expected 'ggml' (%#x)", magic, GGML_MAGIC);
  }
  if (rc) {
    delete M;
    return rc;
  }
  *out = M;
  return RW_OK;
}

void rw_rocm_model_free(rw_model *m) { delete m; }

int rw_rocm_model_hparams(const rw_model *m, int32_t *hp) {
  if (!m || !hp) return fail(RW_EINVAL, "model or hparams is NULL");
  memcpy(hp, m->hp, sizeof m->hp);
  return RW_OK;
}

int rw_rocm_model_mel_filters(const rw_model *m, const float **data, size_t *n_mel, size_t *n_fft) {
  if (!m) return fail(RW_EINVAL, "model is NULL");
  if (data) *data = m->mel.data();
  if (n_mel) *n_mel = m->n_mel;
  if (n_fft) *n_fft = m->n_fft;
  return RW_OK;
}

int rw_rocm_model_vocab_size(const rw_model *m, size_t *n) {
  if (!m || !n) return fail(RW_EINVAL, "model or n is NULL");
  *n = m->vocab.size();
  return RW_OK;
}

int rw_rocm_model_token(const rw_model *m, size_t id, const uint8_t **bytes, size_t *len) {
  if (!m || !bytes || !len) return fail(RW_EINVAL, "model, bytes or len is NULL");
  if (id >= m->vocab.size()) return fail(RW_EINVAL, "token id %zu out of range (%zu tokens)", id, m->vocab.size());
  *bytes = (const uint8_t *)m->vocab[id].data();
  *len = m->vocab[id].size();
  return RW_OK;
}

int rw_rocm_model_tensor_count(const rw_model *m, size_t *n) {
  if (!m || !n) return fail(RW_EINVAL, "model or n is NULL");
  *n = m->tensors.size();
  return RW_OK;
}

int rw_rocm_model_tensor_name(const rw_model *m, size_t i, const char **name) {
  if (!m || !name) return fail(RW_EINVAL, "model or name is NULL");
  if (i >= m->tensors.size()) return fail(RW_EINVAL, "tensor index %zu out of range", i);
  *name = m->tensors[i].name.c_str();
  return RW_OK;
}

int rw_rocm_model_tensor(const rw_model *m, const char *name, int *dtype, int *ndims, size_t *shape) {
  const rw_model::Tensor *t = find(m, name);
  if (!t) return fail(RW_EINVAL, "no tensor '%s'", name ? name : "(null)");
  if (dtype) *dtype = t->dtype;
  if (ndims) *ndims = t->ndims;
  if (shape)
    for (int d = 0; d < 3; ++d) shape[d] = d < t->ndims ? t->shape[d] : 1;
  return t->quant2d ? 1 : 0;
}

int rw_rocm_model_weight(const rw_model *m, const char *name, const rw_weight **w) {
  const rw_model::Tensor *t = find(m, name);
  if (!t || !w) return fail(RW_EINVAL, "no tensor '%s'", name ? name : "(null)");
  if (!t->quant2d) return fail(RW_EINVAL, "tensor '%s' is dense, not a quantized matrix", name);
  if (!t->w) return fail(RW_EINVAL, "tensor '%s' was not uploaded (parse-only load)", name);
  *w = t->w;
  return RW_OK;
}

int rw_rocm_model_dense(const rw_model *m, const char *name, const float **data, size_t *len) {
  const rw_model::Tensor *t = find(m, name);
  if (!t || !data || !len) return fail(RW_EINVAL, "no tensor '%s'", name ? name : "(null)");
  if (t->quant2d) return fail(RW_EINVAL, "tensor '%s' is a quantized matrix, not dense", name);
  *data = t->dense.data();
  *len = t->dense.size();
  return RW_OK;
}

int rw_rocm_model_raw(const rw_model *m, const char *name, const uint8_t **raw, size_t *len) {
  const rw_model::Tensor *t = find(m, name);
  if (!t || !raw || !len) return fail(RW_EINVAL, "no tensor '%s'", name ? name : "(null)");
  *raw = t->raw;
  *len = t->raw_len;
  return RW_OK;
}

}  // extern "C"
