// safetensors.cpp -- C entry points of include/ullm/weights_io.h.
//
// Files are read with pread (no mapping is kept across calls), validated
// completely at open (header JSON, dtypes, shapes, offsets tiling the data
// region), and optionally hashed with SHA-256 against the digest a model lock
// records (reference docs/models/model-lock.md: "reject ... missing file, or
// content mismatch").  Weights are built through ullm_linear_weight_create
// from host buffers, so a loaded weight is indistinguishable from one
// uploaded or quantized directly.  Saving exports canonical encodings through
// ullm_linear_weight_export and writes them to a temporary file that is
// renamed into place.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstring>
#include <memory>
#include <mutex>
#include <set>
#include <string>
#include <unordered_set>
#include <vector>

#include "abi_common.hpp"
#include "json_lite.hpp"
#include "sha256.hpp"
#include "ullm/weights_io.h"

struct ullm_safetensors_t {
  struct Tensor {
    uint32_t dtype = 0;
    std::vector<uint64_t> shape;
    uint64_t begin = 0, end = 0;  // relative to the data region
  };
  std::string path;
  int fd = -1;
  uint64_t size = 0;
  uint64_t data_start = 0;
  std::map<std::string, Tensor> tensors;
  std::vector<std::string> names;  // sorted (byte order)
  std::map<std::string, std::string> metadata;
  mutable std::mutex hash_mutex;
  mutable bool hashed = false;
  mutable uint8_t sha[32] = {0};
  ~ullm_safetensors_t() {
    if (fd >= 0) {
      ::close(fd);
    }
  }
};

namespace {

using ullm::write_error;
using ullm::write_errorf;

constexpr uint64_t kMaxHeader = uint64_t(100) << 20;  // as the format's readers cap it

std::mutex g_files_mutex;
std::unordered_set<const ullm_safetensors_t *> g_files;

bool live(const ullm_safetensors_t *f) {
  std::lock_guard<std::mutex> lock(g_files_mutex);
  return g_files.count(f) != 0;
}

ullm_status_t lookup_file(const ullm_safetensors_t *f, ullm_error_sink_t *sink) {
  if (f == nullptr) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT, "safetensors handle is null");
  }
  if (!live(f)) {
    return write_error(sink, ULLM_STATUS_HIP_INVALID_HANDLE,
                       "safetensors handle is not live");
  }
  return ULLM_STATUS_OK;
}

struct DtypeName {
  const char *name;
  uint32_t id;
  uint32_t bytes;
};
constexpr DtypeName kDtypes[] = {
    {"BOOL", ULLM_ST_DTYPE_BOOL, 1},       {"U8", ULLM_ST_DTYPE_U8, 1},
    {"I8", ULLM_ST_DTYPE_I8, 1},           {"F8_E4M3", ULLM_ST_DTYPE_F8_E4M3, 1},
    {"F8_E5M2", ULLM_ST_DTYPE_F8_E5M2, 1}, {"U16", ULLM_ST_DTYPE_U16, 2},
    {"I16", ULLM_ST_DTYPE_I16, 2},         {"F16", ULLM_ST_DTYPE_F16, 2},
    {"BF16", ULLM_ST_DTYPE_BF16, 2},       {"U32", ULLM_ST_DTYPE_U32, 4},
    {"I32", ULLM_ST_DTYPE_I32, 4},         {"F32", ULLM_ST_DTYPE_F32, 4},
    {"U64", ULLM_ST_DTYPE_U64, 8},         {"I64", ULLM_ST_DTYPE_I64, 8},
    {"F64", ULLM_ST_DTYPE_F64, 8},
};

const DtypeName *dtype_by_name(const std::string &s) {
  for (const auto &d : kDtypes) {
    if (s == d.name) {
      return &d;
    }
  }
  return nullptr;
}

// Whole-buffer pread (retries short reads).
bool read_at(int fd, void *dst, uint64_t bytes, uint64_t offset) {
  char *p = static_cast<char *>(dst);
  while (bytes != 0) {
    const ssize_t r = ::pread(fd, p, bytes < (uint64_t(1) << 30) ? bytes : (uint64_t(1) << 30),
                              static_cast<off_t>(offset));
    if (r < 0 && errno == EINTR) {
      continue;
    }
    if (r <= 0) {
      return false;
    }
    p += r;
    bytes -= uint64_t(r);
    offset += uint64_t(r);
  }
  return true;
}

bool hash_file(int fd, uint64_t size, uint8_t out[32]) {
  ullm::Sha256 h;
  std::vector<char> buf(uint64_t(16) << 20);
  for (uint64_t off = 0; off < size;) {
    const uint64_t n = std::min<uint64_t>(buf.size(), size - off);
    if (!read_at(fd, buf.data(), n, off)) {
      return false;
    }
    h.update(buf.data(), n);
    off += n;
  }
  h.finish(out);
  return true;
}

// Header validation; throws std::runtime_error with the reason.
void parse_header(ullm_safetensors_t &f, const std::string &text) {
  ullm::json::Parser parser(text.data(), text.size());
  const ullm::json::Value root = parser.parse_document();
  if (root.kind != ullm::json::Value::kObject) {
    throw std::runtime_error("header is not a JSON object");
  }
  const uint64_t data_bytes = f.size - f.data_start;
  std::vector<std::pair<uint64_t, uint64_t>> spans;
  for (const auto &kv : root.o) {
    if (kv.first == "__metadata__") {
      if (kv.second.kind != ullm::json::Value::kObject) {
        throw std::runtime_error("__metadata__ is not an object");
      }
      for (const auto &m : kv.second.o) {
        if (m.second.kind != ullm::json::Value::kString) {
          throw std::runtime_error("__metadata__ value of '" + m.first +
                                   "' is not a string");
        }
        f.metadata[m.first] = m.second.s;
      }
      continue;
    }
    const ullm::json::Value &t = kv.second;
    if (t.kind != ullm::json::Value::kObject) {
      throw std::runtime_error("tensor '" + kv.first + "' is not an object");
    }
    const auto dt = t.o.find("dtype");
    const auto sh = t.o.find("shape");
    const auto of = t.o.find("data_offsets");
    if (dt == t.o.end() || sh == t.o.end() || of == t.o.end() || t.o.size() != 3) {
      throw std::runtime_error("tensor '" + kv.first +
                               "' needs exactly dtype, shape and data_offsets");
    }
    if (dt->second.kind != ullm::json::Value::kString) {
      throw std::runtime_error("tensor '" + kv.first + "': dtype is not a string");
    }
    const DtypeName *d = dtype_by_name(dt->second.s);
    if (d == nullptr) {
      throw std::runtime_error("tensor '" + kv.first + "': unknown dtype " + dt->second.s);
    }
    ullm_safetensors_t::Tensor rec;
    rec.dtype = d->id;
    if (sh->second.kind != ullm::json::Value::kArray ||
        sh->second.a.size() > ULLM_ST_MAX_RANK) {
      throw std::runtime_error("tensor '" + kv.first + "': bad shape");
    }
    uint64_t elems = 1;
    for (const auto &dim : sh->second.a) {
      if (dim.kind != ullm::json::Value::kInt || dim.negative) {
        throw std::runtime_error("tensor '" + kv.first + "': bad shape entry");
      }
      if (dim.u != 0 && elems > UINT64_MAX / dim.u) {
        throw std::runtime_error("tensor '" + kv.first + "': shape overflows");
      }
      elems *= dim.u;
      rec.shape.push_back(dim.u);
    }
    if (of->second.kind != ullm::json::Value::kArray || of->second.a.size() != 2 ||
        of->second.a[0].kind != ullm::json::Value::kInt ||
        of->second.a[1].kind != ullm::json::Value::kInt ||
        of->second.a[0].negative || of->second.a[1].negative) {
      throw std::runtime_error("tensor '" + kv.first + "': bad data_offsets");
    }
    rec.begin = of->second.a[0].u;
    rec.end = of->second.a[1].u;
    if (rec.begin > rec.end || rec.end > data_bytes) {
      throw std::runtime_error("tensor '" + kv.first + "': data_offsets out of range");
    }
    if (elems > UINT64_MAX / d->bytes || rec.end - rec.begin != elems * d->bytes) {
      throw std::runtime_error("tensor '" + kv.first +
                               "': byte range does not match dtype and shape");
    }
    spans.emplace_back(rec.begin, rec.end);
    f.tensors.emplace(kv.first, std::move(rec));
    f.names.push_back(kv.first);
  }
  // The tensors tile the data region: sorted by start, each starts where the
  // previous ended, the last ends at the end of the file.
  std::sort(spans.begin(), spans.end());
  uint64_t at = 0;
  for (const auto &s : spans) {
    if (s.first != at) {
      throw std::runtime_error("tensor data regions overlap or leave a gap");
    }
    at = s.second;
  }
  if (at != data_bytes) {
    throw std::runtime_error("tensor data does not end at the end of the file");
  }
  std::sort(f.names.begin(), f.names.end());
}

ullm_status_t copy_string(const std::string &s, char *out, uint64_t capacity,
                          uint64_t *length, ullm_error_sink_t *sink) {
  if (length != nullptr) {
    *length = s.size();
  }
  if (capacity == 0) {
    return s.empty() ? ULLM_STATUS_OK : ULLM_STATUS_BUFFER_TOO_SMALL;
  }
  if (out == nullptr) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT, "output buffer is null");
  }
  const uint64_t n = std::min<uint64_t>(s.size(), capacity - 1);
  std::memcpy(out, s.data(), n);
  out[n] = '\0';
  return n == s.size() ? ULLM_STATUS_OK
                       : write_error(sink, ULLM_STATUS_BUFFER_TOO_SMALL,
                                     "output buffer is too small");
}

// f16 bits -> f32 (IEEE binary16, subnormals and specials kept).
float f16_to_f32_host(uint16_t h) {
  const uint32_t sign = uint32_t(h >> 15) << 31;
  const uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0x1f) {
    bits = sign | 0x7f800000u | (man << 13);
  } else if (exp != 0) {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  } else if (man == 0) {
    bits = sign;
  } else {  // subnormal: normalise
    uint32_t e = 113;
    while ((man & 0x400u) == 0) {
      man <<= 1;
      --e;
    }
    bits = sign | (e << 23) | ((man & 0x3ffu) << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

const ullm_safetensors_t::Tensor *find_tensor(const ullm_safetensors_t *f,
                                               const char *name,
                                               ullm_error_sink_t *sink,
                                               ullm_status_t *st) {
  if (name == nullptr) {
    *st = write_error(sink, ULLM_STATUS_INVALID_ARGUMENT, "tensor name is null");
    return nullptr;
  }
  const auto it = f->tensors.find(name);
  if (it == f->tensors.end()) {
    *st = write_errorf(sink, ULLM_STATUS_INVALID_ARGUMENT,
                       std::string("no tensor named '") + name + "'");
    return nullptr;
  }
  *st = ULLM_STATUS_OK;
  return &it->second;
}

ullm_status_t read_tensor(const ullm_safetensors_t *f,
                          const ullm_safetensors_t::Tensor &t, void *dst,
                          ullm_error_sink_t *sink) {
  if (!read_at(f->fd, dst, t.end - t.begin, f->data_start + t.begin)) {
    return write_errorf(sink, ULLM_STATUS_INVALID_ARGUMENT,
                        "read failed: " + f->path + ": " + std::strerror(errno));
  }
  return ULLM_STATUS_OK;
}

ullm_status_t load_weight(const ullm_linear_weight_load_desc_t *d,
                          ullm_linear_weight_t **out, ullm_error_sink_t *sink) {
  const ullm_safetensors_t *f = d->file;
  if (d->values == nullptr || d->value_parts == 0) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT, "no value tensors named");
  }
  ullm_status_t st;
  const ullm_safetensors_t::Tensor *first = find_tensor(f, d->values[0], sink, &st);
  if (first == nullptr) {
    return st;
  }
  ullm_linear_weight_desc_t wd{};
  wd.struct_size = sizeof(wd);
  wd.abi_version = ULLM_HIP_ABI_VERSION;
  wd.encoding = d->encoding;
  wd.layout = d->layout;
  wd.memory = ULLM_MEMORY_HOST;
  wd.device = d->device;
  wd.stream = d->stream;
  const uint32_t vt = first->dtype;
  const bool float_src = vt == ULLM_ST_DTYPE_F32 || vt == ULLM_ST_DTYPE_BF16 ||
                         vt == ULLM_ST_DTYPE_F16;
  std::vector<float> wf;
  std::vector<uint8_t> vbytes, sbytes, zbytes;
  std::vector<float> row_scales;
  if (float_src) {
    if (d->scales != nullptr || d->zeros != nullptr) {
      return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "float weights take no scales or zeros");
    }
    uint64_t n = 0, k = 0;
    std::vector<const ullm_safetensors_t::Tensor *> parts;
    for (uint32_t i = 0; i < d->value_parts; ++i) {
      const ullm_safetensors_t::Tensor *t = find_tensor(f, d->values[i], sink, &st);
      if (t == nullptr) {
        return st;
      }
      if (t->dtype != vt || t->shape.size() != 2) {
        return write_errorf(sink, ULLM_STATUS_INVALID_ARGUMENT,
                            std::string("tensor '") + d->values[i] +
                                "' must be a 2-D tensor of the first part's dtype");
      }
      if (i == 0) {
        k = t->shape[1];
      } else if (t->shape[1] != k) {
        return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                           "stacked parts disagree on K");
      }
      n += t->shape[0];
      parts.push_back(t);
    }
    if (n == 0 || k == 0) {
      return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT, "empty weight");
    }
    wf.resize(n * k);
    uint64_t row = 0;
    std::vector<uint8_t> raw;
    for (const auto *t : parts) {
      const uint64_t cnt = t->shape[0] * k;
      float *dst = wf.data() + row * k;
      if (vt == ULLM_ST_DTYPE_F32) {
        st = read_tensor(f, *t, dst, sink);
      } else {
        raw.resize(cnt * 2);
        st = read_tensor(f, *t, raw.data(), sink);
        const uint16_t *h = reinterpret_cast<const uint16_t *>(raw.data());
        for (uint64_t i = 0; st == ULLM_STATUS_OK && i < cnt; ++i) {
          if (vt == ULLM_ST_DTYPE_BF16) {
            const uint32_t bits = uint32_t(h[i]) << 16;
            std::memcpy(dst + i, &bits, 4);
          } else {
            dst[i] = f16_to_f32_host(h[i]);
          }
        }
      }
      if (st != ULLM_STATUS_OK) {
        return st;
      }
      row += t->shape[0];
    }
    wd.source = ULLM_LINEAR_SOURCE_F32;
    wd.n = n;
    wd.k = k;
    wd.values = wf.data();
  } else {
    if (d->value_parts != 1) {
      return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "encoded weights are loaded from one tensor");
    }
    const ullm_safetensors_t::Tensor *sc = find_tensor(f, d->scales, sink, &st);
    if (sc == nullptr) {
      return st;
    }
    if (first->shape.size() != 2) {
      return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "encoded values must be 2-D");
    }
    wd.source = ULLM_LINEAR_SOURCE_ENCODED;
    wd.n = first->shape[0];
    if (d->encoding == ULLM_LINEAR_ENCODING_FP8_E4M3_ROW) {
      if (vt != ULLM_ST_DTYPE_F8_E4M3 || sc->dtype != ULLM_ST_DTYPE_F32) {
        return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                           "FP8 weights need F8_E4M3 values and F32 scales");
      }
      if (d->zeros != nullptr) {
        return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT, "FP8 weights take no zeros");
      }
      wd.k = first->shape[1];
      uint64_t scount = 1;
      for (const uint64_t s : sc->shape) {
        scount *= s;
      }
      const bool per_row = (sc->shape.size() == 1 && sc->shape[0] == wd.n) ||
                           (sc->shape.size() == 2 && sc->shape[0] == wd.n &&
                            sc->shape[1] == 1);
      const bool per_tensor = scount == 1;
      if (!per_row && !per_tensor) {
        return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                           "FP8 scales must have shape [N], [N, 1], [] or [1]");
      }
      vbytes.resize(wd.n * wd.k);
      row_scales.resize(wd.n);
      st = read_tensor(f, *first, vbytes.data(), sink);
      if (st == ULLM_STATUS_OK) {
        st = read_tensor(f, *sc, row_scales.data(), sink);
      }
      if (st != ULLM_STATUS_OK) {
        return st;
      }
      if (per_tensor && wd.n > 1 && !per_row) {
        std::fill(row_scales.begin() + 1, row_scales.end(), row_scales[0]);
      }
      wd.values = vbytes.data();
      wd.scales = row_scales.data();
    } else if (d->encoding == ULLM_LINEAR_ENCODING_AQ4_G128) {
      const ullm_safetensors_t::Tensor *zr = find_tensor(f, d->zeros, sink, &st);
      if (zr == nullptr) {
        return st;
      }
      wd.k = first->shape[1] * 8;
      const uint64_t groups = wd.k / 128;
      if (vt != ULLM_ST_DTYPE_U32 || sc->dtype != ULLM_ST_DTYPE_F16 ||
          zr->dtype != ULLM_ST_DTYPE_F16) {
        return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                           "AQ4 weights need U32 values and F16 scales and zeros");
      }
      const std::vector<uint64_t> gshape = {wd.n, groups};
      if (sc->shape != gshape || zr->shape != gshape) {
        return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                           "AQ4 scales and zeros must have shape [N, K/128]");
      }
      vbytes.resize(first->end - first->begin);
      sbytes.resize(sc->end - sc->begin);
      zbytes.resize(zr->end - zr->begin);
      st = read_tensor(f, *first, vbytes.data(), sink);
      if (st == ULLM_STATUS_OK) {
        st = read_tensor(f, *sc, sbytes.data(), sink);
      }
      if (st == ULLM_STATUS_OK) {
        st = read_tensor(f, *zr, zbytes.data(), sink);
      }
      if (st != ULLM_STATUS_OK) {
        return st;
      }
      wd.values = vbytes.data();
      wd.scales = sbytes.data();
      wd.zeros = zbytes.data();
    } else {
      return write_error(sink, ULLM_STATUS_UNSUPPORTED, "unknown weight encoding");
    }
  }
  return ullm_linear_weight_create(&wd, out, sink);
}

struct OutTensor {
  std::string name;
  const char *dtype;
  std::vector<uint64_t> shape;
  std::vector<uint8_t> bytes;
};

std::string header_json(const std::vector<OutTensor> &ts,
                        const std::vector<std::pair<std::string, std::string>> &meta) {
  std::string h = "{\"__metadata__\":{";
  for (std::size_t i = 0; i < meta.size(); ++i) {
    h += (i ? "," : "") + ullm::json::quote(meta[i].first) + ":" +
         ullm::json::quote(meta[i].second);
  }
  h += "}";
  uint64_t at = 0;
  for (const auto &t : ts) {
    h += "," + ullm::json::quote(t.name) + ":{\"dtype\":\"" + t.dtype + "\",\"shape\":[";
    for (std::size_t i = 0; i < t.shape.size(); ++i) {
      h += (i ? "," : "") + std::to_string(t.shape[i]);
    }
    h += "],\"data_offsets\":[" + std::to_string(at) + "," +
         std::to_string(at + t.bytes.size()) + "]}";
    at += t.bytes.size();
  }
  h += "}";
  while (h.size() % 8 != 0) {  // data region 8-byte aligned, as writers pad it
    h += ' ';
  }
  return h;
}

ullm_status_t save_weights(const ullm_linear_weights_save_desc_t *d, uint8_t *sha256,
                           ullm_error_sink_t *sink) {
  if (d->path == nullptr || d->count == 0 || d->names == nullptr ||
      d->weights == nullptr) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                       "path, names and weights are required");
  }
  if (d->metadata_count != 0 &&
      (d->metadata_keys == nullptr || d->metadata_values == nullptr)) {
    return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT, "metadata arrays are null");
  }
  std::vector<OutTensor> ts;
  std::vector<std::pair<std::string, std::string>> meta = {{"format", "ullm-linear"}};
  std::set<std::string> seen;
  for (uint64_t i = 0; i < d->count; ++i) {
    if (d->names[i] == nullptr || d->names[i][0] == '\0' ||
        !seen.insert(d->names[i]).second) {
      return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "weight names must be non-empty and unique");
    }
    const std::string name = d->names[i];
    ullm_linear_weight_info_t info{};
    info.struct_size = sizeof(info);
    info.abi_version = ULLM_HIP_ABI_VERSION;
    ullm_status_t st = ullm_linear_weight_query(d->weights[i], &info, sink);
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    const bool fp8 = info.encoding == ULLM_LINEAR_ENCODING_FP8_E4M3_ROW;
    const uint64_t n = info.n, k = info.k;
    ullm_linear_weight_export_desc_t ex{};
    ex.struct_size = sizeof(ex);
    ex.abi_version = ULLM_HIP_ABI_VERSION;
    ex.memory = ULLM_MEMORY_HOST;
    if (fp8) {
      OutTensor v{name + ".weight", "F8_E4M3", {n, k}, std::vector<uint8_t>(n * k)};
      OutTensor s{name + ".weight_scale", "F32", {n}, std::vector<uint8_t>(n * 4)};
      ex.values = v.bytes.data();
      ex.scales = s.bytes.data();
      st = ullm_linear_weight_export(d->weights[i], &ex, sink);
      ts.push_back(std::move(v));
      ts.push_back(std::move(s));
    } else {
      const uint64_t g = k / 128;
      OutTensor v{name + ".qweight", "U32", {n, k / 8}, std::vector<uint8_t>(n * k / 2)};
      OutTensor s{name + ".scales", "F16", {n, g}, std::vector<uint8_t>(n * g * 2)};
      OutTensor z{name + ".zeros", "F16", {n, g}, std::vector<uint8_t>(n * g * 2)};
      ex.values = v.bytes.data();
      ex.scales = s.bytes.data();
      ex.zeros = z.bytes.data();
      st = ullm_linear_weight_export(d->weights[i], &ex, sink);
      ts.push_back(std::move(v));
      ts.push_back(std::move(s));
      ts.push_back(std::move(z));
    }
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    meta.emplace_back(name + ".encoding", fp8 ? "fp8_e4m3_row" : "aq4_g128");
    meta.emplace_back(name + ".layout",
                      info.layout == ULLM_LINEAR_LAYOUT_GATED_PAIRS ? "gated_pairs" : "plain");
  }
  std::set<std::string> keys;
  for (const auto &m : meta) {
    keys.insert(m.first);
  }
  for (uint64_t i = 0; i < d->metadata_count; ++i) {
    if (d->metadata_keys[i] == nullptr || d->metadata_values[i] == nullptr ||
        !keys.insert(d->metadata_keys[i]).second) {
      return write_error(sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "metadata keys must be non-null, unique and not reserved");
    }
    meta.emplace_back(d->metadata_keys[i], d->metadata_values[i]);
  }
  // Tensor names may not collide across weights either ("a.weight" from "a"
  // and a weight literally named "a.weight" would).
  std::set<std::string> tnames;
  for (const auto &t : ts) {
    if (!tnames.insert(t.name).second || t.name == "__metadata__") {
      return write_errorf(sink, ULLM_STATUS_INVALID_ARGUMENT,
                          "tensor name '" + t.name + "' would repeat");
    }
  }
  const std::string header = header_json(ts, meta);
  const std::string tmp = std::string(d->path) + ".tmp";
  const int fd = ::open(tmp.c_str(), O_WRONLY | O_CREAT | O_TRUNC, 0644);
  if (fd < 0) {
    return write_errorf(sink, ULLM_STATUS_INVALID_ARGUMENT,
                        "cannot create " + tmp + ": " + std::strerror(errno));
  }
  ullm::Sha256 h;
  bool ok = true;
  auto put = [&](const void *p, uint64_t n) {
    h.update(p, n);
    const char *c = static_cast<const char *>(p);
    while (ok && n != 0) {
      const ssize_t w = ::write(fd, c, n < (uint64_t(1) << 30) ? n : (uint64_t(1) << 30));
      if (w < 0 && errno == EINTR) {
        continue;
      }
      if (w <= 0) {
        ok = false;
        break;
      }
      c += w;
      n -= uint64_t(w);
    }
  };
  uint8_t len[8];
  for (int i = 0; i < 8; ++i) {
    len[i] = static_cast<uint8_t>(uint64_t(header.size()) >> (8 * i));
  }
  put(len, 8);
  put(header.data(), header.size());
  for (const auto &t : ts) {
    put(t.bytes.data(), t.bytes.size());
  }
  ok = (::fsync(fd) == 0) && ok;
  ok = (::close(fd) == 0) && ok;
  if (!ok || ::rename(tmp.c_str(), d->path) != 0) {
    ::unlink(tmp.c_str());
    return write_errorf(sink, ULLM_STATUS_INVALID_ARGUMENT,
                        std::string("writing ") + d->path + " failed: " +
                            std::strerror(errno));
  }
  uint8_t digest[32];
  h.finish(digest);
  if (sha256 != nullptr) {
    std::memcpy(sha256, digest, 32);
  }
  return ULLM_STATUS_OK;
}

}  // namespace

extern "C" ULLM_HIP_API ullm_status_t ullm_safetensors_open(
    const ullm_safetensors_open_desc_t *desc, ullm_safetensors_t **file,
    ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "safetensors open", {
    ullm_status_t st = ullm::validate_header(desc, error_sink, "open descriptor is null");
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    if (!ullm::all_zero(desc->reserved)) {
      return write_error(error_sink, ULLM_STATUS_RESERVED_NONZERO,
                         "open descriptor reserved fields must be zero");
    }
    if (file == nullptr || desc->path == nullptr) {
      return write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "path or handle output is null");
    }
    *file = nullptr;
    auto f = std::make_unique<ullm_safetensors_t>();
    f->path = desc->path;
    f->fd = ::open(desc->path, O_RDONLY | O_CLOEXEC);
    if (f->fd < 0) {
      return write_errorf(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                          "cannot open " + f->path + ": " + std::strerror(errno));
    }
    struct stat sb;
    if (::fstat(f->fd, &sb) != 0 || !S_ISREG(sb.st_mode)) {
      return write_errorf(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                          f->path + " is not a regular file");
    }
    f->size = uint64_t(sb.st_size);
    if (desc->expected_size != 0 && desc->expected_size != f->size) {
      return write_errorf(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                          f->path + ": size " + std::to_string(f->size) +
                              " does not match the expected " +
                              std::to_string(desc->expected_size));
    }
    if (desc->expected_sha256 != nullptr) {
      if (!hash_file(f->fd, f->size, f->sha)) {
        return write_errorf(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                            "read failed: " + f->path);
      }
      f->hashed = true;
      if (std::memcmp(f->sha, desc->expected_sha256, 32) != 0) {
        return write_errorf(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                            f->path + ": SHA-256 does not match the expected digest");
      }
    }
    uint8_t len[8];
    if (f->size < 8 || !read_at(f->fd, len, 8, 0)) {
      return write_errorf(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                          f->path + ": shorter than the 8-byte header length");
    }
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; --i) {
      hlen = (hlen << 8) | len[i];
    }
    if (hlen == 0 || hlen > kMaxHeader || hlen > f->size - 8) {
      return write_errorf(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                          f->path + ": header length " + std::to_string(hlen) +
                              " is out of range");
    }
    std::string text(hlen, '\0');
    if (!read_at(f->fd, &text[0], hlen, 8)) {
      return write_errorf(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                          "read failed: " + f->path);
    }
    if (text[0] != '{') {
      return write_errorf(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                          f->path + ": header does not start with '{'");
    }
    f->data_start = 8 + hlen;
    try {
      parse_header(*f, text);
    } catch (const std::runtime_error &e) {
      return write_errorf(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                          f->path + ": " + e.what());
    }
    {
      std::lock_guard<std::mutex> lock(g_files_mutex);
      g_files.insert(f.get());
    }
    *file = f.release();
    return ULLM_STATUS_OK;
  });
}

extern "C" ULLM_HIP_API ullm_status_t ullm_safetensors_close(
    ullm_safetensors_t **file, ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "safetensors close", {
    if (file == nullptr || *file == nullptr) {
      return write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "safetensors handle is null");
    }
    {
      std::lock_guard<std::mutex> lock(g_files_mutex);
      if (g_files.erase(*file) == 0) {
        return write_error(error_sink, ULLM_STATUS_HIP_INVALID_HANDLE,
                           "safetensors handle is not live");
      }
    }
    delete *file;
    *file = nullptr;
    return ULLM_STATUS_OK;
  });
}

extern "C" ULLM_HIP_API ullm_status_t ullm_safetensors_tensor_count(
    const ullm_safetensors_t *file, uint64_t *count, ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "safetensors tensor count", {
    const ullm_status_t st = lookup_file(file, error_sink);
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    if (count == nullptr) {
      return write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT, "count output is null");
    }
    *count = file->names.size();
    return ULLM_STATUS_OK;
  });
}

extern "C" ULLM_HIP_API ullm_status_t ullm_safetensors_tensor_name(
    const ullm_safetensors_t *file, uint64_t index, char *name, uint64_t capacity,
    uint64_t *length, ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "safetensors tensor name", {
    const ullm_status_t st = lookup_file(file, error_sink);
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    if (index >= file->names.size()) {
      return write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "tensor index out of range");
    }
    return copy_string(file->names[index], name, capacity, length, error_sink);
  });
}

extern "C" ULLM_HIP_API ullm_status_t ullm_safetensors_tensor_info(
    const ullm_safetensors_t *file, const char *name,
    ullm_safetensors_tensor_info_t *info, ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "safetensors tensor info", {
    ullm_status_t st = lookup_file(file, error_sink);
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    st = ullm::validate_header(info, error_sink, "tensor info output is null");
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    if (!ullm::all_zero(info->reserved)) {
      return write_error(error_sink, ULLM_STATUS_RESERVED_NONZERO,
                         "tensor info reserved fields must be zero");
    }
    const ullm_safetensors_t::Tensor *t = find_tensor(file, name, error_sink, &st);
    if (t == nullptr) {
      return st;
    }
    info->dtype = t->dtype;
    info->rank = static_cast<uint32_t>(t->shape.size());
    for (uint32_t i = 0; i < ULLM_ST_MAX_RANK; ++i) {
      info->shape[i] = i < t->shape.size() ? t->shape[i] : 0;
    }
    info->offset = file->data_start + t->begin;
    info->bytes = t->end - t->begin;
    return ULLM_STATUS_OK;
  });
}

extern "C" ULLM_HIP_API ullm_status_t ullm_safetensors_metadata(
    const ullm_safetensors_t *file, const char *key, char *value, uint64_t capacity,
    uint64_t *length, ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "safetensors metadata", {
    const ullm_status_t st = lookup_file(file, error_sink);
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    if (key == nullptr) {
      return write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT, "metadata key is null");
    }
    const auto it = file->metadata.find(key);
    if (it == file->metadata.end()) {
      return write_errorf(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                          std::string("no metadata key '") + key + "'");
    }
    return copy_string(it->second, value, capacity, length, error_sink);
  });
}

extern "C" ULLM_HIP_API ullm_status_t ullm_safetensors_file_sha256(
    const ullm_safetensors_t *file, uint8_t sha256[32], ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "safetensors sha256", {
    const ullm_status_t st = lookup_file(file, error_sink);
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    if (sha256 == nullptr) {
      return write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT, "digest output is null");
    }
    std::lock_guard<std::mutex> lock(file->hash_mutex);
    if (!file->hashed) {
      if (!hash_file(file->fd, file->size, file->sha)) {
        return write_errorf(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                            "read failed: " + file->path);
      }
      file->hashed = true;
    }
    std::memcpy(sha256, file->sha, 32);
    return ULLM_STATUS_OK;
  });
}

extern "C" ULLM_HIP_API ullm_status_t ullm_linear_weight_load(
    const ullm_linear_weight_load_desc_t *desc, ullm_linear_weight_t **weight,
    ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "weight load", {
    ullm_status_t st = ullm::validate_header(desc, error_sink, "load descriptor is null");
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    if (!ullm::all_zero(desc->reserved)) {
      return write_error(error_sink, ULLM_STATUS_RESERVED_NONZERO,
                         "load descriptor reserved fields must be zero");
    }
    if (weight == nullptr) {
      return write_error(error_sink, ULLM_STATUS_INVALID_ARGUMENT,
                         "weight output pointer is null");
    }
    *weight = nullptr;
    st = lookup_file(desc->file, error_sink);
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    return load_weight(desc, weight, error_sink);
  });
}

extern "C" ULLM_HIP_API ullm_status_t ullm_linear_weights_save(
    const ullm_linear_weights_save_desc_t *desc, uint8_t *sha256,
    ullm_error_sink_t *error_sink) {
  ULLM_ENTRY(error_sink, "weights save", {
    const ullm_status_t st =
        ullm::validate_header(desc, error_sink, "save descriptor is null");
    if (st != ULLM_STATUS_OK) {
      return st;
    }
    if (!ullm::all_zero(desc->reserved)) {
      return write_error(error_sink, ULLM_STATUS_RESERVED_NONZERO,
                         "save descriptor reserved fields must be zero");
    }
    return save_weights(desc, sha256, error_sink);
  });
}
