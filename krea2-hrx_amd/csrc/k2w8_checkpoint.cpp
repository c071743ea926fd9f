// Checkpoint upload for the W8A8 path: a memory-mapped .safetensors reader
// (src/checkpoint/file.rs), the device layout of the ConvRot block weights
// (src/checkpoint/plan.rs:88-264) and the upload that fills one device allocation
// from it (src/session/weights.rs:48-100).
//
// Host code only. The layout is the reference's, so the GEMM kernels consume the
// uploaded operands unchanged: qkvg = wq | wk | wv | attn.gate rows, gu = mlp.gate and
// mlp.up interleaved 16 rows at a time (the SwiGLU epilogue's pairing), wo and down as
// they are; every operand at the GEMM pitch of its K, scales gathered in row order,
// spans 256-byte aligned in name order.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "krea2_w8a8.h"

// The C ABI's error channel (k2w8_api.cpp).
int k2w8_fail_invalid(const char *message);
int k2w8_fail_runtime(const char *stage, hipError_t e);
int k2w8_succeed();

namespace {

std::string format(const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  return buf;
}

struct Error {
  std::string message;
};

// ---- safetensors header ---------------------------------------------------------

struct Entry {
  int dtype = K2W8_DTYPE_OTHER;
  std::vector<int64_t> shape;
  uint64_t begin = 0, end = 0;  // byte range within the data section
};

int dtype_code(const std::string &s) {
  if (s == "I8") return K2W8_DTYPE_I8;
  if (s == "F32") return K2W8_DTYPE_F32;
  if (s == "BF16") return K2W8_DTYPE_BF16;
  if (s == "F16") return K2W8_DTYPE_F16;
  if (s == "U8") return K2W8_DTYPE_U8;
  if (s == "I32") return K2W8_DTYPE_I32;
  return K2W8_DTYPE_OTHER;
}

int64_t dtype_bytes(const std::string &s) {
  if (s == "BOOL" || s == "U8" || s == "I8" || s == "F8_E4M3" || s == "F8_E5M2") return 1;
  if (s == "F16" || s == "BF16" || s == "I16" || s == "U16") return 2;
  if (s == "F32" || s == "I32" || s == "U32") return 4;
  if (s == "F64" || s == "I64" || s == "U64") return 8;
  return 0;
}

// A minimal JSON reader for the header: one object of objects, with strings, integer
// arrays and (in __metadata__) string values; anything else is rejected.
class Json {
 public:
  Json(const char *p, size_t n) : p_(p), end_(p + n) {}

  std::map<std::string, Entry> header() {
    std::map<std::string, Entry> out;
    expect('{');
    if (peek() == '}') {
      ++p_;
      return out;
    }
    for (;;) {
      std::string name = string();
      expect(':');
      if (name == "__metadata__") {
        skip_string_map();
      } else {
        if (out.count(name)) fail("duplicate tensor " + name);
        out[name] = entry(name);
      }
      if (peek() == ',') {
        ++p_;
        continue;
      }
      expect('}');
      break;
    }
    ws();
    if (p_ != end_) fail("trailing bytes after the header object");
    return out;
  }

 private:
  [[noreturn]] void fail(const std::string &what) { throw Error{"invalid header: " + what}; }

  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) ++p_;
  }
  char peek() {
    ws();
    if (p_ >= end_) fail("unexpected end");
    return *p_;
  }
  void expect(char c) {
    if (peek() != c) fail(std::string("expected '") + c + "'");
    ++p_;
  }

  std::string string() {
    expect('"');
    std::string s;
    while (p_ < end_ && *p_ != '"') {
      char c = *p_++;
      if (c == '\\') {
        if (p_ >= end_) fail("unterminated escape");
        char e = *p_++;
        switch (e) {
          case '"': s += '"'; break;
          case '\\': s += '\\'; break;
          case '/': s += '/'; break;
          case 'b': s += '\b'; break;
          case 'f': s += '\f'; break;
          case 'n': s += '\n'; break;
          case 'r': s += '\r'; break;
          case 't': s += '\t'; break;
          case 'u': {
            if (end_ - p_ < 4) fail("short \\u escape");
            unsigned v = 0;
            for (int i = 0; i < 4; ++i) {
              char h = *p_++;
              v <<= 4;
              if (h >= '0' && h <= '9') v |= h - '0';
              else if (h >= 'a' && h <= 'f') v |= h - 'a' + 10;
              else if (h >= 'A' && h <= 'F') v |= h - 'A' + 10;
              else fail("bad \\u escape");
            }
            // UTF-8 of a BMP code point (names are ASCII in practice).
            if (v < 0x80) {
              s += (char)v;
            } else if (v < 0x800) {
              s += (char)(0xC0 | (v >> 6));
              s += (char)(0x80 | (v & 0x3F));
            } else {
              s += (char)(0xE0 | (v >> 12));
              s += (char)(0x80 | ((v >> 6) & 0x3F));
              s += (char)(0x80 | (v & 0x3F));
            }
            break;
          }
          default: fail("bad escape");
        }
      } else {
        s += c;
      }
    }
    if (p_ >= end_) fail("unterminated string");
    ++p_;
    return s;
  }

  uint64_t integer() {
    ws();
    if (p_ >= end_ || *p_ < '0' || *p_ > '9') fail("expected a non-negative integer");
    uint64_t v = 0;
    while (p_ < end_ && *p_ >= '0' && *p_ <= '9') {
      const uint64_t d = (uint64_t)(*p_++ - '0');
      if (v > (UINT64_MAX - d) / 10) fail("integer overflow");
      v = v * 10 + d;
    }
    return v;
  }

  std::vector<uint64_t> integers() {
    std::vector<uint64_t> v;
    expect('[');
    if (peek() == ']') {
      ++p_;
      return v;
    }
    for (;;) {
      v.push_back(integer());
      if (peek() == ',') {
        ++p_;
        continue;
      }
      expect(']');
      return v;
    }
  }

  void skip_string_map() {
    expect('{');
    if (peek() == '}') {
      ++p_;
      return;
    }
    for (;;) {
      string();
      expect(':');
      string();
      if (peek() == ',') {
        ++p_;
        continue;
      }
      expect('}');
      return;
    }
  }

  Entry entry(const std::string &name) {
    Entry e;
    std::string dtype;
    bool have_dtype = false, have_shape = false, have_offsets = false;
    expect('{');
    for (;;) {
      std::string key = string();
      expect(':');
      if (key == "dtype") {
        dtype = string();
        have_dtype = true;
      } else if (key == "shape") {
        for (uint64_t d : integers()) {
          if (d > (uint64_t)INT64_MAX) fail("shape of " + name);
          e.shape.push_back((int64_t)d);
        }
        have_shape = true;
      } else if (key == "data_offsets") {
        std::vector<uint64_t> o = integers();
        if (o.size() != 2 || o[0] > o[1]) fail("data_offsets of " + name);
        e.begin = o[0];
        e.end = o[1];
        have_offsets = true;
      } else {
        fail("unknown key " + key + " in " + name);
      }
      if (peek() == ',') {
        ++p_;
        continue;
      }
      expect('}');
      break;
    }
    if (!have_dtype || !have_shape || !have_offsets) fail("incomplete entry " + name);
    e.dtype = dtype_code(dtype);
    const int64_t size = dtype_bytes(dtype);
    if (size == 0) fail("unknown dtype " + dtype + " of " + name);
    uint64_t elems = 1;
    for (int64_t d : e.shape) {
      if (d != 0 && elems > UINT64_MAX / (uint64_t)d) fail("shape of " + name);
      elems *= (uint64_t)d;
    }
    if (elems > UINT64_MAX / (uint64_t)size || elems * (uint64_t)size != e.end - e.begin)
      fail("byte size of " + name + " does not match its dtype and shape");
    return e;
  }

  const char *p_, *end_;
};

// A tensor every transformer checkpoint carries (file.rs:46).
const char *kAnchor = "blocks.0.attn.wq.weight";

// file.rs:53-63: strip the namespace a whole-model save wraps every tensor name in.
std::map<std::string, Entry> unwrap_model(std::map<std::string, Entry> entries) {
  const std::string anchor = kAnchor;
  std::string prefix;
  bool found = false;
  for (const auto &kv : entries) {
    const std::string &n = kv.first;
    if (n.size() >= anchor.size() && n.compare(n.size() - anchor.size(), anchor.size(), anchor) == 0) {
      prefix = n.substr(0, n.size() - anchor.size());
      found = true;
      break;
    }
  }
  if (!found || prefix.empty() || prefix.back() != '.') return entries;
  for (const auto &kv : entries)
    if (kv.first.compare(0, prefix.size(), prefix) != 0) return entries;
  std::map<std::string, Entry> out;
  for (auto &kv : entries) out[kv.first.substr(prefix.size())] = kv.second;
  return out;
}

}  // namespace

struct k2w8_checkpoint {
  std::string path;
  const uint8_t *map = nullptr;
  size_t size = 0;
  const uint8_t *data = nullptr;  // start of the data section
  size_t data_size = 0;
  std::map<std::string, Entry> entries;

  ~k2w8_checkpoint() {
    if (map) munmap(const_cast<uint8_t *>(map), size);
  }

  const Entry &get(const std::string &name) const {
    auto it = entries.find(name);
    if (it == entries.end()) throw Error{format("missing tensor %s in %s", name.c_str(), path.c_str())};
    return it->second;
  }
  bool has(const std::string &name) const { return entries.count(name) != 0; }
  const uint8_t *bytes(const Entry &e) const { return data + e.begin; }

  // file.rs:124-129
  int64_t block_count() const {
    int64_t i = 0;
    while (i < (int64_t)entries.size() && has(format("blocks.%lld.attn.wq.weight", (long long)i))) ++i;
    return i;
  }
};

namespace {

struct Segment {
  std::string tensor;
  int64_t first = 0, last = 0;  // rows [first, last)
};

struct Span {
  int64_t device_offset = 0, device_bytes = 0;
  int64_t rows = 0, row_bytes = 0, device_row_bytes = 0;
  std::vector<Segment> segments;
  std::vector<uint8_t> host;  // bytes assembled on the host (gathered scales, upcast vectors)
  int64_t file_bytes() const { return host.empty() ? rows * row_bytes : (int64_t)host.size(); }
};

// plan.rs:61-74
const Entry &int8_rows(const k2w8_checkpoint &file, const std::string &name) {
  const Entry &t = file.get(name + ".weight");
  if (t.dtype != K2W8_DTYPE_I8 || t.shape.size() != 2)
    throw Error{format("%s.weight is not int8 ConvRot rows (%s)", name.c_str(), file.path.c_str())};
  if (t.shape[0] == 0 || t.shape[1] == 0)
    throw Error{format("invalid weight shape or size in %s", name.c_str())};
  return t;
}

// plan.rs:76-85
const Entry &scales(const k2w8_checkpoint &file, const std::string &name, int64_t rows) {
  const Entry &t = file.get(name + ".weight_scale");
  if (t.dtype != K2W8_DTYPE_F32) throw Error{format("%s.weight_scale is not float32", name.c_str())};
  if ((int64_t)(t.end - t.begin) != rows * 4) throw Error{format("scale count in %s", name.c_str())};
  return t;
}

// plan.rs:154-230: one GEMM operand and its scales; group 0 concatenates the parts'
// rows, group g interleaves them g rows at a time.
void operand(const k2w8_checkpoint &file, const std::string &out, const std::vector<std::string> &parts,
             int64_t group, Span &weights, Span &scale_span) {
  std::vector<const Entry *> tensors;
  for (const auto &part : parts) tensors.push_back(&int8_rows(file, part));
  const int64_t row_bytes = tensors[0]->shape[1];
  int64_t rows = 0;
  for (const Entry *t : tensors) {
    if (t->shape[1] != row_bytes) throw Error{format("mismatched K in %s", out.c_str())};
    rows += t->shape[0];
  }
  const int64_t pitch = k2w8_shape_gemm_pitch(row_bytes);
  weights = Span{};
  weights.rows = rows;
  weights.row_bytes = row_bytes;
  weights.device_row_bytes = pitch;
  weights.device_bytes = rows * pitch;
  std::vector<uint8_t> scale_bytes((size_t)rows * 4);
  int64_t written = 0;
  if (group == 0) {
    for (size_t i = 0; i < parts.size(); ++i) {
      const int64_t count = tensors[i]->shape[0];
      weights.segments.push_back(Segment{parts[i] + ".weight", 0, count});
      const Entry &src = scales(file, parts[i], count);
      memcpy(scale_bytes.data() + written * 4, file.bytes(src), (size_t)count * 4);
      written += count;
    }
  } else {
    if (tensors.size() != 2 || tensors[0]->shape[0] != tensors[1]->shape[0] ||
        tensors[0]->shape[0] % group != 0)
      throw Error{format("interleave shape in %s", out.c_str())};
    const int64_t half = tensors[0]->shape[0];
    const Entry *src[2] = {&scales(file, parts[0], half), &scales(file, parts[1], half)};
    for (int64_t start = 0; start < half; start += group) {
      for (int p = 0; p < 2; ++p) {
        weights.segments.push_back(Segment{parts[p] + ".weight", start, start + group});
        memcpy(scale_bytes.data() + written * 4, file.bytes(*src[p]) + start * 4, (size_t)group * 4);
        written += group;
      }
    }
  }
  scale_span = Span{};
  scale_span.device_bytes = (int64_t)scale_bytes.size();
  scale_span.host = std::move(scale_bytes);
}

// plan.rs:233-264: an f32 vector as it is, or upcast exactly from bf16.
Span vector(const k2w8_checkpoint &file, const std::string &name) {
  const Entry &t = file.get(name);
  Span s;
  const int64_t nbytes = (int64_t)(t.end - t.begin);
  if (t.dtype == K2W8_DTYPE_BF16) {
    s.host.resize((size_t)nbytes * 2);
    const uint8_t *src = file.bytes(t);
    for (int64_t i = 0; i < nbytes / 2; ++i) {
      const uint32_t bits = (uint32_t)(src[2 * i] | (src[2 * i + 1] << 8)) << 16;
      memcpy(s.host.data() + 4 * i, &bits, 4);
    }
    s.device_bytes = (int64_t)s.host.size();
    return s;
  }
  if (t.dtype != K2W8_DTYPE_F32) throw Error{format("%s is not float32", name.c_str())};
  s.device_bytes = nbytes;
  s.rows = 1;
  s.row_bytes = nbytes;
  s.device_row_bytes = nbytes;
  s.segments.push_back(Segment{name, 0, 1});
  return s;
}

}  // namespace

struct k2w8_plan {
  std::map<std::string, Span> spans;
  std::vector<std::string> names;  // the spans' names in order
  int64_t total_bytes = 0;
  int64_t layers = 0;
};

namespace {

// plan.rs:88-143
std::unique_ptr<k2w8_plan> plan_for(const k2w8_checkpoint &file) {
  auto plan = std::make_unique<k2w8_plan>();
  const int64_t layers = file.block_count();
  if (layers == 0) throw Error{format("no transformer blocks in %s", file.path.c_str())};
  for (int64_t block = 0; block < layers; ++block) {
    const std::string p = format("blocks.%lld", (long long)block);
    Span q, s;
    operand(file, p + ".qkvg", {p + ".attn.wq", p + ".attn.wk", p + ".attn.wv", p + ".attn.gate"}, 0, q, s);
    plan->spans[p + ".qkvg.q"] = std::move(q);
    plan->spans[p + ".qkvg.s"] = std::move(s);
    const std::pair<const char *, std::string> single[2] = {{"wo", p + ".attn.wo"}, {"down", p + ".mlp.down"}};
    for (const auto &os : single) {
      operand(file, p + "." + os.first, {os.second}, 0, q, s);
      plan->spans[p + "." + os.first + ".q"] = std::move(q);
      plan->spans[p + "." + os.first + ".s"] = std::move(s);
    }
    operand(file, p + ".gu", {p + ".mlp.gate", p + ".mlp.up"}, 16, q, s);
    plan->spans[p + ".gu.q"] = std::move(q);
    plan->spans[p + ".gu.s"] = std::move(s);
    const std::pair<const char *, std::string> vectors[4] = {
        {"prenorm", p + ".prenorm.scale"},
        {"postnorm", p + ".postnorm.scale"},
        {"qnorm", p + ".attn.qknorm.qnorm.scale"},
        {"knorm", p + ".attn.qknorm.knorm.scale"}};
    for (const auto &v : vectors) plan->spans[p + "." + v.first] = vector(file, v.second);
  }
  // Spans start at 256-byte boundaries in name order.
  int64_t total = 0;
  for (auto &kv : plan->spans) {
    kv.second.device_offset = total;
    total += (kv.second.device_bytes + 255) / 256 * 256;
    plan->names.push_back(kv.first);
  }
  plan->total_bytes = total;
  plan->layers = layers;
  return plan;
}

}  // namespace

extern "C" {

int k2w8_checkpoint_open(const char *path, k2w8_checkpoint **out) {
  if (!path || !out) return k2w8_fail_invalid("checkpoint_open: null argument");
  *out = nullptr;
  const std::string p = path;
  if (p.size() < 12 || p.compare(p.size() - 12, 12, ".safetensors") != 0)
    return k2w8_fail_invalid(format("%s is not a ComfyUI checkpoint (.safetensors)", path).c_str());
  auto file = std::make_unique<k2w8_checkpoint>();
  file->path = p;
  try {
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) throw Error{format("cannot read %s: %s", path, strerror(errno))};
    struct stat st;
    if (fstat(fd, &st) != 0) {
      close(fd);
      throw Error{format("cannot read %s: %s", path, strerror(errno))};
    }
    file->size = (size_t)st.st_size;
    if (file->size < 8) {
      close(fd);
      throw Error{format("cannot read %s: shorter than a safetensors header", path)};
    }
    void *m = mmap(nullptr, file->size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) throw Error{format("cannot read %s: %s", path, strerror(errno))};
    file->map = static_cast<const uint8_t *>(m);
    uint64_t header_len = 0;
    for (int i = 0; i < 8; ++i) header_len |= (uint64_t)file->map[i] << (8 * i);
    if (header_len > file->size - 8)
      throw Error{format("cannot read %s: header longer than the file", path)};
    file->data = file->map + 8 + header_len;
    file->data_size = file->size - 8 - (size_t)header_len;
    std::map<std::string, Entry> entries;
    try {
      entries = Json(reinterpret_cast<const char *>(file->map + 8), (size_t)header_len).header();
    } catch (const Error &e) {
      throw Error{format("cannot read %s: %s", path, e.message.c_str())};
    }
    for (const auto &kv : entries)
      if (kv.second.end > file->data_size)
        throw Error{format("cannot read %s: tensor %s reaches past the data", path, kv.first.c_str())};
    file->entries = unwrap_model(std::move(entries));
  } catch (const Error &e) {
    return k2w8_fail_invalid(e.message.c_str());
  }
  *out = file.release();
  return k2w8_succeed();
}

void k2w8_checkpoint_close(k2w8_checkpoint *file) { delete file; }

int64_t k2w8_checkpoint_block_count(const k2w8_checkpoint *file) {
  return file ? file->block_count() : 0;
}

int k2w8_checkpoint_tensor(const k2w8_checkpoint *file, const char *name, k2w8_tensor *out) {
  if (!file || !name || !out) return k2w8_fail_invalid("checkpoint_tensor: null argument");
  try {
    const Entry &e = file->get(name);
    if (e.shape.size() > 8) throw Error{format("%s has more than 8 dimensions", name)};
    memset(out, 0, sizeof *out);
    out->dtype = e.dtype;
    out->ndim = (int32_t)e.shape.size();
    for (size_t i = 0; i < e.shape.size(); ++i) out->shape[i] = e.shape[i];
    out->data = file->bytes(e);
    out->nbytes = (int64_t)(e.end - e.begin);
  } catch (const Error &e) {
    return k2w8_fail_invalid(e.message.c_str());
  }
  return k2w8_succeed();
}

int k2w8_plan_for_checkpoint(const k2w8_checkpoint *file, k2w8_plan **out) {
  if (!file || !out) return k2w8_fail_invalid("plan_for_checkpoint: null argument");
  *out = nullptr;
  try {
    *out = plan_for(*file).release();
  } catch (const Error &e) {
    return k2w8_fail_invalid(e.message.c_str());
  }
  return k2w8_succeed();
}

void k2w8_plan_free(k2w8_plan *plan) { delete plan; }

int64_t k2w8_plan_total_bytes(const k2w8_plan *plan) { return plan ? plan->total_bytes : 0; }
int64_t k2w8_plan_layers(const k2w8_plan *plan) { return plan ? plan->layers : 0; }
int64_t k2w8_plan_span_count(const k2w8_plan *plan) { return plan ? (int64_t)plan->names.size() : 0; }

const char *k2w8_plan_span_name(const k2w8_plan *plan, int64_t index) {
  if (!plan || index < 0 || index >= (int64_t)plan->names.size()) return nullptr;
  return plan->names[(size_t)index].c_str();
}

int k2w8_plan_span(const k2w8_plan *plan, const char *name, k2w8_span *out) {
  if (!plan || !name || !out) return k2w8_fail_invalid("plan_span: null argument");
  auto it = plan->spans.find(name);
  if (it == plan->spans.end()) return k2w8_fail_invalid(format("no span named %s", name).c_str());
  const Span &s = it->second;
  out->device_offset = s.device_offset;
  out->device_bytes = s.device_bytes;
  out->rows = s.rows;
  out->row_bytes = s.row_bytes;
  out->device_row_bytes = s.device_row_bytes;
  out->file_bytes = s.file_bytes();
  out->segments = (int64_t)s.segments.size();
  return k2w8_succeed();
}

int k2w8_plan_upload(void *stream, const k2w8_plan *plan, const k2w8_checkpoint *file,
                     void *device, int64_t device_bytes) {
  const char *stage = "plan_upload";
  if (!plan || !file || !device) return k2w8_fail_invalid("plan_upload: null argument");
  if (device_bytes < plan->total_bytes)
    return k2w8_fail_invalid(format("plan_upload: the allocation holds %lld bytes, the plan needs %lld",
                                    (long long)device_bytes, (long long)plan->total_bytes).c_str());
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint8_t *base = static_cast<uint8_t *>(device);
  // Padding stays zero (weights.rs:3-6): clear the allocation, then place the rows.
  hipError_t e = hipMemsetAsync(base, 0, (size_t)plan->total_bytes, s);
  if (e != hipSuccess) return k2w8_fail_runtime(stage, e);
  try {
    for (const auto &kv : plan->spans) {
      const Span &span = kv.second;
      uint8_t *dst = base + span.device_offset;
      if (!span.host.empty()) {
        e = hipMemcpyAsync(dst, span.host.data(), span.host.size(), hipMemcpyHostToDevice, s);
        if (e != hipSuccess) return k2w8_fail_runtime(stage, e);
        continue;
      }
      const int64_t width = span.row_bytes;
      const int64_t pitch = span.device_row_bytes;
      int64_t row = 0;
      for (const Segment &seg : span.segments) {
        const Entry &t = file->get(seg.tensor);
        const int64_t rows = seg.last - seg.first;
        const uint8_t *src = file->bytes(t) + seg.first * width;
        if (rows == 0) continue;
        // Rows at the device pitch straight from the mapped file.
        e = hipMemcpy2DAsync(dst + row * pitch, (size_t)pitch, src, (size_t)width, (size_t)width,
                             (size_t)rows, hipMemcpyHostToDevice, s);
        if (e != hipSuccess) return k2w8_fail_runtime(stage, e);
        row += rows;
      }
    }
  } catch (const Error &err) {
    return k2w8_fail_invalid(err.message.c_str());
  }
  // The plan's host bytes must outlive the copies, and a failed upload should surface
  // here rather than at the first dispatch (weights.rs:96-98).
  e = hipStreamSynchronize(s);
  if (e != hipSuccess) return k2w8_fail_runtime(stage, e);
  return k2w8_succeed();
}

}  // extern "C"
