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
#include <set>
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

  // Blocks are numbered from 0 without gaps; a block exists when its first attention
  // projection does (the rule of src/checkpoint/file.rs:115-119): the count is the first number
  // missing from the checkpoint's `blocks.<n>.attn.wq.weight` names.
  int64_t block_count() const {
    static const std::string head = "blocks.", tail = ".attn.wq.weight";
    std::set<int64_t> present;
    for (const auto &kv : entries) {
      const std::string &n = kv.first;
      if (n.size() <= head.size() + tail.size() || n.compare(0, head.size(), head) != 0 ||
          n.compare(n.size() - tail.size(), tail.size(), tail) != 0)
        continue;
      const std::string digits = n.substr(head.size(), n.size() - head.size() - tail.size());
      // Only the decimal form `{i}` names block i: no sign, no leading zero.
      if (digits.empty() || digits.size() > 9 || digits.find_first_not_of("0123456789") != std::string::npos ||
          (digits.size() > 1 && digits[0] == '0'))
        continue;
      present.insert(std::stoll(digits));
    }
    // The reference counts at most one block per tensor of the file.
    int64_t count = 0;
    while (count < (int64_t)entries.size() && present.count(count)) ++count;
    return count;
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

// A GEMM operand's rows on the device (the layout of plan.rs:61-85, 154-230): int8
// weight rows of K bytes, each padded to the GEMM pitch, with one f32 scale per row in a
// span of their own. The device rows are a sequence of runs of source rows; the scales
// follow the same runs.
struct RowRun {
  int part;               // index into the operand's parts
  int64_t first, count;   // source rows [first, first + count)
};

// The device row order of `parts` (their row counts in `rows`): the parts one after
// another (group 0), or taken in turns, `group` rows of each part per turn. The turns
// need every part to have the same number of rows, a whole number of groups.
std::vector<RowRun> row_order(const std::string &operand, const std::vector<int64_t> &rows, int64_t group) {
  std::vector<RowRun> runs;
  if (group == 0) {
    for (size_t p = 0; p < rows.size(); ++p) runs.push_back(RowRun{(int)p, 0, rows[p]});
    return runs;
  }
  for (int64_t r : rows)
    if (r != rows[0] || r % group != 0)
      throw Error{format("%s takes its parts %lld rows at a time in turn: they need equal row counts "
                         "that are whole multiples of it", operand.c_str(), (long long)group)};
  for (int64_t first = 0; first < rows[0]; first += group)
    for (size_t p = 0; p < rows.size(); ++p) runs.push_back(RowRun{(int)p, first, group});
  return runs;
}

// One operand: its weight span (rows gathered straight from the file) and its scale
// span (assembled on the host in the same row order).
void operand(const k2w8_checkpoint &file, const std::string &out, const std::vector<std::string> &parts,
             int64_t group, Span &weights, Span &scale_span) {
  std::vector<const Entry *> w(parts.size()), sc(parts.size());
  std::vector<int64_t> rows(parts.size());
  for (size_t p = 0; p < parts.size(); ++p) {
    w[p] = &file.get(parts[p] + ".weight");
    if (w[p]->dtype != K2W8_DTYPE_I8 || w[p]->shape.size() != 2 || w[p]->shape[0] == 0 || w[p]->shape[1] == 0)
      throw Error{format("%s.weight in %s must be a non-empty int8 matrix of ConvRot rows", parts[p].c_str(),
                         file.path.c_str())};
    rows[p] = w[p]->shape[0];
    if (w[p]->shape[1] != w[0]->shape[1])
      throw Error{format("%s: %s has rows of %lld bytes and %s of %lld; one operand has one K", out.c_str(),
                         parts[0].c_str(), (long long)w[0]->shape[1], parts[p].c_str(), (long long)w[p]->shape[1])};
    sc[p] = &file.get(parts[p] + ".weight_scale");
    if (sc[p]->dtype != K2W8_DTYPE_F32 || (int64_t)(sc[p]->end - sc[p]->begin) != rows[p] * 4)
      throw Error{format("%s.weight_scale must hold one float32 per weight row (%lld)", parts[p].c_str(),
                         (long long)rows[p])};
  }
  const std::vector<RowRun> runs = row_order(out, rows, group);
  const int64_t k = w[0]->shape[1];
  weights = Span{};
  weights.row_bytes = k;
  weights.device_row_bytes = k2w8_shape_gemm_pitch(k);
  std::vector<uint8_t> scale_bytes;
  for (const RowRun &run : runs) {
    weights.segments.push_back(Segment{parts[run.part] + ".weight", run.first, run.first + run.count});
    weights.rows += run.count;
    const uint8_t *src = file.bytes(*sc[run.part]) + run.first * 4;
    scale_bytes.insert(scale_bytes.end(), src, src + run.count * 4);
  }
  weights.device_bytes = weights.rows * weights.device_row_bytes;
  scale_span = Span{};
  scale_span.device_bytes = (int64_t)scale_bytes.size();
  scale_span.host = std::move(scale_bytes);
}

// A norm vector (plan.rs:233-264): float32 as stored, or bfloat16 widened exactly (the
// bf16 bits become the high half of the f32).
Span vector(const k2w8_checkpoint &file, const std::string &name) {
  const Entry &t = file.get(name);
  const int64_t nbytes = (int64_t)(t.end - t.begin);
  Span s;
  if (t.dtype == K2W8_DTYPE_F32) {
    s.rows = 1;
    s.row_bytes = s.device_row_bytes = s.device_bytes = nbytes;
    s.segments.push_back(Segment{name, 0, 1});
    return s;
  }
  if (t.dtype != K2W8_DTYPE_BF16) throw Error{format("%s must be float32 or bfloat16", name.c_str())};
  const uint8_t *src = file.bytes(t);
  s.host.resize((size_t)nbytes * 2);
  for (int64_t i = 0; i < nbytes / 2; ++i) {
    const uint32_t widened = ((uint32_t)src[2 * i] | (uint32_t)src[2 * i + 1] << 8) << 16;
    memcpy(s.host.data() + 4 * i, &widened, 4);
  }
  s.device_bytes = (int64_t)s.host.size();
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

// What each block uploads (the spans of plan.rs:88-143): four GEMM operands, named by
// suffix, from their source tensors (the gate|up pair in turns of 16 rows, the layout
// gemm_i8_swiglu reads), and four norm vectors.
struct OperandSource {
  const char *span;
  std::vector<const char *> parts;
  int64_t group;
};
const OperandSource kOperands[] = {
    {"qkvg", {"attn.wq", "attn.wk", "attn.wv", "attn.gate"}, 0},
    {"wo", {"attn.wo"}, 0},
    {"gu", {"mlp.gate", "mlp.up"}, 16},
    {"down", {"mlp.down"}, 0},
};
const std::pair<const char *, const char *> kVectors[] = {
    {"prenorm", "prenorm.scale"},
    {"postnorm", "postnorm.scale"},
    {"qnorm", "attn.qknorm.qnorm.scale"},
    {"knorm", "attn.qknorm.knorm.scale"},
};

std::unique_ptr<k2w8_plan> plan_for(const k2w8_checkpoint &file) {
  auto plan = std::make_unique<k2w8_plan>();
  plan->layers = file.block_count();
  if (plan->layers == 0)
    throw Error{format("no transformer blocks in %s (no blocks.0.attn.wq.weight)", file.path.c_str())};
  for (int64_t b = 0; b < plan->layers; ++b) {
    const std::string block = format("blocks.%lld.", (long long)b);
    for (const OperandSource &op : kOperands) {
      std::vector<std::string> parts;
      for (const char *part : op.parts) parts.push_back(block + part);
      Span weights, scales;
      operand(file, block + op.span, parts, op.group, weights, scales);
      plan->spans[block + op.span + ".q"] = std::move(weights);
      plan->spans[block + op.span + ".s"] = std::move(scales);
    }
    for (const auto &v : kVectors) plan->spans[block + v.first] = vector(file, block + v.second);
  }
  // Device placement: the spans in name order (the map's order), each at the next
  // 256-byte boundary.
  for (auto &kv : plan->spans) {
    kv.second.device_offset = plan->total_bytes;
    plan->total_bytes += (kv.second.device_bytes + 255) / 256 * 256;
    plan->names.push_back(kv.first);
  }
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
