// Safetensors checkpoints on the host: header parsing with the reference
// reader's bounds and span checks (parse_shard, logan-qwen4/src/lib.rs
// :326-421), single files and sharded directories (StFile::open / open_dir,
// :508-595), the engine-name aliases (register, :460-503), and the geometry
// rules of the MLX quantized loaders (:11818-12078). No device code: the
// upload into HBM is loader.hip.
#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <memory>
#include <set>

#include "../../include/logan_hip.h"
#include "stfile.hpp"

namespace lh {

namespace {
thread_local std::string t_last_error;
}
void set_last_error(const std::string &m) { t_last_error = m; }

namespace st {
namespace {

// ---- a small JSON reader: enough for safetensors headers and index files.
// Objects keep their last value per key and iterate in key order (the order
// serde_json's default map gives the reference's reader). Numbers keep their
// text so u64 offsets are read exactly.
struct JVal {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } k = Null;
  bool b = false;
  std::string s;  // Str: decoded text; Num: the literal
  std::vector<JVal> a;
  std::map<std::string, JVal> o;

  const JVal *get(const char *key) const {
    if (k != Obj) return nullptr;
    auto it = o.find(key);
    return it == o.end() ? nullptr : &it->second;
  }
  // as_u64: a non-negative integer literal that fits 64 bits
  bool u64(uint64_t *v) const {
    if (k != Num || s.empty() || s[0] == '-') return false;
    uint64_t r = 0;
    for (char c : s) {
      if (c < '0' || c > '9') return false;
      uint64_t d = (uint64_t)(c - '0');
      if (r > (UINT64_MAX - d) / 10) return false;
      r = r * 10 + d;
    }
    *v = r;
    return true;
  }
};

struct JParser {
  const char *p, *end;
  std::string err;
  int depth = 0;

  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool fail(const char *m) {
    if (err.empty()) err = m;
    return false;
  }
  static void put_utf8(std::string &out, uint32_t cp) {
    if (cp < 0x80) {
      out += (char)cp;
    } else if (cp < 0x800) {
      out += (char)(0xC0 | (cp >> 6));
      out += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      out += (char)(0xE0 | (cp >> 12));
      out += (char)(0x80 | ((cp >> 6) & 0x3F));
      out += (char)(0x80 | (cp & 0x3F));
    } else {
      out += (char)(0xF0 | (cp >> 18));
      out += (char)(0x80 | ((cp >> 12) & 0x3F));
      out += (char)(0x80 | ((cp >> 6) & 0x3F));
      out += (char)(0x80 | (cp & 0x3F));
    }
  }
  bool hex4(uint32_t *v) {
    if (end - p < 4) return fail("truncated \\u escape");
    uint32_t r = 0;
    for (int i = 0; i < 4; ++i) {
      char c = *p++;
      r <<= 4;
      if (c >= '0' && c <= '9') r |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') r |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') r |= (uint32_t)(c - 'A' + 10);
      else return fail("invalid \\u escape");
    }
    *v = r;
    return true;
  }
  bool str(std::string *out) {
    if (p >= end || *p != '"') return fail("expected string");
    ++p;
    out->clear();
    while (p < end) {
      unsigned char c = (unsigned char)*p++;
      if (c == '"') return true;
      if (c < 0x20) return fail("control character in string");
      if (c != '\\') {
        *out += (char)c;
        continue;
      }
      if (p >= end) break;
      char e = *p++;
      switch (e) {
        case '"': *out += '"'; break;
        case '\\': *out += '\\'; break;
        case '/': *out += '/'; break;
        case 'b': *out += '\b'; break;
        case 'f': *out += '\f'; break;
        case 'n': *out += '\n'; break;
        case 'r': *out += '\r'; break;
        case 't': *out += '\t'; break;
        case 'u': {
          uint32_t cp;
          if (!hex4(&cp)) return false;
          if (cp >= 0xD800 && cp < 0xDC00) {
            uint32_t lo;
            if (end - p < 2 || p[0] != '\\' || p[1] != 'u') return fail("lone surrogate");
            p += 2;
            if (!hex4(&lo) || lo < 0xDC00 || lo >= 0xE000) return fail("lone surrogate");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          } else if (cp >= 0xDC00 && cp < 0xE000) {
            return fail("lone surrogate");
          }
          put_utf8(*out, cp);
          break;
        }
        default: return fail("invalid escape");
      }
    }
    return fail("unterminated string");
  }
  bool num(JVal *v) {
    const char *s = p;
    if (p < end && *p == '-') ++p;
    if (p >= end || *p < '0' || *p > '9') return fail("invalid number");
    if (*p == '0') ++p;
    else while (p < end && *p >= '0' && *p <= '9') ++p;
    if (p < end && *p == '.') {
      ++p;
      if (p >= end || *p < '0' || *p > '9') return fail("invalid number");
      while (p < end && *p >= '0' && *p <= '9') ++p;
    }
    if (p < end && (*p == 'e' || *p == 'E')) {
      ++p;
      if (p < end && (*p == '+' || *p == '-')) ++p;
      if (p >= end || *p < '0' || *p > '9') return fail("invalid number");
      while (p < end && *p >= '0' && *p <= '9') ++p;
    }
    v->k = JVal::Num;
    v->s.assign(s, (size_t)(p - s));
    return true;
  }
  bool lit(const char *w) {
    size_t n = strlen(w);
    if ((size_t)(end - p) < n || memcmp(p, w, n) != 0) return fail("invalid literal");
    p += n;
    return true;
  }
  bool val(JVal *v) {
    ws();
    if (p >= end) return fail("unexpected end of input");
    if (++depth > 128) return fail("nesting too deep");
    bool ok;
    char c = *p;
    if (c == '{') {
      ++p;
      v->k = JVal::Obj;
      ws();
      ok = true;
      if (p < end && *p == '}') {
        ++p;
      } else {
        for (;;) {
          std::string key;
          ws();
          if (!str(&key)) { ok = false; break; }
          ws();
          if (p >= end || *p != ':') { ok = fail("expected ':'"); break; }
          ++p;
          JVal item;
          if (!val(&item)) { ok = false; break; }
          v->o[key] = std::move(item);
          ws();
          if (p < end && *p == ',') { ++p; continue; }
          if (p < end && *p == '}') { ++p; break; }
          ok = fail("expected ',' or '}'");
          break;
        }
      }
    } else if (c == '[') {
      ++p;
      v->k = JVal::Arr;
      ws();
      ok = true;
      if (p < end && *p == ']') {
        ++p;
      } else {
        for (;;) {
          JVal item;
          if (!val(&item)) { ok = false; break; }
          v->a.push_back(std::move(item));
          ws();
          if (p < end && *p == ',') { ++p; continue; }
          if (p < end && *p == ']') { ++p; break; }
          ok = fail("expected ',' or ']'");
          break;
        }
      }
    } else if (c == '"') {
      v->k = JVal::Str;
      ok = str(&v->s);
    } else if (c == 't') {
      v->k = JVal::Bool;
      v->b = true;
      ok = lit("true");
    } else if (c == 'f') {
      v->k = JVal::Bool;
      ok = lit("false");
    } else if (c == 'n') {
      ok = lit("null");
    } else {
      ok = num(v);
    }
    --depth;
    return ok;
  }
  bool doc(JVal *v) {
    if (!val(v)) return false;
    ws();
    if (p != end) return fail("trailing characters");
    return true;
  }
};

bool parse_json(const char *data, size_t n, JVal *out, std::string *err) {
  JParser jp{data, data + n, {}};
  if (!jp.doc(out)) {
    *err = jp.err;
    return false;
  }
  return true;
}

bool read_all(int fd, uint64_t off, void *dst, size_t n) {
  char *d = (char *)dst;
  while (n) {
    ssize_t r = pread(fd, d, n, (off_t)off);
    if (r < 0 && errno == EINTR) continue;
    if (r <= 0) return false;
    d += r;
    off += (uint64_t)r;
    n -= (size_t)r;
  }
  return true;
}

bool read_text(const std::string &path, std::string *out, std::string *err) {
  int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) {
    *err = path + ": " + strerror(errno);
    return false;
  }
  struct stat sb;
  bool ok = fstat(fd, &sb) == 0;
  if (ok) {
    out->resize((size_t)sb.st_size);
    ok = read_all(fd, 0, &(*out)[0], out->size());
  }
  if (!ok) *err = path + ": " + strerror(errno ? errno : EIO);
  close(fd);
  return ok;
}

struct ShardEntry {
  std::string name;
  Tensor t;
};

// parse_shard (lib.rs:326-421): header length, header JSON, and for every
// tensor its dtype, shape, data_offsets, the range inside the file and
// span == elements x dtype width. Returns the open descriptor.
int parse_shard(const std::string &path, std::vector<ShardEntry> *out, std::string *err) {
  int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) {
    *err = path + ": " + strerror(errno);
    return -1;
  }
  auto fail = [&](const std::string &m) {
    *err = m;
    close(fd);
    return -1;
  };
  struct stat sb;
  if (fstat(fd, &sb) != 0) return fail(path + ": " + strerror(errno));
  const uint64_t file_len = (uint64_t)sb.st_size;
  unsigned char nbuf[8];
  if (!read_all(fd, 0, nbuf, 8)) return fail(path + ": failed to fill whole buffer");
  uint64_t n = 0;
  for (int i = 7; i >= 0; --i) n = (n << 8) | nbuf[i];
  if (n > UINT64_MAX - 8) return fail(path + ": header length overflow");
  const uint64_t data_start = 8 + n;
  if (data_start > file_len)
    return fail(path + ": header extends past EOF (" + std::to_string(data_start) + " > " +
                std::to_string(file_len) + ")");
  std::string hdr((size_t)n, '\0');
  if (n && !read_all(fd, 8, &hdr[0], (size_t)n)) return fail(path + ": failed to fill whole buffer");
  JVal root;
  std::string jerr;
  if (!parse_json(hdr.data(), hdr.size(), &root, &jerr)) return fail(path + ": " + jerr);
  if (root.k != JVal::Obj) return fail(path + ": header is not an object");
  for (const auto &kv : root.o) {
    const std::string &name = kv.first;
    if (name == "__metadata__") continue;
    const JVal &spec = kv.second;
    const JVal *dt = spec.get("dtype");
    if (!dt || dt->k != JVal::Str) return fail(name + ": missing dtype");
    if (!element_bytes(dt->s))
      return fail(name + ": unsupported dtype `" + dt->s +
                  "` (supported: F32, I32, I64, U32, U8, BF16, F16, F8_E4M3, F8_E4M3FN)");
    const JVal *sh = spec.get("shape");
    if (!sh || sh->k != JVal::Arr) return fail(name + ": missing shape");
    Tensor t;
    t.dtype = dt->s;
    for (const JVal &d : sh->a) {
      uint64_t v;
      if (!d.u64(&v)) return fail(name + ": invalid shape");
      t.shape.push_back(v);
    }
    const JVal *offs = spec.get("data_offsets");
    if (!offs || offs->k != JVal::Arr) return fail(name + ": missing data_offsets");
    if (offs->a.size() != 2) return fail(name + ": invalid data_offsets");
    uint64_t begin, endo;
    if (!offs->a[0].u64(&begin)) return fail(name + ": invalid start offset");
    if (!offs->a[1].u64(&endo)) return fail(name + ": invalid end offset");
    if (endo < begin || endo > UINT64_MAX - data_start || data_start + endo > file_len)
      return fail(name + ": tensor range is outside " + path);
    // elements as the reference counts them: the product of the dims, at
    // least 1; the expected span saturates
    unsigned __int128 el = 1;
    bool big = false;
    for (uint64_t d : t.shape) {
      el *= d;
      if (el > (unsigned __int128)UINT64_MAX) big = true, el = (unsigned __int128)UINT64_MAX;
    }
    uint64_t elems = big ? UINT64_MAX : (uint64_t)el;
    if (elems == 0) elems = 1;
    unsigned __int128 ex = (unsigned __int128)elems * (unsigned)element_bytes(t.dtype);
    uint64_t expected = ex > (unsigned __int128)UINT64_MAX ? UINT64_MAX : (uint64_t)ex;
    if (endo - begin != expected)
      return fail(name + ": span " + std::to_string(endo - begin) + " != " + std::to_string(elems) +
                  " x \"" + t.dtype + "\" = " + std::to_string(expected));
    t.offset = data_start + begin;
    t.len = endo - begin;
    out->push_back({name, std::move(t)});
  }
  return fd;
}

// register (lib.rs:460-503): the checkpoint's own name, plus the engine's
// spelling where an HF / MLX prefix is present and the checkpoint does not
// itself define that spelling. (The in-layer PLE alias of the reference is
// outside the quantized hot path and not registered here.)
void register_name(std::map<std::string, Tensor> &m, const std::string &name, const Tensor &t) {
  static const char *const kFrom[3] = {"model.language_model.", "language_model.model.",
                                       "language_model.lm_head."};
  static const char *const kTo[3] = {"model.", "model.", "lm_head."};
  for (int i = 0; i < 3; ++i) {
    size_t n = strlen(kFrom[i]);
    if (name.compare(0, n, kFrom[i]) == 0) {
      std::string alias = std::string(kTo[i]) + name.substr(n);
      if (!m.count(alias)) m[alias] = t;
    }
  }
  m[name] = t;
}

}  // namespace

File::~File() {
  for (int fd : fds)
    if (fd >= 0) close(fd);
}

int element_bytes(const std::string &d) {
  if (d == "F32" || d == "I32" || d == "U32") return 4;
  if (d == "BF16" || d == "F16") return 2;
  if (d == "U8" || d == "F8_E4M3" || d == "F8_E4M3FN") return 1;
  if (d == "I64") return 8;
  return 0;
}

std::string shape_str(const std::vector<uint64_t> &s) {
  std::string r = "[";
  for (size_t i = 0; i < s.size(); ++i) {
    if (i) r += ", ";
    r += std::to_string(s[i]);
  }
  return r + "]";
}

File *open_file(const std::string &path, std::string *err) {
  std::vector<ShardEntry> ents;
  int fd = parse_shard(path, &ents, err);
  if (fd < 0) return nullptr;
  File *f = new File();
  f->fds.push_back(fd);
  f->paths.push_back(path);
  for (auto &e : ents) f->tensors[e.name] = std::move(e.t);  // no aliases
  return f;
}

File *open_dir(const std::string &dir, std::string *err) {
  std::unique_ptr<File> f(new File());
  const std::string index = dir + "/model.safetensors.index.json";
  struct stat sb;
  if (stat(index.c_str(), &sb) == 0 && S_ISREG(sb.st_mode)) {
    std::string raw, jerr;
    if (!read_text(index, &raw, err)) return nullptr;
    JVal root;
    if (!parse_json(raw.data(), raw.size(), &root, &jerr)) {
      *err = index + ": " + jerr;
      return nullptr;
    }
    const JVal *map = root.get("weight_map");
    if (!map || map->k != JVal::Obj) {
      *err = index + ": missing weight_map";
      return nullptr;
    }
    // deterministic shard order: sorted, deduplicated file names
    std::set<std::string> shards;
    for (const auto &kv : map->o)
      if (kv.second.k == JVal::Str) shards.insert(kv.second.s);
    int id = 0;
    for (const std::string &sh : shards) {
      std::vector<ShardEntry> ents;
      const std::string path = dir + "/" + sh;
      int fd = parse_shard(path, &ents, err);
      if (fd < 0) return nullptr;
      f->fds.push_back(fd);
      f->paths.push_back(path);
      for (auto &e : ents) {
        e.t.shard = id;
        register_name(f->tensors, e.name, e.t);
      }
      ++id;
    }
    if (f->tensors.empty()) {
      *err = index + ": weight_map names no tensors";
      return nullptr;
    }
  } else {
    const std::string single = dir + "/model.safetensors";
    if (!(stat(single.c_str(), &sb) == 0 && S_ISREG(sb.st_mode))) {
      *err = dir + ": neither model.safetensors.index.json nor model.safetensors";
      return nullptr;
    }
    std::vector<ShardEntry> ents;
    int fd = parse_shard(single, &ents, err);
    if (fd < 0) return nullptr;
    f->fds.push_back(fd);
    f->paths.push_back(single);
    for (auto &e : ents) register_name(f->tensors, e.name, e.t);
  }
  return f.release();
}

namespace {

const Tensor *find(const File &f, const std::string &name) {
  auto it = f.tensors.find(name);
  return it == f.tensors.end() ? nullptr : &it->second;
}

bool ends_with_weight(const std::string &name, std::string *base) {
  static const char kSuf[] = ".weight";
  const size_t n = sizeof(kSuf) - 1;
  if (name.size() < n || name.compare(name.size() - n, n, kSuf) != 0) return false;
  *base = name.substr(0, name.size() - n);
  return true;
}

// payload_range (lib.rs:726-760): within + len inside the payload
bool region(const Tensor &t, const std::string &name, uint64_t within, uint64_t len, Region *r,
            std::string *err) {
  if (within > UINT64_MAX - len) {
    *err = name + ": requested byte range overflows";
    return false;
  }
  if (within + len > t.len) {
    *err = name + ": requested byte range " + std::to_string(within) + ".." +
           std::to_string(within + len) + " exceeds payload length " + std::to_string(t.len);
    return false;
  }
  r->shard = t.shard;
  r->file_off = t.offset + within;
  r->len = len;
  return true;
}

// the inferred code width: words * 32 / I, exactly
bool infer_bits(const std::string &name, uint64_t words, long long i, int *bits,
                std::string *err) {
  if (words > UINT64_MAX / 32) {
    *err = name + ": packed row bit count overflows";
    return false;
  }
  const uint64_t row_bits = words * 32;
  if (row_bits % (uint64_t)i) {
    *err = name + ": " + std::to_string(words) + " U32 words cannot represent " +
           std::to_string(i) + " logical columns exactly";
    return false;
  }
  const uint64_t b = row_bits / (uint64_t)i;
  if (b > 255) {
    *err = name + ": inferred bit width overflows u8";
    return false;
  }
  *bits = (int)b;
  return true;
}

bool good_bits(int b) { return b == 4 || b == 5 || b == 6 || b == 8; }

}  // namespace

bool plan_dense(const File &f, const std::string &name, long long o, long long i, QuantPlan *p,
                std::string *err) {
  *p = QuantPlan();
  if (o <= 0 || i <= 0) {
    *err = name + ": quantized matrix dimensions must be non-zero";
    return false;
  }
  const Tensor *w = find(f, name);
  if (!w) {
    *err = "missing tensor " + name;
    return false;
  }
  if (w->dtype != "U32" || w->shape.size() != 2 || w->shape[0] != (uint64_t)o) {
    *err = name + ": expected U32 packed matrix with " + std::to_string(o) + " rows, got " +
           w->dtype + "/" + shape_str(w->shape);
    return false;
  }
  int bits;
  if (!infer_bits(name, w->shape[1], i, &bits, err)) return false;
  if (!good_bits(bits)) {
    *err = name + ": inferred unsupported MLX quantization width " + std::to_string(bits) +
           " from " + shape_str(w->shape) + " -> " + std::to_string(o) + "x" + std::to_string(i);
    return false;
  }
  std::string base;
  if (!ends_with_weight(name, &base)) {
    *err = name + ": quantized matrix name must end in .weight";
    return false;
  }
  const std::string sname = base + ".scales";
  const Tensor *s = find(f, sname);
  if (!s) {
    *err = "missing quantization sidecar " + sname;
    return false;
  }
  p->E = 1;
  p->O = (int)o;
  p->I = (int)i;
  p->bits = bits;
  if (!region(*w, name, 0, w->len, &p->w, err)) return false;
  if (s->dtype == "BF16" || s->dtype == "F16") {
    if (s->shape.size() != 2 || s->shape[0] != (uint64_t)o || s->shape[1] == 0) {
      *err = sname + ": expected [rows, groups] BF16/F16 scales for " + std::to_string(o) +
             " rows, got " + s->dtype + "/" + shape_str(s->shape);
      return false;
    }
    const uint64_t groups = s->shape[1];
    if ((uint64_t)i % groups) {
      *err = sname + ": " + std::to_string(groups) + " groups do not divide " + std::to_string(i) +
             " logical columns";
      return false;
    }
    const std::string bname = base + ".biases";
    const Tensor *b = find(f, bname);
    if (!b) {
      *err = "missing affine quantization sidecar " + bname;
      return false;
    }
    if (b->dtype != s->dtype || b->shape != s->shape) {
      *err = bname + ": expected " + s->dtype + " shape " + shape_str(s->shape) + ", got " +
             b->dtype + "/" + shape_str(b->shape);
      return false;
    }
    p->kind = 1;
    p->group_size = (int)((uint64_t)i / groups);
    p->aux_fp16 = s->dtype == "F16";
    return region(*s, sname, 0, s->len, &p->sc, err) && region(*b, bname, 0, b->len, &p->bi, err);
  }
  if (s->dtype == "U8") {
    if (bits != 4) {
      *err = name + ": U8 scale sidecar identifies MLX MXFP4, but inferred weight width is " +
             std::to_string(bits);
      return false;
    }
    const uint64_t want = ((uint64_t)i + 31) / 32;
    if (s->shape != std::vector<uint64_t>{(uint64_t)o, want}) {
      *err = sname + ": expected MLX MXFP4 scale shape [" + std::to_string(o) + ", " +
             std::to_string(want) + "], got " + shape_str(s->shape);
      return false;
    }
    p->kind = 2;
    p->group_size = 32;
    return region(*s, sname, 0, s->len, &p->sc, err);
  }
  *err = sname + ": unsupported MLX quantization scale dtype " + s->dtype +
         "; expected BF16/F16 affine or U8 MXFP4";
  return false;
}

bool plan_experts(const File &f, const std::string &name, long long e0, long long ne,
                  long long experts, long long o, long long i, QuantPlan *p, std::string *err) {
  *p = QuantPlan();
  if (e0 < 0 || ne < 1 || experts < 1 || e0 >= experts || ne > experts - e0 || o <= 0 || i <= 0) {
    *err = name + ": invalid expert geometry expert=" + std::to_string(e0) + "/" +
           std::to_string(experts) + " matrix=" + std::to_string(o) + "x" + std::to_string(i);
    if (ne != 1) *err += " count=" + std::to_string(ne);
    return false;
  }
  const Tensor *w = find(f, name);
  if (!w) {
    *err = "missing tensor " + name;
    return false;
  }
  if (w->dtype != "U32" || w->shape.size() != 3 || w->shape[0] != (uint64_t)experts ||
      w->shape[1] != (uint64_t)o) {
    *err = name + ": expected stacked U32 [" + std::to_string(experts) + ", " + std::to_string(o) +
           ", words], got " + w->dtype + "/" + shape_str(w->shape);
    return false;
  }
  const uint64_t words = w->shape[2];
  int bits;
  if (!infer_bits(name, words, i, &bits, err)) return false;
  if (!good_bits(bits)) {
    *err = name + ": unsupported MLX expert bit width " + std::to_string(bits);
    return false;
  }
  std::string base;
  if (!ends_with_weight(name, &base)) {
    *err = name + ": quantized expert name must end in .weight";
    return false;
  }
  const std::string sname = base + ".scales";
  const Tensor *s = find(f, sname);
  if (!s) {
    *err = "missing expert sidecar " + sname;
    return false;
  }
  if (s->shape.size() != 3 || s->shape[0] != (uint64_t)experts || s->shape[1] != (uint64_t)o ||
      s->shape[2] == 0) {
    *err = sname + ": expected [" + std::to_string(experts) + ", " + std::to_string(o) +
           ", groups], got " + shape_str(s->shape);
    return false;
  }
  const uint64_t groups = s->shape[2];
  if ((uint64_t)i % groups) {
    *err = sname + ": " + std::to_string(groups) + " groups do not divide " + std::to_string(i) +
           " logical columns";
    return false;
  }
  const uint64_t gs = (uint64_t)i / groups;
  // all sizes below are bounded by the (validated) payload lengths
  const uint64_t wslice = (uint64_t)o * words * 4;
  if (!region(*w, name, (uint64_t)e0 * wslice, (uint64_t)ne * wslice, &p->w, err)) return false;
  p->E = (int)ne;
  p->O = (int)o;
  p->I = (int)i;
  p->bits = bits;
  p->group_size = (int)gs;
  if (s->dtype == "BF16" || s->dtype == "F16") {
    const uint64_t pslice = (uint64_t)o * groups * 2;
    const std::string bname = base + ".biases";
    const Tensor *b = find(f, bname);
    if (!b) {
      *err = "missing affine expert sidecar " + bname;
      return false;
    }
    if (b->dtype != s->dtype || b->shape != s->shape) {
      *err = bname + ": expected " + s->dtype + " shape " + shape_str(s->shape) + ", got " +
             b->dtype + "/" + shape_str(b->shape);
      return false;
    }
    p->kind = 1;
    p->aux_fp16 = s->dtype == "F16";
    return region(*s, sname, (uint64_t)e0 * pslice, (uint64_t)ne * pslice, &p->sc, err) &&
           region(*b, bname, (uint64_t)e0 * pslice, (uint64_t)ne * pslice, &p->bi, err);
  }
  if (s->dtype == "U8") {
    if (bits != 4 || gs != 32) {
      *err = name + ": MLX MXFP4 expert requires 4-bit/group-32, got " + std::to_string(bits) +
             "-bit/group-" + std::to_string(gs);
      return false;
    }
    const uint64_t sslice = (uint64_t)o * groups;
    p->kind = 2;
    return region(*s, sname, (uint64_t)e0 * sslice, (uint64_t)ne * sslice, &p->sc, err);
  }
  *err = sname + ": unsupported MLX expert scale dtype " + s->dtype;
  return false;
}

}  // namespace st
}  // namespace lh

// ------------------------------------------------------------------------
// C ABI: checkpoint index
// ------------------------------------------------------------------------

struct LoganHipStFile {
  lh::st::File *f;
};

extern "C" {

const char *logan_hip_last_error(void) { return lh::t_last_error.c_str(); }

LoganHipStFile *logan_hip_st_open(const char *path) {
  if (!path) {
    lh::set_last_error("null path");
    return nullptr;
  }
  std::string err;
  lh::st::File *f = lh::st::open_file(path, &err);
  if (!f) {
    lh::set_last_error(err);
    return nullptr;
  }
  return new LoganHipStFile{f};
}

LoganHipStFile *logan_hip_st_open_dir(const char *dir) {
  if (!dir) {
    lh::set_last_error("null path");
    return nullptr;
  }
  std::string err;
  lh::st::File *f = lh::st::open_dir(dir, &err);
  if (!f) {
    lh::set_last_error(err);
    return nullptr;
  }
  return new LoganHipStFile{f};
}

void logan_hip_st_close(LoganHipStFile *st) {
  if (!st) return;
  delete st->f;
  delete st;
}

int logan_hip_st_shard_count(const LoganHipStFile *st) {
  return st ? (int)st->f->fds.size() : 0;
}

int logan_hip_st_tensor(const LoganHipStFile *st, const char *name, char *dtype, size_t dtype_cap,
                        uint64_t *shape, int max_dims, int *ndim, uint64_t *nbytes) {
  if (!st || !name) return 0;
  auto it = st->f->tensors.find(name);
  if (it == st->f->tensors.end()) return 0;
  const lh::st::Tensor &t = it->second;
  if (dtype && dtype_cap) {
    size_t n = std::min(dtype_cap - 1, t.dtype.size());
    memcpy(dtype, t.dtype.data(), n);
    dtype[n] = 0;
  }
  if (ndim) *ndim = (int)t.shape.size();
  if (shape)
    for (int i = 0; i < max_dims && i < (int)t.shape.size(); ++i) shape[i] = t.shape[i];
  if (nbytes) *nbytes = t.len;
  return 1;
}

int logan_hip_st_dtype_count(const LoganHipStFile *st, const char *dtype) {
  if (!st || !dtype) return 0;
  // distinct payloads, not names: an alias shares its payload
  std::set<std::pair<int, uint64_t>> seen;
  int n = 0;
  for (const auto &kv : st->f->tensors) {
    const lh::st::Tensor &t = kv.second;
    if (t.dtype == dtype && seen.insert({t.shard, t.offset}).second) ++n;
  }
  return n;
}

int logan_hip_st_read(const LoganHipStFile *st, const char *name, uint64_t within, uint64_t len,
                      void *dst) {
  if (!st || !name || (!dst && len)) {
    lh::set_last_error("null argument");
    return 0;
  }
  auto it = st->f->tensors.find(name);
  if (it == st->f->tensors.end()) {
    lh::set_last_error(std::string("missing tensor ") + name);
    return 0;
  }
  lh::st::Region r;
  std::string err;
  if (!lh::st::region(it->second, name, within, len, &r, &err)) {
    lh::set_last_error(err);
    return 0;
  }
  if (!lh::st::read_all(st->f->fds[r.shard], r.file_off, dst, (size_t)r.len)) {
    lh::set_last_error(std::string(name) + ": " + strerror(errno ? errno : EIO));
    return -1;
  }
  return 1;
}

static int plan_to_c(const lh::st::QuantPlan &p, LoganHipQuantWt *out) {
  memset(out, 0, sizeof(*out));
  out->kind = p.kind;
  out->E = p.E;
  out->O = p.O;
  out->I = p.I;
  out->bits = p.bits;
  out->group_size = p.group_size;
  out->aux_fp16 = p.aux_fp16;
  out->weight_bytes = p.w.len;
  out->scale_bytes = p.sc.len;
  out->bias_bytes = p.bi.len;
  return 1;
}

int logan_hip_plan_mlx_quantized(const LoganHipStFile *st, const char *name, int O, int I,
                                 LoganHipQuantWt *out) {
  if (!st || !name || !out) {
    lh::set_last_error("null argument");
    return 0;
  }
  lh::st::QuantPlan p;
  std::string err;
  if (!lh::st::plan_dense(*st->f, name, O, I, &p, &err)) {
    lh::set_last_error(err);
    return 0;
  }
  return plan_to_c(p, out);
}

int logan_hip_plan_mlx_quantized_experts(const LoganHipStFile *st, const char *name, int e0,
                                         int count, int experts, int O, int I,
                                         LoganHipQuantWt *out) {
  if (!st || !name || !out) {
    lh::set_last_error("null argument");
    return 0;
  }
  lh::st::QuantPlan p;
  std::string err;
  if (!lh::st::plan_experts(*st->f, name, e0, count, experts, O, I, &p, &err)) {
    lh::set_last_error(err);
    return 0;
  }
  return plan_to_c(p, out);
}

}  // extern "C"

// for loader.hip
namespace lh {
namespace st {
bool plan_lookup(const LoganHipStFile *h, const File **f) {
  if (!h) return false;
  *f = h->f;
  return true;
}
bool pread_all(int fd, uint64_t off, void *dst, size_t n) { return read_all(fd, off, dst, n); }
}  // namespace st
}  // namespace lh
