// Host-only checkpoint parsing (no HIP, so it also builds on its own for a host
// sanitizer run):
//   parseHeaderJson   src/weights.zig:70-121
//   inferQuantSpec    src/weights.zig:130-185
//   sanitizeName      src/weights.zig:186-202
//   checkShardFile    src/weights.zig:239-255
//   WeightMap.load    src/weights.zig:257-300 (the index and shard headers)
#include "checkpoint.h"

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <utility>
#include <vector>

namespace qmm {

constexpr size_t kMaxDim = 8;  // the most dimensions an array handle holds

// ---------------------------------------------------------------- minimal JSON (objects keep file order)
struct JVal {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  bool b = false;
  double num = 0;
  bool is_int = false;
  long long ival = 0;
  std::string str;
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;
  const JVal *get(const char *k) const {
    for (auto &kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
};

class JParser {
 public:
  JParser(const char *p, size_t n) : p_(p), e_(p + n) {}
  bool parse(JVal &out) {
    ws();
    if (!value(out, 0)) return false;
    ws();
    return p_ == e_;
  }

 private:
  const char *p_, *e_;
  void ws() {
    while (p_ < e_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  bool lit(const char *s) {
    size_t n = std::strlen(s);
    if ((size_t)(e_ - p_) < n || std::memcmp(p_, s, n) != 0) return false;
    p_ += n;
    return true;
  }
  bool string(std::string &out) {
    if (p_ >= e_ || *p_ != '"') return false;
    ++p_;
    while (p_ < e_ && *p_ != '"') {
      char c = *p_++;
      if ((unsigned char)c < 0x20) return false;
      if (c == '\\') {
        if (p_ >= e_) return false;
        char d = *p_++;
        switch (d) {
          case '"': out += '"'; break;
          case '\\': out += '\\'; break;
          case '/': out += '/'; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'n': out += '\n'; break;
          case 'r': out += '\r'; break;
          case 't': out += '\t'; break;
          case 'u': {
            if (e_ - p_ < 4) return false;
            unsigned cp = 0;
            for (int i = 0; i < 4; ++i) {
              char h = *p_++;
              cp <<= 4;
              if (h >= '0' && h <= '9') cp |= h - '0';
              else if (h >= 'a' && h <= 'f') cp |= h - 'a' + 10;
              else if (h >= 'A' && h <= 'F') cp |= h - 'A' + 10;
              else return false;
            }
            if (cp < 0x80) {
              out += (char)cp;
            } else if (cp < 0x800) {
              out += (char)(0xC0 | (cp >> 6));
              out += (char)(0x80 | (cp & 0x3F));
            } else {
              out += (char)(0xE0 | (cp >> 12));
              out += (char)(0x80 | ((cp >> 6) & 0x3F));
              out += (char)(0x80 | (cp & 0x3F));
            }
            break;
          }
          default: return false;
        }
      } else {
        out += c;
      }
    }
    if (p_ >= e_) return false;
    ++p_;
    return true;
  }
  bool number(JVal &v) {
    const char *s = p_;
    if (p_ < e_ && *p_ == '-') ++p_;
    if (p_ >= e_ || !(*p_ >= '0' && *p_ <= '9')) return false;
    while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
    bool integer = true;
    if (p_ < e_ && *p_ == '.') {
      integer = false;
      ++p_;
      if (p_ >= e_ || !(*p_ >= '0' && *p_ <= '9')) return false;
      while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    if (p_ < e_ && (*p_ == 'e' || *p_ == 'E')) {
      integer = false;
      ++p_;
      if (p_ < e_ && (*p_ == '+' || *p_ == '-')) ++p_;
      if (p_ >= e_ || !(*p_ >= '0' && *p_ <= '9')) return false;
      while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    std::string t(s, p_);
    v.kind = JVal::Num;
    v.num = std::strtod(t.c_str(), nullptr);
    v.is_int = integer;
    if (integer) v.ival = std::strtoll(t.c_str(), nullptr, 10);
    return true;
  }
  bool value(JVal &v, int depth) {
    if (depth > 64 || p_ >= e_) return false;
    char c = *p_;
    if (c == '{') {
      ++p_;
      v.kind = JVal::Obj;
      ws();
      if (p_ < e_ && *p_ == '}') {
        ++p_;
        return true;
      }
      for (;;) {
        ws();
        std::string k;
        if (!string(k)) return false;
        ws();
        if (p_ >= e_ || *p_ != ':') return false;
        ++p_;
        ws();
        JVal child;
        if (!value(child, depth + 1)) return false;
        v.obj.emplace_back(std::move(k), std::move(child));
        ws();
        if (p_ < e_ && *p_ == ',') {
          ++p_;
          continue;
        }
        if (p_ < e_ && *p_ == '}') {
          ++p_;
          return true;
        }
        return false;
      }
    }
    if (c == '[') {
      ++p_;
      v.kind = JVal::Arr;
      ws();
      if (p_ < e_ && *p_ == ']') {
        ++p_;
        return true;
      }
      for (;;) {
        ws();
        JVal child;
        if (!value(child, depth + 1)) return false;
        v.arr.push_back(std::move(child));
        ws();
        if (p_ < e_ && *p_ == ',') {
          ++p_;
          continue;
        }
        if (p_ < e_ && *p_ == ']') {
          ++p_;
          return true;
        }
        return false;
      }
    }
    if (c == '"') {
      v.kind = JVal::Str;
      return string(v.str);
    }
    if (c == 't') { v.kind = JVal::Bool; v.b = true; return lit("true"); }
    if (c == 'f') { v.kind = JVal::Bool; v.b = false; return lit("false"); }
    if (c == 'n') { v.kind = JVal::Null; return lit("null"); }
    return number(v);
  }
};

// ---------------------------------------------------------------- header parse
size_t dsize(DType d) { return d == DType::BF16 ? 2 : (d == DType::U8 ? 1 : 4); }
qmm_dtype to_qmm(DType d) {
  switch (d) {
    case DType::BF16: return QMM_BFLOAT16;
    case DType::F32: return QMM_FLOAT32;
    case DType::U32: return QMM_UINT32;
    default: return QMM_UINT8;
  }
}

bool ends_with(const std::string &s, const char *suf) {
  size_t n = std::strlen(suf);
  return s.size() >= n && s.compare(s.size() - n, n, suf) == 0;
}
static bool starts_with(const std::string &s, const char *pre) { return s.rfind(pre, 0) == 0; }

// parseHeaderJson (src/weights.zig:70-121): dtype whitelist, integer shapes,
// conv1d.weight must end in 1; data_offsets are read when present.
int parse_header(const char *json, size_t len, std::vector<TensorInfo> &out) {
  JVal root;
  JParser p(json, len);
  if (!p.parse(root) || root.kind != JVal::Obj) return QMM_WE_BAD_HEADER;
  for (auto &kv : root.obj) {
    if (kv.first == "__metadata__") continue;
    const JVal &o = kv.second;
    if (o.kind != JVal::Obj) return QMM_WE_BAD_HEADER;
    const JVal *dt = o.get("dtype"), *sh = o.get("shape");
    if (!dt || !sh || dt->kind != JVal::Str || sh->kind != JVal::Arr) return QMM_WE_BAD_HEADER;
    TensorInfo t;
    t.name = kv.first;
    if (dt->str == "BF16") t.dtype = DType::BF16;
    else if (dt->str == "F32") t.dtype = DType::F32;
    else if (dt->str == "U32") t.dtype = DType::U32;
    else if (dt->str == "U8") t.dtype = DType::U8;
    else return QMM_WE_UNSUPPORTED_DTYPE;
    for (auto &d : sh->arr) {
      // dimensions are non-negative and fit an int (the shape type of an array)
      if (d.kind != JVal::Num || !d.is_int || d.ival < 0 || d.ival > INT32_MAX) return QMM_WE_BAD_HEADER;
      t.shape.push_back(d.ival);
    }
    if (t.name.find("conv1d.weight") != std::string::npos) {
      if (t.shape.empty() || t.shape.back() != 1) return QMM_WE_UNSUPPORTED_LAYOUT;
    }
    if (const JVal *offs = o.get("data_offsets")) {
      if (offs->kind == JVal::Arr && offs->arr.size() == 2 && offs->arr[0].kind == JVal::Num &&
          offs->arr[1].kind == JVal::Num && offs->arr[0].is_int && offs->arr[1].is_int) {
        t.off0 = offs->arr[0].ival;
        t.off1 = offs->arr[1].ival;
      }
    }
    out.push_back(std::move(t));
  }
  return 0;
}

static const TensorInfo *find_info(const std::vector<TensorInfo> &v, const std::string &name) {
  for (auto &t : v)
    if (t.name == name) return &t;
  return nullptr;
}

// inferQuantSpec (src/weights.zig:130-185).
int infer_quant_spec(const std::vector<TensorInfo> &infos, qmm_quant_spec *spec) {
  *spec = qmm_quant_spec{QMM_QUANT_NONE, 0, 0};
  const TensorInfo *sc = nullptr;
  for (auto &t : infos)
    if (ends_with(t.name, ".scales")) {
      sc = &t;
      break;
    }
  if (!sc) {
    for (auto &t : infos)
      if (t.dtype == DType::U32 || t.dtype == DType::U8) return QMM_WE_NONSTANDARD_QUANT;
    return 0;
  }
  if (sc->shape.size() != 2) return QMM_WE_NONSTANDARD_QUANT;
  if (sc->dtype != DType::U8) return QMM_WE_AFFINE_UNSUPPORTED;
  const std::string prefix = sc->name.substr(0, sc->name.size() - 7);
  if (prefix.empty()) return QMM_WE_NONSTANDARD_QUANT;
  const TensorInfo *w = find_info(infos, prefix + ".weight");
  if (!w || w->dtype != DType::U32 || w->shape.size() != 2) return QMM_WE_NONSTANDARD_QUANT;
  const long long packed = w->shape[1], groups = sc->shape[1];
  if (packed <= 0 || groups <= 0 || packed % groups != 0) return QMM_WE_NONSTANDARD_QUANT;
  const long long r = packed / groups;  // group * bits / 32
  qmm_quant_spec sp;
  if (r == 8)
    sp = qmm_quant_spec{QMM_QUANT_MXFP8, 32, 8};
  else if (r == 2)
    sp = qmm_quant_spec{QMM_QUANT_NVFP4, 16, 4};
  else
    return QMM_WE_NONSTANDARD_QUANT;
  for (auto &t : infos) {
    if (ends_with(t.name, ".scales")) {
      if (t.dtype != DType::U8 || t.shape.size() != 2) return QMM_WE_INCONSISTENT_QUANT;
      const TensorInfo *w2 = find_info(infos, t.name.substr(0, t.name.size() - 7) + ".weight");
      if (!w2 || w2->dtype != DType::U32 || w2->shape.size() != 2) return QMM_WE_NONSTANDARD_QUANT;
      if (t.shape[1] <= 0 || w2->shape[1] % t.shape[1] != 0 || w2->shape[1] / t.shape[1] != r)
        return QMM_WE_INCONSISTENT_QUANT;
    }
    if (t.dtype == DType::U32 && ends_with(t.name, ".weight")) {
      if (!find_info(infos, t.name.substr(0, t.name.size() - 7) + ".scales")) return QMM_WE_INCONSISTENT_QUANT;
    }
  }
  *spec = sp;
  return 0;
}

// sanitizeName (src/weights.zig:186-202): vision keys dropped, HF names remapped.
bool sanitize_name(const std::string &name, std::string &out) {
  if (starts_with(name, "vision_tower") || starts_with(name, "model.visual")) return false;
  if (starts_with(name, "model.language_model")) {
    out = "language_model.model" + name.substr(std::strlen("model.language_model"));
    return true;
  }
  if (starts_with(name, "language_model.")) {
    out = name;
    return true;
  }
  out = "language_model." + name;
  return true;
}

static int read_file(const std::string &path, std::string &out) {
  FILE *f = std::fopen(path.c_str(), "rb");
  if (!f) return QMM_WE_IO;
  std::fseek(f, 0, SEEK_END);
  long n = std::ftell(f);
  std::fseek(f, 0, SEEK_SET);
  out.resize(n > 0 ? (size_t)n : 0);
  size_t got = n > 0 ? std::fread(&out[0], 1, (size_t)n, f) : 0;
  std::fclose(f);
  return got == out.size() ? 0 : QMM_WE_IO;
}

bool pread_all(int fd, void *buf, size_t n, long long off) {
  char *p = (char *)buf;
  while (n) {
    ssize_t r = ::pread(fd, p, n, (off_t)off);
    if (r <= 0) return false;
    p += r;
    n -= (size_t)r;
    off += r;
  }
  return true;
}

// checkShardFile (src/weights.zig:239-255): 8-byte LE length + header JSON only.
static int read_shard_header(int fd, std::vector<TensorInfo> &infos, uint64_t *data_start) {
  unsigned char lenbuf[8];
  if (!pread_all(fd, lenbuf, 8, 0)) return QMM_WE_IO;
  uint64_t n = 0;
  for (int i = 7; i >= 0; --i) n = (n << 8) | lenbuf[i];
  if (n == 0 || n > 256ull * 1024 * 1024) return QMM_WE_BAD_HEADER;
  std::string hdr(n, '\0');
  if (!pread_all(fd, &hdr[0], n, 8)) return QMM_WE_IO;
  *data_start = 8 + n;
  return parse_header(hdr.data(), hdr.size(), infos);
}


CheckpointPlan::~CheckpointPlan() { close_files(); }

void CheckpointPlan::close_files() {
  for (int fd : fds) ::close(fd);
  fds.clear();
}

int plan_checkpoint(const std::string &dir, CheckpointPlan &plan, std::string *err) {
  std::string idx;
  int rc = read_file(dir + "/model.safetensors.index.json", idx);
  if (rc) {
    *err = "cannot read " + dir + "/model.safetensors.index.json";
    return rc;
  }
  JVal root;
  JParser jp(idx.data(), idx.size());
  if (!jp.parse(root) || root.kind != JVal::Obj) return QMM_WE_BAD_INDEX_JSON;
  const JVal *wm = root.get("weight_map");
  if (!wm || wm->kind != JVal::Obj) return QMM_WE_BAD_INDEX_JSON;
  for (auto &kv : wm->obj) {  // the shards, ordered and unique
    if (kv.second.kind != JVal::Str) return QMM_WE_BAD_INDEX_JSON;
    bool seen = false;
    for (auto &sh : plan.shards) seen |= sh == kv.second.str;
    if (!seen) plan.shards.push_back(kv.second.str);
  }
  plan.infos.resize(plan.shards.size());  // sized once: items point into it
  for (size_t si = 0; si < plan.shards.size(); ++si) {
    const std::string path = dir + "/" + plan.shards[si];
    int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) {
      *err = "cannot open " + path;
      return QMM_WE_IO;
    }
    plan.fds.push_back(fd);
    uint64_t data_start = 0;
    rc = read_shard_header(fd, plan.infos[si], &data_start);
    if (rc) return rc;
    plan.data_starts.push_back(data_start);
    for (auto &t : plan.infos[si]) {
      std::string kept;
      if (!sanitize_name(t.name, kept)) continue;
      if (plan.index.count(kept)) return QMM_WE_DUPLICATE_TENSOR;
      // bytes = prod(shape) * dtype size, rejected if it overflows 64 bits, and they
      // must be exactly the tensor's data_offsets range
      uint64_t bytes = dsize(t.dtype);
      bool over = false;
      for (long long d : t.shape) over = over || __builtin_mul_overflow(bytes, (uint64_t)d, &bytes);
      if (over || t.off0 < 0 || t.off1 < t.off0 || (uint64_t)(t.off1 - t.off0) != bytes ||
          t.shape.size() > kMaxDim)
        return QMM_WE_BAD_HEADER;
      plan.index.emplace(kept, plan.items.size());
      plan.items.push_back(CheckpointItem{si, &t, kept, bytes});
    }
  }
  return 0;
}

}  // namespace qmm

using namespace qmm;

extern "C" {


int qmm_parse_header_json(const char *json, size_t len, size_t *n_tensors) {
  std::vector<TensorInfo> infos;
  int rc = parse_header(json, len, infos);
  if (n_tensors) *n_tensors = infos.size();
  return rc;
}

int qmm_infer_quant_spec_json(const char *json, size_t len, qmm_quant_spec *spec, size_t *n_tensors) {
  std::vector<TensorInfo> infos;
  int rc = parse_header(json, len, infos);
  if (n_tensors) *n_tensors = infos.size();
  if (rc) return rc;
  qmm_quant_spec sp;
  rc = infer_quant_spec(infos, &sp);
  if (rc == 0 && spec) *spec = sp;
  return rc;
}

int qmm_sanitize_name(const char *name, char *out, size_t out_len) {
  std::string kept;
  if (!sanitize_name(name, kept)) return 0;
  if (kept.size() + 1 > out_len) return -1;
  std::memcpy(out, kept.c_str(), kept.size() + 1);
  return 1;
}

}  // extern "C"
