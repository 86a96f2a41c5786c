// Host mirror of mlx-runner's weight loading and linear dispatch:
//   parseHeaderJson   src/weights.zig:70-121
//   inferQuantSpec    src/weights.zig:130-185
//   sanitizeName      src/weights.zig:186-202
//   WeightMap.load    src/weights.zig:257-352 (here: raw bytes at data_offsets -> HBM)
//   namedLinearQ      src/model.zig:213-233, qlinear :244-260, linear :200-211
//
// The loader reads each tensor's bytes at its `data_offsets` (which the
// reference ignores, src/weights.zig:91-92) in chunks of at most 1 GiB through
// a pinned staging buffer, and copies them to HBM unchanged: U32 packed
// weights and U8 scales land exactly as the kernels consume them.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "../../include/qmm.h"
#include "qmm_internal.h"

namespace qmm {

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
enum class DType { BF16, F32, U32, U8 };

struct TensorInfo {
  std::string name;
  DType dtype;
  std::vector<long long> shape;
  long long off0 = -1, off1 = -1;  // data_offsets, relative to the data section
};

static size_t dsize(DType d) { return d == DType::BF16 ? 2 : (d == DType::U8 ? 1 : 4); }
static qmm_dtype to_qmm(DType d) {
  switch (d) {
    case DType::BF16: return QMM_BFLOAT16;
    case DType::F32: return QMM_FLOAT32;
    case DType::U32: return QMM_UINT32;
    default: return QMM_UINT8;
  }
}

static bool ends_with(const std::string &s, const char *suf) {
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
      if (d.kind != JVal::Num || !d.is_int) return QMM_WE_BAD_HEADER;
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

// ---------------------------------------------------------------- WeightMap
struct WeightMap {
  std::unordered_map<std::string, Arr *> map;
  std::vector<void *> buffers;  // hipMalloc'd tensor buffers
  qmm_quant_spec quant{QMM_QUANT_NONE, 0, 0};
  ~WeightMap() {
    for (auto &kv : map) delete kv.second;  // buffers freed below
    for (void *b : buffers) (void)hipFree(b);
  }
};

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

static bool pread_all(int fd, void *buf, size_t n, off_t off) {
  char *p = (char *)buf;
  while (n) {
    ssize_t r = ::pread(fd, p, n, off);
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

int load_weights(const std::string &dir, hipStream_t st, WeightMap **out) {
  std::string idx;
  int rc = read_file(dir + "/model.safetensors.index.json", idx);
  if (rc) {
    fail("[qmm_weights_load] cannot read %s/model.safetensors.index.json", dir.c_str());
    return rc;
  }
  JVal root;
  JParser jp(idx.data(), idx.size());
  if (!jp.parse(root) || root.kind != JVal::Obj) return QMM_WE_BAD_INDEX_JSON;
  const JVal *wm = root.get("weight_map");
  if (!wm || wm->kind != JVal::Obj) return QMM_WE_BAD_INDEX_JSON;
  std::vector<std::string> shards;  // ordered, unique
  for (auto &kv : wm->obj) {
    if (kv.second.kind != JVal::Str) return QMM_WE_BAD_INDEX_JSON;
    bool seen = false;
    for (auto &s : shards) seen |= s == kv.second.str;
    if (!seen) shards.push_back(kv.second.str);
  }
  std::unique_ptr<WeightMap> m(new WeightMap());
  // 1) every shard's header: the tensors to load, with their file and data offset
  struct Item {
    size_t shard;          // index into fds
    const TensorInfo *t;
    std::string kept;      // name after sanitize_name
    size_t bytes;
    void *dev = nullptr;   // destination in HBM
  };
  std::vector<int> fds;
  std::vector<uint64_t> data_starts;
  std::vector<std::vector<TensorInfo>> shard_infos(shards.size());
  auto close_all = [&]() {
    for (int fd : fds) ::close(fd);
    fds.clear();
  };
  std::vector<Item> items;
  std::unordered_map<std::string, size_t> index;  // kept name -> items index
  for (size_t si = 0; si < shards.size(); ++si) {
    const std::string path = dir + "/" + shards[si];
    int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) {
      close_all();
      fail("[qmm_weights_load] cannot open %s", path.c_str());
      return QMM_WE_IO;
    }
    fds.push_back(fd);
    uint64_t data_start = 0;
    rc = read_shard_header(fd, shard_infos[si], &data_start);
    if (rc) {
      close_all();
      return rc;
    }
    data_starts.push_back(data_start);
    for (auto &t : shard_infos[si]) {
      std::string kept;
      if (!sanitize_name(t.name, kept)) continue;
      if (index.count(kept)) {
        close_all();
        return QMM_WE_DUPLICATE_TENSOR;
      }
      long long numel = 1;
      for (long long d : t.shape) numel *= d;
      const size_t bytes = (size_t)numel * dsize(t.dtype);
      if (t.off0 < 0 || t.off1 < t.off0 || (size_t)(t.off1 - t.off0) != bytes || t.shape.size() > QMM_MAX_DIM) {
        close_all();
        return QMM_WE_BAD_HEADER;
      }
      index.emplace(kept, items.size());
      items.push_back(Item{si, &t, kept, bytes});
    }
  }

  // 2) placement.  The packed weights (and, separately, the scales) of projections
  //    that share their input are placed back to back in one allocation, so one
  //    grouped call runs them as one matrix: each member's rows follow the previous
  //    member's.  Everything else gets its own allocation.
  static const std::vector<std::vector<const char *>> kGroups = {
      {"linear_attn.in_proj_qkv", "linear_attn.in_proj_z", "linear_attn.in_proj_b", "linear_attn.in_proj_a"},
      {"self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"},
      {"mlp.gate_proj", "mlp.up_proj"},
  };
  auto alloc = [&](void **dev, size_t bytes, const std::string &what) -> int {
    *dev = nullptr;
    if (!bytes) return 0;
    hipError_t e = hipMalloc(dev, bytes);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      fail("[qmm_weights_load] Unable to allocate %zu bytes for %s (out of memory)", bytes, what.c_str());
      return QMM_WE_IO;
    }
    m->buffers.push_back(*dev);
    return 0;
  };
  for (const char *kind : {".weight", ".scales"}) {
    const DType want = std::strcmp(kind, ".weight") == 0 ? DType::U32 : DType::U8;
    for (const auto &g : kGroups) {
      // the first member's tensors name the layers that have this group
      const std::string first = std::string(g[0]) + kind;
      for (auto &it : items) {
        if (!ends_with(it.kept, first.c_str()) || it.kept.size() == first.size() ||
            it.kept[it.kept.size() - first.size() - 1] != '.')
          continue;
        const std::string prefix = it.kept.substr(0, it.kept.size() - first.size());
        std::vector<Item *> mem;
        for (const char *name : g) {
          auto f = index.find(prefix + name + kind);
          if (f == index.end()) break;
          Item *x = &items[f->second];
          if (x->dev || x->t->dtype != want || x->t->shape.size() != 2 || x->t->shape[1] != it.t->shape[1]) break;
          mem.push_back(x);
        }
        if (mem.size() != g.size()) continue;
        // every member starts 256-byte aligned, as its own allocation would
        size_t total = 0;
        bool aligned = true;
        for (size_t j = 0; j < mem.size(); ++j) {
          aligned = aligned && (j + 1 == mem.size() || mem[j]->bytes % 256 == 0);
          total += mem[j]->bytes;
        }
        if (!aligned || !total) continue;
        void *base = nullptr;
        if (alloc(&base, total, prefix + g[0] + kind)) {
          close_all();
          return QMM_WE_IO;
        }
        size_t off = 0;
        for (Item *x : mem) {
          x->dev = (char *)base + off;
          off += x->bytes;
        }
      }
    }
  }
  for (auto &it : items) {
    if (it.dev || !it.bytes) continue;
    if (alloc(&it.dev, it.bytes, it.t->name)) {
      close_all();
      return QMM_WE_IO;
    }
  }

  // 3) raw copies: file -> pinned stage -> HBM, reads of at most 1 GiB
  const size_t kStage = 64ull << 20, kMaxRead = 1ull << 30;
  void *stage[2] = {nullptr, nullptr};
  hipEvent_t done[2];
  for (int i = 0; i < 2; ++i) {
    if (hipHostMalloc(&stage[i], kStage, hipHostMallocDefault) != hipSuccess) {
      (void)hipGetLastError();
      for (int j = 0; j < i; ++j) (void)hipHostFree(stage[j]);
      close_all();
      fail("[qmm_weights_load] Unable to allocate pinned staging buffer (out of memory)");
      return QMM_WE_IO;
    }
    (void)hipEventCreateWithFlags(&done[i], hipEventDisableTiming);
  }
  int cur = 0;
  bool used[2] = {false, false};
  auto cleanup = [&]() {
    (void)hipStreamSynchronize(st);
    for (int i = 0; i < 2; ++i) {
      (void)hipHostFree(stage[i]);
      (void)hipEventDestroy(done[i]);
    }
    close_all();
  };
  for (auto &it : items) {
    const int fd = fds[it.shard];
    const uint64_t data_start = data_starts[it.shard];
    size_t done_bytes = 0;
    while (done_bytes < it.bytes) {
      size_t n = it.bytes - done_bytes;
      if (n > kStage) n = kStage;
      if (n > kMaxRead) n = kMaxRead;
      if (used[cur]) (void)hipEventSynchronize(done[cur]);
      if (!pread_all(fd, stage[cur], n, (off_t)(data_start + it.t->off0 + done_bytes))) {
        cleanup();
        fail("[qmm_weights_load] short read in %s", (dir + "/" + shards[it.shard]).c_str());
        return QMM_WE_IO;
      }
      hipError_t e = hipMemcpyAsync((char *)it.dev + done_bytes, stage[cur], n, hipMemcpyHostToDevice, st);
      if (e == hipSuccess) e = hipEventRecord(done[cur], st);
      if (e != hipSuccess) {
        cleanup();
        fail_hip(e, "qmm_weights_load");
        return QMM_WE_IO;
      }
      used[cur] = true;
      cur ^= 1;
      done_bytes += n;
    }
    std::vector<int> shp(it.t->shape.begin(), it.t->shape.end());
    Arr *a = new_arr(shp.data(), (int)shp.size(), to_qmm(it.t->dtype));
    a->data = it.dev;
    a->owned = false;  // the map owns the buffer
    m->map.emplace(it.kept, a);
  }
  std::vector<TensorInfo> all;
  for (auto &v : shard_infos)
    for (auto &t : v) all.push_back(t);
  cleanup();
  rc = infer_quant_spec(all, &m->quant);
  if (rc) return rc;
  *out = m.release();
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

int qmm_weights_load(qmm_weight_map *res, const char *model_dir, qmm_stream s) {
  if (!res || !model_dir) return finish(fail("[qmm_weights_load] null argument"));
  WeightMap *m = nullptr;
  int rc = load_weights(model_dir, stream_of(s), &m);
  if (rc) return finish(rc);
  res->ctx = m;
  return finish(0);
}

int qmm_weights_free(qmm_weight_map m) {
  delete (WeightMap *)m.ctx;
  return 0;
}

qmm_array qmm_weights_get(qmm_weight_map m, const char *name) {
  WeightMap *w = (WeightMap *)m.ctx;
  if (!w || !name) return qmm_array{nullptr};
  auto it = w->map.find(name);
  return qmm_array{it == w->map.end() ? nullptr : it->second};
}

size_t qmm_weights_count(qmm_weight_map m) { return m.ctx ? ((WeightMap *)m.ctx)->map.size() : 0; }

qmm_quant_spec qmm_weights_quant(qmm_weight_map m) {
  return m.ctx ? ((WeightMap *)m.ctx)->quant : qmm_quant_spec{QMM_QUANT_NONE, 0, 0};
}

// namedLinearQ (src/model.zig:213-233) -> qlinear (src/model.zig:244-260) or linear (:200-211).
int qmm_named_linear_q(qmm_array *res, qmm_weight_map m, qmm_array x, const char *name, qmm_stream s) {
  WeightMap *wm = (WeightMap *)m.ctx;
  if (!wm || !name) return finish(fail("[named_linear_q] null weight map or name"));
  qmm_array w = qmm_weights_get(m, name);
  if (!w.ctx) return QMM_WE_MISSING_WEIGHT;
  if (wm->quant.mode == QMM_QUANT_NONE) return qmm_linear(res, x, w, s);
  std::string n(name);
  if (!ends_with(n, ".weight")) return QMM_WE_MISSING_WEIGHT;
  const std::string sname = n.substr(0, n.size() - 7) + ".scales";
  qmm_array sc = qmm_weights_get(m, sname.c_str());
  if (!sc.ctx) {
    if (((Arr *)w.ctx)->dtype == QMM_UINT32) return QMM_WE_MISSING_WEIGHT;
    return qmm_linear(res, x, w, s);
  }
  const char *mode = wm->quant.mode == QMM_QUANT_MXFP8 ? "mxfp8" : "nvfp4";
  return qmm_quantized_matmul(res, x, w, sc, qmm_array{nullptr}, true,
                              qmm_optional_int{(int)wm->quant.group_size, true},
                              qmm_optional_int{(int)wm->quant.bits, true}, mode, s);
}

// Several projections of one x by checkpoint names (the GDN layer's in_proj_qkv /
// z / b / a, src/model.zig:1066-1074; attention's q / k / v, :929-944): one grouped
// call (qmm_quantized_matmul_group) when every weight is packed with scales,
// otherwise named_linear_q per name.  res[i] is the result for names[i].
int qmm_named_linear_q_group(qmm_array *res, size_t n, qmm_weight_map m, qmm_array x, const char *const *names,
                             qmm_stream s) {
  WeightMap *wm = (WeightMap *)m.ctx;
  if (!wm || !names || !res) return finish(fail("[named_linear_q_group] null weight map, names or results"));
  if (n < 1 || n > 4) return finish(fail("[named_linear_q_group] takes 1 to 4 names, got %zu", n));
  qmm_array w[4], sc[4];
  bool packed = wm->quant.mode != QMM_QUANT_NONE;
  for (size_t i = 0; i < n; ++i) {
    if (!names[i]) return finish(fail("[named_linear_q_group] null name"));
    w[i] = qmm_weights_get(m, names[i]);
    if (!w[i].ctx) return QMM_WE_MISSING_WEIGHT;
    const std::string nm(names[i]);
    sc[i] = ends_with(nm, ".weight") ? qmm_weights_get(m, (nm.substr(0, nm.size() - 7) + ".scales").c_str())
                                     : qmm_array{nullptr};
    packed = packed && sc[i].ctx && ((Arr *)w[i].ctx)->dtype == QMM_UINT32;
  }
  if (packed) {
    const char *mode = wm->quant.mode == QMM_QUANT_MXFP8 ? "mxfp8" : "nvfp4";
    return qmm_quantized_matmul_group(res, n, x, w, sc, qmm_optional_int{(int)wm->quant.group_size, true},
                                      qmm_optional_int{(int)wm->quant.bits, true}, mode, s);
  }
  for (size_t i = 0; i < n; ++i) {
    const int rc = qmm_named_linear_q(&res[i], m, x, names[i], s);
    if (rc) return rc;
  }
  return 0;
}

// mlpForwardQ (src/model.zig:905-915): down(silu(gate(x)) * up(x)), the projections
// named as in the checkpoint ("....mlp.gate_proj.weight" etc.).  When gate and up
// are packed with scales the first three ops run fused (qmm_mlp_gate_up_silu);
// otherwise each goes through named_linear_q and the activation is qmm_silu_mul.
int qmm_mlp_forward_q(qmm_array *res, qmm_weight_map m, qmm_array x, const char *gate_name, const char *down_name,
                      const char *up_name, qmm_stream s) {
  WeightMap *wm = (WeightMap *)m.ctx;
  if (!wm || !gate_name || !down_name || !up_name) return finish(fail("[mlp_forward_q] null weight map or name"));
  auto scales_of = [&](const char *name) -> qmm_array {
    std::string n(name);
    if (!ends_with(n, ".weight")) return qmm_array{nullptr};
    return qmm_weights_get(m, (n.substr(0, n.size() - 7) + ".scales").c_str());
  };
  qmm_array wg = qmm_weights_get(m, gate_name), wu = qmm_weights_get(m, up_name);
  if (!wg.ctx || !wu.ctx) return QMM_WE_MISSING_WEIGHT;
  qmm_array sg = scales_of(gate_name), su = scales_of(up_name);
  qmm_array h{nullptr};
  int rc;
  if (wm->quant.mode != QMM_QUANT_NONE && sg.ctx && su.ctx) {
    const char *mode = wm->quant.mode == QMM_QUANT_MXFP8 ? "mxfp8" : "nvfp4";
    rc = qmm_mlp_gate_up_silu(&h, x, wg, sg, wu, su, qmm_optional_int{(int)wm->quant.group_size, true},
                              qmm_optional_int{(int)wm->quant.bits, true}, mode, s);
  } else {
    qmm_array g{nullptr}, u{nullptr};
    rc = qmm_named_linear_q(&g, m, x, gate_name, s);
    if (!rc) rc = qmm_named_linear_q(&u, m, x, up_name, s);
    if (!rc) rc = qmm_silu_mul(&h, g, u, s);
    if (g.ctx) qmm_array_free(g);
    if (u.ctx) qmm_array_free(u);
  }
  if (!rc) rc = qmm_named_linear_q(res, m, h, down_name, s);
  if (h.ctx) qmm_array_free(h);
  return rc;
}

}  // extern "C"
