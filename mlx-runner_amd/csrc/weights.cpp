// Host mirror of mlx-runner's weight loading and linear dispatch (the header and
// index parsing is in checkpoint.cpp):
//   WeightMap.load    src/weights.zig:257-352 (here: raw bytes at data_offsets -> HBM)
//   namedLinearQ      src/model.zig:213-233, qlinear :244-260, linear :200-211
//
// The loader reads each tensor's bytes at its `data_offsets` (which the
// reference ignores, src/weights.zig:91-92) in chunks of at most 1 GiB through
// a pinned staging buffer, and copies them to HBM unchanged: U32 packed
// weights and U8 scales land exactly as the kernels consume them.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "../../include/qmm.h"
#include "checkpoint.h"
#include "qmm_internal.h"

namespace qmm {

// ---------------------------------------------------------------- WeightMap
struct WeightMap {
  std::unordered_map<std::string, Arr *> map;
  std::vector<void *> buffers;  // hipMalloc'd tensor buffers
  qmm_quant_spec quant{QMM_QUANT_NONE, 0, 0};
  ~WeightMap() {
    for (auto &kv : map) {  // the tensor buffers are freed below; a scales handle's tile-major copy here
      release_tiled(kv.second);
      delete kv.second;
    }
    for (void *b : buffers) (void)hipFree(b);
  }
};

int load_weights(const std::string &dir, hipStream_t st, WeightMap **out) {
  CheckpointPlan plan;
  std::string err;
  int rc = plan_checkpoint(dir, plan, &err);
  if (rc) {
    if (!err.empty()) fail("[qmm_weights_load] %s", err.c_str());
    return rc;
  }
  std::unique_ptr<WeightMap> m(new WeightMap());
  auto &items = plan.items;
  auto &index = plan.index;
  std::vector<void *> dev(items.size(), nullptr);  // destination of each item in HBM
  auto close_all = [&]() { plan.close_files(); };

  // 2) placement.  The packed weights (and, separately, the scales) of projections
  //    that share their input are placed back to back in one allocation, so one
  //    grouped call runs them as one matrix: each member's rows follow the previous
  //    member's.  Everything else gets its own allocation.
  static const std::vector<std::vector<const char *>> kGroups = {
      {"linear_attn.in_proj_qkv", "linear_attn.in_proj_z", "linear_attn.in_proj_b", "linear_attn.in_proj_a"},
      {"self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"},
      {"mlp.gate_proj", "mlp.up_proj"},
  };
  auto alloc = [&](void **p, size_t bytes, const std::string &what) -> int {
    *p = nullptr;
    if (!bytes) return 0;
    hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      fail("[qmm_weights_load] Unable to allocate %zu bytes for %s (out of memory)", bytes, what.c_str());
      return QMM_WE_IO;
    }
    m->buffers.push_back(*p);
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
        std::vector<size_t> mem;  // items indices of the members
        for (const char *name : g) {
          auto f = index.find(prefix + name + kind);
          if (f == index.end()) break;
          const CheckpointItem &x = items[f->second];
          if (dev[f->second] || x.t->dtype != want || x.t->shape.size() != 2 || x.t->shape[1] != it.t->shape[1])
            break;
          mem.push_back(f->second);
        }
        if (mem.size() != g.size()) continue;
        // every member starts 256-byte aligned, as its own allocation would
        size_t total = 0;
        bool aligned = true;
        for (size_t j = 0; j < mem.size(); ++j) {
          aligned = aligned && (j + 1 == mem.size() || items[mem[j]].bytes % 256 == 0);
          total += items[mem[j]].bytes;
        }
        if (!aligned || !total) continue;
        void *base = nullptr;
        if (alloc(&base, total, prefix + g[0] + kind)) {
          close_all();
          return QMM_WE_IO;
        }
        size_t off = 0;
        for (size_t j : mem) {
          dev[j] = (char *)base + off;
          off += items[j].bytes;
        }
      }
    }
  }
  for (size_t i = 0; i < items.size(); ++i) {
    if (dev[i] || !items[i].bytes) continue;
    if (alloc(&dev[i], items[i].bytes, items[i].t->name)) {
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
    const hipError_t e = hipEventCreateWithFlags(&done[i], hipEventDisableTiming);
    if (e != hipSuccess) {
      for (int j = 0; j <= i; ++j) (void)hipHostFree(stage[j]);
      for (int j = 0; j < i; ++j) (void)hipEventDestroy(done[j]);
      close_all();
      fail_hip(e, "qmm_weights_load");
      return QMM_WE_IO;
    }
  }
  int cur = 0;
  bool used[2] = {false, false};
  // waits for the copies in flight (a failed one reports here), then frees the staging
  auto cleanup = [&]() -> hipError_t {
    const hipError_t e = hipStreamSynchronize(st);
    for (int i = 0; i < 2; ++i) {
      (void)hipHostFree(stage[i]);
      (void)hipEventDestroy(done[i]);
    }
    close_all();
    return e;
  };
  for (size_t i = 0; i < items.size(); ++i) {
    const CheckpointItem &it = items[i];
    const int fd = plan.fds[it.shard];
    const uint64_t data_start = plan.data_starts[it.shard];
    size_t done_bytes = 0;
    while (done_bytes < it.bytes) {
      size_t n = it.bytes - done_bytes;
      if (n > kStage) n = kStage;
      if (n > kMaxRead) n = kMaxRead;
      if (used[cur]) {  // the copy out of this staging buffer must be done before it is refilled
        const hipError_t e = hipEventSynchronize(done[cur]);
        if (e != hipSuccess) {
          (void)cleanup();
          fail_hip(e, "qmm_weights_load");
          return QMM_WE_IO;
        }
      }
      if (!pread_all(fd, stage[cur], n, (long long)(data_start + it.t->off0 + done_bytes))) {
        (void)cleanup();
        fail("[qmm_weights_load] short read in %s", (dir + "/" + plan.shards[it.shard]).c_str());
        return QMM_WE_IO;
      }
      hipError_t e = hipMemcpyAsync((char *)dev[i] + done_bytes, stage[cur], n, hipMemcpyHostToDevice, st);
      if (e == hipSuccess) e = hipEventRecord(done[cur], st);
      if (e != hipSuccess) {
        (void)cleanup();
        fail_hip(e, "qmm_weights_load");
        return QMM_WE_IO;
      }
      used[cur] = true;
      cur ^= 1;
      done_bytes += n;
    }
    std::vector<int> shp(it.t->shape.begin(), it.t->shape.end());
    Arr *a = new_arr(shp.data(), (int)shp.size(), to_qmm(it.t->dtype));
    a->data = dev[i];
    a->owned = false;  // the map owns the buffer
    m->map.emplace(it.kept, a);
  }
  std::vector<TensorInfo> all;
  for (auto &v : plan.infos)
    for (auto &t : v) all.push_back(t);
  const hipError_t e = cleanup();
  if (e != hipSuccess) {
    fail_hip(e, "qmm_weights_load");
    return QMM_WE_IO;
  }
  rc = infer_quant_spec(all, &m->quant);
  if (rc) return rc;
  *out = m.release();
  return 0;
}

}  // namespace qmm

using namespace qmm;

extern "C" {

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
