// Host-only checkpoint parsing (no HIP): the safetensors header and index rules of
// mlx-runner's weight loader, shared by the HBM loader (weights.cpp) and the C ABI.
//   parseHeaderJson   src/weights.zig:70-121
//   inferQuantSpec    src/weights.zig:130-185
//   sanitizeName      src/weights.zig:186-202
//   checkShardFile    src/weights.zig:239-255
#pragma once
#include <stdint.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/qmm.h"

namespace qmm {

enum class DType { BF16, F32, U32, U8 };

struct TensorInfo {
  std::string name;
  DType dtype;
  std::vector<long long> shape;    // each in [0, INT32_MAX]
  long long off0 = -1, off1 = -1;  // data_offsets, relative to the data section
};

size_t dsize(DType d);
qmm_dtype to_qmm(DType d);
bool ends_with(const std::string &s, const char *suf);

int parse_header(const char *json, size_t len, std::vector<TensorInfo> &out);
int infer_quant_spec(const std::vector<TensorInfo> &infos, qmm_quant_spec *spec);
bool sanitize_name(const std::string &name, std::string &out);

// One tensor to load: its shard, header entry, name after sanitize_name and byte count.
struct CheckpointItem {
  size_t shard;
  const TensorInfo *t;
  std::string kept;
  uint64_t bytes;
};

// A sharded checkpoint's index and shard headers, read and checked; the shard files
// stay open (closed with the plan) for the loader's reads.
struct CheckpointPlan {
  std::vector<std::string> shards;
  std::vector<int> fds;
  std::vector<uint64_t> data_starts;             // file offset of each shard's data section
  std::vector<std::vector<TensorInfo>> infos;    // per shard
  std::vector<CheckpointItem> items;             // the tensors to load, in shard order
  std::unordered_map<std::string, size_t> index; // kept name -> items index
  CheckpointPlan() = default;
  CheckpointPlan(const CheckpointPlan &) = delete;
  CheckpointPlan &operator=(const CheckpointPlan &) = delete;
  ~CheckpointPlan();
  void close_files();
};

// Reads dir/model.safetensors.index.json and every shard's header (WeightMap.load's
// first half, src/weights.zig:257-300): returns 0 or a QMM_WE_* code, with a message
// in *err for the I/O failures.
int plan_checkpoint(const std::string &dir, CheckpointPlan &plan, std::string *err);

// pread until n bytes are read (false on error or end of file).
bool pread_all(int fd, void *buf, size_t n, long long off);

}  // namespace qmm
