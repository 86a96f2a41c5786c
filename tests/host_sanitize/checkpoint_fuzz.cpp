// Host sanitizer driver for the checkpoint parser (mlx-runner_amd/csrc/checkpoint.cpp),
// built with g++ -fsanitize=address,undefined by tests/test_host_sanitize.py.
//
//   checkpoint_fuzz header <file>...        parse each file as one safetensors header JSON
//   checkpoint_fuzz mutate <n> <file>...    n seeded mutations of each header, parsed
//   checkpoint_fuzz dir <dir>...            read each checkpoint directory's index and headers
//
// Prints one line per case: "<what> rc=<code>".  Every return code must be 0 or a
// QMM_WE_* code; the sanitizers abort on any memory or undefined-behaviour error.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <sstream>
#include <string>

#include "../../mlx-runner_amd/csrc/checkpoint.h"

static std::string slurp(const char *path) {
  std::ifstream f(path, std::ios::binary);
  std::stringstream ss;
  ss << f.rdbuf();
  return ss.str();
}

static bool valid_rc(int rc) { return rc == 0 || (rc >= QMM_WE_BAD_INDEX_JSON && rc <= QMM_WE_MISSING_WEIGHT); }

static int parse_both(const std::string &h) {
  size_t n = 0;
  qmm_quant_spec spec;
  const int a = qmm_parse_header_json(h.data(), h.size(), &n);
  const int b = qmm_infer_quant_spec_json(h.data(), h.size(), &spec, &n);
  if (!valid_rc(a) || !valid_rc(b)) {
    std::printf("invalid return code %d / %d\n", a, b);
    std::exit(3);
  }
  // the names a header holds go through the remap too
  char out[64];
  (void)qmm_sanitize_name(h.c_str(), out, sizeof out);
  return b;
}

int main(int argc, char **argv) {
  if (argc < 3) return 2;
  const std::string mode = argv[1];
  if (mode == "header") {
    for (int i = 2; i < argc; ++i) std::printf("%s rc=%d\n", argv[i], parse_both(slurp(argv[i])));
    return 0;
  }
  if (mode == "mutate") {
    const int n = std::atoi(argv[2]);
    uint64_t st = 0x9E3779B97F4A7C15ull;
    auto rnd = [&]() {  // splitmix64
      st += 0x9E3779B97F4A7C15ull;
      uint64_t z = st;
      z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
      z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
      return z ^ (z >> 31);
    };
    static const char *const kTokens[] = {"-1", "2147483648", "9223372036854775807", "99999999999999999999",
                                          "1e309", "\"", "\\u00", "{", "}", "[", "]", ",", ":", "null", "-",
                                          "0.5", "\"shape\"", "\"dtype\"", "\"U32\"", "\"data_offsets\""};
    for (int f = 3; f < argc; ++f) {
      const std::string base = slurp(argv[f]);
      int counts[2] = {0, 0};
      for (int k = 0; k < n; ++k) {
        std::string h = base;
        const int edits = 1 + (int)(rnd() % 4);
        for (int e = 0; e < edits && !h.empty(); ++e) {
          const size_t at = rnd() % h.size();
          switch (rnd() % 4) {
            case 0: h[at] = (char)(rnd() & 0xFF); break;                   // flip a byte
            case 1: h.resize(at); break;                                   // truncate
            case 2: h.insert(at, kTokens[rnd() % (sizeof kTokens / sizeof *kTokens)]); break;
            default: h.erase(at, 1 + rnd() % 8); break;                    // drop a few bytes
          }
        }
        counts[parse_both(h) == 0] += 1;
      }
      std::printf("%s mutations=%d accepted=%d rejected=%d\n", argv[f], n, counts[1], counts[0]);
    }
    return 0;
  }
  if (mode == "dir") {
    for (int i = 2; i < argc; ++i) {
      qmm::CheckpointPlan plan;
      std::string err;
      const int rc = qmm::plan_checkpoint(argv[i], plan, &err);
      if (!valid_rc(rc)) return 3;
      std::printf("%s rc=%d tensors=%zu\n", argv[i], rc, plan.items.size());
    }
    return 0;
  }
  return 2;
}
