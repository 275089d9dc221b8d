// flags.cpp -- the ANNC_FLAGS switch set.
//
// Same flag table, defaults, grammar and diagnostics as the reference parser
// (annc/service/cpu/annc_flags.cc:10-130):
//   * tokens are separated by spaces only; each must start with "--";
//   * "--key" or "--key=value"; value "true", "1" or "" enables, anything
//     else disables;
//   * "--gemm-opt" / "--graph-opt" enable every flag of type GEMM_OPT /
//     GRAPH_OPT whatever their value (so --gemm-opt leaves matmul-add,
//     matmul-add-relu and batch-matmul alone);
//   * an unknown key is reported on stderr and still stored;
//   * a token without "--" stops parsing.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "annc_hip.h"

namespace {

enum class OptType { kGraphOpt, kGemmOpt, kTfOpt, kNone };

struct FlagDef {
  const char* name;
  bool default_value;
  OptType type;
};

const std::vector<FlagDef>& flag_table() {
  static const std::vector<FlagDef> table = {
      {"matmul", false, OptType::kGemmOpt},
      {"layout-matmul", false, OptType::kGemmOpt},
      {"batch-matmul", false, OptType::kNone},
      {"matmul-add", false, OptType::kNone},
      {"matmul-add-relu", false, OptType::kNone},
      {"sps-emd-2", false, OptType::kGraphOpt},
      {"pooling", false, OptType::kNone},
      {"disable-tf-matmul-fusion", false, OptType::kGemmOpt},
      {"annc-pass", true, OptType::kTfOpt},
  };
  return table;
}

class FlagSet {
 public:
  FlagSet() { reset(); }

  void reset() {
    values_.clear();
    for (const FlagDef& f : flag_table()) values_[f.name] = f.default_value;
  }

  void parse(const std::string& str) {
    size_t pos = 0;
    const size_t n = str.size();
    auto skip_spaces = [&](size_t p) {
      while (p < n && str[p] == ' ') ++p;
      return p;
    };
    while (pos < n) {
      pos = skip_spaces(pos);
      if (pos >= n) break;
      if (str.compare(pos, 2, "--") != 0) {
        std::fprintf(stderr,
                     "[ANNC ERROR] Invalid flag syntax: expected '--' at position%zu in: %s\n",
                     pos, str.c_str());
        break;
      }
      pos += 2;
      const size_t key_start = pos;
      while (pos < n && str[pos] != '=' && str[pos] != ' ') ++pos;
      const bool has_value = pos < n && str[pos] == '=';
      std::string key = str.substr(key_start, pos - key_start);
      std::string value = "true";
      if (has_value) {
        size_t val_end = pos + 1;
        while (val_end < n && str[val_end] != ' ') ++val_end;
        value = str.substr(pos + 1, val_end - pos - 1);
        pos = val_end;
      } else {
        pos = skip_spaces(pos);
      }
      if (key == "graph-opt" || key == "gemm-opt") {
        const OptType group = key == "graph-opt" ? OptType::kGraphOpt : OptType::kGemmOpt;
        for (const FlagDef& f : flag_table())
          if (f.type == group) values_[f.name] = true;
        continue;
      }
      if (values_.find(key) == values_.end()) {
        std::fprintf(stderr, "[ANNC ERROR] Unknown flag: '%s'. Valid flags are:", key.c_str());
        for (const FlagDef& f : flag_table()) std::fprintf(stderr, "%s\n", f.name);
      }
      const bool enable = value == "true" || value == "1" || value.empty();
      values_[key] = enable;
      if (enable) std::printf("enabled flag : --%s\n", key.c_str());
    }
    std::fflush(stdout);
  }

  bool enabled(const std::string& name) const {
    auto it = values_.find(name);
    return it != values_.end() && it->second;
  }

  std::string dump() const {
    std::string s;
    for (const auto& kv : values_) s += kv.first + "=" + (kv.second ? "1" : "0") + "\n";
    return s;
  }

 private:
  std::map<std::string, bool> values_;
};

std::mutex g_flags_mu;

FlagSet& flags() {
  static FlagSet* set = [] {
    FlagSet* s = new FlagSet();
    const char* env = std::getenv("ANNC_FLAGS");
    if (env && env[0] != '\0') s->parse(env);
    return s;
  }();
  return *set;
}

}  // namespace

extern "C" {

int annc_flag_enabled(const char* name) {
  if (!name) return 0;
  std::lock_guard<std::mutex> lock(g_flags_mu);
  return flags().enabled(name) ? 1 : 0;
}

void annc_flags_reset(const char* str) {
  std::lock_guard<std::mutex> lock(g_flags_mu);
  flags().reset();
  if (str && str[0] != '\0') flags().parse(str);
}

int64_t annc_flags_dump(char* buf, int64_t len) {
  std::lock_guard<std::mutex> lock(g_flags_mu);
  std::string s = flags().dump();
  if (buf && len > 0) {
    size_t k = s.size() < static_cast<size_t>(len - 1) ? s.size() : static_cast<size_t>(len - 1);
    std::memcpy(buf, s.data(), k);
    buf[k] = '\0';
  }
  return static_cast<int64_t>(s.size());
}

}  // extern "C"
