// Safetensors pack reader: a directory of *.safetensors shards + config.json, each shard mmapped read-only once.
// Reference: core/pack.h:19-74, core/pack.mm:52-174 (header parse, one mapping per file).
#pragma once
#include <map>
#include <string>
#include <vector>

#include "common.h"

namespace ijah {

struct TensorInfo {
  int dtype = -1;
  int ndim = 0;
  int64_t shape[NE_MAX_DIMS] = {0};
  uint64_t nbytes = 0;
  int file = -1;
  uint64_t file_offset = 0;    // absolute offset of the data in the shard
  const void *host = nullptr;  // inside the read-only mapping
  int64_t numel() const {
    int64_t n = 1;
    for (int i = 0; i < ndim; i++) n *= shape[i];
    return n;
  }
};

class Pack {
 public:
  static std::unique_ptr<Pack> open(const std::string &dir);
  ~Pack();
  const TensorInfo *info(const std::string &name) const;
  bool has(const std::string &name) const { return info(name) != nullptr; }
  // the tensor, checked for dtype and dims (-1 = any); throws with the tensor name on mismatch
  const TensorInfo &need(const std::string &name, int dtype, std::initializer_list<int64_t> shape) const;
  const std::vector<std::string> &names() const { return names_; }
  const std::string &config() const { return config_; }
  const std::string &file(int i) const { return files_[i]; }

 private:
  std::string dir_, config_;
  std::vector<std::string> files_;
  std::vector<std::pair<void *, size_t>> maps_;
  std::map<std::string, TensorInfo> tensors_;
  std::vector<std::string> names_;
};

int dtype_from_name(const std::string &s);  // "BF16" -> NE_BF16, -1 if unknown
const char *dtype_name(int dt);
int dtype_size(int dt);

}  // namespace ijah

struct ne_pack {
  std::unique_ptr<ijah::Pack> pack;
  std::map<std::string, ne_buf *> bufs;  // pack-owned device copies, made on first ne_tensor_info
};
