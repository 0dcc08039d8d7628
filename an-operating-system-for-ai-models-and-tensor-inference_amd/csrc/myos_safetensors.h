// Read-only SafeTensors map (8-byte little-endian header length, JSON header,
// payload). Mirrors crates/weight_loader: SafeTensorsMmap::open/parse
// (mmap.rs:82-100) and SafeTensorsWeights::parse (safe_tensors.rs:30-43).
#pragma once
#include <stddef.h>
#include <stdint.h>

#include <map>
#include <string>
#include <vector>

namespace myos {

enum class StDType { F32, F16, BF16 };

struct StTensor {
  StDType dtype;
  std::vector<size_t> shape;
  const uint8_t *data;  // points into the mapping
  size_t nbytes;
};

class SafeTensorsFile {
 public:
  SafeTensorsFile() = default;
  ~SafeTensorsFile();
  SafeTensorsFile(const SafeTensorsFile &) = delete;
  SafeTensorsFile &operator=(const SafeTensorsFile &) = delete;

  // Returns a MYOS_E_* status: IO (open/map), PARSE (header, dtype outside
  // F32/F16/BF16, empty or duplicate name, offsets), W_LENGTH (payload length
  // disagrees with shape x dtype).
  int open(const char *path);
  const StTensor *find(const std::string &name) const;
  // bf16_tensor (qwen25_bf16.rs:72-82): W_MISSING, W_DTYPE, W_SHAPE or OK.
  int bf16(const std::string &name, const std::vector<size_t> &expect,
           const uint16_t **out) const;
  size_t size() const { return tensors_.size(); }
  size_t file_bytes() const { return len_; }

 private:
  void *map_ = nullptr;
  size_t len_ = 0;
  std::map<std::string, StTensor> tensors_;
};

}  // namespace myos
