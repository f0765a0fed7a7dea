// C++17 face of the QWENBIN1 archive code: infer::ModelArchive
// (include/infer/archive.hpp:22-52 of Greedy-cy/qwen2.5-jetson-inference),
// ModelConfig::load (include/infer/model_config.hpp:7-24) and the exporter
// of tools/export_model.py:273-396, with the same names and meaning.  Errors
// throw infer::Error with the reference's messages.  Header-only over the C
// ABI of include/infer_archive.h; link with libinfer_linear.so.  Host-only:
// nothing here touches the GPU.
#pragma once

#include <cstddef>
#include <cstdint>
#include <optional>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

#include "infer/linear_dispatch.hpp"
#include "infer/linear_hip.hpp"
#include "infer_archive.h"

namespace infer {

// infer::DType (include/infer/common.hpp:10) is linear_dispatch.hpp's; the
// archive ABI numbers its dtypes the same way.
static_assert(static_cast<int>(DType::kFloat32) == INFER_HIP_DTYPE_FLOAT32 &&
                  static_cast<int>(DType::kBFloat16) == INFER_HIP_DTYPE_BFLOAT16 &&
                  static_cast<int>(DType::kInt8) == INFER_HIP_DTYPE_INT8,
              "archive dtype codes");
using Shape = std::vector<int64_t>;

// include/infer/archive.hpp:7-11.
struct QuantizationInfo {
  int group_size{0};
  int axis{1};
  std::string scale_tensor;
};

// include/infer/archive.hpp:13-20 (plus the recorded SHA-256).
struct TensorRecord {
  std::string name;
  Shape shape;
  DType dtype{DType::kFloat32};
  uint64_t offset{0};
  uint64_t nbytes{0};
  std::optional<QuantizationInfo> quant;
  std::string sha256;
};

// include/infer/archive.hpp:22-52: a read-only mapping of one archive.
class ModelArchive {
 public:
  ModelArchive() = default;
  explicit ModelArchive(const std::string& path) { open(path); }
  ~ModelArchive() { close(); }
  ModelArchive(const ModelArchive&) = delete;
  ModelArchive& operator=(const ModelArchive&) = delete;
  ModelArchive(ModelArchive&& other) noexcept { *this = std::move(other); }
  ModelArchive& operator=(ModelArchive&& other) noexcept {
    if (this != &other) {
      close();
      handle_ = other.handle_;
      path_ = std::move(other.path_);
      records_ = std::move(other.records_);
      index_ = std::move(other.index_);
      other.handle_ = nullptr;
    }
    return *this;
  }

  void open(const std::string& path) {
    close();
    hip::check(infer_hip_archive_open(path.c_str(), &handle_));
    path_ = path;
    const int count = infer_hip_archive_tensor_count(handle_);
    for (int i = 0; i < count; ++i) {
      infer_hip_tensor_record r;
      hip::check(infer_hip_archive_record(handle_, i, &r));
      TensorRecord rec;
      rec.name = r.name;
      rec.shape.assign(r.shape, r.shape + r.ndim);
      rec.dtype = static_cast<DType>(r.dtype);
      rec.offset = r.offset;
      rec.nbytes = r.nbytes;
      if (r.quant_group_size > 0) {
        rec.quant = QuantizationInfo{r.quant_group_size, r.quant_axis, r.scale_tensor};
      }
      rec.sha256 = r.sha256;
      index_.emplace(rec.name, records_.size());
      records_.push_back(std::move(rec));
    }
  }
  void close() {
    (void)infer_hip_archive_close(handle_);
    handle_ = nullptr;
    records_.clear();
    index_.clear();
  }
  const TensorRecord& record(std::string_view name) const {
    return records_[position(name)];
  }
  const void* data(std::string_view name) const {
    return infer_hip_archive_data(handle_, static_cast<int>(position(name)));
  }
  bool contains(std::string_view name) const { return index_.count(std::string(name)) != 0; }
  const std::vector<TensorRecord>& records() const { return records_; }
  uint64_t data_offset() const { return infer_hip_archive_data_offset(handle_); }
  size_t mapped_bytes() const { return infer_hip_archive_mapped_bytes(handle_); }
  const std::string& path() const { return path_; }
  std::string precision() const { return infer_hip_archive_precision(handle_); }
  // tools/export_model.py:148-199 (alignment and SHA-256 of every payload).
  void verify() const { hip::check(infer_hip_archive_verify(handle_)); }

 private:
  size_t position(std::string_view name) const {
    const auto it = index_.find(std::string(name));
    if (it == index_.end()) throw Error("missing tensor: " + std::string(name));
    return it->second;
  }

  infer_hip_archive* handle_{nullptr};
  std::string path_;
  std::vector<TensorRecord> records_;
  std::unordered_map<std::string, size_t> index_;
};

// include/infer/model_config.hpp:7-24 (the fields this runtime reads).
struct ModelConfig {
  infer_hip_model_config c{};
  int max_position_embeddings{0};

  static ModelConfig load(const std::string& path) {
    ModelConfig m;
    hip::check(infer_hip_model_config_load(path.c_str(), &m.c, &m.max_position_embeddings));
    return m;
  }
};

// One FP32 source tensor of an export (a safetensors tensor read by the
// caller), row-major.
struct SourceTensor {
  std::string name;
  Shape shape;
  const float* data{nullptr};
};

// export() (tools/export_model.py:273-368) over FP32 tensors in memory.
inline infer_hip_export_report export_archive(const std::string& destination,
                                              const std::vector<SourceTensor>& tensors,
                                              const std::string& precision, int group_size = 64,
                                              const std::string& source = "") {
  std::vector<infer_hip_export_tensor> table;
  table.reserve(tensors.size());
  for (const SourceTensor& t : tensors) {
    table.push_back(infer_hip_export_tensor{t.name.c_str(), static_cast<int>(t.shape.size()),
                                            t.shape.data(), t.data});
  }
  infer_hip_export_report report{};
  hip::check(infer_hip_archive_export(destination.c_str(), precision.c_str(), group_size,
                                      table.data(), static_cast<int>(table.size()),
                                      source.c_str(), &report));
  return report;
}

}  // namespace infer
