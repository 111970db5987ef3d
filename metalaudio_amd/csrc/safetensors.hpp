// SafeTensors reader (SafeTensorsLoader.swift:41-660): an 8-byte little-endian header length, a
// UTF-8 JSON header {name: {"dtype", "shape", "data_offsets": [begin, end]}, "__metadata__": {…}}
// and the raw tensor bytes (offsets relative to the end of the header). Host-only; tensors are
// converted to fp32 on read (F32, F16, BF16, I32, I64, I16, I8, U8, BOOL, as the reference).
#pragma once

#include <cstdint>
#include <cstdio>
#include <map>
#include <string>
#include <vector>

namespace mnn {

enum StDType { ST_F32 = 0, ST_F16, ST_BF16, ST_I32, ST_I64, ST_I16, ST_I8, ST_U8, ST_BOOL };

struct StTensorInfo {
  StDType dtype = ST_F32;
  std::vector<int64_t> shape;
  uint64_t begin = 0, end = 0;  // byte offsets in the data section
  int64_t count() const;        // elements the byte range holds (end - begin) / dtype size
};

class SafeTensorsFile {
 public:
  // Largest accepted JSON header (SafeTensorsLoader.maxHeaderSize).
  static constexpr uint64_t kMaxHeader = 100ull * 1024 * 1024;
  explicit SafeTensorsFile(const std::string& path);
  ~SafeTensorsFile();
  SafeTensorsFile(const SafeTensorsFile&) = delete;
  SafeTensorsFile& operator=(const SafeTensorsFile&) = delete;
  // availableTensors (sorted names)
  const std::vector<std::string>& names() const { return names_; }
  const StTensorInfo& info(const std::string& name) const;
  // loadTensor(name:): all of the tensor's elements as fp32; NaN / Inf are rejected
  void read_f32(const std::string& name, float* out, size_t count) const;
  const std::map<std::string, std::string>& metadata() const { return meta_; }

 private:
  std::string path_;
  FILE* f_ = nullptr;
  uint64_t data_start_ = 0, data_size_ = 0;
  std::map<std::string, StTensorInfo> infos_;
  std::vector<std::string> names_;
  std::map<std::string, std::string> meta_;
};

size_t st_dtype_size(StDType t);
// IEEE half -> single (exact: every half is a float).
float st_half_to_float(uint16_t h);

}  // namespace mnn

namespace mnn {

// "MTLA" binary model file (BinaryModelLoader, Model.swift:401-679): header magic 0x4D544C41,
// version (2, or the legacy 1), tensor count, CRC-32 of everything after the header (v2 only),
// reserved; then per tensor: name length, rank, data type (0 = f32), data bytes (u32 each),
// UTF-8 name, u32 dims, fp32 data. Read whole, validated like the reference (name < 1024 bytes,
// rank <= 16, overflow-checked element counts, declared bytes == 4 * elements, bounds).
class MtlaFile {
 public:
  static constexpr uint32_t kMagic = 0x4D544C41u;
  explicit MtlaFile(const std::string& path);
  const std::vector<std::string>& names() const { return names_; }
  const std::vector<int64_t>& shape(const std::string& name) const;
  const std::vector<float>& data(const std::string& name) const;

 private:
  std::map<std::string, std::pair<std::vector<int64_t>, std::vector<float>>> t_;
  std::vector<std::string> names_;
};

// BinaryModelLoader.save: version 2, tensors in name order, CRC-32 over the entries.
void mtla_write(const std::string& path,
                const std::map<std::string, std::pair<std::vector<int64_t>, std::vector<float>>>& t);

// Reflected CRC-32 (polynomial 0xEDB88320), as computeCRC32 (Model.swift:431-449).
uint32_t crc32_ieee(const unsigned char* p, size_t n, uint32_t crc = 0);

}  // namespace mnn
