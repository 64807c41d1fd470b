// gguf.h -- GGUF v3 container: reader (mmap or owned bytes) and writer.
//
// Mirrors Tsuskov/talos src/gguf/{mod,reader,dtype}.rs: header, typed
// metadata (UINT32=4, INT32=5, FLOAT32=6, BOOL=7, STRING=8, ARRAY=9 with
// STRING/INT32/FLOAT32 elements), tensor index, 32-byte aligned data section.
// Errors are thrown as talos::Error with the reference's messages.
#pragma once
#include <cstddef>
#include <cstdint>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

namespace talos {

struct Error : std::runtime_error {
  using std::runtime_error::runtime_error;
};

// A failed backend call: keeps the talos_status it returned.
struct BackendError : Error {
  BackendError(int status, const char* msg) : Error(msg ? msg : "backend error"), status(status) {}
  int status;
};

// GGML tensor types (src/gguf/dtype.rs:22-41).
enum class GgmlType : uint32_t { F32 = 0, Q4_0 = 2, Q8_0 = 8, Q6K = 14 };
bool ggml_type_from_u32(uint32_t tag, GgmlType* out);
size_t block_elems(GgmlType t);
size_t block_bytes(GgmlType t);
// dequantize (src/gguf/dtype.rs:64-121): n elements, n % block_elems == 0.
void dequantize(GgmlType t, const uint8_t* raw, float* out, size_t n);

struct MetaValue {
  enum Kind { U32, F32, Bool, Str, ArrStr, ArrI32, ArrF32 } kind = U32;
  uint32_t u32 = 0;
  float f32 = 0.f;
  bool b = false;
  std::string str;
  std::vector<std::string> arr_str;
  std::vector<int32_t> arr_i32;
  std::vector<float> arr_f32;
};

struct TensorInfo {
  std::string name;
  std::vector<uint64_t> dims;  // ne order: a row-major [rows, cols] has dims [cols, rows]
  GgmlType dtype = GgmlType::F32;
  uint64_t offset = 0;         // relative to the data section
  size_t elem_count() const;
};

class GgufFile {
 public:
  static GgufFile open(const std::string& path);       // mmap (reader.rs:177-185)
  static GgufFile from_bytes(std::vector<uint8_t> b);  // reader.rs:189-191
  GgufFile(GgufFile&&) noexcept;
  GgufFile& operator=(GgufFile&&) noexcept;
  GgufFile(const GgufFile&) = delete;
  ~GgufFile();

  const MetaValue* metadata(const std::string& key) const;
  bool get_u32(const std::string& key, uint32_t* out) const;
  bool get_f32(const std::string& key, float* out) const;
  const std::string* get_str(const std::string& key) const;
  const std::vector<std::string>* get_arr_str(const std::string& key) const;
  const std::vector<int32_t>* get_arr_i32(const std::string& key) const;
  const std::vector<float>* get_arr_f32(const std::string& key) const;

  const std::vector<TensorInfo>& tensors() const { return tensors_; }
  const TensorInfo* tensor_info(const std::string& name) const;
  // Zero-copy F32 view (reader.rs:302-324).
  const float* tensor_f32(const std::string& name, size_t* n) const;
  // Raw bytes + type (reader.rs:328-351).
  const uint8_t* tensor_raw(const std::string& name, size_t* len, GgmlType* type) const;

  const uint8_t* data() const { return data_; }
  size_t size() const { return size_; }

 private:
  GgufFile() = default;
  void parse();
  std::vector<uint8_t> owned_;
  void* map_ = nullptr;
  size_t map_len_ = 0;
  const uint8_t* data_ = nullptr;
  size_t size_ = 0;
  std::map<std::string, MetaValue> meta_;
  std::vector<TensorInfo> tensors_;
  std::map<std::string, size_t> by_name_;
  size_t data_start_ = 0;
};

// Writer with the byte layout the reader expects (as the reference's test
// writers do, tests/gqa.rs:25-108 and tests/forward_gpu.rs:288-371).
class GgufWriter {
 public:
  void u32(const std::string& k, uint32_t v);
  void f32(const std::string& k, float v);
  void boolean(const std::string& k, bool v);
  void str(const std::string& k, const std::string& v);
  void arr_str(const std::string& k, const std::vector<std::string>& v);
  void arr_i32(const std::string& k, const std::vector<int32_t>& v);
  void arr_f32(const std::string& k, const std::vector<float>& v);
  // dims in ne order; `bytes` already in the type's block layout.
  void tensor(const std::string& name, std::vector<uint64_t> dims, GgmlType t, std::vector<uint8_t> bytes);
  // Declare a tensor whose bytes are written later by finish_fill().
  void tensor_sized(const std::string& name, std::vector<uint64_t> dims, GgmlType t, size_t nbytes);
  std::vector<uint8_t> finish() const;
  // Lay out the file, then let fill(i, dst) write tensor i's bytes in place.
  template <class Fill>
  std::vector<uint8_t> finish_fill(Fill fill) const {
    std::vector<size_t> offs;
    std::vector<uint8_t> buf = layout(&offs);
    for (size_t i = 0; i < tensors_.size(); ++i) fill(i, buf.data() + offs[i]);
    return buf;
  }

 private:
  std::vector<uint8_t> kv_;
  uint64_t n_kv_ = 0;
  struct T {
    std::string name;
    std::vector<uint64_t> dims;
    GgmlType type;
    std::vector<uint8_t> bytes;
    size_t nbytes;
  };
  // Header + zero-filled data section; offs[i] = absolute offset of tensor i.
  std::vector<uint8_t> layout(std::vector<size_t>* offs) const;
  std::vector<T> tensors_;
};

}  // namespace talos
