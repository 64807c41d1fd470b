// gguf.cpp -- GGUF v3 reader/writer (see gguf.h).
#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>

namespace talos {

namespace {
constexpr size_t kAlign = 32;  // reader.rs:22
enum : uint32_t { T_UINT32 = 4, T_INT32 = 5, T_FLOAT32 = 6, T_BOOL = 7, T_STRING = 8, T_ARRAY = 9 };

float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      const float v = (float)man * 5.9604644775390625e-8f;
      return sign ? -v : v;
    }
  } else if (exp == 31) {
    bits = sign | 0x7F800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

struct Cursor {
  const uint8_t* b;
  size_t len, pos = 0;
  const uint8_t* take(size_t n) {
    if (n > len - pos) throw Error("GGUF data ends early: wanted " + std::to_string(n) + " bytes at " +
                                   std::to_string(pos) + ")");
    const uint8_t* p = b + pos;
    pos += n;
    return p;
  }
  uint32_t u32() {
    uint32_t v;
    memcpy(&v, take(4), 4);
    return v;
  }
  int32_t i32() {
    int32_t v;
    memcpy(&v, take(4), 4);
    return v;
  }
  uint64_t u64() {
    uint64_t v;
    memcpy(&v, take(8), 8);
    return v;
  }
  float f32() {
    float v;
    memcpy(&v, take(4), 4);
    return v;
  }
  std::string str() {
    const uint64_t n = u64();
    if (n > len - pos) throw Error("GGUF data ends early: wanted " + std::to_string(n) + " bytes at " +
                                   std::to_string(pos) + ")");
    const uint8_t* p = take((size_t)n);
    return std::string(reinterpret_cast<const char*>(p), (size_t)n);
  }
};

// reader.rs:135-171
MetaValue read_value(Cursor& c, uint32_t tag) {
  MetaValue v;
  switch (tag) {
    case T_UINT32: v.kind = MetaValue::U32; v.u32 = c.u32(); return v;
    case T_FLOAT32: v.kind = MetaValue::F32; v.f32 = c.f32(); return v;
    case T_BOOL: v.kind = MetaValue::Bool; v.b = c.take(1)[0] != 0; return v;
    case T_STRING: v.kind = MetaValue::Str; v.str = c.str(); return v;
    case T_ARRAY: {
      const uint32_t inner = c.u32();
      const uint64_t count = c.u64();
      if (inner == T_STRING) {
        v.kind = MetaValue::ArrStr;
        for (uint64_t i = 0; i < count; ++i) v.arr_str.push_back(c.str());
      } else if (inner == T_INT32) {
        v.kind = MetaValue::ArrI32;
        if (count > (c.len - c.pos) / 4) c.take(c.len - c.pos + 1);
        for (uint64_t i = 0; i < count; ++i) v.arr_i32.push_back(c.i32());
      } else if (inner == T_FLOAT32) {
        v.kind = MetaValue::ArrF32;
        if (count > (c.len - c.pos) / 4) c.take(c.len - c.pos + 1);
        for (uint64_t i = 0; i < count; ++i) v.arr_f32.push_back(c.f32());
      } else {
        throw Error("GGUF array holds values of unknown type " + std::to_string(inner));
      }
      return v;
    }
    default:
      throw Error("GGUF metadata value of unknown type " + std::to_string(tag));
  }
}

void put_u32(std::vector<uint8_t>& b, uint32_t v) {
  const uint8_t* p = reinterpret_cast<const uint8_t*>(&v);
  b.insert(b.end(), p, p + 4);
}
void put_u64(std::vector<uint8_t>& b, uint64_t v) {
  const uint8_t* p = reinterpret_cast<const uint8_t*>(&v);
  b.insert(b.end(), p, p + 8);
}
void put_str(std::vector<uint8_t>& b, const std::string& s) {
  put_u64(b, s.size());
  b.insert(b.end(), s.begin(), s.end());
}
}  // namespace

bool ggml_type_from_u32(uint32_t tag, GgmlType* out) {  // dtype.rs:33-41
  switch (tag) {
    case 0: *out = GgmlType::F32; return true;
    case 8: *out = GgmlType::Q8_0; return true;
    case 2: *out = GgmlType::Q4_0; return true;
    case 14: *out = GgmlType::Q6K; return true;
  }
  return false;
}

size_t block_elems(GgmlType t) { return t == GgmlType::F32 ? 1 : t == GgmlType::Q6K ? 256 : 32; }
size_t block_bytes(GgmlType t) {
  return t == GgmlType::F32 ? 4 : t == GgmlType::Q8_0 ? 34 : t == GgmlType::Q4_0 ? 18 : 210;
}

void dequantize(GgmlType t, const uint8_t* raw, float* out, size_t n) {
  switch (t) {
    case GgmlType::F32:
      memcpy(out, raw, n * 4);
      return;
    case GgmlType::Q8_0:
      for (size_t blk = 0; blk < n / 32; ++blk) {
        const uint8_t* b = raw + blk * 34;
        const float d = f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
        for (int j = 0; j < 32; ++j) out[blk * 32 + j] = d * (float)(int8_t)b[2 + j];
      }
      return;
    case GgmlType::Q4_0:
      for (size_t blk = 0; blk < n / 32; ++blk) {
        const uint8_t* b = raw + blk * 18;
        const float d = f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
        for (int j = 0; j < 16; ++j) {
          out[blk * 32 + j] = d * (float)((int)(b[2 + j] & 0x0F) - 8);
          out[blk * 32 + j + 16] = d * (float)((int)(b[2 + j] >> 4) - 8);
        }
      }
      return;
    case GgmlType::Q6K:
      for (size_t sb = 0; sb < n / 256; ++sb) {
        const uint8_t* b = raw + sb * 210;
        const float d = f16_to_f32((uint16_t)(b[208] | (b[209] << 8)));
        for (int h = 0; h < 2; ++h) {
          const uint8_t *ql = b + h * 64, *qh = b + 128 + h * 32;
          const int8_t* sc = reinterpret_cast<const int8_t*>(b + 192 + h * 8);
          float* y = out + sb * 256 + h * 128;
          for (int l = 0; l < 32; ++l) {
            const int is = l / 16;
            const int q1 = (int)((ql[l] & 0xF) | ((qh[l] & 0x03) << 4)) - 32;
            const int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 0x03) << 4)) - 32;
            const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 0x03) << 4)) - 32;
            const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 0x03) << 4)) - 32;
            y[l] = d * (float)sc[is] * (float)q1;
            y[l + 32] = d * (float)sc[is + 2] * (float)q2;
            y[l + 64] = d * (float)sc[is + 4] * (float)q3;
            y[l + 96] = d * (float)sc[is + 6] * (float)q4;
          }
        }
      }
      return;
  }
}

size_t TensorInfo::elem_count() const {
  size_t n = 1;
  for (uint64_t d : dims) n *= (size_t)d;
  return n;
}

GgufFile::GgufFile(GgufFile&& o) noexcept { *this = std::move(o); }
GgufFile& GgufFile::operator=(GgufFile&& o) noexcept {
  if (this != &o) {
    if (map_) munmap(map_, map_len_);
    owned_ = std::move(o.owned_);
    map_ = o.map_;
    map_len_ = o.map_len_;
    data_ = map_ ? static_cast<const uint8_t*>(map_) : owned_.data();
    size_ = o.size_;
    meta_ = std::move(o.meta_);
    tensors_ = std::move(o.tensors_);
    by_name_ = std::move(o.by_name_);
    data_start_ = o.data_start_;
    o.map_ = nullptr;
    o.data_ = nullptr;
    o.size_ = 0;
  }
  return *this;
}
GgufFile::~GgufFile() {
  if (map_) munmap(map_, map_len_);
}

GgufFile GgufFile::open(const std::string& path) {
  const int fd = ::open(path.c_str(), O_RDONLY);
  if (fd < 0) throw Error("opening " + path);
  struct stat st;
  if (fstat(fd, &st) != 0) {
    ::close(fd);
    throw Error("opening " + path);
  }
  GgufFile g;
  if (st.st_size > 0) {
    void* m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m == MAP_FAILED) throw Error("mmapping " + path);
    g.map_ = m;
    g.map_len_ = (size_t)st.st_size;
    g.data_ = static_cast<const uint8_t*>(m);
    g.size_ = (size_t)st.st_size;
  } else {
    ::close(fd);
  }
  g.parse();
  return g;
}

GgufFile GgufFile::from_bytes(std::vector<uint8_t> b) {
  GgufFile g;
  g.owned_ = std::move(b);
  g.data_ = g.owned_.data();
  g.size_ = g.owned_.size();
  g.parse();
  return g;
}

void GgufFile::parse() {  // reader.rs:193-246
  Cursor c{data_, size_};
  const uint8_t* magic = c.take(4);
  if (memcmp(magic, "GGUF", 4) != 0) throw Error("file does not start with the GGUF magic");
  const uint32_t version = c.u32();
  if (version != 3) throw Error("GGUF version " + std::to_string(version) + " is not read here (only version 3)");
  const uint64_t n_t = c.u64(), n_kv = c.u64();
  for (uint64_t i = 0; i < n_kv; ++i) {
    std::string key = c.str();
    const uint32_t tag = c.u32();
    try {
      meta_[key] = read_value(c, tag);
    } catch (const Error& e) {
      throw Error("metadata entry \"" + key + "\": " + e.what());
    }
  }
  for (uint64_t i = 0; i < n_t; ++i) {
    TensorInfo t;
    t.name = c.str();
    const uint32_t nd = c.u32();
    if (nd > (c.len - c.pos) / 8) c.take(c.len - c.pos + 1);
    for (uint32_t d = 0; d < nd; ++d) t.dims.push_back(c.u64());
    const uint32_t tag = c.u32();
    if (!ggml_type_from_u32(tag, &t.dtype))
      throw Error("tensor \"" + t.name + "\": ggml type tag not handled: " + std::to_string(tag));
    t.offset = c.u64();
    by_name_[t.name] = tensors_.size();
    tensors_.push_back(std::move(t));
  }
  data_start_ = (c.pos + kAlign - 1) / kAlign * kAlign;
  if (data_start_ > size_)
    throw Error("tensor data would start at byte " + std::to_string(data_start_) + " of a " + std::to_string(size_) + "-byte file");
}

const MetaValue* GgufFile::metadata(const std::string& key) const {
  auto it = meta_.find(key);
  return it == meta_.end() ? nullptr : &it->second;
}
bool GgufFile::get_u32(const std::string& key, uint32_t* out) const {
  const MetaValue* v = metadata(key);
  if (!v || v->kind != MetaValue::U32) return false;
  *out = v->u32;
  return true;
}
bool GgufFile::get_f32(const std::string& key, float* out) const {
  const MetaValue* v = metadata(key);
  if (!v || v->kind != MetaValue::F32) return false;
  *out = v->f32;
  return true;
}
const std::string* GgufFile::get_str(const std::string& key) const {
  const MetaValue* v = metadata(key);
  return v && v->kind == MetaValue::Str ? &v->str : nullptr;
}
const std::vector<std::string>* GgufFile::get_arr_str(const std::string& key) const {
  const MetaValue* v = metadata(key);
  return v && v->kind == MetaValue::ArrStr ? &v->arr_str : nullptr;
}
const std::vector<int32_t>* GgufFile::get_arr_i32(const std::string& key) const {
  const MetaValue* v = metadata(key);
  return v && v->kind == MetaValue::ArrI32 ? &v->arr_i32 : nullptr;
}
const std::vector<float>* GgufFile::get_arr_f32(const std::string& key) const {
  const MetaValue* v = metadata(key);
  return v && v->kind == MetaValue::ArrF32 ? &v->arr_f32 : nullptr;
}

const TensorInfo* GgufFile::tensor_info(const std::string& name) const {
  auto it = by_name_.find(name);
  return it == by_name_.end() ? nullptr : &tensors_[it->second];
}

const float* GgufFile::tensor_f32(const std::string& name, size_t* n) const {
  const TensorInfo* t = tensor_info(name);
  if (!t) throw Error("model has no tensor \"" + name + "\"");
  if (t->dtype != GgmlType::F32) throw Error("tensor \"" + name + "\" must be stored as F32");
  size_t len;
  GgmlType ty;
  const uint8_t* p = tensor_raw(name, &len, &ty);
  *n = len / 4;
  return reinterpret_cast<const float*>(p);
}

const uint8_t* GgufFile::tensor_raw(const std::string& name, size_t* len, GgmlType* type) const {
  const TensorInfo* t = tensor_info(name);
  if (!t) throw Error("model has no tensor \"" + name + "\"");
  uint64_t elems = 1;
  for (uint64_t d : t->dims) {
    if (d && elems > UINT64_MAX / d) throw Error("tensor size overflows 64 bits");
    elems *= d;
  }
  const size_t blk = block_elems(t->dtype);
  if (elems % blk)
    throw Error("tensor \"" + name + "\" has " + std::to_string(elems) + " elems, not a multiple of block " +
                std::to_string(blk));
  const uint64_t blen = elems / blk * block_bytes(t->dtype);
  const uint64_t start = (uint64_t)data_start_ + t->offset;
  if (start < t->offset || start + blen < start || start + blen > size_)
    throw Error("tensor \"" + name + "\" runs past the end of the file");
  *len = (size_t)blen;
  *type = t->dtype;
  return data_ + start;
}

// ---- writer
void GgufWriter::u32(const std::string& k, uint32_t v) {
  put_str(kv_, k);
  put_u32(kv_, T_UINT32);
  put_u32(kv_, v);
  ++n_kv_;
}
void GgufWriter::f32(const std::string& k, float v) {
  put_str(kv_, k);
  put_u32(kv_, T_FLOAT32);
  uint32_t b;
  memcpy(&b, &v, 4);
  put_u32(kv_, b);
  ++n_kv_;
}
void GgufWriter::boolean(const std::string& k, bool v) {
  put_str(kv_, k);
  put_u32(kv_, T_BOOL);
  kv_.push_back(v ? 1 : 0);
  ++n_kv_;
}
void GgufWriter::str(const std::string& k, const std::string& v) {
  put_str(kv_, k);
  put_u32(kv_, T_STRING);
  put_str(kv_, v);
  ++n_kv_;
}
void GgufWriter::arr_str(const std::string& k, const std::vector<std::string>& v) {
  put_str(kv_, k);
  put_u32(kv_, T_ARRAY);
  put_u32(kv_, T_STRING);
  put_u64(kv_, v.size());
  for (const auto& s : v) put_str(kv_, s);
  ++n_kv_;
}
void GgufWriter::arr_i32(const std::string& k, const std::vector<int32_t>& v) {
  put_str(kv_, k);
  put_u32(kv_, T_ARRAY);
  put_u32(kv_, T_INT32);
  put_u64(kv_, v.size());
  for (int32_t x : v) put_u32(kv_, (uint32_t)x);
  ++n_kv_;
}
void GgufWriter::arr_f32(const std::string& k, const std::vector<float>& v) {
  put_str(kv_, k);
  put_u32(kv_, T_ARRAY);
  put_u32(kv_, T_FLOAT32);
  put_u64(kv_, v.size());
  for (float x : v) {
    uint32_t b;
    memcpy(&b, &x, 4);
    put_u32(kv_, b);
  }
  ++n_kv_;
}
void GgufWriter::tensor(const std::string& name, std::vector<uint64_t> dims, GgmlType t, std::vector<uint8_t> bytes) {
  const size_t n = bytes.size();
  tensors_.push_back({name, std::move(dims), t, std::move(bytes), n});
}
void GgufWriter::tensor_sized(const std::string& name, std::vector<uint64_t> dims, GgmlType t, size_t nbytes) {
  tensors_.push_back({name, std::move(dims), t, {}, nbytes});
}

std::vector<uint8_t> GgufWriter::layout(std::vector<size_t>* abs_offs) const {
  std::vector<uint8_t> buf;
  buf.insert(buf.end(), {'G', 'G', 'U', 'F'});
  put_u32(buf, 3);
  put_u64(buf, tensors_.size());
  put_u64(buf, n_kv_);
  buf.insert(buf.end(), kv_.begin(), kv_.end());
  std::vector<uint64_t> offs;
  uint64_t off = 0;
  for (const auto& t : tensors_) {
    offs.push_back(off);
    off = (off + t.nbytes + kAlign - 1) / kAlign * kAlign;
  }
  for (size_t i = 0; i < tensors_.size(); ++i) {
    const auto& t = tensors_[i];
    put_str(buf, t.name);
    put_u32(buf, (uint32_t)t.dims.size());
    for (uint64_t d : t.dims) put_u64(buf, d);
    put_u32(buf, (uint32_t)t.type);
    put_u64(buf, offs[i]);
  }
  while (buf.size() % kAlign) buf.push_back(0);
  const size_t data_start = buf.size();
  buf.resize(data_start + off, 0);
  abs_offs->clear();
  for (uint64_t o : offs) abs_offs->push_back(data_start + (size_t)o);
  return buf;
}

std::vector<uint8_t> GgufWriter::finish() const {
  std::vector<size_t> offs;
  std::vector<uint8_t> buf = layout(&offs);
  for (size_t i = 0; i < tensors_.size(); ++i)
    if (!tensors_[i].bytes.empty()) memcpy(buf.data() + offs[i], tensors_[i].bytes.data(), tensors_[i].bytes.size());
  return buf;
}

}  // namespace talos
