// gguf.cpp — GGUF container reader (GgufLoader.LoadMeta, SharpMind.Model/Format/GgufLoader.cs:124-177).
//
// Layout (little endian): u32 magic "GGUF", u32 version, i64 tensor count, i64 metadata count;
// metadata entries (string key, u32 value type, value; strings are u64 length + UTF-8 bytes,
// arrays are u32 element type + u64 length + elements); tensor entries (string name, u32 n_dims,
// u64 dims[n_dims] innermost first, u32 ggml type, u64 offset into the data section); the data
// section starts at the next multiple of general.alignment (default 32).
#include "gguf.hpp"

#include <cstdio>
#include <cstring>
#include <memory>

#include "common.hpp"

namespace smhip {

namespace {

struct Reader {
  FILE* f;
  bool ok = true;
  template <class T>
  T get() {
    T v{};
    if (ok && fread(&v, sizeof(T), 1, f) != 1) ok = false;
    return v;
  }
  std::string str() {
    const uint64_t n = get<uint64_t>();
    if (!ok || n > ((uint64_t)1 << 30)) { ok = false; return {}; }
    std::string s((size_t)n, '\0');
    if (n && fread(s.data(), 1, (size_t)n, f) != (size_t)n) ok = false;
    return s;
  }
  void skip(int64_t n) {
    if (ok && fseeko(f, (off_t)n, SEEK_CUR) != 0) ok = false;
  }
};

// size of a scalar value type; 0 for string / array
int scalar_size(uint32_t t) {
  switch (t) {
    case 0: case 1: case 7: return 1;  // u8, i8, bool
    case 2: case 3: return 2;          // u16, i16
    case 4: case 5: case 6: return 4;  // u32, i32, f32
    case 10: case 11: case 12: return 8;  // u64, i64, f64
    default: return 0;
  }
}

bool read_int(Reader& r, uint32_t t, int64_t* v) {
  switch (t) {
    case 0: *v = r.get<uint8_t>(); return true;
    case 1: *v = r.get<int8_t>(); return true;
    case 2: *v = r.get<uint16_t>(); return true;
    case 3: *v = r.get<int16_t>(); return true;
    case 4: *v = r.get<uint32_t>(); return true;
    case 5: *v = r.get<int32_t>(); return true;
    case 7: *v = r.get<uint8_t>(); return true;
    case 10: *v = (int64_t)r.get<uint64_t>(); return true;
    case 11: *v = r.get<int64_t>(); return true;
    default: return false;
  }
}

// skips one value of type t (arrays may nest)
void skip_value(Reader& r, uint32_t t, int depth = 0) {
  if (t == 8) { r.str(); return; }
  if (t == 9) {
    const uint32_t et = r.get<uint32_t>();
    const uint64_t n = r.get<uint64_t>();
    if (!r.ok || depth > 4) { r.ok = false; return; }
    if (const int sz = scalar_size(et)) { r.skip((int64_t)n * sz); return; }
    if (et != 8 && et != 9) { r.ok = false; return; }
    for (uint64_t i = 0; i < n && r.ok; i++) skip_value(r, et, depth + 1);
    return;
  }
  if (const int sz = scalar_size(t)) { r.skip(sz); return; }
  r.ok = false;
}

}  // namespace

bool GgufFile::int_value(const std::string& key, int64_t* v) const {
  for (const auto& kv : ints)
    if (kv.first == key) { *v = kv.second; return true; }
  return false;
}
const std::string* GgufFile::string_value(const std::string& key) const {
  for (const auto& kv : strings)
    if (kv.first == key) return &kv.second;
  return nullptr;
}
const GgufTensor* GgufFile::find(const std::string& name) const {
  for (const auto& t : tensors)
    if (t.name == name) return &t;
  return nullptr;
}

int64_t gguf_tensor_bytes(uint32_t type, const std::vector<int64_t>& dims) {
  if (dims.empty()) return -1;
  int64_t rows = 1;
  for (size_t i = 1; i < dims.size(); i++) rows *= dims[i];
  const int64_t ne0 = dims[0];
  switch (type) {
    case 0: return rows * ne0 * 4;   // F32
    case 1: return rows * ne0 * 2;   // F16
    case 8: return ne0 % 32 ? -1 : rows * (ne0 / 32) * 34;     // Q8_0: 34-byte blocks of 32
    case 12: return ne0 % 256 ? -1 : rows * (ne0 / 256) * 144;  // Q4_K: 144-byte blocks of 256
    default: return -1;
  }
}

int gguf_parse(const std::string& path, GgufFile* out) {
  struct Closer { void operator()(FILE* f) const { if (f) fclose(f); } };
  std::unique_ptr<FILE, Closer> f(fopen(path.c_str(), "rb"));
  if (!f) return fail(SMHIP_EINVAL, "gguf: cannot open " + path);
  Reader r{f.get()};
  const uint32_t magic = r.get<uint32_t>();
  if (!r.ok || magic != 0x46554747u) return fail(SMHIP_EINVAL, "gguf: not a GGUF file: " + path);
  out->version = r.get<uint32_t>();
  const int64_t n_tensors = r.get<int64_t>(), n_kv = r.get<int64_t>();
  if (!r.ok || n_tensors < 0 || n_kv < 0 || n_tensors > (1 << 24) || n_kv > (1 << 24))
    return fail(SMHIP_EINVAL, "gguf: bad header in " + path);
  int64_t alignment = 32;
  for (int64_t i = 0; i < n_kv && r.ok; i++) {
    std::string key = r.str();
    const uint32_t t = r.get<uint32_t>();
    int64_t v;
    if (!r.ok) break;
    if (t == 8) {
      out->strings.emplace_back(std::move(key), r.str());
    } else if (read_int(r, t, &v)) {
      if (key == "general.alignment") alignment = v;
      out->ints.emplace_back(std::move(key), v);
    } else {
      skip_value(r, t);
    }
  }
  if (!r.ok) return fail(SMHIP_EINVAL, "gguf: truncated metadata in " + path);
  if (alignment <= 0 || (alignment & (alignment - 1))) return fail(SMHIP_EINVAL, "gguf: bad general.alignment");
  out->tensors.resize((size_t)n_tensors);
  for (auto& t : out->tensors) {
    t.name = r.str();
    const uint32_t nd = r.get<uint32_t>();
    if (!r.ok || nd == 0 || nd > 8) return fail(SMHIP_EINVAL, "gguf: bad tensor entry in " + path);
    t.dims.resize(nd);
    for (auto& d : t.dims) d = (int64_t)r.get<uint64_t>();
    t.type = r.get<uint32_t>();
    t.offset = r.get<uint64_t>();
    if (!r.ok) return fail(SMHIP_EINVAL, "gguf: truncated tensor table in " + path);
  }
  const off_t pos = ftello(f.get());
  out->data_offset = ((uint64_t)pos + alignment - 1) & ~(uint64_t)(alignment - 1);
  return SMHIP_OK;
}

}  // namespace smhip

using namespace smhip;

extern "C" {

int smhip_gguf_tensor_count(const char* path, int64_t* count) {
  SMHIP_REQUIRE(path && count, "gguf_tensor_count: null argument");
  GgufFile g;
  if (int rc = gguf_parse(path, &g)) return rc;
  *count = (int64_t)g.tensors.size();
  return SMHIP_OK;
}

int smhip_gguf_tensor_info(const char* path, int64_t index, char* name, int64_t cap, int* ggml_type, int* n_dims,
                           int64_t* dims, int64_t* file_offset) {
  SMHIP_REQUIRE(path && name && cap > 0 && ggml_type && n_dims && dims && file_offset,
                "gguf_tensor_info: null argument");
  GgufFile g;
  if (int rc = gguf_parse(path, &g)) return rc;
  SMHIP_REQUIRE(index >= 0 && index < (int64_t)g.tensors.size(), "gguf_tensor_info: index out of range");
  const GgufTensor& t = g.tensors[(size_t)index];
  SMHIP_REQUIRE((int64_t)t.name.size() < cap, "gguf_tensor_info: name buffer too small");
  memcpy(name, t.name.c_str(), t.name.size() + 1);
  *ggml_type = (int)t.type;
  *n_dims = (int)t.dims.size();
  for (size_t i = 0; i < 8; i++) dims[i] = i < t.dims.size() ? t.dims[i] : 1;
  *file_offset = (int64_t)(g.data_offset + t.offset);
  return SMHIP_OK;
}

}  // extern "C"
