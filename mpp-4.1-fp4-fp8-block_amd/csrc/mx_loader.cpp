// mx_loader.cpp - on-disk MXFP4 weights (safetensors) -> device, no repack.
//
// The reference's weight layout (docs/MXFP4-MPP41-GUIDE.md:43-55): data
// row-major [n][k/2], two E2M1 per byte, low nibble = even k; one E8M0 byte
// per (row, 32-wide k block) at scales[row * (k/32) + kb].  MXFP4 checkpoints
// store a matrix as a uint8 "blocks" tensor [..., n, k/32, 16] (or
// [..., n, k/2]) plus a uint8 "scales" tensor [..., n, k/32]; with the same
// bytes in the same order that is exactly this layout, and leading
// dimensions (experts) give the stacked [E][n][k/2] + [E][n][k/32] form the
// MoE entry point takes.  So loading is: parse the header, check the shapes,
// copy the two byte ranges to device memory.
//
// safetensors: 8-byte little-endian header size, then a JSON object
// {name: {"dtype", "shape", "data_offsets": [begin, end]}, "__metadata__":
// {...}}, then the data region (offsets are relative to its start).
#include <hip/hip_runtime.h>

#include <cerrno>
#include <climits>
#include <cstdlib>

#include <cctype>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/mxfp4hip.h"

namespace {

struct TensorInfo {
  std::string dtype;
  std::vector<long long> shape;
  unsigned long long begin = 0, end = 0;  // relative to the data region
};

// A minimal JSON reader for the safetensors header: objects, arrays,
// strings, integers, and (skipped) other scalars.
class Json {
 public:
  explicit Json(const std::string& s) : s_(s) {}
  bool ok() const { return ok_; }

  // Walk the top-level object; for `want` fill `out`.  Returns whether found.
  bool find(const std::string& want, TensorInfo* out) {
    pos_ = 0;
    ok_ = true;
    bool found = false;
    ws();
    if (!eat('{')) return false;
    ws();
    if (peek() == '}') return false;
    while (ok_) {
      std::string key;
      if (!str(&key)) return false;
      ws();
      if (!eat(':')) return false;
      ws();
      if (key == want) {
        if (!tensor(out)) return false;
        found = true;
      } else if (!skip()) {
        return false;
      }
      ws();
      if (peek() == ',') { pos_++; ws(); continue; }
      if (eat('}')) break;
      return ok_ = false;
    }
    return found && ok_;
  }

 private:
  const std::string& s_;
  size_t pos_ = 0;
  bool ok_ = true;

  char peek() const { return pos_ < s_.size() ? s_[pos_] : '\0'; }
  void ws() {
    while (pos_ < s_.size() && std::isspace((unsigned char)s_[pos_])) pos_++;
  }
  bool eat(char c) {
    if (peek() != c) return ok_ = false;
    pos_++;
    return true;
  }
  bool str(std::string* out) {
    if (!eat('"')) return false;
    out->clear();
    while (pos_ < s_.size() && s_[pos_] != '"') {
      char c = s_[pos_++];
      if (c == '\\') {
        if (pos_ >= s_.size()) return ok_ = false;
        const char e = s_[pos_++];
        if (e == 'u') {  // keep \uXXXX verbatim (names are ASCII in practice)
          if (pos_ + 4 > s_.size()) return ok_ = false;
          out->append("\\u").append(s_, pos_, 4);
          pos_ += 4;
          continue;
        }
        c = e == 'n' ? '\n' : e == 't' ? '\t' : e == 'r' ? '\r' : e == 'b' ? '\b' : e == 'f' ? '\f' : e;
      }
      out->push_back(c);
    }
    return eat('"');
  }
  // The header is untrusted: a value outside long long fails the parse
  // (strtoll with an errno check) instead of throwing across the C ABI.
  bool integer(long long* v) {
    const size_t start = pos_;
    if (peek() == '-') pos_++;
    while (std::isdigit((unsigned char)peek())) pos_++;
    if (pos_ == start || (pos_ == start + 1 && s_[start] == '-')) return ok_ = false;
    const std::string digits = s_.substr(start, pos_ - start);
    errno = 0;
    char* endp = nullptr;
    const long long r = std::strtoll(digits.c_str(), &endp, 10);
    if (errno == ERANGE || endp != digits.c_str() + digits.size()) return ok_ = false;
    *v = r;
    return true;
  }
  bool int_array(std::vector<long long>* out) {
    if (!eat('[')) return false;
    out->clear();
    ws();
    if (peek() == ']') { pos_++; return true; }
    while (ok_) {
      long long v;
      ws();
      if (!integer(&v)) return false;
      out->push_back(v);
      ws();
      if (peek() == ',') { pos_++; continue; }
      return eat(']');
    }
    return false;
  }
  bool tensor(TensorInfo* t) {
    if (!eat('{')) return false;
    bool have_dtype = false, have_shape = false, have_off = false;
    ws();
    while (ok_ && peek() != '}') {
      std::string key;
      if (!str(&key)) return false;
      ws();
      if (!eat(':')) return false;
      ws();
      if (key == "dtype") {
        if (!str(&t->dtype)) return false;
        have_dtype = true;
      } else if (key == "shape") {
        if (!int_array(&t->shape)) return false;
        have_shape = true;
      } else if (key == "data_offsets") {
        std::vector<long long> o;
        if (!int_array(&o) || o.size() != 2 || o[0] < 0 || o[1] < o[0]) return ok_ = false;
        t->begin = (unsigned long long)o[0];
        t->end = (unsigned long long)o[1];
        have_off = true;
      } else if (!skip()) {
        return false;
      }
      ws();
      if (peek() == ',') { pos_++; ws(); }
    }
    return eat('}') && have_dtype && have_shape && have_off;
  }
  bool skip() {  // any JSON value
    ws();
    const char c = peek();
    if (c == '"') { std::string tmp; return str(&tmp); }
    if (c == '{' || c == '[') {
      const char close = c == '{' ? '}' : ']';
      pos_++;
      ws();
      if (peek() == close) { pos_++; return true; }
      while (ok_) {
        if (c == '{') {
          std::string k;
          if (!str(&k)) return false;
          ws();
          if (!eat(':')) return false;
        }
        if (!skip()) return false;
        ws();
        if (peek() == ',') { pos_++; ws(); continue; }
        return eat(close);
      }
      return false;
    }
    while (pos_ < s_.size() && s_[pos_] != ',' && s_[pos_] != '}' && s_[pos_] != ']' &&
           !std::isspace((unsigned char)s_[pos_]))
      pos_++;
    return true;
  }
};

struct File {
  FILE* f = nullptr;
  ~File() {
    if (f) std::fclose(f);
  }
};

// Header of `path`: JSON text and the data region's file offset.
int read_header(const char* path, std::string* json, unsigned long long* data_start, unsigned long long* file_size,
                std::string* err) {
  File fh;
  fh.f = std::fopen(path, "rb");
  if (!fh.f) { *err = std::string("Could not open ") + path + "."; return MX_EINVAL; }
  unsigned char len8[8];
  if (std::fread(len8, 1, 8, fh.f) != 8) { *err = "Not a safetensors file (short header)."; return MX_EINVAL; }
  unsigned long long n = 0;
  for (int i = 7; i >= 0; i--) n = (n << 8) | len8[i];
  if (n == 0 || n > (100ull << 20)) { *err = "Not a safetensors file (header size)."; return MX_EINVAL; }
  json->resize((size_t)n);
  if (std::fread(&(*json)[0], 1, (size_t)n, fh.f) != n) { *err = "Truncated safetensors header."; return MX_EINVAL; }
  if (std::fseek(fh.f, 0, SEEK_END) != 0) { *err = "Could not size the file."; return MX_EINVAL; }
  *file_size = (unsigned long long)std::ftell(fh.f);
  *data_start = 8 + n;
  return MX_OK;
}

int find_tensor(const char* path, const char* name, TensorInfo* t, unsigned long long* data_start, std::string* err) {
  std::string json;
  unsigned long long size = 0;
  if (int rc = read_header(path, &json, data_start, &size, err)) return rc;
  Json j(json);
  if (!j.find(name, t)) {
    *err = j.ok() ? std::string("Tensor ") + name + " is not in " + path + "." : "Malformed safetensors header.";
    return MX_EINVAL;
  }
  if (*data_start + t->end > size) { *err = std::string("Tensor ") + name + " runs past the end of the file."; return MX_EINVAL; }
  return MX_OK;
}

// Copy file bytes [off, off + n) to device memory through two pinned
// staging buffers (the read of one chunk overlaps the copy of the previous).
int upload_range(const char* path, unsigned long long off, size_t n, void* dst, hipStream_t st, std::string* err) {
  File fh;
  fh.f = std::fopen(path, "rb");
  if (!fh.f) { *err = std::string("Could not open ") + path + "."; return MX_EINVAL; }
  if (std::fseek(fh.f, (long)off, SEEK_SET) != 0) { *err = "Seek failed."; return MX_EINVAL; }
  const size_t chunk = 32u << 20;
  void* stage[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
  int rc = MX_OK;
  for (int i = 0; i < 2 && !rc; i++) {
    if (hipHostMalloc(&stage[i], chunk, hipHostMallocDefault) != hipSuccess ||
        hipEventCreateWithFlags(&done[i], hipEventDisableTiming) != hipSuccess) {
      *err = "Could not allocate pinned staging memory.";
      rc = MX_ENOMEM;
    }
  }
  size_t copied = 0;
  for (int i = 0; rc == MX_OK && copied < n; i ^= 1) {
    const size_t len = n - copied < chunk ? n - copied : chunk;
    if (hipEventSynchronize(done[i]) != hipSuccess) { *err = "Staging copy failed."; rc = MX_EGPU; break; }
    if (std::fread(stage[i], 1, len, fh.f) != len) { *err = "Short read of tensor data."; rc = MX_EINVAL; break; }
    if (hipMemcpyAsync(static_cast<char*>(dst) + copied, stage[i], len, hipMemcpyHostToDevice, st) != hipSuccess ||
        hipEventRecord(done[i], st) != hipSuccess) {
      *err = "Copy to the device failed.";
      rc = MX_EGPU;
      break;
    }
    copied += len;
  }
  if (hipStreamSynchronize(st) != hipSuccess && rc == MX_OK) { *err = "Copy to the device failed."; rc = MX_EGPU; }
  for (int i = 0; i < 2; i++) {
    if (done[i]) (void)hipEventDestroy(done[i]);
    if (stage[i]) (void)hipHostFree(stage[i]);
  }
  return rc;
}

}  // namespace

// Implemented in mx_api.cpp: context internals the loader needs.
hipStream_t mx_ctx_stream(mx_ctx* ctx);
int mx_ctx_error(mx_ctx* ctx, int code, const char* message);

extern "C" {

int mx_safetensors_find(const char* path, const char* name, char* dtype_out, size_t dtype_len,
                        long long* shape_out, int max_dims, int* ndim_out, unsigned long long* offset_out,
                        unsigned long long* nbytes_out) {
  if (!path || !name) return MX_EINVAL;
  TensorInfo t;
  unsigned long long data_start = 0;
  std::string err;
  if (int rc = find_tensor(path, name, &t, &data_start, &err)) return rc;
  if (dtype_out && dtype_len) std::snprintf(dtype_out, dtype_len, "%s", t.dtype.c_str());
  if (ndim_out) *ndim_out = (int)t.shape.size();
  if (shape_out)
    for (int i = 0; i < max_dims && i < (int)t.shape.size(); i++) shape_out[i] = t.shape[(size_t)i];
  if (offset_out) *offset_out = data_start + t.begin;
  if (nbytes_out) *nbytes_out = t.end - t.begin;
  return MX_OK;
}

int mx_load_mxfp4(mx_ctx* ctx, const char* path, const char* blocks_name, const char* scales_name,
                  mx_qmatrix* out, int* count_out, int* n_out, int* k_out) {
  if (!ctx) return MX_EINVAL;
  if (!path || !blocks_name || !scales_name || !out)
    return mx_ctx_error(ctx, MX_EINVAL, "loader arguments must not be null.");
  TensorInfo b, s;
  unsigned long long ds = 0;
  std::string err;
  if (find_tensor(path, blocks_name, &b, &ds, &err) || find_tensor(path, scales_name, &s, &ds, &err))
    return mx_ctx_error(ctx, MX_EINVAL, err.c_str());
  if (b.dtype != "U8" || s.dtype != "U8")
    return mx_ctx_error(ctx, MX_EINVAL, "MXFP4 blocks and scales must be U8 tensors.");
  // blocks [..., n, k/32, 16] or [..., n, k/2]; scales [..., n, k/32]
  if (s.shape.size() < 2) return mx_ctx_error(ctx, MX_EINVAL, "MXFP4 scales must have at least 2 dimensions.");
  const size_t lead = s.shape.size() - 2;
  const long long n = s.shape[lead], kb = s.shape[lead + 1];
  long long count = 1;
  bool overflow = false;
  for (size_t i = 0; i < lead; i++) overflow = overflow || __builtin_mul_overflow(count, s.shape[i], &count);
  bool match = false;
  if (b.shape.size() == s.shape.size() + 1)
    match = b.shape[lead] == n && b.shape[lead + 1] == kb && b.shape[lead + 2] == 16;
  else if (b.shape.size() == s.shape.size())
    match = b.shape[lead] == n && b.shape[lead + 1] == kb * 16;
  for (size_t i = 0; match && i < lead; i++) match = b.shape[i] == s.shape[i];
  if (!match || n <= 0 || kb <= 0 || count <= 0)
    return mx_ctx_error(ctx, MX_EINVAL, "MXFP4 blocks and scales shapes do not match ([..., n, k/32, 16] and [..., n, k/32]).");
  // counts are returned as int, and the byte sizes must not wrap
  long long scale_ll = 0, data_ll = 0;
  if (overflow || n > INT_MAX || kb > INT_MAX / 32 || count > INT_MAX ||
      __builtin_mul_overflow(count, n, &scale_ll) || __builtin_mul_overflow(scale_ll, kb, &scale_ll) ||
      __builtin_mul_overflow(scale_ll, 16LL, &data_ll))
    return mx_ctx_error(ctx, MX_EINVAL, "MXFP4 tensor shape is too large.");
  const unsigned long long data_bytes = (unsigned long long)data_ll, scale_bytes = (unsigned long long)scale_ll;
  if (b.end - b.begin != data_bytes || s.end - s.begin != scale_bytes)
    return mx_ctx_error(ctx, MX_EINVAL, "MXFP4 tensor byte sizes do not match their shapes.");
  void* d = nullptr;
  void* sc = nullptr;
  if (hipMalloc(&d, data_bytes) != hipSuccess || hipMalloc(&sc, scale_bytes) != hipSuccess) {
    if (d) (void)hipFree(d);
    (void)hipGetLastError();
    return mx_ctx_error(ctx, MX_ENOMEM, "Could not create device buffers for the MXFP4 weights.");
  }
  hipStream_t st = mx_ctx_stream(ctx);
  int rc = upload_range(path, ds + b.begin, (size_t)data_bytes, d, st, &err);
  if (!rc) rc = upload_range(path, ds + s.begin, (size_t)scale_bytes, sc, st, &err);
  if (rc) {
    (void)hipFree(d);
    (void)hipFree(sc);
    return mx_ctx_error(ctx, rc, err.c_str());
  }
  out->data = d;
  out->scales = sc;
  if (count_out) *count_out = (int)count;
  if (n_out) *n_out = (int)n;
  if (k_out) *k_out = (int)(kb * 32);
  return MX_OK;
}

}  // extern "C"
