// whisper.cpp GGML file parsing (main/model/GgmlLoader.java:95-220 reads the same layout):
//   int32 magic 0x67676d6c; 11 int32 hparams (n_vocab, n_audio_ctx, n_audio_state, n_audio_head,
//   n_audio_layer, n_text_ctx, n_text_state, n_text_head, n_text_layer, n_mels, ftype);
//   mel filters (int32 n_mel, int32 n_fft, float[n_mel*n_fft]); vocab (int32 count, then count x
//   {int32 len, bytes}); then tensors until end of file: int32 n_dims, int32 name_len, int32 type,
//   int32 ne[n_dims], name bytes, data (no alignment padding).
// The file is memory-mapped; tensor data is handed to model creation without copies.

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <vector>

#include "w4h_host.h"

namespace {

constexpr int32_t kMagic = 0x67676D6C;

struct Mapped {
  void* base = MAP_FAILED;
  size_t size = 0;
  ~Mapped() {
    if (base != MAP_FAILED) munmap(base, size);
  }
};

struct Parsed {
  w4h_dims dims{};
  w4h_encoder_dims edims{};
  std::vector<w4h_tensor> tensors;
  std::vector<std::string> names;
  int64_t data_bytes = 0;
};

int64_t type_bytes(int32_t type, int64_t n, bool* ok) {
  *ok = true;
  switch (type) {
    case 0: return n * 4;            // F32
    case 1: return n * 2;            // F16
    case 2: return (n / 32) * 18;    // Q4_0
    case 3: return (n / 32) * 20;    // Q4_1
    case 6: return (n / 32) * 22;    // Q5_0
    case 7: return (n / 32) * 24;    // Q5_1
    case 8: return (n / 32) * 34;    // Q8_0
    default: *ok = false; return 0;
  }
}

int map_file(const char* path, Mapped& m) {
  int fd = open(path, O_RDONLY);
  if (fd < 0) return w4h::fail(W4H_ERR_IO, "cannot open %s", path);
  struct stat st;
  if (fstat(fd, &st) != 0) {
    close(fd);
    return w4h::fail(W4H_ERR_IO, "cannot stat %s", path);
  }
  m.size = (size_t)st.st_size;
  if (m.size < 4) {
    close(fd);
    return w4h::fail(W4H_ERR_FORMAT, "not a GGML file (%zu bytes): %s", m.size, path);
  }
  m.base = mmap(nullptr, m.size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (m.base == MAP_FAILED) return w4h::fail(W4H_ERR_IO, "cannot map %s", path);
  return W4H_OK;
}

int parse(const Mapped& mf, Parsed& out) {
  const unsigned char* p = static_cast<const unsigned char*>(mf.base);
  const size_t size = mf.size;
  size_t pos = 0;
  auto rd32 = [&](int32_t* v) -> bool {
    if (pos + 4 > size) return false;
    memcpy(v, p + pos, 4);
    pos += 4;
    return true;
  };
  int32_t magic;
  if (!rd32(&magic) || magic != kMagic) return w4h::fail(W4H_ERR_FORMAT, "not a GGML file (magic 0x%08X)", (unsigned)magic);
  int32_t hp[11];
  for (int i = 0; i < 11; i++)
    if (!rd32(&hp[i])) return w4h::fail(W4H_ERR_FORMAT, "truncated GGML header");
  out.dims.n_vocab = hp[0];
  out.dims.n_audio_ctx = hp[1];
  out.dims.n_text_ctx = hp[5];
  out.dims.n_text_state = hp[6];
  out.dims.n_text_head = hp[7];
  out.dims.n_text_layer = hp[8];
  out.edims.n_mels = hp[9];
  out.edims.n_audio_ctx = hp[1];
  out.edims.n_audio_state = hp[2];
  out.edims.n_audio_head = hp[3];
  out.edims.n_audio_layer = hp[4];
  int32_t n_mel, n_fft;
  if (!rd32(&n_mel) || !rd32(&n_fft) || n_mel < 0 || n_fft < 0) return w4h::fail(W4H_ERR_FORMAT, "bad mel filter header");
  const size_t mel_bytes = (size_t)n_mel * (size_t)n_fft * 4;
  if (pos + mel_bytes > size) return w4h::fail(W4H_ERR_FORMAT, "truncated mel filters");
  pos += mel_bytes;
  int32_t nvocab;
  if (!rd32(&nvocab) || nvocab < 0) return w4h::fail(W4H_ERR_FORMAT, "bad vocab header");
  for (int i = 0; i < nvocab; i++) {
    int32_t len;
    if (!rd32(&len) || len < 0 || pos + (size_t)len > size) return w4h::fail(W4H_ERR_FORMAT, "truncated vocab");
    pos += (size_t)len;
  }
  while (pos + 12 <= size) {
    int32_t n_dims, name_len, type;
    rd32(&n_dims);
    rd32(&name_len);
    rd32(&type);
    // the reference stops at the first implausible header (main/model/GgmlLoader.java:153-158)
    if (n_dims < 1 || n_dims > 4 || name_len < 1 || name_len > 256 || type < 0 || type > 15) break;
    w4h_tensor t{};
    t.n_dims = n_dims;
    t.type = type;
    int64_t n = 1;
    for (int i = 0; i < n_dims; i++) {
      int32_t ne;
      if (!rd32(&ne) || ne < 0) return w4h::fail(W4H_ERR_FORMAT, "truncated tensor header");
      t.ne[i] = ne;
      n *= ne;
    }
    for (int i = n_dims; i < 4; i++) t.ne[i] = 1;
    if (pos + (size_t)name_len > size) return w4h::fail(W4H_ERR_FORMAT, "truncated tensor name");
    std::string name(reinterpret_cast<const char*>(p + pos), (size_t)name_len);
    pos += (size_t)name_len;
    while (!name.empty() && (name.back() == ' ' || name.back() == '\0')) name.pop_back();
    bool ok;
    const int64_t bytes = type_bytes(type, n, &ok);
    if (!ok) return w4h::fail(W4H_ERR_FORMAT, "tensor %s: unsupported GGML type %d", name.c_str(), type);
    if (pos + (size_t)bytes > size) return w4h::fail(W4H_ERR_FORMAT, "tensor %s: data truncated", name.c_str());
    t.data = p + pos;
    pos += (size_t)bytes;
    out.data_bytes += bytes;
    out.names.push_back(name);
    out.tensors.push_back(t);
  }
  for (size_t i = 0; i < out.tensors.size(); i++) out.tensors[i].name = out.names[i].c_str();
  return W4H_OK;
}

}  // namespace

extern "C" {

int w4h_ggml_inspect(const char* path, w4h_dims* dims, int32_t* n_tensors, int64_t* data_bytes) {
  if (!path) return w4h::fail(W4H_ERR_INVALID, "null path");
  Mapped mf;
  int rc = map_file(path, mf);
  if (rc) return rc;
  Parsed ps;
  if ((rc = parse(mf, ps))) return rc;
  if (dims) *dims = ps.dims;
  if (n_tensors) *n_tensors = (int32_t)ps.tensors.size();
  if (data_bytes) *data_bytes = ps.data_bytes;
  return W4H_OK;
}

int w4h_ggml_read_tensor(const char* path, const char* name, int32_t* type, int32_t* n_dims, int64_t ne[4], void* dst,
                         int64_t dst_bytes) {
  if (!path || !name) return w4h::fail(W4H_ERR_INVALID, "null argument");
  Mapped mf;
  int rc = map_file(path, mf);
  if (rc) return rc;
  Parsed ps;
  if ((rc = parse(mf, ps))) return rc;
  for (size_t i = 0; i < ps.tensors.size(); i++) {
    if (ps.names[i] != name) continue;
    const w4h_tensor& t = ps.tensors[i];
    int64_t n = 1;
    for (int j = 0; j < t.n_dims; j++) n *= t.ne[j];
    bool ok;
    const int64_t bytes = type_bytes(t.type, n, &ok);
    if (type) *type = t.type;
    if (n_dims) *n_dims = t.n_dims;
    if (ne)
      for (int j = 0; j < 4; j++) ne[j] = t.ne[j];
    if (dst) {
      if (dst_bytes < bytes) return w4h::fail(W4H_ERR_INVALID, "destination holds %lld bytes, tensor needs %lld",
                                              (long long)dst_bytes, (long long)bytes);
      memcpy(dst, t.data, (size_t)bytes);
    }
    return W4H_OK;
  }
  return w4h::fail(W4H_ERR_NOT_FOUND, "missing tensor: %s", name);
}

int w4h_model_load_ggml(const char* path, int32_t device, w4h_model** out) {
  if (!path || !out) return w4h::fail(W4H_ERR_INVALID, "null argument");
  Mapped mf;
  int rc = map_file(path, mf);
  if (rc) return rc;
  Parsed ps;
  if ((rc = parse(mf, ps))) return rc;
  if (ps.tensors.empty()) return w4h::fail(W4H_ERR_FORMAT, "GGML file has no tensors: %s", path);
  return w4h_model_create(&ps.dims, ps.tensors.data(), (int32_t)ps.tensors.size(), device, out);
}

int w4h_encoder_load_ggml(const char* path, int32_t device, w4h_encoder** out) {
  if (!path || !out) return w4h::fail(W4H_ERR_INVALID, "null argument");
  Mapped mf;
  int rc = map_file(path, mf);
  if (rc) return rc;
  Parsed ps;
  if ((rc = parse(mf, ps))) return rc;
  if (ps.tensors.empty()) return w4h::fail(W4H_ERR_FORMAT, "GGML file has no tensors: %s", path);
  return w4h_encoder_create(&ps.edims, ps.tensors.data(), (int32_t)ps.tensors.size(), device, out);
}

}  // extern "C"
