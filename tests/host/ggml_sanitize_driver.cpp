// Drives the GGML file parser (whisper4j_amd/csrc/w4h_ggml.cpp) over the files named on the command
// line, for a build with AddressSanitizer and UndefinedBehaviorSanitizer: every file is inspected and
// each of its tensors read back, and every outcome must be a return code (never a memory error or
// undefined behaviour).  Model and encoder creation, the only device steps the parser reaches, are
// stubbed out.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/w4h.h"

namespace w4h {
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  return code;
}
}  // namespace w4h

extern "C" int w4h_model_create(const w4h_dims*, const w4h_tensor*, int32_t, int32_t, w4h_model**) {
  return W4H_ERR_DEVICE;
}
extern "C" int w4h_encoder_create(const w4h_encoder_dims*, const w4h_tensor*, int32_t, int32_t, w4h_encoder**) {
  return W4H_ERR_DEVICE;
}

int main(int argc, char** argv) {
  int ok = 0, refused = 0;
  for (int i = 1; i < argc; i++) {
    w4h_dims d{};
    int32_t n = 0;
    int64_t bytes = 0;
    int rc = w4h_ggml_inspect(argv[i], &d, &n, &bytes);
    if (rc == W4H_OK) {
      ++ok;
      // names are read from a second file listing ("<file>.names", one per line) when present
      std::string lst = std::string(argv[i]) + ".names";
      if (FILE* f = fopen(lst.c_str(), "r")) {
        char name[256];
        while (fgets(name, sizeof name, f)) {
          name[strcspn(name, "\n")] = 0;
          int32_t type = 0, nd = 0;
          int64_t ne[4];
          if (w4h_ggml_read_tensor(argv[i], name, &type, &nd, ne, nullptr, 0) == W4H_OK) {
            int64_t cnt = 1;
            for (int j = 0; j < nd; j++) cnt *= ne[j];
            std::vector<unsigned char> buf((size_t)(cnt * 4 + 64));
            (void)w4h_ggml_read_tensor(argv[i], name, &type, &nd, ne, buf.data(), (int64_t)buf.size());
            (void)w4h_ggml_read_tensor(argv[i], name, &type, &nd, ne, buf.data(), 1);  // too small: refused
          }
        }
        fclose(f);
      }
    } else {
      ++refused;
    }
    w4h_model* m = nullptr;
    (void)w4h_model_load_ggml(argv[i], 0, &m);
  }
  printf("parsed %d, refused %d\n", ok, refused);
  return 0;
}
