// Loader fuzz driver (CPU, sanitizer build): opens each shard directory given
// on the command line and walks every entry point that parses index, registry
// or shard bytes: param_info, staging_size, load_layer, pack_layer, blob_tensor.
#include "nf4stream.h"
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>
int main(int argc, char **argv) {
  const char *names[] = {"model.layers.0.q", "model.layers.0.norm", "model.layers.1.q",
                         "model.layers.1.norm", "missing"};
  int opened = 0;
  for (int a = 1; a < argc; ++a) {
    nf4s_loader *L = nullptr;
    if (nf4s_loader_open(argv[a], &L) != 0) continue;
    ++opened;
    for (const char *n : names) {
      nf4s_param_info pi;
      nf4s_loader_param_info(L, n, &pi);
      int64_t b = 0;
      nf4s_loader_staging_size(L, n, &b);
    }
    for (uint32_t l = 0; l < 3; ++l) {
      const uint8_t *d = nullptr;
      int64_t len = 0;
      if (nf4s_loader_load_layer(L, l, &d, &len) == 0 && d && len > 0) {
        volatile uint8_t s = 0;
        for (int64_t i = 0; i < len; i += 4096) s ^= d[i];
        s ^= d[len - 1];
      }
    }
    const char *pk[] = {"model.layers.0.q", "model.layers.1.q"};
    nf4s_blob_entry ent[2];
    int64_t bytes = 0;
    if (nf4s_loader_pack_layer(L, pk, 2, nullptr, 0, ent, &bytes) == 0 && bytes > 0 &&
        bytes < (1 << 26)) {
      std::vector<uint8_t> buf((size_t)bytes);
      if (nf4s_loader_pack_layer(L, pk, 2, buf.data(), bytes, ent, &bytes) == 0) {
        for (int i = 0; i < 2; ++i) {
          nf4s_tensor t;
          nf4s_blob_tensor(&ent[i], buf.data(), &t);
        }
      }
    }
    nf4s_loader_close(L);
  }
  printf("opened %d of %d\n", opened, argc - 1);
  return 0;
}
