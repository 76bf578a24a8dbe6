// Host-only driver for the GGUF parser under AddressSanitizer / UBSan: opens
// every file named on the command line and walks everything a loader reads
// (version, metadata entries and lookups, tensor table, model config). Exit
// status 0 unless a sanitizer reports an error.
#include <cstdio>

#include "../../include/zinc_hip.h"

int main(int argc, char **argv) {
    int opened = 0;
    for (int i = 1; i < argc; i++) {
        zh_gguf *f = nullptr;
        if (zh_gguf_open(argv[i], &f) != ZH_OK) continue;
        opened++;
        (void)zh_gguf_version(f);
        (void)zh_gguf_data_offset(f);
        for (uint64_t m = 0; m < zh_gguf_metadata_count(f); m++) {
            const char *key = nullptr;
            uint32_t t = 0, et = 0;
            uint64_t n = 0;
            if (zh_gguf_metadata_entry(f, m, &key, &t, &et, &n) == ZH_OK && key) {
                uint32_t u32;
                uint64_t u64;
                float f32;
                int b;
                const char *s;
                uint64_t len;
                (void)zh_gguf_get_u32(f, key, &u32);
                (void)zh_gguf_get_u64(f, key, &u64);
                (void)zh_gguf_get_f32(f, key, &f32);
                (void)zh_gguf_get_bool(f, key, &b);
                (void)zh_gguf_get_string(f, key, &s, &len);
            }
        }
        for (uint64_t t = 0; t < zh_gguf_tensor_count(f); t++) {
            const char *name = nullptr;
            uint32_t nd = 0, type = 0;
            uint64_t dims[4], off = 0, bytes = 0;
            if (zh_gguf_tensor_info(f, t, &name, &nd, dims, &type, &off, &bytes) == ZH_OK && name)
                (void)zh_gguf_find_tensor(f, name);
        }
        zh_model_config cfg;
        (void)zh_gguf_model_config(f, 0, &cfg);
        zh_gguf_close(f);
    }
    printf("opened %d of %d\n", opened, argc - 1);
    return 0;
}
