/* Test driver (sanitizer tier): opens every GGUF file named on the command
 * line with libmiattn's loader (anetransformers_amd/csrc/mia_gguf.c, built
 * into this executable with AddressSanitizer and UBSan) and, when the open
 * succeeds, walks everything the API exposes: config, header, every tensor's
 * record and bytes in the mapping, lookups by name.  Prints one line per file
 * (name, status); a sanitizer report aborts the run. */
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "../../include/mia_gguf.h"
#include "../../include/miattn.h"

/* The library's error and device entry points the loader calls, stubbed:
 * this build has no device. */
static char g_msg[512];
int mia_internal_set_error(int code, const char *msg) {
    snprintf(g_msg, sizeof g_msg, "%s", msg ? msg : "");
    return code;
}
int mia_malloc(void **dptr, size_t bytes) { (void)dptr; (void)bytes; return MIA_ERR_NO_DEVICE; }
int mia_free(void *dptr) { (void)dptr; return MIA_OK; }
int mia_memcpy_h2d(void *d, const void *s, size_t n) { (void)d; (void)s; (void)n; return MIA_ERR_NO_DEVICE; }

static int walk(mia_gguf *f) {
    mia_gguf_config c;
    uint32_t version;
    int bos, eos, unk;
    if (mia_gguf_get_config(f, &c) || mia_gguf_get_header(f, &version, &bos, &eos, &unk)) return 1;
    const size_t off = mia_gguf_data_offset(f), nbytes = mia_gguf_data_bytes(f);
    (void)off;
    const int n = mia_gguf_n_tensors(f);
    uint64_t sum = 0;
    for (int i = 0; i < n; ++i) {
        mia_gguf_tensor t, u;
        if (mia_gguf_tensor_at(f, i, &t)) return 1;
        if (t.offset + t.bytes > nbytes) return 2;  /* an accepted tensor must lie in the data */
        const unsigned char *p = (const unsigned char *)mia_gguf_host_data(f, &t);
        if (!p && t.bytes) return 3;
        for (uint64_t b = 0; b < t.bytes; ++b) sum += p[b];
        if (mia_gguf_find(f, t.name, &u)) return 4;
        uint32_t bb, bv;
        mia_gguf_type_block(t.type, &bb, &bv);
    }
    mia_gguf_tensor none;
    if (mia_gguf_tensor_at(f, n, &none) == MIA_OK) return 5;  /* past the end is an error */
    void *dev = NULL;
    size_t db = 0;
    if (mia_gguf_upload(f, &dev, &db) == MIA_OK) return 6;    /* no device in this build */
    printf("  walked %d tensors, byte sum %llu\n", n, (unsigned long long)sum);
    return 0;
}

int main(int argc, char **argv) {
    int bad = 0;
    for (int a = 1; a < argc; ++a) {
        mia_gguf *f = NULL;
        const int rc = mia_gguf_open(argv[a], &f);
        printf("%s %d %s\n", argv[a], rc, rc ? g_msg : "");
        if (rc == MIA_OK) {
            const int w = walk(f);
            if (w) {
                printf("  walk failed (%d)\n", w);
                bad = 1;
            }
            mia_gguf_close(f);
        } else if (f != NULL) {
            printf("  a failed open returned a handle\n");
            bad = 1;
        }
    }
    return bad;
}
