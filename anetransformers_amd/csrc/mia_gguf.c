/*
 * mia_gguf.c -- GGUF v2/v3 parsing over a read-only mapping and the upload of
 * the tensor data section to device memory (include/mia_gguf.h).
 *
 * The file layout (the GGUF format, which mistral/gguf_loader.h:150-320 reads):
 *   u32 magic "GGUF", u32 version, u64 n_tensors, u64 n_kv,
 *   n_kv x (string key, u32 value type, value),
 *   n_tensors x (string name, u32 n_dims, n_dims x u64 ne, u32 type, u64 offset),
 *   padding to the alignment, then the data section.
 * Strings are a u64 length and the bytes; arrays are a u32 element type, a
 * u64 count and the elements.  All little-endian.
 */
#define _GNU_SOURCE
#include <fcntl.h>
#include <limits.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "../../include/mia_gguf.h"
#include "../../include/miattn.h"

int mia_internal_set_error(int code, const char *msg);

enum {
    V_U8 = 0, V_I8 = 1, V_U16 = 2, V_I16 = 3, V_U32 = 4, V_I32 = 5, V_F32 = 6, V_BOOL = 7,
    V_STR = 8, V_ARR = 9, V_U64 = 10, V_I64 = 11, V_F64 = 12
};

struct mia_gguf {
    int fd;
    const uint8_t *map;
    size_t size;
    size_t data_off;
    uint32_t version;
    uint32_t n_tensors;
    mia_gguf_tensor *tensors;
    mia_gguf_config cfg;
    int bos_id, eos_id, unk_id;
};

typedef struct {
    const uint8_t *p;
    size_t pos, size;
    int bad;
} reader;

static int fail(int code, const char *msg) { return mia_internal_set_error(code, msg); }

static int take(reader *r, size_t n) {
    if (r->bad || n > r->size - r->pos) {
        r->bad = 1;
        return 0;
    }
    return 1;
}

static uint64_t get(reader *r, size_t n) { /* little-endian unsigned of n <= 8 bytes */
    uint64_t v = 0;
    if (!take(r, n)) return 0;
    for (size_t i = 0; i < n; i++) v |= (uint64_t)r->p[r->pos + i] << (8 * i);
    r->pos += n;
    return v;
}

static const char *get_str(reader *r, uint64_t *len) {
    *len = get(r, 8);
    if (r->bad || !take(r, *len)) return NULL;
    const char *s = (const char *)r->p + r->pos;
    r->pos += *len;
    return s;
}

static size_t scalar_size(uint32_t t) {
    switch (t) {
    case V_U8: case V_I8: case V_BOOL: return 1;
    case V_U16: case V_I16: return 2;
    case V_U32: case V_I32: case V_F32: return 4;
    case V_U64: case V_I64: case V_F64: return 8;
    default: return 0;
    }
}

static void skip_value(reader *r, uint32_t t, int depth) {
    size_t n = scalar_size(t);
    if (n) {
        if (take(r, n)) r->pos += n;
    } else if (t == V_STR) {
        uint64_t len;
        get_str(r, &len);
    } else if (t == V_ARR && depth < 8) {
        uint32_t et = (uint32_t)get(r, 4);
        uint64_t count = get(r, 8);
        size_t es = scalar_size(et);
        if (es) {
            if (count > (r->size - r->pos) / es) r->bad = 1;
            else r->pos += count * es;
        } else {
            for (uint64_t i = 0; i < count && !r->bad; i++) skip_value(r, et, depth + 1);
        }
    } else {
        r->bad = 1; /* unknown type or nesting too deep */
    }
}

/* Integer value of a numeric scalar, as gguf_read_uint does for the config
 * keys (signed types sign-extended); *ok = 0 (value skipped) otherwise. */
static int64_t read_int(reader *r, uint32_t t, int *ok) {
    *ok = 1;
    switch (t) {
    case V_U8: case V_BOOL: return (int64_t)get(r, 1);
    case V_I8: return (int8_t)get(r, 1);
    case V_U16: return (int64_t)get(r, 2);
    case V_I16: return (int16_t)get(r, 2);
    case V_U32: return (int64_t)get(r, 4);
    case V_I32: return (int32_t)get(r, 4);
    case V_U64: return (int64_t)get(r, 8);
    case V_I64: return (int64_t)get(r, 8);
    default: *ok = 0; skip_value(r, t, 0); return 0;
    }
}

static float read_float(reader *r, uint32_t t, int *ok) {
    if (t == V_F32) {
        uint32_t b = (uint32_t)get(r, 4);
        float f;
        memcpy(&f, &b, 4);
        *ok = 1;
        return f;
    }
    if (t == V_F64) {
        uint64_t b = get(r, 8);
        double d;
        memcpy(&d, &b, 8);
        *ok = 1;
        return (float)d;
    }
    int64_t v = read_int(r, t, ok);
    return (float)(uint64_t)v; /* gguf_loader.h:125: (float) of the unsigned read */
}

static int key_is(const char *k, uint64_t len, const char *want) {
    size_t n = strlen(want);
    return len == n && memcmp(k, want, n) == 0;
}

/* "llama.<s>" or "mistral.<s>" (gguf_loader.h:192-216 accepts both). */
static int arch_key(const char *k, uint64_t len, const char *suffix) {
    char a[128], b[128];
    snprintf(a, sizeof(a), "llama.%s", suffix);
    snprintf(b, sizeof(b), "mistral.%s", suffix);
    return key_is(k, len, a) || key_is(k, len, b);
}

int mia_gguf_type_block(uint32_t type, uint32_t *block_bytes, uint32_t *block_values) {
    /* ggml block sizes: bytes per block, values per block */
    static const uint32_t tab[][3] = {
        {0, 4, 1},     {1, 2, 1},     {2, 18, 32},   {3, 20, 32},   {6, 22, 32},
        {7, 24, 32},   {8, 34, 32},   {9, 36, 32},   {10, 84, 256}, {11, 110, 256},
        {12, 144, 256}, {13, 176, 256}, {14, 210, 256}, {15, 292, 256},
    };
    for (size_t i = 0; i < sizeof(tab) / sizeof(tab[0]); i++) {
        if (tab[i][0] == type) {
            if (block_bytes) *block_bytes = tab[i][1];
            if (block_values) *block_values = tab[i][2];
            return MIA_OK;
        }
    }
    if (block_bytes) *block_bytes = 0;
    if (block_values) *block_values = 0;
    return MIA_ERR_UNSUPPORTED;
}

static int parse(mia_gguf *f) {
    reader r = {f->map, 0, f->size, 0};
    if ((uint32_t)get(&r, 4) != 0x46554747u || r.bad) return fail(MIA_ERR_INVALID, "not a GGUF file");
    f->version = (uint32_t)get(&r, 4);
    if (f->version != 2 && f->version != 3)
        return fail(MIA_ERR_UNSUPPORTED, "GGUF version not 2 or 3");
    uint64_t n_tensors = get(&r, 8), n_kv = get(&r, 8);
    if (r.bad || n_tensors > (f->size / 32) || n_tensors > INT_MAX || n_kv > f->size / 12)
        return fail(MIA_ERR_INVALID, "GGUF header counts exceed the file");
    f->n_tensors = (uint32_t)n_tensors;

    /* defaults of gguf_loader.h:166-171 */
    f->cfg.rope_theta = 10000.0f;
    f->cfg.rms_eps = 1e-5f;
    f->cfg.sliding_window = 4096;
    f->bos_id = 1;
    f->eos_id = 2;
    f->unk_id = 0;
    uint64_t alignment = 32;

    for (uint64_t i = 0; i < n_kv && !r.bad; i++) {
        uint64_t kl;
        const char *k = get_str(&r, &kl);
        uint32_t vt = (uint32_t)get(&r, 4);
        if (r.bad) break;
        int ok = 0;
        int *ip = NULL;
        float *fp = NULL;
        if (arch_key(k, kl, "embedding_length")) ip = &f->cfg.dim;
        else if (arch_key(k, kl, "feed_forward_length")) ip = &f->cfg.hidden_dim;
        else if (arch_key(k, kl, "block_count")) ip = &f->cfg.n_layers;
        else if (arch_key(k, kl, "attention.head_count")) ip = &f->cfg.n_heads;
        else if (arch_key(k, kl, "attention.head_count_kv")) ip = &f->cfg.n_kv_heads;
        else if (arch_key(k, kl, "context_length")) ip = &f->cfg.max_seq_len;
        else if (arch_key(k, kl, "rope.freq_base")) fp = &f->cfg.rope_theta;
        else if (arch_key(k, kl, "attention.layer_norm_rms_epsilon")) fp = &f->cfg.rms_eps;
        else if (key_is(k, kl, "mistral.attention.sliding_window")) ip = &f->cfg.sliding_window;
        else if (key_is(k, kl, "tokenizer.ggml.bos_token_id")) ip = &f->bos_id;
        else if (key_is(k, kl, "tokenizer.ggml.eos_token_id")) ip = &f->eos_id;
        else if (key_is(k, kl, "tokenizer.ggml.unknown_token_id")) ip = &f->unk_id;
        if (ip) {
            int64_t v = read_int(&r, vt, &ok);
            if (ok) *ip = (int)v;
        } else if (fp) {
            float v = read_float(&r, vt, &ok);
            if (ok) *fp = v;
        } else if (key_is(k, kl, "general.alignment")) {
            int64_t v = read_int(&r, vt, &ok);
            if (ok) {
                if (v <= 0 || (v & (v - 1)) || v > (1 << 20))
                    return fail(MIA_ERR_INVALID, "general.alignment not a power of two");
                alignment = (uint64_t)v;
            }
        } else if (key_is(k, kl, "tokenizer.ggml.tokens") && vt == V_ARR) {
            size_t save = r.pos;
            get(&r, 4);
            uint64_t count = get(&r, 8);
            if (!r.bad && count <= INT_MAX) f->cfg.vocab_size = (int)count;
            r.pos = save;
            skip_value(&r, vt, 0);
        } else {
            skip_value(&r, vt, 0);
        }
    }
    if (r.bad) return fail(MIA_ERR_INVALID, "GGUF metadata runs past the end of the file");
    if (f->cfg.dim > 0 && f->cfg.n_heads > 0) f->cfg.head_dim = f->cfg.dim / f->cfg.n_heads;

    f->tensors = (mia_gguf_tensor *)calloc(n_tensors ? n_tensors : 1, sizeof(mia_gguf_tensor));
    if (!f->tensors) return fail(MIA_ERR_INVALID, "out of host memory");
    for (uint64_t i = 0; i < n_tensors; i++) {
        mia_gguf_tensor *t = &f->tensors[i];
        uint64_t nl;
        const char *name = get_str(&r, &nl);
        t->n_dims = (uint32_t)get(&r, 4);
        if (r.bad || t->n_dims < 1 || t->n_dims > 4)
            return fail(MIA_ERR_INVALID, "GGUF tensor info is truncated or has more than 4 dims");
        size_t cpy = nl < sizeof(t->name) - 1 ? (size_t)nl : sizeof(t->name) - 1;
        memcpy(t->name, name, cpy);
        t->name[cpy] = '\0';
        for (uint32_t d = 0; d < 4; d++) t->ne[d] = d < t->n_dims ? get(&r, 8) : 1;
        t->type = (uint32_t)get(&r, 4);
        t->offset = get(&r, 8);
        if (r.bad) return fail(MIA_ERR_INVALID, "GGUF tensor info runs past the end of the file");
    }
    f->data_off = (r.pos + alignment - 1) & ~(size_t)(alignment - 1);
    if (f->data_off > f->size) return fail(MIA_ERR_INVALID, "GGUF data section starts past the end");
    const uint64_t data_len = f->size - f->data_off;
    for (uint32_t i = 0; i < f->n_tensors; i++) {
        mia_gguf_tensor *t = &f->tensors[i];
        uint32_t bb, bv;
        uint64_t nel = 1;
        for (uint32_t d = 0; d < t->n_dims; d++) {
            if (t->ne[d] && nel > UINT64_MAX / t->ne[d])
                return fail(MIA_ERR_INVALID, "GGUF tensor element count overflows");
            nel *= t->ne[d];
        }
        t->bytes = 0;
        if (mia_gguf_type_block(t->type, &bb, &bv) == MIA_OK) {
            if (nel % bv) return fail(MIA_ERR_INVALID, "GGUF tensor is not a whole number of blocks");
            t->bytes = nel / bv * bb;
        }
        if (t->offset > data_len || t->bytes > data_len - t->offset)
            return fail(MIA_ERR_INVALID, "GGUF tensor lies outside the data section");
    }
    return MIA_OK;
}

int mia_gguf_open(const char *path, mia_gguf **out) {
    if (!path || !out) return fail(MIA_ERR_INVALID, "NULL argument");
    *out = NULL;
    int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(MIA_ERR_INVALID, "cannot open the GGUF file");
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        close(fd);
        return fail(MIA_ERR_INVALID, "GGUF file too short");
    }
    void *map = mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (map == MAP_FAILED) {
        close(fd);
        return fail(MIA_ERR_INVALID, "cannot map the GGUF file");
    }
    madvise(map, (size_t)st.st_size, MADV_SEQUENTIAL);
    mia_gguf *f = (mia_gguf *)calloc(1, sizeof(mia_gguf));
    if (!f) {
        munmap(map, (size_t)st.st_size);
        close(fd);
        return fail(MIA_ERR_INVALID, "out of host memory");
    }
    f->fd = fd;
    f->map = (const uint8_t *)map;
    f->size = (size_t)st.st_size;
    int rc = parse(f);
    if (rc) {
        mia_gguf_close(f);
        return rc;
    }
    *out = f;
    return MIA_OK;
}

void mia_gguf_close(mia_gguf *f) {
    if (!f) return;
    free(f->tensors);
    if (f->map) munmap((void *)f->map, f->size);
    if (f->fd >= 0) close(f->fd);
    free(f);
}

int mia_gguf_get_config(const mia_gguf *f, mia_gguf_config *cfg) {
    if (!f || !cfg) return fail(MIA_ERR_INVALID, "NULL argument");
    *cfg = f->cfg;
    return MIA_OK;
}

int mia_gguf_get_header(const mia_gguf *f, uint32_t *version, int *bos_id, int *eos_id,
                        int *unk_id) {
    if (!f) return fail(MIA_ERR_INVALID, "NULL argument");
    if (version) *version = f->version;
    if (bos_id) *bos_id = f->bos_id;
    if (eos_id) *eos_id = f->eos_id;
    if (unk_id) *unk_id = f->unk_id;
    return MIA_OK;
}

int mia_gguf_n_tensors(const mia_gguf *f) { return f ? (int)f->n_tensors : 0; }

int mia_gguf_tensor_at(const mia_gguf *f, int index, mia_gguf_tensor *t) {
    if (!f || !t || index < 0 || (uint32_t)index >= f->n_tensors)
        return fail(MIA_ERR_INVALID, "tensor index out of range");
    *t = f->tensors[index];
    return MIA_OK;
}

int mia_gguf_find(const mia_gguf *f, const char *name, mia_gguf_tensor *t) {
    if (!f || !name || !t) return fail(MIA_ERR_INVALID, "NULL argument");
    for (uint32_t i = 0; i < f->n_tensors; i++) {
        if (strcmp(f->tensors[i].name, name) == 0) {
            *t = f->tensors[i];
            return MIA_OK;
        }
    }
    return fail(MIA_ERR_INVALID, "tensor not in the GGUF file");
}

const void *mia_gguf_host_data(const mia_gguf *f, const mia_gguf_tensor *t) {
    if (!f || !t) return NULL;
    return f->map + f->data_off + t->offset;
}

size_t mia_gguf_data_offset(const mia_gguf *f) { return f ? f->data_off : 0; }

size_t mia_gguf_data_bytes(const mia_gguf *f) { return f ? f->size - f->data_off : 0; }

int mia_gguf_upload(const mia_gguf *f, void **dev, size_t *bytes) {
    if (!f || !dev || !bytes) return fail(MIA_ERR_INVALID, "NULL argument");
    const size_t n = f->size - f->data_off;
    void *d = NULL;
    int rc = mia_malloc(&d, n);
    if (rc) return rc;
    const size_t piece = (size_t)64 << 20;
    for (size_t off = 0; off < n; off += piece) {
        size_t len = n - off < piece ? n - off : piece;
        rc = mia_memcpy_h2d((char *)d + off, f->map + f->data_off + off, len);
        if (rc) {
            mia_free(d);
            return rc;
        }
    }
    *dev = d;
    *bytes = n;
    return MIA_OK;
}
