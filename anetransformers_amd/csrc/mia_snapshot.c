/*
 * mia_snapshot.c -- KV-ring snapshots: the device ring of every layer written
 * to host memory or a file and read back, for a session that is saved and
 * resumed or moved to another process.
 *
 * The reference keeps its ring in host memory (KVCache, mistral/kv_cache.h:
 * 10-20) and has no snapshot of it; the format below carries exactly that
 * struct's sizes and cursors and its two arrays as they lie in memory, so a
 * reference-side loader can read the header fields into a KVCache and the two
 * payloads straight into k_cache / v_cache.
 *
 * Layout, little-endian, 64-byte header:
 *    0  char[8]  "MIAKVRG1"
 *    8  u32      header bytes (64)
 *   12  u32      element bytes (2: IEEE fp16)
 *   16  i32 x 7  n_layers, n_kv_heads, head_dim, max_seq, kv_dim, pos, len
 *               (KVCache's int fields in its order)
 *   44  u32      0
 *   48  u64      bytes of each payload: n_layers * max_seq * kv_dim * 2
 *   56  u64      0
 *   64  k_cache  [n_layers][max_seq][n_kv_heads][head_dim] fp16
 *       v_cache  the same
 */
#define _FILE_OFFSET_BITS 64
#define _POSIX_C_SOURCE 200809L
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/types.h>

#include "../../include/mia_dropin.h"

int mia_internal_set_error(int code, const char *msg);

#define SNAP_HDR 64
static const char kMagic[8] = {'M', 'I', 'A', 'K', 'V', 'R', 'G', '1'};

static void put_u32(uint8_t *p, uint32_t v) {
    for (int i = 0; i < 4; i++) p[i] = (uint8_t)(v >> (8 * i));
}
static void put_u64(uint8_t *p, uint64_t v) {
    for (int i = 0; i < 8; i++) p[i] = (uint8_t)(v >> (8 * i));
}
static uint32_t get_u32(const uint8_t *p) {
    uint32_t v = 0;
    for (int i = 0; i < 4; i++) v |= (uint32_t)p[i] << (8 * i);
    return v;
}
static uint64_t get_u64(const uint8_t *p) {
    uint64_t v = 0;
    for (int i = 0; i < 8; i++) v |= (uint64_t)p[i] << (8 * i);
    return v;
}

/* payload bytes of one array, 0 for a bad shape */
static uint64_t payload_bytes(int n_layers, int n_kv_heads, int head_dim, int max_seq) {
    if (n_layers <= 0 || n_kv_heads <= 0 || head_dim <= 0 || max_seq <= 0) return 0;
    const uint64_t kv_dim = (uint64_t)n_kv_heads * (uint64_t)head_dim;
    if (kv_dim > INT32_MAX) return 0;
    return (uint64_t)n_layers * (uint64_t)max_seq * kv_dim * 2u;
}

size_t mia_kv_snapshot_bytes(int n_layers, int n_kv_heads, int head_dim, int max_seq) {
    const uint64_t p = payload_bytes(n_layers, n_kv_heads, head_dim, max_seq);
    return p ? (size_t)(SNAP_HDR + 2 * p) : 0;
}

static void write_header(uint8_t *h, int n_layers, int n_kv_heads, int head_dim, int max_seq,
                         int pos, int len, uint64_t payload) {
    memset(h, 0, SNAP_HDR);
    memcpy(h, kMagic, 8);
    put_u32(h + 8, SNAP_HDR);
    put_u32(h + 12, 2);
    const int f[7] = {n_layers, n_kv_heads, head_dim, max_seq, n_kv_heads * head_dim, pos, len};
    for (int i = 0; i < 7; i++) put_u32(h + 16 + 4 * i, (uint32_t)f[i]);
    put_u64(h + 48, payload);
}

/* header fields -> f[7]; MIA_OK or MIA_ERR_INVALID with the reason */
static int read_header(const uint8_t *h, size_t avail, int f[7], uint64_t *payload) {
    if (avail < SNAP_HDR) return mia_internal_set_error(MIA_ERR_INVALID, "snapshot: short header");
    if (memcmp(h, kMagic, 8) != 0)
        return mia_internal_set_error(MIA_ERR_INVALID, "snapshot: not a KV-ring snapshot");
    if (get_u32(h + 8) != SNAP_HDR || get_u32(h + 12) != 2)
        return mia_internal_set_error(MIA_ERR_INVALID, "snapshot: unknown header or element size");
    for (int i = 0; i < 7; i++) f[i] = (int)get_u32(h + 16 + 4 * i);
    *payload = get_u64(h + 48);
    if ((int64_t)f[4] != (int64_t)f[1] * f[2] ||
        *payload != payload_bytes(f[0], f[1], f[2], f[3]) || *payload == 0)
        return mia_internal_set_error(MIA_ERR_INVALID, "snapshot: inconsistent sizes");
    if (f[5] < 0 || f[6] < 0 || f[6] > f[3])
        return mia_internal_set_error(MIA_ERR_INVALID, "snapshot: bad pos / len");
    return MIA_OK;
}

int mia_kv_snapshot_info(const void *src, size_t src_bytes, int *n_layers, int *n_kv_heads,
                         int *head_dim, int *max_seq, int *pos, int *len) {
    if (!src) return mia_internal_set_error(MIA_ERR_INVALID, "snapshot: NULL pointer");
    int f[7];
    uint64_t payload;
    int rc = read_header((const uint8_t *)src, src_bytes, f, &payload);
    if (rc) return rc;
    if (n_layers) *n_layers = f[0];
    if (n_kv_heads) *n_kv_heads = f[1];
    if (head_dim) *head_dim = f[2];
    if (max_seq) *max_seq = f[3];
    if (pos) *pos = f[5];
    if (len) *len = f[6];
    return MIA_OK;
}

int mia_kv_snapshot_save(void *dst, size_t dst_bytes, const uint16_t *k_cache,
                         const uint16_t *v_cache, int n_layers, int n_kv_heads, int head_dim,
                         int max_seq, int pos, int len) {
    if (!dst || !k_cache || !v_cache)
        return mia_internal_set_error(MIA_ERR_INVALID, "snapshot: NULL pointer");
    const uint64_t p = payload_bytes(n_layers, n_kv_heads, head_dim, max_seq);
    if (p == 0) return mia_internal_set_error(MIA_ERR_INVALID, "snapshot: bad ring shape");
    if (pos < 0 || len < 0 || len > max_seq)
        return mia_internal_set_error(MIA_ERR_INVALID, "snapshot: bad pos / len");
    if (dst_bytes < SNAP_HDR + 2 * p)
        return mia_internal_set_error(MIA_ERR_INVALID, "snapshot: destination too small");
    uint8_t *d = (uint8_t *)dst;
    write_header(d, n_layers, n_kv_heads, head_dim, max_seq, pos, len, p);
    int rc = mia_memcpy_d2h(d + SNAP_HDR, k_cache, (size_t)p);
    if (rc) return rc;
    return mia_memcpy_d2h(d + SNAP_HDR + p, v_cache, (size_t)p);
}

int mia_kv_snapshot_load(const void *src, size_t src_bytes, uint16_t *k_cache, uint16_t *v_cache,
                         int n_layers, int n_kv_heads, int head_dim, int max_seq, int *pos,
                         int *len) {
    if (!src || !k_cache || !v_cache)
        return mia_internal_set_error(MIA_ERR_INVALID, "snapshot: NULL pointer");
    int f[7];
    uint64_t p;
    int rc = read_header((const uint8_t *)src, src_bytes, f, &p);
    if (rc) return rc;
    if (f[0] != n_layers || f[1] != n_kv_heads || f[2] != head_dim || f[3] != max_seq)
        return mia_internal_set_error(MIA_ERR_INVALID, "snapshot: ring shape differs");
    if (src_bytes < SNAP_HDR + 2 * p)
        return mia_internal_set_error(MIA_ERR_INVALID, "snapshot: truncated");
    const uint8_t *s = (const uint8_t *)src;
    rc = mia_memcpy_h2d(k_cache, s + SNAP_HDR, (size_t)p);
    if (rc) return rc;
    rc = mia_memcpy_h2d(v_cache, s + SNAP_HDR + p, (size_t)p);
    if (rc) return rc;
    if (pos) *pos = f[5];
    if (len) *len = f[6];
    return MIA_OK;
}

/* ---- files, through a bounded host buffer ------------------------------- */

#define SNAP_CHUNK ((size_t)64 << 20)

static int copy_to_file(FILE *fp, const uint16_t *dev, uint64_t bytes, uint8_t *buf) {
    for (uint64_t off = 0; off < bytes; off += SNAP_CHUNK) {
        const size_t n = (size_t)(bytes - off < SNAP_CHUNK ? bytes - off : SNAP_CHUNK);
        int rc = mia_memcpy_d2h(buf, (const uint8_t *)dev + off, n);
        if (rc) return rc;
        if (fwrite(buf, 1, n, fp) != n)
            return mia_internal_set_error(MIA_ERR_INVALID, "snapshot: write failed");
    }
    return MIA_OK;
}

static int copy_from_file(FILE *fp, uint16_t *dev, uint64_t bytes, uint8_t *buf) {
    for (uint64_t off = 0; off < bytes; off += SNAP_CHUNK) {
        const size_t n = (size_t)(bytes - off < SNAP_CHUNK ? bytes - off : SNAP_CHUNK);
        if (fread(buf, 1, n, fp) != n)
            return mia_internal_set_error(MIA_ERR_INVALID, "snapshot: truncated file");
        int rc = mia_memcpy_h2d((uint8_t *)dev + off, buf, n);
        if (rc) return rc;
    }
    return MIA_OK;
}

int mia_dropin_kv_save(const KVCache *c, const char *path) {
    if (!c || !path || !c->k_cache || !c->v_cache)
        return mia_internal_set_error(MIA_ERR_INVALID, "kv_save: NULL pointer");
    const uint64_t p = payload_bytes(c->n_layers, c->n_kv_heads, c->head_dim, c->max_seq);
    if (p == 0 || c->kv_dim != c->n_kv_heads * c->head_dim)
        return mia_internal_set_error(MIA_ERR_INVALID, "kv_save: bad ring shape");
    if (c->pos < 0 || c->len < 0 || c->len > c->max_seq)
        return mia_internal_set_error(MIA_ERR_INVALID, "kv_save: bad pos / len");
    uint8_t *buf = (uint8_t *)malloc(SNAP_CHUNK);
    if (!buf) return mia_internal_set_error(MIA_ERR_INVALID, "kv_save: out of host memory");
    FILE *fp = fopen(path, "wb");
    int rc = fp ? MIA_OK : mia_internal_set_error(MIA_ERR_INVALID, "kv_save: cannot open file");
    if (!rc) {
        uint8_t h[SNAP_HDR];
        write_header(h, c->n_layers, c->n_kv_heads, c->head_dim, c->max_seq, c->pos, c->len, p);
        if (fwrite(h, 1, SNAP_HDR, fp) != SNAP_HDR)
            rc = mia_internal_set_error(MIA_ERR_INVALID, "kv_save: write failed");
    }
    if (!rc) rc = copy_to_file(fp, (const uint16_t *)c->k_cache, p, buf);
    if (!rc) rc = copy_to_file(fp, (const uint16_t *)c->v_cache, p, buf);
    if (fp && fclose(fp) != 0 && !rc)
        rc = mia_internal_set_error(MIA_ERR_INVALID, "kv_save: write failed");
    free(buf);
    return rc;
}

int mia_dropin_kv_load(KVCache *c, const char *path) {
    if (!c || !path || !c->k_cache || !c->v_cache)
        return mia_internal_set_error(MIA_ERR_INVALID, "kv_load: NULL pointer");
    FILE *fp = fopen(path, "rb");
    if (!fp) return mia_internal_set_error(MIA_ERR_INVALID, "kv_load: cannot open file");
    uint8_t h[SNAP_HDR];
    int f[7];
    uint64_t p = 0;
    const size_t got = fread(h, 1, SNAP_HDR, fp);
    int rc = read_header(h, got, f, &p);
    if (!rc && (f[0] != c->n_layers || f[1] != c->n_kv_heads || f[2] != c->head_dim ||
                f[3] != c->max_seq))
        rc = mia_internal_set_error(MIA_ERR_INVALID, "kv_load: ring shape differs");
    if (!rc) {  // the whole file is there before the cache is touched
        if (fseeko(fp, 0, SEEK_END) != 0 || ftello(fp) < (off_t)(SNAP_HDR + 2 * p) ||
            fseeko(fp, SNAP_HDR, SEEK_SET) != 0)
            rc = mia_internal_set_error(MIA_ERR_INVALID, "kv_load: truncated file");
    }
    uint8_t *buf = rc ? NULL : (uint8_t *)malloc(SNAP_CHUNK);
    if (!rc && !buf) rc = mia_internal_set_error(MIA_ERR_INVALID, "kv_load: out of host memory");
    if (!rc) rc = copy_from_file(fp, (uint16_t *)c->k_cache, p, buf);
    if (!rc) rc = copy_from_file(fp, (uint16_t *)c->v_cache, p, buf);
    fclose(fp);
    free(buf);
    if (!rc) {
        c->pos = f[5];
        c->len = f[6];
    }
    return rc;
}
