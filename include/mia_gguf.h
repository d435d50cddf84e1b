/*
 * mia_gguf.h -- GGUF (v2/v3) weight files mapped on the host and uploaded to
 * the MI355X in their own block layout, so the Q4_0 tensors feed
 * mia_q4_0_matvec* directly.  Part of libmiattn.so; plain C.
 *
 * Replaces mistral/gguf_loader.h's parsing (gguf_open, gguf_find, gguf_data,
 * gguf_tensor_bytes, gguf_close) for the weights; the tokenizer arrays are
 * skipped (only their length, the vocabulary size, is kept).  Differences:
 *   - every read is bounds-checked: a truncated or inconsistent file is an
 *     error (MIA_ERR_INVALID), not a read past the mapping;
 *   - general.alignment is honoured (the GGUF rule; gguf_loader.h:280 always
 *     uses 32, the default, which is what Mistral files carry);
 *   - tensor byte sizes are known for every ggml block type
 *     (gguf_loader.h:361-371 returns 0 for Q4_1, Q5_x, Q2_K, Q3_K, Q5_K, Q6_K);
 *   - versions other than 2 and 3 are refused (v1 has 32-bit counts).
 * Errors return a mia_status; the message is in mia_last_error().
 */
#ifndef MIA_GGUF_H
#define MIA_GGUF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mia_gguf mia_gguf; /* a mapped file (opaque) */

/* GGUFTensor (mistral/gguf_loader.h:43-49) plus the tensor's byte size. */
typedef struct {
    char name[256];
    uint32_t n_dims;
    uint64_t ne[4];  /* ne[0] = columns (in_dim), ne[1] = rows; unused dims 1 */
    uint32_t type;   /* GGML_TYPE_* (gguf_loader.h:31-39) */
    uint64_t offset; /* from the start of the data section */
    uint64_t bytes;
} mia_gguf_tensor;

/* MistralConfig (mistral/gguf_loader.h:52-64), same fields and order, filled
 * from the same keys with the same defaults (gguf_loader.h:166-171, 192-228). */
typedef struct {
    int dim;
    int hidden_dim;
    int n_layers;
    int n_heads;
    int n_kv_heads;
    int head_dim;
    int vocab_size;
    int max_seq_len;
    float rope_theta;
    float rms_eps;
    int sliding_window;
} mia_gguf_config;

int mia_gguf_open(const char *path, mia_gguf **out);
void mia_gguf_close(mia_gguf *f);
int mia_gguf_get_config(const mia_gguf *f, mia_gguf_config *cfg);
/* version, and the tokenizer's bos / eos / unk ids (defaults 1, 2, 0). */
int mia_gguf_get_header(const mia_gguf *f, uint32_t *version, int *bos_id, int *eos_id,
                        int *unk_id);
int mia_gguf_n_tensors(const mia_gguf *f);
int mia_gguf_tensor_at(const mia_gguf *f, int index, mia_gguf_tensor *t);
/* gguf_find: MIA_ERR_INVALID if absent. */
int mia_gguf_find(const mia_gguf *f, const char *name, mia_gguf_tensor *t);
/* gguf_data: the tensor's bytes in the host mapping. */
const void *mia_gguf_host_data(const mia_gguf *f, const mia_gguf_tensor *t);
/* Offset of the data section in the file, and its length (to the file end). */
size_t mia_gguf_data_offset(const mia_gguf *f);
size_t mia_gguf_data_bytes(const mia_gguf *f);
/* Bytes per block and values per block of a ggml type (0, 0 if unknown). */
int mia_gguf_type_block(uint32_t type, uint32_t *block_bytes, uint32_t *block_values);

/* Copies the whole data section into one device allocation (*dev, *bytes;
 * free with mia_free), as the Metal backend wraps the mapping in one buffer
 * (mistral/metal_matvec.h:185-192): tensor t is then at (char *)*dev +
 * t.offset, in the file's layout.  Synchronous; copied from the mapping in
 * 64 MiB pieces. */
int mia_gguf_upload(const mia_gguf *f, void **dev, size_t *bytes);

#ifdef __cplusplus
}
#endif
#endif
