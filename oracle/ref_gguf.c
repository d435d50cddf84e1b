/*
 * ref_gguf.c -- test infrastructure: exposes the reference's own GGUF parser
 * (mistral/gguf_loader.h, header-only C over POSIX mmap, which builds as it
 * lies in the reference tree) to the CPU tests, which check libmiattn's
 * loader against it.  Built by `make -C oracle ref` into oracle/_ref/ only
 * when the reference tree is present; nothing here is shipped or timed.
 */
#include "gguf_loader.h"

void *ref_gguf_open(const char *path) { return gguf_open(path); }

void ref_gguf_close(void *h) { gguf_close((GGUFFile *)h); }

/* ints: dim, hidden_dim, n_layers, n_heads, n_kv_heads, head_dim, vocab_size,
 * max_seq_len, sliding_window, version, n_tensors, bos, eos, unk;
 * floats: rope_theta, rms_eps. */
void ref_gguf_config(void *h, int *ints, float *floats) {
    GGUFFile *f = (GGUFFile *)h;
    MistralConfig *c = &f->cfg;
    int v[14] = {c->dim, c->hidden_dim, c->n_layers, c->n_heads, c->n_kv_heads, c->head_dim,
                 c->vocab_size, c->max_seq_len, c->sliding_window, (int)f->version,
                 (int)f->n_tensors, f->bos_id, f->eos_id, f->unk_id};
    memcpy(ints, v, sizeof(v));
    floats[0] = c->rope_theta;
    floats[1] = c->rms_eps;
}

void ref_gguf_tensor(void *h, int i, char *name, uint32_t *n_dims, uint64_t *ne, uint32_t *type,
                     uint64_t *offset, uint64_t *bytes) {
    GGUFFile *f = (GGUFFile *)h;
    GGUFTensor *t = &f->tensors[i];
    memcpy(name, t->name, GGUF_MAX_NAME);
    *n_dims = t->n_dims;
    memcpy(ne, t->ne, sizeof(t->ne));
    *type = t->type;
    *offset = t->offset;
    *bytes = gguf_tensor_bytes(t);
}

long ref_gguf_data_offset(void *h) {
    GGUFFile *f = (GGUFFile *)h;
    return (long)(f->data_start - (uint8_t *)f->mmap_base);
}
