/* sp_model_load.c -- .sp-model / .sp-tokenizer mmap loader.
 *
 * Follows the validation order of core/io_format/sp_model_load.c:119-186:
 * magic, version_major, header_size, CRC-32 over [0,360), file_size, arch_struct
 * sizing, table offset, 65536-aligned data region, table/data bounds, tokenizer
 * SHA-256 == header.tokenizer_hash, tokenizer magic, vocab agreement, and the
 * first/last-block 0xA5 sentinel sample of every Spinor tensor.  Tensor lookup
 * is a binary search on the xxh64-sorted table with a name check over the run of
 * equal hashes (sp_model_load.c:214-228).  Nothing proportional to tensor data
 * is allocated: the mapping is the in-memory layout. */
#include "sp_model_abi.h"
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

struct sp_model {
    const uint8_t *map;   uint64_t map_len;  int fd;
    const uint8_t *tmap;  uint64_t tmap_len; int tfd;
    sp_model_header hdr;
    const sp_tensor_entry *table;
    const uint8_t *data;
    qwen3_model *qm;
    void (*qm_free)(qwen3_model *);
};

static const uint8_t *map_ro(const char *path, uint64_t *len, int *fd) {
    *fd = open(path, O_RDONLY);
    if (*fd < 0) return NULL;
    struct stat st;
    if (fstat(*fd, &st) != 0 || st.st_size <= 0) return NULL;
    *len = (uint64_t)st.st_size;
    void *p = mmap(NULL, (size_t)*len, PROT_READ, MAP_PRIVATE, *fd, 0);
    return p == MAP_FAILED ? NULL : (const uint8_t *)p;
}

static sp_status reject(sp_model *m, sp_status st, const char *why) {
    sp_set_error(why);
    sp_model_unload(m);
    return st;
}

static sp_status spinor_sample(const sp_model *m) {
    for (uint32_t i = 0; i < m->hdr.tensor_count; i++) {
        const sp_tensor_entry *e = &m->table[i];
        if (e->dtype_id != (uint32_t)SP_DT_SPINOR63) continue;
        const uint8_t *t = (const uint8_t *)sp_model_tensor_data(m, e);
        uint64_t bs = e->block_size, bc = e->block_count;
        if (!t || !bs || !bc || bs * bc > e->size_bytes) {
            sp_set_error("sp_model_load: Spinor tensor has invalid block geometry");
            return SP_EBADFORMAT;
        }
        if (t[bs - 1] != SP_SPINOR_SENTINEL || t[(bc - 1) * bs + bs - 1] != SP_SPINOR_SENTINEL) {
            sp_set_error("sp_model_load: Spinor block sentinel != 0xA5");
            return SP_ESPINOR_BADBLOCK;
        }
    }
    return SP_OK;
}

sp_status sp_model_load(const char *model_path, const char *tok_path, sp_model **out) {
    if (!model_path || !tok_path || !out) { sp_set_error("sp_model_load: null arg"); return SP_EBADARG; }
    *out = NULL;
    sp_model *m = (sp_model *)calloc(1, sizeof *m);
    if (!m) { sp_set_error("sp_model_load: OOM handle"); return SP_ENOMEM; }
    m->fd = m->tfd = -1;

    m->map = map_ro(model_path, &m->map_len, &m->fd);
    if (!m->map) return reject(m, SP_EIO, "sp_model_load: cannot open/mmap .sp-model");
    if (m->map_len < SP_HEADER_SIZE) return reject(m, SP_EBADFORMAT, "sp_model_load: file shorter than header");
    memcpy(&m->hdr, m->map, SP_HEADER_SIZE);
    const sp_model_header *h = &m->hdr;
    if (h->magic != SP_MODEL_MAGIC) return reject(m, SP_EBADFORMAT, "sp_model_load: bad magic (not SPMD)");
    if (h->version_major != SP_MODEL_VER_MAJOR) return reject(m, SP_EBADFORMAT, "sp_model_load: unsupported version_major");
    if (h->header_size != SP_HEADER_SIZE) return reject(m, SP_EBADFORMAT, "sp_model_load: header_size != 512");
    if (sp_crc32(m->map, SP_HEADER_CRC_COVER) != h->header_crc32)
        return reject(m, SP_EBADFORMAT, "sp_model_load: header CRC-32 mismatch");
    if (h->file_size != m->map_len) return reject(m, SP_EBADFORMAT, "sp_model_load: file_size != stat size");
    if (h->arch_struct_capacity != 256u || h->arch_struct_size > 256u)
        return reject(m, SP_EBADFORMAT, "sp_model_load: bad arch_struct sizing");
    if (h->tensor_table_offset != SP_HEADER_SIZE)
        return reject(m, SP_EBADFORMAT, "sp_model_load: tensor_table_offset invalid");
    if (h->tensor_data_offset % SP_DATA_REGION_ALIGN)
        return reject(m, SP_EBADFORMAT, "sp_model_load: tensor_data_offset not 65536-aligned");
    uint64_t tend = h->tensor_table_offset + (uint64_t)h->tensor_count * SP_TENSOR_ENTRY_SIZE;
    if (tend < h->tensor_table_offset || tend > m->map_len ||
        h->tensor_data_offset < tend || h->tensor_data_offset > m->map_len)
        return reject(m, SP_EBADFORMAT, "sp_model_load: table/data offsets out of range");
    m->table = (const sp_tensor_entry *)(m->map + h->tensor_table_offset);
    m->data = m->map + h->tensor_data_offset;

    m->tmap = map_ro(tok_path, &m->tmap_len, &m->tfd);
    if (!m->tmap) return reject(m, SP_EIO, "sp_model_load: cannot open/mmap .sp-tokenizer");
    if (m->tmap_len < SP_TOK_HEADER_SIZE) return reject(m, SP_EBADFORMAT, "sp_model_load: tokenizer shorter than header");
    uint8_t dg[32];
    sp_sha256(m->tmap, (size_t)m->tmap_len, dg);
    if (memcmp(dg, h->tokenizer_hash, 32) != 0)
        return reject(m, SP_ETOKENIZER_HASH, "sp_model_load: tokenizer SHA-256 != header.tokenizer_hash");
    const sp_tok_header *th = (const sp_tok_header *)m->tmap;
    if (th->magic != SP_TOK_MAGIC) return reject(m, SP_EBADFORMAT, "sp_model_load: tokenizer bad magic (not SPTK)");
    if (th->vocab_size != h->vocab_size) return reject(m, SP_EVOCAB, "sp_model_load: tokenizer vocab != model vocab");
    sp_status st = spinor_sample(m);
    if (st != SP_OK) { sp_model_unload(m); return st; }
    *out = m;
    return SP_OK;
}

void sp_model_unload(sp_model *m) {
    if (!m) return;
    if (m->qm && m->qm_free) m->qm_free(m->qm);   /* arena aliases the mapping: free first */
    if (m->map) munmap((void *)m->map, (size_t)m->map_len);
    if (m->tmap) munmap((void *)m->tmap, (size_t)m->tmap_len);
    if (m->fd >= 0) close(m->fd);
    if (m->tfd >= 0) close(m->tfd);
    free(m);
}

const sp_model_header *sp_model_get_header(const sp_model *m) { return m ? &m->hdr : NULL; }
uint32_t sp_model_tensor_count(const sp_model *m) { return m ? m->hdr.tensor_count : 0u; }
const sp_tensor_entry *sp_model_tensor_at(const sp_model *m, uint32_t i) {
    return (m && i < m->hdr.tensor_count) ? &m->table[i] : NULL;
}

const sp_tensor_entry *sp_model_find_tensor(const sp_model *m, const char *name) {
    if (!m || !name) return NULL;
    const uint64_t key = sp_xxh64(name, strlen(name), 0);
    uint32_t lo = 0, hi = m->hdr.tensor_count;
    while (lo < hi) {                      /* first entry with hash >= key */
        uint32_t mid = lo + (hi - lo) / 2u;
        if (m->table[mid].name_hash < key) lo = mid + 1u; else hi = mid;
    }
    for (; lo < m->hdr.tensor_count && m->table[lo].name_hash == key; lo++)
        if (strncmp(m->table[lo].name, name, sizeof m->table[lo].name) == 0) return &m->table[lo];
    return NULL;
}

const void *sp_model_tensor_data(const sp_model *m, const sp_tensor_entry *e) {
    if (!m || !e) return NULL;
    uint64_t region = m->map_len - m->hdr.tensor_data_offset;
    if (e->offset_in_data > region || e->size_bytes > region - e->offset_in_data) return NULL;
    return m->data + e->offset_in_data;
}

const void *sp_model_tokenizer_blob(const sp_model *m, uint64_t *size_out) {
    if (!m || !m->tmap) return NULL;
    const sp_tok_header *th = (const sp_tok_header *)m->tmap;
    if (th->blob_offset > m->tmap_len || th->blob_size > m->tmap_len - th->blob_offset) return NULL;
    if (size_out) *size_out = th->blob_size;
    return m->tmap + th->blob_offset;
}

/* arch query: core/io_format/sp_model_arch.c:22-35 -- copy min(arch_struct_size,
 * sizeof) bytes, zero tail = "unspecified" for appended fields. */
sp_status sp_model_arch(const sp_model *m, sp_arch_info *out) {
    if (!m || !out) { sp_set_error("sp_model_arch: null arg"); return SP_EBADARG; }
    memset(out, 0, sizeof *out);
    size_t n = m->hdr.arch_struct_size;
    if (n > sizeof *out) n = sizeof *out;
    memcpy(out, m->hdr.arch_struct, n);
    return SP_OK;
}

void sp_model_store_qm(sp_model *m, qwen3_model *qm, void (*free_fn)(qwen3_model *)) {
    if (m) { m->qm = qm; m->qm_free = free_fn; }
}
qwen3_model *sp_model_borrow_qm(const sp_model *m) { return m ? m->qm : NULL; }
