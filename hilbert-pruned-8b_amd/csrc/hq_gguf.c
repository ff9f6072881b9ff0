/* hq_gguf.c - read-only GGUF mapping and tensor table (include/hq_gguf.h).
 *
 * The container format (GGUF v2/v3, little-endian): "GGUF", u32 version, u64 tensor count, u64
 * metadata count; each metadata entry is a u64-length key, a u32 value type and the value (scalars
 * of 1/2/4/8 bytes, strings as u64 length + bytes, arrays as u32 element type + u64 count +
 * elements); each tensor entry is a u64-length name, u32 n_dims, n_dims u64 extents (ne[0]
 * contiguous), u32 ggml type and a u64 offset into the data section, which starts at the end of
 * the header rounded up to general.alignment (32 when absent). This follows the same file format
 * as the reference reader (cleanroom-transformer/src/gguf.c:134-219), with its limits: version 2
 * or 3, at most 2^20 entries of each kind, names under 256 bytes, at most 4 dimensions, each
 * extent in 1 .. 2^32 and at most 2^40 elements, a power-of-two alignment, nested arrays at most 4
 * deep. Tensor data is checked against the file size when a matrix view is taken (:324-344).
 */
#define _POSIX_C_SOURCE 200809L
#include "hq_gguf.h"

#include <fcntl.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "hq_internal.h"

enum { T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 };

typedef struct {
    const unsigned char *key;
    uint64_t key_len;
    uint32_t type;
    const unsigned char *val;
} kv_t;

typedef struct {
    char name[256];
    uint32_t n_dims;
    uint64_t ne[4];
    int type;
    uint64_t offset; /* from the start of the data section */
} tinfo_t;

struct hq_gguf {
    unsigned char *map;
    size_t size, data_off;
    kv_t *kv;
    size_t n_kv;
    tinfo_t *t;
    size_t n_t;
};

typedef struct {
    const unsigned char *p, *end;
    int bad;
} rd_t;

static uint64_t take(rd_t *r, size_t n) {
    if (r->bad || (size_t)(r->end - r->p) < n) {
        r->bad = 1;
        return 0;
    }
    uint64_t v = 0;
    for (size_t i = 0; i < n; i++) v |= (uint64_t)r->p[i] << (8 * i);
    r->p += n;
    return v;
}

static size_t scalar_bytes(uint32_t t) {
    switch (t) {
    case T_U8: case T_I8: case T_BOOL: return 1;
    case T_U16: case T_I16: return 2;
    case T_U32: case T_I32: case T_F32: return 4;
    case T_U64: case T_I64: case T_F64: return 8;
    default: return 0;
    }
}

static void skip(rd_t *r, uint32_t t, int depth) {
    if (depth > 4) {
        r->bad = 1;
        return;
    }
    if (t == T_STR) {
        const uint64_t n = take(r, 8);
        if (r->bad || n > (uint64_t)(r->end - r->p)) r->bad = 1;
        else r->p += n;
        return;
    }
    if (t == T_ARR) {
        const uint32_t et = (uint32_t)take(r, 4);
        const uint64_t n = take(r, 8);
        const size_t es = scalar_bytes(et);
        if (r->bad) return;
        if (es) {
            if (n > (uint64_t)(r->end - r->p) / es) r->bad = 1;
            else r->p += n * es;
        } else {
            for (uint64_t i = 0; i < n && !r->bad; i++) skip(r, et, depth + 1);
        }
        return;
    }
    const size_t es = scalar_bytes(t);
    if (!es) r->bad = 1;
    else take(r, es);
}

void hq_gguf_close(hq_gguf *g) {
    if (!g) return;
    if (g->map) munmap(g->map, g->size);
    free(g->kv);
    free(g->t);
    free(g);
}

int hq_gguf_open(const char *path, hq_gguf **out) {
    *out = NULL;
    if (!path) return hq_internal_fail("hq_gguf_open: no path");
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return hq_internal_fail("hq_gguf_open: cannot open %s", path);
    struct stat sb;
    if (fstat(fd, &sb) || !S_ISREG(sb.st_mode) || sb.st_size < 24) {
        close(fd);
        return hq_internal_fail("hq_gguf_open: %s is not a GGUF file", path);
    }
    void *map = mmap(NULL, (size_t)sb.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) return hq_internal_fail("hq_gguf_open: cannot map %s", path);
    hq_gguf *g = (hq_gguf *)calloc(1, sizeof *g);
    if (!g) {
        munmap(map, (size_t)sb.st_size);
        return hq_internal_fail("hq_gguf_open: out of memory");
    }
    g->map = (unsigned char *)map;
    g->size = (size_t)sb.st_size;
    rd_t r = {g->map, g->map + g->size, 0};
    const uint32_t magic = (uint32_t)take(&r, 4), version = (uint32_t)take(&r, 4);
    const uint64_t nt = take(&r, 8), nkv = take(&r, 8);
    if (magic != 0x46554747u) {
        hq_gguf_close(g);
        return hq_internal_fail("hq_gguf_open: %s: not a GGUF file", path);
    }
    if (version < 2 || version > 3) {
        hq_gguf_close(g);
        return hq_internal_fail("hq_gguf_open: %s: GGUF version %u (2 or 3 supported)", path, version);
    }
    if (nkv > (1u << 20) || nt > (1u << 20)) {
        hq_gguf_close(g);
        return hq_internal_fail("hq_gguf_open: %s: implausible header (%llu tensors, %llu metadata entries)", path,
                                (unsigned long long)nt, (unsigned long long)nkv);
    }
    g->kv = (kv_t *)calloc(nkv ? nkv : 1, sizeof *g->kv);
    g->t = (tinfo_t *)calloc(nt ? nt : 1, sizeof *g->t);
    if (!g->kv || !g->t) {
        hq_gguf_close(g);
        return hq_internal_fail("hq_gguf_open: out of memory");
    }
    uint64_t alignment = 32;
    for (uint64_t i = 0; i < nkv && !r.bad; i++) {
        const uint64_t kl = take(&r, 8);
        if (r.bad || kl > (uint64_t)(r.end - r.p)) {
            r.bad = 1;
            break;
        }
        kv_t *e = &g->kv[g->n_kv++];
        e->key = r.p;
        e->key_len = kl;
        r.p += kl;
        e->type = (uint32_t)take(&r, 4);
        e->val = r.p;
        skip(&r, e->type, 0);
        if (!r.bad && kl == 17 && !memcmp(e->key, "general.alignment", 17) && e->type == T_U32) {
            rd_t v = {e->val, r.end, 0};
            alignment = take(&v, 4);
        }
    }
    for (uint64_t i = 0; i < nt && !r.bad; i++) {
        tinfo_t *t = &g->t[g->n_t];
        const uint64_t nl = take(&r, 8);
        if (r.bad || nl > (uint64_t)(r.end - r.p) || nl >= sizeof t->name) {
            r.bad = 1;
            break;
        }
        memcpy(t->name, r.p, (size_t)nl);
        t->name[nl] = 0;
        r.p += nl;
        t->n_dims = (uint32_t)take(&r, 4);
        if (t->n_dims > 4) {
            r.bad = 1;
            break;
        }
        uint64_t count = 1;
        for (uint32_t d = 0; d < t->n_dims; d++) {
            t->ne[d] = take(&r, 8);
            if (t->ne[d] == 0 || t->ne[d] > (1ull << 32) || (count *= t->ne[d]) > (1ull << 40)) r.bad = 1;
        }
        for (uint32_t d = t->n_dims; d < 4; d++) t->ne[d] = 1;
        t->type = (int)take(&r, 4);
        t->offset = take(&r, 8);
        g->n_t++;
    }
    if (r.bad || alignment == 0 || (alignment & (alignment - 1)) || alignment > (1u << 20)) {
        hq_gguf_close(g);
        return hq_internal_fail("hq_gguf_open: %s: truncated or malformed GGUF header", path);
    }
    const size_t end = (size_t)(r.p - g->map);
    g->data_off = (end + (size_t)alignment - 1) / (size_t)alignment * (size_t)alignment;
    *out = g;
    return 0;
}

size_t hq_gguf_n_tensors(const hq_gguf *g) { return g ? g->n_t : 0; }

int hq_gguf_tensor_info(const hq_gguf *g, size_t i, const char **name, int *ggml_type, uint32_t *n_dims, uint64_t ne[4],
                        uint64_t *file_offset) {
    if (!g || i >= g->n_t) return hq_internal_fail("hq_gguf_tensor_info: no tensor %zu", i);
    const tinfo_t *t = &g->t[i];
    if (name) *name = t->name;
    if (ggml_type) *ggml_type = t->type;
    if (n_dims) *n_dims = t->n_dims;
    if (ne) memcpy(ne, t->ne, sizeof t->ne);
    if (file_offset) *file_offset = (uint64_t)g->data_off + t->offset;
    return 0;
}

int hq_gguf_find(const hq_gguf *g, const char *name, size_t *index) {
    if (!g || !name) return hq_internal_fail("hq_gguf_find: null argument");
    for (size_t i = 0; i < g->n_t; i++)
        if (!strcmp(g->t[i].name, name)) {
            if (index) *index = i;
            return 0;
        }
    return hq_internal_fail("hq_gguf_find: no tensor %s", name);
}

int hq_gguf_get_uint(const hq_gguf *g, const char *key, uint64_t *out) {
    if (!g || !key || !out) return hq_internal_fail("hq_gguf_get_uint: null argument");
    const size_t n = strlen(key);
    for (size_t i = 0; i < g->n_kv; i++) {
        const kv_t *e = &g->kv[i];
        if (e->key_len != n || memcmp(e->key, key, n)) continue;
        if (e->type != T_U8 && e->type != T_U16 && e->type != T_U32 && e->type != T_U64) break;
        rd_t v = {e->val, g->map + g->size, 0};
        *out = take(&v, scalar_bytes(e->type));
        return v.bad ? hq_internal_fail("hq_gguf_get_uint: %s truncated", key) : 0;
    }
    return hq_internal_fail("hq_gguf_get_uint: no unsigned value %s", key);
}

int hq_gguf_wmat(const hq_gguf *g, const char *name, uint32_t perm_heads, hq_wmat_t *out) {
    size_t i;
    if (!out) return hq_internal_fail("hq_gguf_wmat: null argument");
    if (hq_gguf_find(g, name, &i)) return -1;
    const tinfo_t *t = &g->t[i];
    const uint64_t per = t->type == HQ_GGML_Q8_0 ? 32 : t->type == HQ_GGML_Q4_K || t->type == HQ_GGML_Q6_K ? 256 : 0;
    const uint64_t bb = t->type == HQ_GGML_Q8_0 ? 34 : t->type == HQ_GGML_Q4_K ? 144 : 210;
    if (!per) return hq_internal_fail("hq_gguf_wmat: tensor %s has ggml type %d (Q8_0, Q4_K or Q6_K supported)", name, t->type);
    if (t->ne[0] % per) return hq_internal_fail("hq_gguf_wmat: tensor %s row length %llu is not whole blocks", name,
                                                (unsigned long long)t->ne[0]);
    const uint64_t rows = t->ne[1] * t->ne[2] * t->ne[3], bytes = t->ne[0] / per * bb * rows;
    if (t->ne[0] > UINT32_MAX || rows > UINT32_MAX) return hq_internal_fail("hq_gguf_wmat: tensor %s too large", name);
    const uint64_t start = (uint64_t)g->data_off + t->offset;
    if (start > g->size || bytes > g->size - start)
        return hq_internal_fail("hq_gguf_wmat: tensor %s lies outside the file (truncated?)", name);
    out->dtype = HQ_DT_GGML;
    out->rows = (uint32_t)rows;
    out->cols = (uint32_t)t->ne[0];
    out->data = g->map + start;
    out->ggml_type = t->type;
    out->perm_heads = perm_heads;
    return 0;
}
