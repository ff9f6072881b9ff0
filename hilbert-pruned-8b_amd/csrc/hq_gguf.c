/* hq_gguf.c - GGUF container reader: a read-only mapping of the file, an index of its metadata and
 * tensor records, and hq_wmat_t views of the quantized matrices (include/hq_gguf.h).
 *
 * Container (GGUF v2 / v3, all integers little-endian):
 *   fixed header   "GGUF", u32 version, u64 tensor count, u64 metadata count      (24 bytes)
 *   metadata       count x { string key, u32 value type, value }
 *   tensor records count x { string name, u32 n_dims, n_dims x u64 extent (ne[0] contiguous),
 *                            u32 ggml type, u64 offset into the data section }
 *   data section   starts at the end of the records rounded up to general.alignment (a u32
 *                  metadata value; 32 when absent)
 * A string is a u64 byte count and the bytes. Value types 0..12 are u8, i8, u16, i16, u32, i32,
 * f32, bool, string, array, u64, i64, f64; an array is a u32 element type, a u64 count and the
 * elements.
 *
 * How this reader works: map_file() maps the whole file; index_file() then makes one forward pass
 * over the bytes with a cursor (positions are offsets into the mapping, every read reports a short
 * file through its return value), appending one entry per metadata value and per tensor record to
 * growable arrays. Nested metadata values are passed with an explicit stack instead of recursion.
 * Tensor names are copied, NUL-terminated, into one string pool, and tensors are found by binary
 * search over a name-sorted index (the first record of a name wins, as a linear scan would).
 *
 * Acceptance: the set of files accepted is the runtime's own reader's
 * (cleanroom-transformer/src/gguf.c:134-219; tests/test_gguf.py checks both readers locate the same
 * bytes and that malformed files are refused): version 2 or 3; at most 2^20 entries of each kind;
 * tensor names under 256 bytes; at most 4 dimensions; each extent in 1 .. 2^32 and at most 2^40
 * elements; nesting of metadata arrays at most 4 deep; a nonzero power-of-two alignment, the last
 * u32 general.alignment entry counting. One difference, on corrupt files only: an extent product
 * that overflows 64 bits is refused here. Tensor bytes are checked against the file size when a
 * matrix view is taken (as src/gguf.c:324-344 does), so a file whose header alone is intact can
 * still be indexed.
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

#define GGUF_MAGIC 0x46554747u /* "GGUF" as a little-endian u32 */
#define HEADER_BYTES 24u
#define MAX_RECORDS (1ull << 20)
#define MAX_NAME_BYTES 255u
#define MAX_DIMS 4u
#define MAX_EXTENT (1ull << 32)
#define MAX_ELEMENTS (1ull << 40)
#define MAX_NEST 4
#define DEFAULT_ALIGNMENT 32u

enum { VT_UINT8 = 0, VT_UINT16 = 2, VT_UINT32 = 4, VT_STRING = 8, VT_ARRAY = 9, VT_UINT64 = 10, VT_KINDS = 13 };

/* Byte width of a fixed-size value type (types 0..12 packed one nibble each, type 0 lowest);
 * 0 for strings, arrays and unknown types. */
static unsigned fixed_width(uint32_t vt) {
    const uint64_t widths = 0x8880014442211ull;
    return vt < VT_KINDS ? (unsigned)((widths >> (4 * vt)) & 15u) : 0u;
}

/* ---------------------------------------------------------------- cursor over the mapping */
typedef struct {
    const uint8_t *buf;
    size_t len, pos;
} cursor_t;

static size_t remaining(const cursor_t *c) { return c->len - c->pos; }

static int advance(cursor_t *c, uint64_t n) {
    if (n > remaining(c)) return -1;
    c->pos += (size_t)n;
    return 0;
}

static uint64_t load_le(const uint8_t *p, unsigned n) {
    uint64_t v = 0;
    while (n--) v = v << 8 | p[n];
    return v;
}

static int read_u32(cursor_t *c, uint32_t *v) {
    if (remaining(c) < 4) return -1;
    *v = (uint32_t)load_le(c->buf + c->pos, 4);
    c->pos += 4;
    return 0;
}

static int read_u64(cursor_t *c, uint64_t *v) {
    if (remaining(c) < 8) return -1;
    *v = load_le(c->buf + c->pos, 8);
    c->pos += 8;
    return 0;
}

/* A length-prefixed string: *at = its offset in the mapping, *n = its length. */
static int read_string(cursor_t *c, size_t *at, uint64_t *n) {
    if (read_u64(c, n)) return -1;
    *at = c->pos;
    return advance(c, *n);
}

/* Passes one metadata value of type vt. Frame f of the stack holds the element type of an array
 * whose elements sit at nesting depth f, and how many of them are still to pass; arrays of
 * fixed-size elements are passed in one step. An element deeper than MAX_NEST is refused, as is an
 * unknown type. */
static int pass_value(cursor_t *c, uint32_t vt) {
    struct {
        uint32_t vt;
        uint64_t left;
    } frame[MAX_NEST + 2];
    int top = 0;
    frame[0].vt = vt;
    frame[0].left = 1;
    for (;;) {
        while (frame[top].left == 0)
            if (top-- == 0) return 0;
        frame[top].left--;
        if (top > MAX_NEST) return -1;
        const uint32_t t = frame[top].vt;
        if (fixed_width(t)) {
            if (advance(c, fixed_width(t))) return -1;
        } else if (t == VT_STRING) {
            size_t at;
            uint64_t n;
            if (read_string(c, &at, &n)) return -1;
        } else if (t == VT_ARRAY) {
            uint32_t et;
            uint64_t n;
            if (read_u32(c, &et) || read_u64(c, &n)) return -1;
            const unsigned w = fixed_width(et);
            if (w) {
                if (n > remaining(c) / w) return -1;
                c->pos += (size_t)(n * w);
            } else {
                top++;
                frame[top].vt = et;
                frame[top].left = n;
            }
        } else {
            return -1;
        }
    }
}

/* ---------------------------------------------------------------- the index */
typedef struct {
    size_t key_at; /* offset of the key bytes in the mapping */
    uint64_t key_len;
    uint32_t vt;
    size_t value_at; /* offset of the value (after the type tag) */
} meta_rec;

typedef struct {
    size_t name_at;    /* offset of the name: in the mapping while indexing, then in the string pool */
    uint64_t name_len;
    uint32_t n_dims;
    uint64_t ne[4];
    int type;
    uint64_t data_rel; /* from the start of the data section */
} tensor_rec;

struct hq_gguf {
    const uint8_t *map;
    size_t size, data_start;
    meta_rec *meta;
    size_t n_meta;
    tensor_rec *tensor;
    size_t n_tensor;
    char *pool;          /* tensor names, NUL-terminated */
    struct name_key {
        const char *name; /* into the pool */
        uint32_t index;
    } *sorted;           /* one per tensor, ordered by (name, index) */
};

/* Appends one zeroed element to a growable array of `*n` elements of `size` bytes with room for
 * `*cap`; returns it, or NULL when out of memory. */
static void *append(void **arr, size_t *n, size_t *cap, size_t size) {
    if (*n == *cap) {
        const size_t grown = *cap ? 2 * *cap : 16;
        void *p = realloc(*arr, grown * size);
        if (!p) return NULL;
        *arr = p;
        *cap = grown;
    }
    void *e = (char *)*arr + (*n)++ * size;
    memset(e, 0, size);
    return e;
}

/* Extents of one tensor record: each in 1 .. MAX_EXTENT, their product at most MAX_ELEMENTS
 * (computed with an overflow check). Unused dimensions are 1. */
static int read_extents(cursor_t *c, tensor_rec *t) {
    uint64_t elements = 1;
    for (uint32_t d = 0; d < MAX_DIMS; d++) t->ne[d] = 1;
    for (uint32_t d = 0; d < t->n_dims; d++) {
        if (read_u64(c, &t->ne[d]) || t->ne[d] < 1 || t->ne[d] > MAX_EXTENT) return -1;
        if (__builtin_mul_overflow(elements, t->ne[d], &elements) || elements > MAX_ELEMENTS) return -1;
    }
    return 0;
}

static int by_name_then_index(const void *a, const void *b) {
    const struct name_key *x = (const struct name_key *)a, *y = (const struct name_key *)b;
    const int s = strcmp(x->name, y->name);
    return s ? s : (x->index > y->index) - (x->index < y->index);
}

/* One pass over the mapping: header, metadata, tensor records; then the data start, the name pool
 * and the sorted index. Returns 0, or -1 for a malformed or truncated file (nothing recorded). */
static int index_file(hq_gguf *g, const char *path) {
    cursor_t c = {g->map, g->size, 0};
    uint32_t magic, version;
    uint64_t n_tensor, n_meta;
    if (read_u32(&c, &magic) || read_u32(&c, &version) || read_u64(&c, &n_tensor) || read_u64(&c, &n_meta))
        return hq_internal_fail("hq_gguf_open: %s: truncated or malformed GGUF header", path);
    if (magic != GGUF_MAGIC) return hq_internal_fail("hq_gguf_open: %s: not a GGUF file", path);
    if (version != 2 && version != 3)
        return hq_internal_fail("hq_gguf_open: %s: GGUF version %u (2 or 3 supported)", path, version);
    if (n_tensor > MAX_RECORDS || n_meta > MAX_RECORDS)
        return hq_internal_fail("hq_gguf_open: %s: implausible header (%llu tensors, %llu metadata entries)", path,
                                (unsigned long long)n_tensor, (unsigned long long)n_meta);
    size_t cap_meta = 0, cap_tensor = 0, pool_bytes = 0;
    uint32_t alignment = DEFAULT_ALIGNMENT;
    int ok = 1;
    for (uint64_t i = 0; ok && i < n_meta; i++) {
        meta_rec *m = (meta_rec *)append((void **)&g->meta, &g->n_meta, &cap_meta, sizeof *m);
        if (!m) return hq_internal_fail("hq_gguf_open: out of memory");
        ok = !read_string(&c, &m->key_at, &m->key_len) && !read_u32(&c, &m->vt);
        m->value_at = c.pos;
        ok = ok && !pass_value(&c, m->vt);
        if (ok && m->vt == VT_UINT32 && m->key_len == 17 && !memcmp(g->map + m->key_at, "general.alignment", 17))
            alignment = (uint32_t)load_le(g->map + m->value_at, 4);
    }
    for (uint64_t i = 0; ok && i < n_tensor; i++) {
        tensor_rec *t = (tensor_rec *)append((void **)&g->tensor, &g->n_tensor, &cap_tensor, sizeof *t);
        uint32_t type = 0;
        if (!t) return hq_internal_fail("hq_gguf_open: out of memory");
        ok = !read_string(&c, &t->name_at, &t->name_len) && t->name_len <= MAX_NAME_BYTES &&
             !read_u32(&c, &t->n_dims) && t->n_dims <= MAX_DIMS && !read_extents(&c, t) && !read_u32(&c, &type) &&
             !read_u64(&c, &t->data_rel);
        t->type = (int)type;
        pool_bytes += ok ? (size_t)t->name_len + 1 : 0;
    }
    if (!ok || alignment == 0 || (alignment & (alignment - 1)))
        return hq_internal_fail("hq_gguf_open: %s: truncated or malformed GGUF header", path);
    g->data_start = (c.pos + alignment - 1) / alignment * alignment;

    g->pool = (char *)malloc(pool_bytes ? pool_bytes : 1);
    g->sorted = (struct name_key *)malloc((g->n_tensor ? g->n_tensor : 1) * sizeof *g->sorted);
    if (!g->pool || !g->sorted) return hq_internal_fail("hq_gguf_open: out of memory");
    size_t at = 0;
    for (size_t i = 0; i < g->n_tensor; i++) {
        tensor_rec *t = &g->tensor[i];
        memcpy(g->pool + at, g->map + t->name_at, (size_t)t->name_len);
        g->pool[at + t->name_len] = '\0';
        t->name_at = at;
        g->sorted[i] = (struct name_key){g->pool + at, (uint32_t)i};
        at += (size_t)t->name_len + 1;
    }
    qsort(g->sorted, g->n_tensor, sizeof *g->sorted, by_name_then_index);
    return 0;
}

/* Maps `path` read-only; files shorter than the fixed header are refused. */
static int map_file(const char *path, const uint8_t **map, size_t *size) {
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return hq_internal_fail("hq_gguf_open: cannot open %s", path);
    struct stat st;
    const int regular = !fstat(fd, &st) && S_ISREG(st.st_mode);
    if (!regular || st.st_size < (off_t)HEADER_BYTES) {
        close(fd);
        return hq_internal_fail("hq_gguf_open: %s is not a GGUF file", path);
    }
    void *p = mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd); /* the mapping keeps the file */
    if (p == MAP_FAILED) return hq_internal_fail("hq_gguf_open: cannot map %s", path);
    *map = (const uint8_t *)p;
    *size = (size_t)st.st_size;
    return 0;
}

void hq_gguf_close(hq_gguf *g) {
    if (!g) return;
    if (g->map) munmap((void *)g->map, g->size);
    free(g->meta);
    free(g->tensor);
    free(g->pool);
    free(g->sorted);
    free(g);
}

int hq_gguf_open(const char *path, hq_gguf **out) {
    if (!out) return hq_internal_fail("hq_gguf_open: null argument");
    *out = NULL;
    if (!path) return hq_internal_fail("hq_gguf_open: no path");
    hq_gguf *g = (hq_gguf *)calloc(1, sizeof *g);
    if (!g) return hq_internal_fail("hq_gguf_open: out of memory");
    if (map_file(path, &g->map, &g->size) || index_file(g, path)) {
        hq_gguf_close(g);
        return -1;
    }
    *out = g;
    return 0;
}

/* ---------------------------------------------------------------- queries */
size_t hq_gguf_n_tensors(const hq_gguf *g) { return g ? g->n_tensor : 0; }

int hq_gguf_tensor_info(const hq_gguf *g, size_t i, const char **name, int *ggml_type, uint32_t *n_dims, uint64_t ne[4],
                        uint64_t *file_offset) {
    if (!g || i >= g->n_tensor) return hq_internal_fail("hq_gguf_tensor_info: no tensor %zu", i);
    const tensor_rec *t = &g->tensor[i];
    if (name) *name = g->pool + t->name_at;
    if (ggml_type) *ggml_type = t->type;
    if (n_dims) *n_dims = t->n_dims;
    if (ne) memcpy(ne, t->ne, sizeof t->ne);
    if (file_offset) *file_offset = (uint64_t)g->data_start + t->data_rel;
    return 0;
}

int hq_gguf_find(const hq_gguf *g, const char *name, size_t *index) {
    if (!g || !name) return hq_internal_fail("hq_gguf_find: null argument");
    size_t lo = 0, hi = g->n_tensor; /* first sorted position whose name is >= `name` */
    while (lo < hi) {
        const size_t mid = lo + (hi - lo) / 2;
        if (strcmp(g->sorted[mid].name, name) < 0) lo = mid + 1;
        else hi = mid;
    }
    if (lo == g->n_tensor || strcmp(g->sorted[lo].name, name)) return hq_internal_fail("hq_gguf_find: no tensor %s", name);
    if (index) *index = g->sorted[lo].index;
    return 0;
}

int hq_gguf_get_uint(const hq_gguf *g, const char *key, uint64_t *out) {
    if (!g || !key || !out) return hq_internal_fail("hq_gguf_get_uint: null argument");
    const size_t n = strlen(key);
    const meta_rec *m = g->meta, *end = g->meta + g->n_meta;
    while (m < end && (m->key_len != n || memcmp(g->map + m->key_at, key, n))) m++;
    const int is_uint = m < end && (m->vt == VT_UINT8 || m->vt == VT_UINT16 || m->vt == VT_UINT32 || m->vt == VT_UINT64);
    if (!is_uint) return hq_internal_fail("hq_gguf_get_uint: no unsigned value %s", key);
    *out = load_le(g->map + m->value_at, fixed_width(m->vt)); /* whole: the indexing pass checked it */
    return 0;
}

int hq_gguf_wmat(const hq_gguf *g, const char *name, uint32_t perm_heads, hq_wmat_t *out) {
    size_t i;
    if (!out) return hq_internal_fail("hq_gguf_wmat: null argument");
    if (hq_gguf_find(g, name, &i)) return -1;
    const tensor_rec *t = &g->tensor[i];
    uint32_t per, bytes;
    if (hq_internal_block_shape(t->type, &per, &bytes))
        return hq_internal_fail("hq_gguf_wmat: tensor %s has ggml type %d (supported: %s)", name, t->type,
                                hq_internal_supported_types());
    const uint64_t cols = t->ne[0], rows = t->ne[1] * t->ne[2] * t->ne[3];
    if (cols % per)
        return hq_internal_fail("hq_gguf_wmat: tensor %s row length %llu is not whole blocks", name,
                                (unsigned long long)cols);
    if (cols > UINT32_MAX || rows > UINT32_MAX) return hq_internal_fail("hq_gguf_wmat: tensor %s too large", name);
    /* rows * cols <= 2^40 elements, so the byte count cannot overflow */
    const uint64_t first = (uint64_t)g->data_start + t->data_rel, span = cols / per * bytes * rows;
    const int inside = t->data_rel <= g->size && first <= g->size && span <= g->size - first;
    if (!inside) return hq_internal_fail("hq_gguf_wmat: tensor %s lies outside the file (truncated?)", name);
    *out = (hq_wmat_t){HQ_DT_GGML, (uint32_t)rows, (uint32_t)cols, g->map + first, t->type, perm_heads};
    return 0;
}
