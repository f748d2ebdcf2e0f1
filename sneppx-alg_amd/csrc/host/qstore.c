/*
 * qstore.c - quantized weights on disk (include/sneppx_qstore.h).
 *
 * A safetensors file is: u64 little-endian header length H, H bytes of JSON
 * ({name: {dtype, shape, data_offsets}, ..., "__metadata__": {k: v}}), then
 * the data block; offsets are relative to the data block.  The reader maps
 * the file, parses the header with a small strict JSON scanner (objects,
 * arrays, strings with escapes, non-negative integers) and checks every
 * tensor against the file size before handing out a pointer.
 */
#define _GNU_SOURCE
#include <errno.h>
#include <fcntl.h>
#include <limits.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "sneppx_qstore.h"
#include "snx_hip.h"
#include "../snx_internal.h"

#define FAIL(...)                       \
    do {                                \
        snx_set_error(__VA_ARGS__);     \
        goto fail;                      \
    } while (0)

static const char* const k_dtype_names[] = {"F32", "F16", "F64", "I64", "I32", "I16",
                                            "I8",  "U8",  "BOOL", "BF16", "F8_E5M2",
                                            "F8_E4M3FN"};
static const size_t k_dtype_size[] = {4, 2, 8, 8, 4, 2, 1, 1, 1, 2, 1, 1};
#define N_DTYPES ((int)(sizeof k_dtype_size / sizeof k_dtype_size[0]))

static int dtype_code(const char* s) {
    for (int i = 0; i < N_DTYPES; i++)
        if (strcmp(s, k_dtype_names[i]) == 0) return i;
    return -1;
}

typedef struct {
    char* name;
    int dtype;   /* -1: a dtype string this library does not know */
    size_t ndim;
    size_t shape[SNEPPX_QST_MAX_DIMS];
    size_t begin, end;
} Entry;

typedef struct {
    char* key;
    char* value;
} Meta;

struct SNEPPXQStore {
    unsigned char* map;
    size_t map_len;
    const unsigned char* data;   /* start of the data block */
    size_t data_len;
    Entry* ent;
    size_t n_ent;
    Meta* meta;
    size_t n_meta;
};

/* ------------------------------------------------------------ JSON scanner */

typedef struct {
    const char* p;
    const char* end;
} Scan;

static void ws(Scan* s) {
    while (s->p < s->end && (*s->p == ' ' || *s->p == '\t' || *s->p == '\n' || *s->p == '\r'))
        s->p++;
}

static int expect(Scan* s, char c) {
    ws(s);
    if (s->p >= s->end || *s->p != c) return -1;
    s->p++;
    return 0;
}

static int peek(Scan* s, char c) {
    ws(s);
    return s->p < s->end && *s->p == c;
}

static void put_utf8(char* out, size_t* n, unsigned cp) {
    if (cp < 0x80) {
        out[(*n)++] = (char)cp;
    } else if (cp < 0x800) {
        out[(*n)++] = (char)(0xC0 | (cp >> 6));
        out[(*n)++] = (char)(0x80 | (cp & 0x3F));
    } else {
        out[(*n)++] = (char)(0xE0 | (cp >> 12));
        out[(*n)++] = (char)(0x80 | ((cp >> 6) & 0x3F));
        out[(*n)++] = (char)(0x80 | (cp & 0x3F));
    }
}

/* JSON string -> malloc'd UTF-8 (surrogate pairs are kept as two 3-byte
 * sequences; tensor names are ASCII in practice). */
static char* string(Scan* s) {
    ws(s);
    if (s->p >= s->end || *s->p != '"') return NULL;
    s->p++;
    const char* q = s->p;
    while (q < s->end && *q != '"') q += (*q == '\\') ? 2 : 1;
    if (q >= s->end) return NULL;
    char* out = (char*)malloc((size_t)(q - s->p) * 3 + 1);
    if (!out) return NULL;
    size_t n = 0;
    while (s->p < q) {
        char c = *s->p++;
        if (c != '\\') {
            out[n++] = c;
            continue;
        }
        c = *s->p++;
        switch (c) {
            case '"': case '\\': case '/': out[n++] = c; break;
            case 'b': out[n++] = '\b'; break;
            case 'f': out[n++] = '\f'; break;
            case 'n': out[n++] = '\n'; break;
            case 'r': out[n++] = '\r'; break;
            case 't': out[n++] = '\t'; break;
            case 'u': {
                unsigned cp = 0;
                for (int i = 0; i < 4; i++) {
                    char h = s->p < q ? *s->p++ : 'x';
                    int v = (h >= '0' && h <= '9') ? h - '0'
                            : (h >= 'a' && h <= 'f') ? h - 'a' + 10
                            : (h >= 'A' && h <= 'F') ? h - 'A' + 10 : -1;
                    if (v < 0) { free(out); return NULL; }
                    cp = cp * 16 + (unsigned)v;
                }
                put_utf8(out, &n, cp);
                break;
            }
            default: free(out); return NULL;
        }
    }
    s->p = q + 1;
    out[n] = 0;
    return out;
}

static int integer(Scan* s, size_t* v) {
    ws(s);
    if (s->p >= s->end || *s->p < '0' || *s->p > '9') return -1;
    size_t x = 0;
    while (s->p < s->end && *s->p >= '0' && *s->p <= '9') {
        size_t d = (size_t)(*s->p++ - '0');
        if (x > (SIZE_MAX - d) / 10) return -1;
        x = x * 10 + d;
    }
    *v = x;
    return 0;
}

/* skip any JSON value (unknown fields) */
static int skip_value(Scan* s) {
    ws(s);
    if (s->p >= s->end) return -1;
    char c = *s->p;
    if (c == '"') {
        char* t = string(s);
        if (!t) return -1;
        free(t);
        return 0;
    }
    if (c == '{' || c == '[') {
        char close = c == '{' ? '}' : ']';
        s->p++;
        if (peek(s, close)) { s->p++; return 0; }
        for (;;) {
            if (c == '{') {
                char* k = string(s);
                if (!k) return -1;
                free(k);
                if (expect(s, ':')) return -1;
            }
            if (skip_value(s)) return -1;
            if (peek(s, ',')) { s->p++; continue; }
            return expect(s, close);
        }
    }
    /* number, true, false, null */
    const char* st = s->p;
    while (s->p < s->end && *s->p != ',' && *s->p != '}' && *s->p != ']' && *s->p != ' ' &&
           *s->p != '\n' && *s->p != '\r' && *s->p != '\t')
        s->p++;
    return s->p > st ? 0 : -1;
}

static int int_array(Scan* s, size_t* out, size_t max_n, size_t* n) {
    if (expect(s, '[')) return -1;
    *n = 0;
    if (peek(s, ']')) { s->p++; return 0; }
    for (;;) {
        size_t v;
        if (integer(s, &v) || *n >= max_n) return -1;
        out[(*n)++] = v;
        if (peek(s, ',')) { s->p++; continue; }
        return expect(s, ']');
    }
}

static int parse_entry(Scan* s, Entry* e) {
    int have_dtype = 0, have_shape = 0, have_off = 0;
    if (expect(s, '{')) return -1;
    if (peek(s, '}')) { s->p++; return -1; }
    for (;;) {
        char* k = string(s);
        if (!k || expect(s, ':')) { free(k); return -1; }
        int rc = 0;
        if (strcmp(k, "dtype") == 0) {
            char* d = string(s);
            if (!d) rc = -1;
            else { e->dtype = dtype_code(d); free(d); have_dtype = 1; }
        } else if (strcmp(k, "shape") == 0) {
            rc = int_array(s, e->shape, SNEPPX_QST_MAX_DIMS, &e->ndim);
            have_shape = 1;
        } else if (strcmp(k, "data_offsets") == 0) {
            size_t off[2], n = 0;
            rc = int_array(s, off, 2, &n);
            if (!rc && n == 2) { e->begin = off[0]; e->end = off[1]; have_off = 1; }
            else rc = -1;
        } else {
            rc = skip_value(s);
        }
        free(k);
        if (rc) return -1;
        if (peek(s, ',')) { s->p++; continue; }
        if (expect(s, '}')) return -1;
        return (have_dtype && have_shape && have_off) ? 0 : -1;
    }
}

static int parse_meta(Scan* s, SNEPPXQStore* st) {
    if (expect(s, '{')) return -1;
    if (peek(s, '}')) { s->p++; return 0; }
    for (;;) {
        char* k = string(s);
        if (!k || expect(s, ':')) { free(k); return -1; }
        if (peek(s, '"')) {
            char* v = string(s);
            if (!v) { free(k); return -1; }
            Meta* nm = (Meta*)realloc(st->meta, (st->n_meta + 1) * sizeof(Meta));
            if (!nm) { free(k); free(v); return -1; }
            st->meta = nm;
            st->meta[st->n_meta].key = k;
            st->meta[st->n_meta].value = v;
            st->n_meta++;
        } else {
            free(k);
            if (skip_value(s)) return -1;
        }
        if (peek(s, ',')) { s->p++; continue; }
        return expect(s, '}');
    }
}

/* ------------------------------------------------------------------ reader */

void SNEPPX_qstore_close(SNEPPXQStore* st) {
    if (!st) return;
    for (size_t i = 0; i < st->n_ent; i++) free(st->ent[i].name);
    for (size_t i = 0; i < st->n_meta; i++) {
        free(st->meta[i].key);
        free(st->meta[i].value);
    }
    free(st->ent);
    free(st->meta);
    if (st->map) munmap(st->map, st->map_len);
    free(st);
}

SNEPPXQStore* SNEPPX_qstore_open(const char* path) {
    SNEPPXQStore* st = NULL;
    int fd = -1;
    if (!path) { snx_set_error("qstore_open: NULL path"); return NULL; }
    snx_clear_error();
    st = (SNEPPXQStore*)calloc(1, sizeof *st);
    if (!st) FAIL("qstore_open: out of host memory");
    fd = open(path, O_RDONLY);
    if (fd < 0) FAIL("qstore_open: cannot open %s (%s)", path, strerror(errno));
    struct stat sb;
    if (fstat(fd, &sb) || sb.st_size < 8) FAIL("qstore_open: %s is not a safetensors file", path);
    st->map_len = (size_t)sb.st_size;
    st->map = (unsigned char*)mmap(NULL, st->map_len, PROT_READ, MAP_PRIVATE, fd, 0);
    if (st->map == MAP_FAILED) { st->map = NULL; FAIL("qstore_open: mmap failed (%s)", strerror(errno)); }
    close(fd);
    fd = -1;

    uint64_t hl = 0;
    for (int i = 7; i >= 0; i--) hl = (hl << 8) | st->map[i];
    if (hl > st->map_len - 8) FAIL("qstore_open: header length %llu exceeds the file",
                                   (unsigned long long)hl);
    Scan s = {(const char*)st->map + 8, (const char*)st->map + 8 + hl};
    if (expect(&s, '{')) FAIL("qstore_open: header is not a JSON object");
    if (!peek(&s, '}')) {
        for (;;) {
            char* key = string(&s);
            if (!key || expect(&s, ':')) { free(key); FAIL("qstore_open: malformed header"); }
            if (strcmp(key, "__metadata__") == 0) {
                free(key);
                if (parse_meta(&s, st)) FAIL("qstore_open: malformed __metadata__");
            } else {
                Entry e;
                memset(&e, 0, sizeof e);
                e.name = key;
                if (parse_entry(&s, &e)) { free(key); FAIL("qstore_open: malformed entry"); }
                Entry* ne = (Entry*)realloc(st->ent, (st->n_ent + 1) * sizeof(Entry));
                if (!ne) { free(key); FAIL("qstore_open: out of host memory"); }
                st->ent = ne;
                st->ent[st->n_ent++] = e;
            }
            if (peek(&s, ',')) { s.p++; continue; }
            if (expect(&s, '}')) FAIL("qstore_open: malformed header");
            break;
        }
    } else {
        s.p++;
    }
    ws(&s);   /* the header may end in spaces (its padding), nothing else */
    if (s.p != s.end) FAIL("qstore_open: bytes after the header object");

    /* data block: 8 + hl, or after the reference writer's zero padding when
     * the recorded length leaves exactly that padding unaccounted for */
    size_t need = 0;
    for (size_t i = 0; i < st->n_ent; i++) {
        Entry* e = &st->ent[i];
        if (e->end < e->begin) FAIL("qstore_open: %s has data_offsets [%zu, %zu]", e->name, e->begin, e->end);
        if (e->end > need) need = e->end;
        if (e->dtype >= 0) {
            size_t cnt = 1;
            for (size_t d = 0; d < e->ndim; d++) {
                if (e->shape[d] && cnt > SIZE_MAX / e->shape[d]) FAIL("qstore_open: %s shape overflows", e->name);
                cnt *= e->shape[d];
            }
            if (cnt > SIZE_MAX / k_dtype_size[e->dtype]) FAIL("qstore_open: %s byte size overflows", e->name);
            if (cnt * k_dtype_size[e->dtype] != e->end - e->begin)
                FAIL("qstore_open: %s holds %zu bytes, its dtype and shape need %zu", e->name,
                     e->end - e->begin, cnt * k_dtype_size[e->dtype]);
        }
    }
    size_t base = 8 + (size_t)hl;
    size_t rest = st->map_len - base;
    size_t pad = (8 - (hl & 7)) & 7;
    if (rest != need && pad && rest == need + pad) {
        int zeros = 1;
        for (size_t i = 0; i < pad; i++) zeros &= st->map[base + i] == 0;
        if (zeros) base += pad;
    }
    if (st->map_len - base < need) FAIL("qstore_open: file is shorter than its tensors need");
    st->data = st->map + base;
    st->data_len = st->map_len - base;
    return st;
fail:
    if (fd >= 0) close(fd);
    SNEPPX_qstore_close(st);
    return NULL;
}

static const Entry* find(const SNEPPXQStore* st, const char* name) {
    if (!st || !name) return NULL;
    for (size_t i = 0; i < st->n_ent; i++)
        if (strcmp(st->ent[i].name, name) == 0) return &st->ent[i];
    return NULL;
}

size_t SNEPPX_qstore_count(const SNEPPXQStore* st) { return st ? st->n_ent : 0; }

const char* SNEPPX_qstore_name(const SNEPPXQStore* st, size_t i) {
    return (st && i < st->n_ent) ? st->ent[i].name : NULL;
}

int SNEPPX_qstore_info(const SNEPPXQStore* st, const char* name, int* dtype, size_t* shape,
                       size_t* ndim, size_t* nbytes) {
    const Entry* e = find(st, name);
    if (!e) return -1;
    if (dtype) *dtype = e->dtype;
    if (ndim) *ndim = e->ndim;
    if (shape)
        for (size_t d = 0; d < e->ndim; d++) shape[d] = e->shape[d];
    if (nbytes) *nbytes = e->end - e->begin;
    return 0;
}

const void* SNEPPX_qstore_data(const SNEPPXQStore* st, const char* name, size_t* nbytes) {
    const Entry* e = find(st, name);
    if (!e) return NULL;
    if (nbytes) *nbytes = e->end - e->begin;
    return st->data + e->begin;
}

int SNEPPX_qstore_read_device(const SNEPPXQStore* st, const char* name, void* d_dst,
                              size_t nbytes, SNEPPXStream stream) {
    const Entry* e = find(st, name);
    if (!e) { snx_set_error("qstore_read_device: no tensor %s", name ? name : "(null)"); return -1; }
    if (!d_dst) { snx_set_error("qstore_read_device: NULL destination"); return -1; }
    if (nbytes != e->end - e->begin) {
        snx_set_error("qstore_read_device: %s holds %zu bytes, not %zu", name, e->end - e->begin, nbytes);
        return -1;
    }
    snx_clear_error();
    if (nbytes == 0) return 0;
    if (snx_hip_memcpy_h2d(d_dst, st->data + e->begin, nbytes, stream)) return -1;
    return snx_hip_stream_sync(stream);
}

const char* SNEPPX_qstore_metadata(const SNEPPXQStore* st, const char* key) {
    if (!st || !key) return NULL;
    for (size_t i = 0; i < st->n_meta; i++)
        if (strcmp(st->meta[i].key, key) == 0) return st->meta[i].value;
    return NULL;
}

/* ------------------------------------------------------------------ writer */

typedef struct {
    char* name;
    int dtype;
    size_t ndim;
    size_t shape[SNEPPX_QST_MAX_DIMS];
    unsigned char* data;
    size_t nbytes;
} WEntry;

struct SNEPPXQStoreWriter {
    char* path;
    WEntry* ent;
    size_t n_ent;
    Meta* meta;
    size_t n_meta;
};

static char* dupstr(const char* s) {
    size_t n = strlen(s) + 1;
    char* d = (char*)malloc(n);
    if (d) memcpy(d, s, n);
    return d;
}

static void free_writer(SNEPPXQStoreWriter* w) {
    if (!w) return;
    for (size_t i = 0; i < w->n_ent; i++) {
        free(w->ent[i].name);
        free(w->ent[i].data);
    }
    for (size_t i = 0; i < w->n_meta; i++) {
        free(w->meta[i].key);
        free(w->meta[i].value);
    }
    free(w->ent);
    free(w->meta);
    free(w->path);
    free(w);
}

SNEPPXQStoreWriter* SNEPPX_qstore_writer_open(const char* path) {
    if (!path) { snx_set_error("qstore_writer_open: NULL path"); return NULL; }
    snx_clear_error();
    SNEPPXQStoreWriter* w = (SNEPPXQStoreWriter*)calloc(1, sizeof *w);
    if (!w || !(w->path = dupstr(path))) {
        free(w);
        snx_set_error("qstore_writer_open: out of host memory");
        return NULL;
    }
    return w;
}

/* shape checks shared by the two add paths; returns the byte size or 0 with
 * the error set (a tensor with a zero dimension has 0 bytes and is allowed) */
static int check_add(SNEPPXQStoreWriter* w, const char* name, int dtype, const size_t* shape,
                     size_t ndim, size_t* nbytes) {
    if (!w || !name || (!shape && ndim)) { snx_set_error("qstore_writer_add: NULL argument"); return -1; }
    if (!*name || strcmp(name, "__metadata__") == 0) { snx_set_error("qstore_writer_add: bad name"); return -1; }
    if (dtype < 0 || dtype >= N_DTYPES) { snx_set_error("qstore_writer_add: unknown dtype %d", dtype); return -1; }
    if (ndim > SNEPPX_QST_MAX_DIMS) { snx_set_error("qstore_writer_add: %zu dims (max %d)", ndim, SNEPPX_QST_MAX_DIMS); return -1; }
    for (size_t i = 0; i < w->n_ent; i++)
        if (strcmp(w->ent[i].name, name) == 0) { snx_set_error("qstore_writer_add: duplicate %s", name); return -1; }
    size_t cnt = 1;
    for (size_t d = 0; d < ndim; d++) {
        if (shape[d] && cnt > SIZE_MAX / shape[d] / 8) { snx_set_error("qstore_writer_add: shape overflows"); return -1; }
        cnt *= shape[d];
    }
    *nbytes = cnt * k_dtype_size[dtype];
    return 0;
}

static int push(SNEPPXQStoreWriter* w, const char* name, int dtype, const size_t* shape,
                size_t ndim, unsigned char* data, size_t nbytes) {
    WEntry* ne = (WEntry*)realloc(w->ent, (w->n_ent + 1) * sizeof(WEntry));
    char* nm = dupstr(name);
    if (!ne || !nm) {
        if (ne) w->ent = ne;
        free(nm);
        free(data);
        snx_set_error("qstore_writer_add: out of host memory");
        return -1;
    }
    w->ent = ne;
    WEntry* e = &w->ent[w->n_ent++];
    memset(e, 0, sizeof *e);
    e->name = nm;
    e->dtype = dtype;
    e->ndim = ndim;
    for (size_t d = 0; d < ndim; d++) e->shape[d] = shape[d];
    e->data = data;
    e->nbytes = nbytes;
    return 0;
}

int SNEPPX_qstore_writer_add_host(SNEPPXQStoreWriter* w, const char* name, int dtype,
                                  const size_t* shape, size_t ndim, const void* data) {
    size_t nbytes;
    if (check_add(w, name, dtype, shape, ndim, &nbytes)) return -1;
    if (nbytes && !data) { snx_set_error("qstore_writer_add_host: NULL data"); return -1; }
    snx_clear_error();
    unsigned char* copy = (unsigned char*)malloc(nbytes ? nbytes : 1);
    if (!copy) { snx_set_error("qstore_writer_add_host: out of host memory"); return -1; }
    if (nbytes) memcpy(copy, data, nbytes);
    return push(w, name, dtype, shape, ndim, copy, nbytes);
}

int SNEPPX_qstore_writer_add_device(SNEPPXQStoreWriter* w, const char* name, int dtype,
                                    const size_t* shape, size_t ndim, const void* d_data,
                                    SNEPPXStream stream) {
    size_t nbytes;
    if (check_add(w, name, dtype, shape, ndim, &nbytes)) return -1;
    if (nbytes && !d_data) { snx_set_error("qstore_writer_add_device: NULL data"); return -1; }
    snx_clear_error();
    unsigned char* copy = (unsigned char*)malloc(nbytes ? nbytes : 1);
    if (!copy) { snx_set_error("qstore_writer_add_device: out of host memory"); return -1; }
    if (nbytes && (snx_hip_memcpy_d2h(copy, d_data, nbytes, stream) || snx_hip_stream_sync(stream))) {
        free(copy);
        return -1;
    }
    return push(w, name, dtype, shape, ndim, copy, nbytes);
}

int SNEPPX_qstore_writer_set_metadata(SNEPPXQStoreWriter* w, const char* key, const char* value) {
    if (!w || !key || !value) { snx_set_error("qstore_writer_set_metadata: NULL argument"); return -1; }
    snx_clear_error();
    for (size_t i = 0; i < w->n_meta; i++)
        if (strcmp(w->meta[i].key, key) == 0) {
            char* v = dupstr(value);
            if (!v) { snx_set_error("qstore_writer_set_metadata: out of host memory"); return -1; }
            free(w->meta[i].value);
            w->meta[i].value = v;
            return 0;
        }
    Meta* nm = (Meta*)realloc(w->meta, (w->n_meta + 1) * sizeof(Meta));
    if (!nm) { snx_set_error("qstore_writer_set_metadata: out of host memory"); return -1; }
    w->meta = nm;
    char* k = dupstr(key);
    char* v = dupstr(value);
    if (!k || !v) {
        free(k);
        free(v);
        snx_set_error("qstore_writer_set_metadata: out of host memory");
        return -1;
    }
    w->meta[w->n_meta].key = k;
    w->meta[w->n_meta].value = v;
    w->n_meta++;
    return 0;
}

/* growable text buffer for the header */
typedef struct {
    char* s;
    size_t n, cap;
    int bad;
} Text;

static void tput(Text* t, const char* s, size_t n) {
    if (t->bad) return;
    if (t->n + n + 1 > t->cap) {
        size_t cap = (t->n + n + 1) * 2 + 256;
        char* ns = (char*)realloc(t->s, cap);
        if (!ns) { t->bad = 1; return; }
        t->s = ns;
        t->cap = cap;
    }
    memcpy(t->s + t->n, s, n);
    t->n += n;
    t->s[t->n] = 0;
}

static void tstr(Text* t, const char* s) { tput(t, s, strlen(s)); }

static void tjson(Text* t, const char* s) {
    tput(t, "\"", 1);
    for (; *s; s++) {
        unsigned char c = (unsigned char)*s;
        char esc[8];
        if (c == '"' || c == '\\') { esc[0] = '\\'; esc[1] = (char)c; tput(t, esc, 2); }
        else if (c < 0x20) { snprintf(esc, sizeof esc, "\\u%04x", c); tput(t, esc, 6); }
        else tput(t, (const char*)&c, 1);
    }
    tput(t, "\"", 1);
}

static void tnum(Text* t, size_t v) {
    char b[32];
    snprintf(b, sizeof b, "%zu", v);
    tstr(t, b);
}

int SNEPPX_qstore_writer_close(SNEPPXQStoreWriter* w) {
    if (!w) { snx_set_error("qstore_writer_close: NULL writer"); return -1; }
    snx_clear_error();
    int rc = -1;
    FILE* f = NULL;
    Text t = {0};
    tstr(&t, "{");
    int first = 1;
    if (w->n_meta) {
        tstr(&t, "\"__metadata__\":{");
        for (size_t i = 0; i < w->n_meta; i++) {
            if (i) tstr(&t, ",");
            tjson(&t, w->meta[i].key);
            tstr(&t, ":");
            tjson(&t, w->meta[i].value);
        }
        tstr(&t, "}");
        first = 0;
    }
    size_t off = 0;
    for (size_t i = 0; i < w->n_ent; i++) {
        const WEntry* e = &w->ent[i];
        if (!first) tstr(&t, ",");
        first = 0;
        tjson(&t, e->name);
        tstr(&t, ":{\"dtype\":\"");
        tstr(&t, k_dtype_names[e->dtype]);
        tstr(&t, "\",\"shape\":[");
        for (size_t d = 0; d < e->ndim; d++) {
            if (d) tstr(&t, ",");
            tnum(&t, e->shape[d]);
        }
        tstr(&t, "],\"data_offsets\":[");
        tnum(&t, off);
        tstr(&t, ",");
        tnum(&t, off + e->nbytes);
        tstr(&t, "]}");
        off += e->nbytes;
    }
    tstr(&t, "}");
    while (!t.bad && t.n % 8) tstr(&t, " ");   /* the data block starts 8-aligned */
    if (t.bad) FAIL("qstore_writer_close: out of host memory");
    f = fopen(w->path, "wb");
    if (!f) FAIL("qstore_writer_close: cannot create %s (%s)", w->path, strerror(errno));
    unsigned char len8[8];
    uint64_t hl = (uint64_t)t.n;
    for (int i = 0; i < 8; i++) len8[i] = (unsigned char)(hl >> (8 * i));
    if (fwrite(len8, 1, 8, f) != 8 || fwrite(t.s, 1, t.n, f) != t.n) FAIL("qstore_writer_close: write failed");
    for (size_t i = 0; i < w->n_ent; i++)
        if (w->ent[i].nbytes && fwrite(w->ent[i].data, 1, w->ent[i].nbytes, f) != w->ent[i].nbytes)
            FAIL("qstore_writer_close: write failed");
    if (fclose(f)) { f = NULL; FAIL("qstore_writer_close: write failed"); }
    f = NULL;
    rc = 0;
fail:
    if (f) fclose(f);
    free(t.s);
    free_writer(w);
    return rc;
}

/* ---------------------------------------------------------- layer helpers */

static void tname(char* out, size_t cap, const char* prefix, const char* suffix) {
    snprintf(out, cap, "%s.%s", prefix, suffix);
}

int SNEPPX_qstore_save_w4(SNEPPXQStoreWriter* w, const char* prefix, const uint32_t* d_qweight,
                          const uint16_t* d_scales, const uint32_t* d_qzeros,
                          const int32_t* d_g_idx, size_t N, size_t K, int group, size_t G,
                          SNEPPXStream stream) {
    char nm[512], val[32];
    if (!w || !prefix || !d_qweight || !d_scales) { snx_set_error("qstore_save_w4: NULL argument"); return -1; }
    if (!N || !K || K % 8 || !G) { snx_set_error("qstore_save_w4: bad shape N=%zu K=%zu G=%zu", N, K, G); return -1; }
    if (!d_g_idx && (group <= 0 || K % (size_t)group || K / (size_t)group != G)) {
        snx_set_error("qstore_save_w4: group %d does not give G=%zu groups of K=%zu", group, G, K);
        return -1;
    }
    size_t s_qw[2] = {N, K / 8}, s_sc[2] = {N, G}, s_qz[2] = {N, (G + 7) / 8}, s_gi[1] = {K};
    tname(nm, sizeof nm, prefix, "qweight");
    if (SNEPPX_qstore_writer_add_device(w, nm, SNEPPX_QST_I32, s_qw, 2, d_qweight, stream)) return -1;
    tname(nm, sizeof nm, prefix, "scales");
    if (SNEPPX_qstore_writer_add_device(w, nm, SNEPPX_QST_F16, s_sc, 2, d_scales, stream)) return -1;
    if (d_qzeros) {
        tname(nm, sizeof nm, prefix, "qzeros");
        if (SNEPPX_qstore_writer_add_device(w, nm, SNEPPX_QST_I32, s_qz, 2, d_qzeros, stream)) return -1;
    }
    if (d_g_idx) {
        tname(nm, sizeof nm, prefix, "g_idx");
        if (SNEPPX_qstore_writer_add_device(w, nm, SNEPPX_QST_I32, s_gi, 1, d_g_idx, stream)) return -1;
    }
    tname(nm, sizeof nm, prefix, "format");
    if (SNEPPX_qstore_writer_set_metadata(w, nm, "w4")) return -1;
    snprintf(val, sizeof val, "%d", d_g_idx ? 0 : group);
    tname(nm, sizeof nm, prefix, "group_size");
    return SNEPPX_qstore_writer_set_metadata(w, nm, val);
}

static int tensor2(const SNEPPXQStore* st, const char* prefix, const char* suffix, int dtype,
                   size_t ndim, size_t* shape) {
    char nm[512];
    int dt;
    size_t nd;
    tname(nm, sizeof nm, prefix, suffix);
    if (SNEPPX_qstore_info(st, nm, &dt, shape, &nd, NULL)) return 1;   /* absent */
    if (dt != dtype || nd != ndim) {
        snx_set_error("qstore: %s has dtype %d / %zu dims, expected %d / %zu", nm, dt, nd, dtype, ndim);
        return -1;
    }
    return 0;
}

int SNEPPX_qstore_query_w4(const SNEPPXQStore* st, const char* prefix, size_t* N, size_t* K,
                           size_t* G, int* group, int* has_zeros, int* has_g_idx) {
    if (!st || !prefix) { snx_set_error("qstore_query_w4: NULL argument"); return -1; }
    snx_clear_error();
    size_t qw[SNEPPX_QST_MAX_DIMS], sc[SNEPPX_QST_MAX_DIMS], qz[SNEPPX_QST_MAX_DIMS], gi[SNEPPX_QST_MAX_DIMS];
    int r = tensor2(st, prefix, "qweight", SNEPPX_QST_I32, 2, qw);
    if (r) { if (r > 0) snx_set_error("qstore_query_w4: no %s.qweight", prefix); return -1; }
    r = tensor2(st, prefix, "scales", SNEPPX_QST_F16, 2, sc);
    if (r) { if (r > 0) snx_set_error("qstore_query_w4: no %s.scales", prefix); return -1; }
    int rz = tensor2(st, prefix, "qzeros", SNEPPX_QST_I32, 2, qz);
    int rg = tensor2(st, prefix, "g_idx", SNEPPX_QST_I32, 1, gi);
    if (rz < 0 || rg < 0) return -1;
    /* every tensor's byte count matched its data_offsets at open, so N K / 2
     * and N G 2 fit in size_t; the kernels also index rows and columns with
     * int */
    size_t n = qw[0], k = qw[1] * 8, g = sc[1];
    if (!n || !k || !g || sc[0] != n || (rz == 0 && (qz[0] != n || qz[1] != (g + 7) / 8)) ||
        (rg == 0 && gi[0] != k) || (rg != 0 && k % g)) {
        snx_set_error("qstore_query_w4: %s tensors have inconsistent shapes", prefix);
        return -1;
    }
    if (n > INT_MAX || qw[1] > INT_MAX / 8 || g > INT_MAX) {
        snx_set_error("qstore_query_w4: %s has N=%zu, K=%zu beyond the kernels' int range", prefix, n, k);
        return -1;
    }
    if (N) *N = n;
    if (K) *K = k;
    if (G) *G = g;
    if (group) *group = rg == 0 ? 0 : (int)(k / g);
    if (has_zeros) *has_zeros = rz == 0;
    if (has_g_idx) *has_g_idx = rg == 0;
    return 0;
}

int SNEPPX_qstore_load_w4(const SNEPPXQStore* st, const char* prefix, uint32_t* d_qweight,
                          uint16_t* d_scales, uint32_t* d_qzeros, int32_t* d_g_idx,
                          SNEPPXStream stream) {
    size_t N, K, G;
    int group, hz, hg;
    char nm[512];
    if (!d_qweight || !d_scales) { snx_set_error("qstore_load_w4: NULL destination"); return -1; }
    if (SNEPPX_qstore_query_w4(st, prefix, &N, &K, &G, &group, &hz, &hg)) return -1;
    if (hz != (d_qzeros != NULL) || hg != (d_g_idx != NULL)) {
        snx_set_error("qstore_load_w4: %s %s zero points and %s g_idx; destinations must match",
                      prefix, hz ? "has" : "has no", hg ? "a" : "no");
        return -1;
    }
    tname(nm, sizeof nm, prefix, "qweight");
    if (SNEPPX_qstore_read_device(st, nm, d_qweight, N * K / 2, stream)) return -1;
    tname(nm, sizeof nm, prefix, "scales");
    if (SNEPPX_qstore_read_device(st, nm, d_scales, N * G * 2, stream)) return -1;
    if (hz) {
        tname(nm, sizeof nm, prefix, "qzeros");
        if (SNEPPX_qstore_read_device(st, nm, d_qzeros, N * ((G + 7) / 8) * 4, stream)) return -1;
    }
    if (hg) {
        tname(nm, sizeof nm, prefix, "g_idx");
        if (SNEPPX_qstore_read_device(st, nm, d_g_idx, K * 4, stream)) return -1;
    }
    return 0;
}

int SNEPPX_qstore_save_w8(SNEPPXQStoreWriter* w, const char* prefix, const int8_t* d_q,
                          const float* d_scales, size_t N, size_t K, SNEPPXStream stream) {
    char nm[512];
    if (!w || !prefix || !d_q || !d_scales) { snx_set_error("qstore_save_w8: NULL argument"); return -1; }
    if (!N || !K) { snx_set_error("qstore_save_w8: empty shape"); return -1; }
    size_t s_q[2] = {N, K}, s_s[1] = {N};
    tname(nm, sizeof nm, prefix, "weight");
    if (SNEPPX_qstore_writer_add_device(w, nm, SNEPPX_QST_I8, s_q, 2, d_q, stream)) return -1;
    tname(nm, sizeof nm, prefix, "weight_scale");
    if (SNEPPX_qstore_writer_add_device(w, nm, SNEPPX_QST_F32, s_s, 1, d_scales, stream)) return -1;
    tname(nm, sizeof nm, prefix, "format");
    return SNEPPX_qstore_writer_set_metadata(w, nm, "w8");
}

int SNEPPX_qstore_query_w8(const SNEPPXQStore* st, const char* prefix, size_t* N, size_t* K) {
    if (!st || !prefix) { snx_set_error("qstore_query_w8: NULL argument"); return -1; }
    snx_clear_error();
    size_t q[SNEPPX_QST_MAX_DIMS], s[SNEPPX_QST_MAX_DIMS];
    int r = tensor2(st, prefix, "weight", SNEPPX_QST_I8, 2, q);
    if (r) { if (r > 0) snx_set_error("qstore_query_w8: no %s.weight", prefix); return -1; }
    r = tensor2(st, prefix, "weight_scale", SNEPPX_QST_F32, 1, s);
    if (r) { if (r > 0) snx_set_error("qstore_query_w8: no %s.weight_scale", prefix); return -1; }
    if (!q[0] || !q[1] || s[0] != q[0]) {
        snx_set_error("qstore_query_w8: %s tensors have inconsistent shapes", prefix);
        return -1;
    }
    if (q[0] > INT_MAX || q[1] > INT_MAX) {
        snx_set_error("qstore_query_w8: %s has N=%zu, K=%zu beyond the kernels' int range", prefix,
                      q[0], q[1]);
        return -1;
    }
    if (N) *N = q[0];
    if (K) *K = q[1];
    return 0;
}

int SNEPPX_qstore_load_w8(const SNEPPXQStore* st, const char* prefix, int8_t* d_q,
                          float* d_scales, SNEPPXStream stream) {
    size_t N, K;
    char nm[512];
    if (!d_q || !d_scales) { snx_set_error("qstore_load_w8: NULL destination"); return -1; }
    if (SNEPPX_qstore_query_w8(st, prefix, &N, &K)) return -1;
    tname(nm, sizeof nm, prefix, "weight");
    if (SNEPPX_qstore_read_device(st, nm, d_q, N * K, stream)) return -1;
    tname(nm, sizeof nm, prefix, "weight_scale");
    return SNEPPX_qstore_read_device(st, nm, d_scales, N * 4, stream);
}
