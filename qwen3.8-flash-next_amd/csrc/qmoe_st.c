/*
 * qmoe_st.c -- checkpoint reader of libqmoe.so: an index over the
 * *.safetensors files of a checkpoint directory and the upload of one MoE
 * layer from it into HBM.  Host C11 only (the upload copies through the
 * context's tensor slots in qmoe_host.c).
 *
 * Follows the reference's reader and loader rules:
 *   c/src/safetensors.c:57-262   header parse and validation, directory scan
 *   c/src/safetensors.c:307-324  lookup (binary search; "language_model." prefix)
 *   c/src/model.c:204-272        q4 iff "<base>.scales" exists, codes U32,
 *                                missing biases read as zero, dense BF16
 *   c/src/model.c:541-547, 1902-1912  MoE tensor names of one layer
 *
 * File format (published safetensors layout): 8-byte little-endian header
 * length N, N bytes of JSON {name: {"dtype", "shape", "data_offsets"}, ...,
 * "__metadata__": {...}}, then the data; offsets are relative to 8 + N.
 */
#define _POSIX_C_SOURCE 200809L /* pread, under -std=c11 */
#include <dirent.h>
#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <hip/hip_runtime_api.h>

#include "qmoe_internal.h"

#define ST_MAX_HEADER (256u << 20) /* larger JSON headers are rejected */
#define ST_MAX_DEPTH 16

static void st_err(qmoe_err *err, const char *fmt, ...) {
    if (!err) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err->msg, sizeof(err->msg), fmt, ap);
    va_end(ap);
}

/* ------------------------------------------------------------ JSON
 * A small recursive-descent parser for the header: objects, arrays,
 * strings (escapes, \u to UTF-8), numbers, true/false/null. */

enum { J_NULL, J_BOOL, J_NUM, J_STR, J_ARR, J_OBJ };

typedef struct jv {
    int type;
    double num;
    int is_int;
    long long inum;
    char *str;         /* J_STR */
    size_t n;          /* J_ARR / J_OBJ entries */
    char **keys;       /* J_OBJ */
    struct jv **items; /* J_ARR / J_OBJ values */
} jv;

typedef struct {
    const char *start, *p, *end;
    char msg[128];
} jparser;

static void jfree(jv *v) {
    if (!v) return;
    free(v->str);
    for (size_t i = 0; i < v->n; i++) {
        if (v->keys) free(v->keys[i]);
        jfree(v->items[i]);
    }
    free(v->keys);
    free(v->items);
    free(v);
}

static void jskip(jparser *ps) {
    while (ps->p < ps->end && (*ps->p == ' ' || *ps->p == '\t' || *ps->p == '\n' || *ps->p == '\r'))
        ps->p++;
}

static int jfail(jparser *ps, const char *what) {
    if (!ps->msg[0]) snprintf(ps->msg, sizeof(ps->msg), "%s at byte %ld", what, (long)(ps->p - ps->start));
    return -1;
}

static int hexval(char c) {
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    if (c >= 'A' && c <= 'F') return c - 'A' + 10;
    return -1;
}

/* parses a string literal at ps->p (which is '"'); returns a malloc'd copy */
static char *jstring(jparser *ps) {
    ps->p++; /* opening quote */
    size_t cap = 32, len = 0;
    char *out = malloc(cap);
    if (!out) return NULL;
    while (ps->p < ps->end && *ps->p != '"') {
        unsigned cp;
        char c = *ps->p++;
        if ((unsigned char)c < 0x20) {
            free(out);
            return NULL;
        }
        if (c != '\\') {
            cp = (unsigned char)c;
            if (len + 1 >= cap) {
                char *o2 = realloc(out, cap *= 2);
                if (!o2) {
                    free(out);
                    return NULL;
                }
                out = o2;
            }
            out[len++] = (char)cp;
            continue;
        }
        if (ps->p >= ps->end) break;
        c = *ps->p++;
        switch (c) {
        case '"': cp = '"'; break;
        case '\\': cp = '\\'; break;
        case '/': cp = '/'; break;
        case 'b': cp = '\b'; break;
        case 'f': cp = '\f'; break;
        case 'n': cp = '\n'; break;
        case 'r': cp = '\r'; break;
        case 't': cp = '\t'; break;
        case 'u': {
            if (ps->end - ps->p < 4) {
                free(out);
                return NULL;
            }
            cp = 0;
            for (int i = 0; i < 4; i++) {
                const int h = hexval(ps->p[i]);
                if (h < 0) {
                    free(out);
                    return NULL;
                }
                cp = cp * 16 + (unsigned)h;
            }
            ps->p += 4;
            /* a surrogate pair becomes one code point */
            if (cp >= 0xD800 && cp < 0xDC00 && ps->end - ps->p >= 6 && ps->p[0] == '\\' &&
                ps->p[1] == 'u') {
                unsigned lo = 0;
                int ok = 1;
                for (int i = 0; i < 4; i++) {
                    const int h = hexval(ps->p[2 + i]);
                    if (h < 0) ok = 0;
                    lo = lo * 16 + (unsigned)(h < 0 ? 0 : h);
                }
                if (ok && lo >= 0xDC00 && lo < 0xE000) {
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    ps->p += 6;
                }
            }
            break;
        }
        default: free(out); return NULL;
        }
        char buf[4];
        int nb;
        if (cp < 0x80) {
            buf[0] = (char)cp;
            nb = 1;
        } else if (cp < 0x800) {
            buf[0] = (char)(0xC0 | (cp >> 6));
            buf[1] = (char)(0x80 | (cp & 0x3F));
            nb = 2;
        } else if (cp < 0x10000) {
            buf[0] = (char)(0xE0 | (cp >> 12));
            buf[1] = (char)(0x80 | ((cp >> 6) & 0x3F));
            buf[2] = (char)(0x80 | (cp & 0x3F));
            nb = 3;
        } else {
            buf[0] = (char)(0xF0 | (cp >> 18));
            buf[1] = (char)(0x80 | ((cp >> 12) & 0x3F));
            buf[2] = (char)(0x80 | ((cp >> 6) & 0x3F));
            buf[3] = (char)(0x80 | (cp & 0x3F));
            nb = 4;
        }
        while (len + (size_t)nb >= cap) {
            char *o2 = realloc(out, cap *= 2);
            if (!o2) {
                free(out);
                return NULL;
            }
            out = o2;
        }
        memcpy(out + len, buf, (size_t)nb);
        len += (size_t)nb;
    }
    if (ps->p >= ps->end) {
        free(out);
        return NULL;
    }
    ps->p++; /* closing quote */
    out[len] = 0;
    return out;
}

static jv *jvalue(jparser *ps, int depth);

/* appends (key, item); objects carry a key per item, arrays none */
static int jpush(jv *v, char *key, jv *item) {
    if (v->type == J_OBJ) {
        char **k2 = realloc(v->keys, (v->n + 1) * sizeof(char *));
        if (!k2) return -1;
        v->keys = k2;
    }
    jv **i2 = realloc(v->items, (v->n + 1) * sizeof(jv *));
    if (!i2) return -1;
    v->items = i2;
    if (v->type == J_OBJ) v->keys[v->n] = key;
    v->items[v->n] = item;
    v->n++;
    return 0;
}

static jv *jvalue(jparser *ps, int depth) {
    jskip(ps);
    if (ps->p >= ps->end || depth > ST_MAX_DEPTH) {
        jfail(ps, depth > ST_MAX_DEPTH ? "nesting too deep" : "unexpected end");
        return NULL;
    }
    jv *v = calloc(1, sizeof(jv));
    if (!v) return NULL;
    const char c = *ps->p;
    if (c == '{' || c == '[') {
        const int obj = c == '{';
        v->type = obj ? J_OBJ : J_ARR;
        ps->p++;
        jskip(ps);
        if (ps->p < ps->end && *ps->p == (obj ? '}' : ']')) {
            ps->p++;
            return v;
        }
        for (;;) {
            char *key = NULL;
            if (obj) {
                jskip(ps);
                if (ps->p >= ps->end || *ps->p != '"' || !(key = jstring(ps))) {
                    jfail(ps, "bad object key");
                    jfree(v);
                    return NULL;
                }
                jskip(ps);
                if (ps->p >= ps->end || *ps->p != ':') {
                    free(key);
                    jfail(ps, "expected ':'");
                    jfree(v);
                    return NULL;
                }
                ps->p++;
            }
            jv *item = jvalue(ps, depth + 1);
            if (!item || jpush(v, key, item)) {
                free(key);
                jfree(item);
                jfree(v);
                return NULL;
            }
            jskip(ps);
            if (ps->p < ps->end && *ps->p == ',') {
                ps->p++;
                continue;
            }
            if (ps->p < ps->end && *ps->p == (obj ? '}' : ']')) {
                ps->p++;
                return v;
            }
            jfail(ps, "expected ',' or a closing bracket");
            jfree(v);
            return NULL;
        }
    }
    if (c == '"') {
        v->type = J_STR;
        if (!(v->str = jstring(ps))) {
            jfail(ps, "bad string");
            jfree(v);
            return NULL;
        }
        return v;
    }
    if (ps->end - ps->p >= 4 && !memcmp(ps->p, "true", 4)) {
        v->type = J_BOOL;
        v->num = 1;
        ps->p += 4;
        return v;
    }
    if (ps->end - ps->p >= 5 && !memcmp(ps->p, "false", 5)) {
        v->type = J_BOOL;
        ps->p += 5;
        return v;
    }
    if (ps->end - ps->p >= 4 && !memcmp(ps->p, "null", 4)) {
        v->type = J_NULL;
        ps->p += 4;
        return v;
    }
    if (c == '-' || (c >= '0' && c <= '9')) {
        /* integers exactly (offsets exceed 2^53 only in files of 8 PiB), others as double */
        char buf[64];
        size_t len = 0;
        int integral = 1;
        while (ps->p < ps->end && len + 1 < sizeof(buf) &&
               *ps->p && (strchr("+-0123456789", *ps->p) || *ps->p == '.' || *ps->p == 'e' || *ps->p == 'E')) {
            if (*ps->p == '.' || *ps->p == 'e' || *ps->p == 'E') integral = 0;
            buf[len++] = *ps->p++;
        }
        buf[len] = 0;
        char *endp = NULL;
        v->type = J_NUM;
        errno = 0;
        if (integral) {
            v->inum = strtoll(buf, &endp, 10);
            v->is_int = errno == 0;
            v->num = (double)v->inum;
        } else {
            v->num = strtod(buf, &endp);
        }
        if (!endp || *endp || errno) {
            jfail(ps, "bad number");
            jfree(v);
            return NULL;
        }
        return v;
    }
    jfail(ps, "unexpected character");
    jfree(v);
    return NULL;
}

static const jv *jget(const jv *o, const char *key) {
    if (!o || o->type != J_OBJ) return NULL;
    for (size_t i = 0; i < o->n; i++)
        if (!strcmp(o->keys[i], key)) return o->items[i];
    return NULL;
}

/* ------------------------------------------------------------ index */

typedef struct {
    char *name;
    qmoe_st_tensor t;
} st_entry;

struct qmoe_st {
    char **paths;
    int *fds;
    int nfiles;
    st_entry *ent;
    size_t n, cap;
};

static const struct {
    const char *name;
    int size;
} DTYPES[QMOE_ST_COUNT] = {
    {"BOOL", 1}, {"U8", 1}, {"I8", 1},  {"U16", 2},  {"I16", 2}, {"U32", 4}, {"I32", 4},
    {"U64", 8},  {"I64", 8}, {"F16", 2}, {"BF16", 2}, {"F32", 4}, {"F64", 8},
};

int qmoe_st_dtype_size(int dtype) { return dtype >= 0 && dtype < QMOE_ST_COUNT ? DTYPES[dtype].size : 0; }

const char *qmoe_st_dtype_name(int dtype) {
    return dtype >= 0 && dtype < QMOE_ST_COUNT ? DTYPES[dtype].name : "?";
}

static int dtype_of(const char *s) {
    for (int i = 0; i < QMOE_ST_COUNT; i++)
        if (!strcmp(DTYPES[i].name, s)) return i;
    return -1;
}

static int add_entry(qmoe_st *ix, const char *name, const qmoe_st_tensor *t) {
    if (ix->n == ix->cap) {
        const size_t cap = ix->cap ? 2 * ix->cap : 256;
        st_entry *e2 = realloc(ix->ent, cap * sizeof(st_entry));
        if (!e2) return -1;
        ix->ent = e2;
        ix->cap = cap;
    }
    char *nm = malloc(strlen(name) + 1);
    if (!nm) return -1;
    strcpy(nm, name);
    ix->ent[ix->n].name = nm;
    ix->ent[ix->n].t = *t;
    ix->n++;
    return 0;
}

typedef struct {
    uint64_t lo, hi;
    const char *name;
} st_range;

static int cmp_range(const void *a, const void *b) {
    const st_range *x = a, *y = b;
    return x->lo < y->lo ? -1 : x->lo > y->lo;
}

/* indexes one file; on failure the entries added from it are dropped */
static int parse_file(qmoe_st *ix, const char *path, int file, qmoe_err *err) {
    const int fd = open(path, O_RDONLY);
    if (fd < 0) {
        st_err(err, "%s: open failed (%s)", path, strerror(errno));
        return -1;
    }
    struct stat sb;
    if (fstat(fd, &sb) != 0) {
        st_err(err, "%s: size query failed (%s)", path, strerror(errno));
        close(fd);
        return -1;
    }
    const uint64_t fsize = (uint64_t)sb.st_size;
    unsigned char lb[8];
    if (fsize < 8 || pread(fd, lb, 8, 0) != 8) {
        st_err(err, "%s: shorter than the 8-byte header length field", path);
        close(fd);
        return -1;
    }
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; i--) hlen = (hlen << 8) | lb[i];
    if (hlen > fsize - 8 || hlen > ST_MAX_HEADER) {
        st_err(err, "%s: header length runs past the end of the file", path);
        close(fd);
        return -1;
    }
    char *hdr = malloc((size_t)hlen + 1);
    if (!hdr) {
        st_err(err, "out of host memory reading %s", path);
        close(fd);
        return -1;
    }
    size_t got = 0;
    while (got < hlen) {
        const ssize_t r = pread(fd, hdr + got, (size_t)hlen - got, (off_t)(8 + got));
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) {
            st_err(err, "%s: header length runs past the end of the file", path);
            free(hdr);
            close(fd);
            return -1;
        }
        got += (size_t)r;
    }
    hdr[hlen] = 0;
    jparser ps = {hdr, hdr, hdr + hlen, {0}};
    jv *root = jvalue(&ps, 0);
    if (root) {
        jskip(&ps);
        if (ps.p != ps.end) {
            jfree(root);
            root = NULL;
            snprintf(ps.msg, sizeof(ps.msg), "trailing bytes after the header object");
        }
    }
    free(hdr);
    if (!root || root->type != J_OBJ) {
        st_err(err, "%s: header is not a JSON object (%s)", path,
               root ? "top level is not an object" : ps.msg);
        jfree(root);
        close(fd);
        return -1;
    }
    const uint64_t base = 8 + hlen;
    const size_t first = ix->n;
    st_range *rg = calloc(root->n ? root->n : 1, sizeof(st_range));
    size_t nr = 0;
    int failed = rg == NULL;
    if (failed) st_err(err, "out of host memory indexing %s", path);
    for (size_t i = 0; i < root->n && !failed; i++) {
        const char *stored = root->keys[i];
        const jv *m = root->items[i];
        if (!strcmp(stored, "__metadata__")) continue;
        const jv *jd = jget(m, "dtype"), *jo = jget(m, "data_offsets"), *js = jget(m, "shape");
        if (!m || m->type != J_OBJ || !jd || jd->type != J_STR || !jo || jo->type != J_ARR ||
            jo->n != 2 || !js || js->type != J_ARR) {
            st_err(err, "%s: entry lacks dtype, shape or data_offsets", stored);
            failed = 1;
            break;
        }
        qmoe_st_tensor t;
        memset(&t, 0, sizeof(t));
        t.dtype = dtype_of(jd->str);
        if (t.dtype < 0) {
            st_err(err, "%s: element type %s is not supported", stored, jd->str);
            failed = 1;
            break;
        }
        const jv *lo = jo->items[0], *hi = jo->items[1];
        if (lo->type != J_NUM || !lo->is_int || hi->type != J_NUM || !hi->is_int || lo->inum < 0 ||
            hi->inum < 0) {
            st_err(err, "%s: data_offsets must be two ordered non-negative integers", stored);
            failed = 1;
            break;
        }
        if (js->n > 8) {
            st_err(err, "%s: more dimensions than the index keeps (8)", stored);
            failed = 1;
            break;
        }
        t.ndim = (int)js->n;
        uint64_t elems = 1;
        int bad = 0;
        for (size_t d = 0; d < js->n; d++) {
            const jv *sv = js->items[d];
            if (sv->type != J_NUM || !sv->is_int || sv->inum < 0 ||
                (sv->inum > 0 && elems > UINT64_MAX / (uint64_t)sv->inum)) {
                bad = 1;
                break;
            }
            t.shape[d] = sv->inum;
            elems *= (uint64_t)sv->inum;
        }
        if (bad || elems > UINT64_MAX / 8) {
            st_err(err, "%s: shape entries must be non-negative integers", stored);
            failed = 1;
            break;
        }
        const uint64_t l = (uint64_t)lo->inum, h = (uint64_t)hi->inum;
        if (h < l || h - l != elems * (uint64_t)DTYPES[t.dtype].size || h > fsize - base) {
            st_err(err, "%s: byte range disagrees with the shape or leaves the file", stored);
            failed = 1;
            break;
        }
        /* duplicates (also across files) are found after the final sort */
        const char *name = strncmp(stored, "language_model.", 15) ? stored : stored + 15;
        t.file = file;
        t.offset = base + l;
        t.nbytes = h - l;
        if (add_entry(ix, name, &t)) {
            st_err(err, "out of host memory indexing %s", path);
            failed = 1;
            break;
        }
        rg[nr].lo = l;
        rg[nr].hi = h;
        rg[nr].name = stored;
        nr++;
    }
    if (!failed && nr > 1) {
        /* sorted by start, two ranges overlap iff a neighbour pair does
         * (empty tensors occupy no bytes) */
        qsort(rg, nr, sizeof(st_range), cmp_range);
        uint64_t reach = 0;
        const char *who = NULL;
        for (size_t i = 0; i < nr; i++) {
            if (rg[i].hi == rg[i].lo) continue;
            if (who && rg[i].lo < reach) {
                st_err(err, "%s: data overlaps another tensor of the file", rg[i].name);
                failed = 1;
                break;
            }
            if (rg[i].hi > reach) reach = rg[i].hi;
            who = rg[i].name;
        }
    }
    free(rg);
    jfree(root);
    if (failed) {
        while (ix->n > first) free(ix->ent[--ix->n].name);
        close(fd);
        return -1;
    }
    ix->paths[file] = malloc(strlen(path) + 1);
    if (!ix->paths[file]) {
        while (ix->n > first) free(ix->ent[--ix->n].name);
        close(fd);
        st_err(err, "out of host memory indexing %s", path);
        return -1;
    }
    strcpy(ix->paths[file], path);
    ix->fds[file] = fd;
    return 0;
}

static int cmp_entry(const void *a, const void *b) {
    return strcmp(((const st_entry *)a)->name, ((const st_entry *)b)->name);
}

static int is_st_file(const char *nm) {
    const size_t len = strlen(nm);
    return len > 12 && !strcmp(nm + len - 12, ".safetensors");
}

static int cmp_str(const void *a, const void *b) { return strcmp(*(char *const *)a, *(char *const *)b); }

void qmoe_st_close(qmoe_st *ix) {
    if (!ix) return;
    for (int i = 0; i < ix->nfiles; i++) {
        if (ix->fds && ix->fds[i] >= 0) close(ix->fds[i]);
        if (ix->paths) free(ix->paths[i]);
    }
    for (size_t i = 0; i < ix->n; i++) free(ix->ent[i].name);
    free(ix->ent);
    free(ix->paths);
    free(ix->fds);
    free(ix);
}

int qmoe_st_open(qmoe_st **out, const char *dir, qmoe_err *err) {
    if (err) err->msg[0] = 0;
    if (!out || !dir) {
        st_err(err, "index or directory pointer is NULL");
        return -1;
    }
    *out = NULL;
    DIR *d = opendir(dir);
    if (!d) {
        st_err(err, "%s: checkpoint directory cannot be listed (%s)", dir, strerror(errno));
        return -1;
    }
    /* file names, sorted so the index does not depend on directory order */
    char **names = NULL;
    int nf = 0, cap = 0, oom = 0;
    struct dirent *de;
    while ((de = readdir(d)) != NULL) {
        if (!is_st_file(de->d_name)) continue;
        if (nf == cap) {
            cap = cap ? 2 * cap : 16;
            char **n2 = realloc(names, (size_t)cap * sizeof(char *));
            if (!n2) {
                oom = 1;
                break;
            }
            names = n2;
        }
        if (!(names[nf] = malloc(strlen(de->d_name) + 1))) {
            oom = 1;
            break;
        }
        strcpy(names[nf++], de->d_name);
    }
    closedir(d);
    int rc = -1;
    qmoe_st *ix = NULL;
    if (oom) {
        st_err(err, "out of host memory listing %s", dir);
        goto done;
    }
    if (nf == 0) {
        st_err(err, "%s: no .safetensors file in the directory", dir);
        goto done;
    }
    qsort(names, (size_t)nf, sizeof(char *), cmp_str);
    ix = calloc(1, sizeof(qmoe_st));
    if (!ix || !(ix->paths = calloc((size_t)nf, sizeof(char *))) ||
        !(ix->fds = malloc((size_t)nf * sizeof(int)))) {
        st_err(err, "out of host memory opening %s", dir);
        goto done;
    }
    ix->nfiles = nf;
    for (int i = 0; i < nf; i++) ix->fds[i] = -1;
    for (int i = 0; i < nf; i++) {
        char path[4096];
        if (snprintf(path, sizeof(path), "%s/%s", dir, names[i]) >= (int)sizeof(path)) {
            st_err(err, "path too long in %s", dir);
            goto done;
        }
        if (parse_file(ix, path, i, err)) goto done;
    }
    if (ix->n) qsort(ix->ent, ix->n, sizeof(st_entry), cmp_entry);
    for (size_t i = 1; i < ix->n; i++)
        if (!strcmp(ix->ent[i - 1].name, ix->ent[i].name)) {
            st_err(err, "%s: tensor name given twice in the checkpoint", ix->ent[i].name);
            goto done;
        }
    *out = ix;
    ix = NULL;
    rc = 0;
done:
    for (int i = 0; i < nf; i++) free(names[i]);
    free(names);
    qmoe_st_close(ix);
    return rc;
}

size_t qmoe_st_count(const qmoe_st *ix) { return ix ? ix->n : 0; }

const char *qmoe_st_name(const qmoe_st *ix, size_t i) { return ix && i < ix->n ? ix->ent[i].name : NULL; }

static const st_entry *find_exact(const qmoe_st *ix, const char *name) {
    size_t lo = 0, hi = ix->n;
    while (lo < hi) {
        const size_t mid = (lo + hi) / 2;
        const int c = strcmp(ix->ent[mid].name, name);
        if (c == 0) return &ix->ent[mid];
        if (c < 0) lo = mid + 1;
        else hi = mid;
    }
    return NULL;
}

static const st_entry *find_entry(const qmoe_st *ix, const char *name) {
    if (!ix || !name) return NULL;
    const st_entry *e = find_exact(ix, name);
    if (e || strncmp(name, "model.", 6)) return e;
    char pre[512];
    if (snprintf(pre, sizeof(pre), "language_model.%s", name) >= (int)sizeof(pre)) return NULL;
    return find_exact(ix, pre);
}

int qmoe_st_find(const qmoe_st *ix, const char *name, qmoe_st_tensor *out) {
    const st_entry *e = find_entry(ix, name);
    if (!e) return 0;
    if (out) *out = e->t;
    return 1;
}

static int read_range(const qmoe_st *ix, const st_entry *e, uint64_t at, void *dst, size_t len,
                      qmoe_err *err) {
    size_t got = 0;
    char *p = dst;
    while (got < len) {
        const ssize_t r = pread(ix->fds[e->t.file], p + got, len - got, (off_t)(e->t.offset + at + got));
        if (r < 0 && errno == EINTR) continue;
        if (r < 0) {
            st_err(err, "%s: data read failed (%s)", e->name, strerror(errno));
            return -1;
        }
        if (r == 0) {
            st_err(err, "%s: file ended inside the tensor data", e->name);
            return -1;
        }
        got += (size_t)r;
    }
    return 0;
}

int qmoe_st_read(const qmoe_st *ix, const char *name, void *dst, size_t cap, qmoe_err *err) {
    if (err) err->msg[0] = 0;
    const st_entry *e = find_entry(ix, name);
    if (!e) {
        st_err(err, "missing tensor %s", name ? name : "(null)");
        return -1;
    }
    if (!dst || cap < e->t.nbytes) {
        st_err(err, "buffer of %zu bytes too small for %s (%llu bytes)", cap, e->name,
               (unsigned long long)e->t.nbytes);
        return -1;
    }
    return read_range(ix, e, 0, dst, (size_t)e->t.nbytes, err);
}

/* ------------------------------------------------------------ layer upload */

/* one tensor of a layer: checkpoint name suffix, slot, expected dtype and shape */
typedef struct {
    const char *suffix; /* after the layer prefix */
    int slot;           /* QH_T_* or QH_HC_* */
    int dtype;
    int ndim;
    int64_t shape[3];
    int optional_zero;  /* biases: absent means zero (model.c:250-256) */
    int dense;          /* must not have .scales (used unquantized by the reference) */
    int widen;          /* BF16 in the file, f32 in the slot (mw_load_f32, model.c:275-294) */
} st_want;

static int check_tensor(const st_entry *e, const st_want *w, qmoe_err *err) {
    if (e->t.dtype != w->dtype) {
        st_err(err, "%s must be %s (got %s)", e->name, DTYPES[w->dtype].name, DTYPES[e->t.dtype].name);
        return -1;
    }
    int ok = e->t.ndim == w->ndim;
    for (int d = 0; ok && d < w->ndim; d++) ok = e->t.shape[d] == w->shape[d];
    if (!ok) {
        char got[160] = "", want[160] = "";
        size_t gl = 0, wl = 0;
        for (int d = 0; d < e->t.ndim && gl < sizeof(got) - 24; d++)
            gl += (size_t)snprintf(got + gl, sizeof(got) - gl, "%s%lld", d ? "," : "", (long long)e->t.shape[d]);
        for (int d = 0; d < w->ndim && wl < sizeof(want) - 24; d++)
            wl += (size_t)snprintf(want + wl, sizeof(want) - wl, "%s%lld", d ? "," : "", (long long)w->shape[d]);
        st_err(err, "%s has shape [%s], the layer config needs [%s]", e->name, got, want);
        return -1;
    }
    return 0;
}

/* where a table's tensors go: the MoE layer slots or the hyper-connection slots */
typedef struct {
    int (*slot)(qmoe_ctx *c, int layer, int t, void **dst, size_t *bytes, int *on_host,
                qmoe_err *err);
    int (*begin)(qmoe_ctx *c, int layer, qmoe_err *err);
    void (*end)(qmoe_ctx *c, int layer);
    const char *dense_what; /* message for q4 weights found without scales */
    const char *quant_what; /* message for a dense tensor found quantized */
} st_target;

/* Locates and checks every tensor of `want` under `prefix` before anything
 * is copied, then copies through a pinned staging buffer, a chunk at a time. */
static int upload_table(qmoe_ctx *ctx, int layer, const qmoe_st *ix, const char *prefix,
                        const st_want *want, int nw, const st_target *tg, qmoe_err *err) {
    const st_entry *found[32];
    if (nw > 32) {
        st_err(err, "tensor table too long");
        return -1;
    }
    for (int i = 0; i < nw; i++) {
        char nm[256];
        snprintf(nm, sizeof(nm), "%s%s", prefix, want[i].suffix);
        found[i] = find_entry(ix, nm);
        if (!found[i]) {
            if (want[i].optional_zero) continue;
            /* name the departures from the reference's loader precisely */
            const size_t sl = strlen(nm);
            if (sl > 7 && !strcmp(nm + sl - 7, ".scales")) {
                char wn[256];
                snprintf(wn, sizeof(wn), "%.*s.weight", (int)(sl - 7), nm);
                if (find_entry(ix, wn)) {
                    st_err(err, "%s has no scales: %s", wn, tg->dense_what);
                    return -1;
                }
            }
            st_err(err, "missing tensor %s", nm);
            return -1;
        }
        if (want[i].dense) {
            char sn[256];
            snprintf(sn, sizeof(sn), "%s%.*s.scales", prefix, (int)(strlen(want[i].suffix) - 7),
                     want[i].suffix);
            if (find_entry(ix, sn)) {
                st_err(err, "%s is quantized: %s", found[i]->name, tg->quant_what);
                return -1;
            }
        }
        if (check_tensor(found[i], &want[i], err)) return -1;
    }

    const size_t chunk = (size_t)64 << 20;
    void *stage = NULL;
    if (qh_host_alloc(&stage, chunk, err)) return -1;
    int rc = tg->begin(ctx, layer, err);
    for (int i = 0; i < nw && rc == 0; i++) {
        void *dst;
        size_t bytes;
        int on_host = 0;
        if (tg->slot(ctx, layer, want[i].slot, &dst, &bytes, &on_host, err)) {
            rc = -1;
            break;
        }
        if (!found[i]) {
            rc = qh_fill_zero(dst, bytes, on_host, err);
            continue;
        }
        const size_t fbytes = want[i].widen ? bytes / 2 : bytes;
        if (found[i]->t.nbytes != fbytes) {
            st_err(err, "%s holds %llu bytes, the slot %zu", found[i]->name,
                   (unsigned long long)found[i]->t.nbytes, fbytes);
            rc = -1;
            break;
        }
        /* widened tensors: half a chunk of bf16 becomes a chunk of f32 */
        const size_t step = want[i].widen ? chunk / 2 : chunk;
        for (size_t at = 0; at < fbytes && rc == 0; at += step) {
            const size_t len = fbytes - at < step ? fbytes - at : step;
            if (want[i].widen) {
                uint16_t *src = (uint16_t *)((char *)stage + chunk / 2);
                rc = read_range(ix, found[i], at, src, len, err);
                float *f = (float *)stage;
                for (size_t e = 0; rc == 0 && e < len / 2; e++) {
                    const uint32_t u = (uint32_t)src[e] << 16;
                    memcpy(&f[e], &u, 4);
                }
                if (rc == 0) rc = qh_copy_to_slot((char *)dst + 2 * at, stage, 2 * len, on_host, err);
            } else {
                rc = read_range(ix, found[i], at, stage, len, err);
                if (rc == 0) rc = qh_copy_to_slot((char *)dst + at, stage, len, on_host, err);
            }
        }
    }
    qh_host_free(stage);
    if (rc == 0) tg->end(ctx, layer);
    return rc;
}

static void moe_end(qmoe_ctx *c, int layer) { qh_layer_end(c, layer, 0, 0); }

int qmoe_upload_layer_st(qmoe_ctx *ctx, int layer, const qmoe_st *ix, int model_layer, qmoe_err *err) {
    if (err) err->msg[0] = 0;
    if (!ix) {
        st_err(err, "index is NULL");
        return -1;
    }
    qmoe_config cfg;
    if (qh_ctx_config(ctx, layer, &cfg, err)) return -1;
    if (model_layer < 0) {
        st_err(err, "model layer %d is negative", model_layer);
        return -1;
    }
    const int64_t H = cfg.hidden, E = cfg.n_experts, I = cfg.moe_inter, g = cfg.group_size;
    const st_want want[] = {
        {"gate.weight", QH_T_ROUTER_W, QMOE_ST_BF16, 2, {E, H}, 0, 1, 0},
        {"switch_mlp.gate_proj.weight", QH_T_GATE_Q, QMOE_ST_U32, 3, {E, I, H / 8}, 0, 0, 0},
        {"switch_mlp.gate_proj.scales", QH_T_GATE_S, QMOE_ST_BF16, 3, {E, I, H / g}, 0, 0, 0},
        {"switch_mlp.gate_proj.biases", QH_T_GATE_B, QMOE_ST_BF16, 3, {E, I, H / g}, 1, 0, 0},
        {"switch_mlp.up_proj.weight", QH_T_UP_Q, QMOE_ST_U32, 3, {E, I, H / 8}, 0, 0, 0},
        {"switch_mlp.up_proj.scales", QH_T_UP_S, QMOE_ST_BF16, 3, {E, I, H / g}, 0, 0, 0},
        {"switch_mlp.up_proj.biases", QH_T_UP_B, QMOE_ST_BF16, 3, {E, I, H / g}, 1, 0, 0},
        {"switch_mlp.down_proj.weight", QH_T_DOWN_Q, QMOE_ST_U32, 3, {E, H, I / 8}, 0, 0, 0},
        {"switch_mlp.down_proj.scales", QH_T_DOWN_S, QMOE_ST_BF16, 3, {E, H, I / g}, 0, 0, 0},
        {"switch_mlp.down_proj.biases", QH_T_DOWN_B, QMOE_ST_BF16, 3, {E, H, I / g}, 1, 0, 0},
        {"shared_expert.gate_proj.weight", QH_T_SH_GATE_Q, QMOE_ST_U32, 2, {I, H / 8}, 0, 0, 0},
        {"shared_expert.gate_proj.scales", QH_T_SH_GATE_S, QMOE_ST_BF16, 2, {I, H / g}, 0, 0, 0},
        {"shared_expert.gate_proj.biases", QH_T_SH_GATE_B, QMOE_ST_BF16, 2, {I, H / g}, 1, 0, 0},
        {"shared_expert.up_proj.weight", QH_T_SH_UP_Q, QMOE_ST_U32, 2, {I, H / 8}, 0, 0, 0},
        {"shared_expert.up_proj.scales", QH_T_SH_UP_S, QMOE_ST_BF16, 2, {I, H / g}, 0, 0, 0},
        {"shared_expert.up_proj.biases", QH_T_SH_UP_B, QMOE_ST_BF16, 2, {I, H / g}, 1, 0, 0},
        {"shared_expert.down_proj.weight", QH_T_SH_DOWN_Q, QMOE_ST_U32, 2, {H, I / 8}, 0, 0, 0},
        {"shared_expert.down_proj.scales", QH_T_SH_DOWN_S, QMOE_ST_BF16, 2, {H, I / g}, 0, 0, 0},
        {"shared_expert.down_proj.biases", QH_T_SH_DOWN_B, QMOE_ST_BF16, 2, {H, I / g}, 1, 0, 0},
        {"shared_expert_gate.weight", QH_T_SHGATE_W, QMOE_ST_BF16, 2, {1, H}, 0, 1, 0},
    };
    const st_target tg = {qh_layer_slot, qh_layer_begin, moe_end,
                          "dense expert weights are not supported (this build runs q4 experts only)",
                          "the router and the shared-expert gate must be dense BF16 "
                          "(model.c:1301, 1396)"};
    char prefix[64];
    snprintf(prefix, sizeof(prefix), "model.layers.%d.mlp.", model_layer);
    return upload_table(ctx, layer, ix, prefix, want, (int)(sizeof(want) / sizeof(want[0])), &tg,
                        err);
}

int qmoe_hc_upload_layer_st(qmoe_ctx *ctx, int layer, const qmoe_st *ix, int model_layer,
                            qmoe_err *err) {
    if (err) err->msg[0] = 0;
    if (!ix) {
        st_err(err, "index is NULL");
        return -1;
    }
    int hc, R, d;
    if (qh_hc_config(ctx, layer, &hc, &R, &d, err)) return -1;
    if (model_layer < 0) {
        st_err(err, "model layer %d is negative", model_layer);
        return -1;
    }
    const int64_t D = (int64_t)hc * d, g = QK_GROUP;
    const st_want want[] = {
        {"hc_norm.weight", QH_HC_NORM, QMOE_ST_BF16, 1, {D}, 0, 1, 1},
        {"input_mix_weight_down.weight", QH_HC_DOWN_Q, QMOE_ST_U32, 2, {R, D / 8}, 0, 0, 0},
        {"input_mix_weight_down.scales", QH_HC_DOWN_S, QMOE_ST_BF16, 2, {R, D / g}, 0, 0, 0},
        {"input_mix_weight_down.biases", QH_HC_DOWN_B, QMOE_ST_BF16, 2, {R, D / g}, 1, 0, 0},
        {"input_mix_weight_up.weight", QH_HC_UP_Q, QMOE_ST_U32, 2, {D, R / 8}, 0, 0, 0},
        {"input_mix_weight_up.scales", QH_HC_UP_S, QMOE_ST_BF16, 2, {D, R / g}, 0, 0, 0},
        {"input_mix_weight_up.biases", QH_HC_UP_B, QMOE_ST_BF16, 2, {D, R / g}, 1, 0, 0},
        {"block_inject_weight.weight", QH_HC_INJECT_W, QMOE_ST_BF16, 2, {hc, D}, 0, 1, 0},
    };
    const st_target tg = {qh_hc_slot, qh_hc_begin, qh_hc_end,
                          "dense mix weights are not supported (this build runs q4 mix weights)",
                          "block_inject_weight must be dense BF16 (model.c:789)"};
    char prefix[96];
    snprintf(prefix, sizeof(prefix), "model.layers.%d.mlp_hyper_connection.", model_layer);
    return upload_table(ctx, layer, ix, prefix, want, (int)(sizeof(want) / sizeof(want[0])), &tg,
                        err);
}
