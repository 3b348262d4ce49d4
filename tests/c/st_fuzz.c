/*
 * st_fuzz.c -- host-only driver of the checkpoint index (qmoe_st.c) and the
 * expert slot cache (qmoe_cache.c) for the sanitizer run
 * (tests/test_sanitize.py builds it with -fsanitize=address,undefined).
 *
 *   st_fuzz DIR...            open each directory's *.safetensors index; for
 *                             an index that opens, look up and read every
 *                             tensor (and once into too small a buffer);
 *                             one line per directory: "ok N" or "refused MSG"
 *   st_fuzz --cache SEED OPS  random sequences of cache operations over
 *                             several shapes and the three policies, with
 *                             the invariants the cache keeps checked
 *
 * The layer upload functions of qmoe_st.c reach the library's context
 * through the qh_* helpers; this driver never calls them, so the helpers
 * are defined here to abort.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "qmoe.h"
#include "qmoe_internal.h"

static void never(const char *what) {
    fprintf(stderr, "st_fuzz: %s called\n", what);
    abort();
}
int qh_ctx_config(qmoe_ctx *c, int layer, qmoe_config *out, qmoe_err *err) { never("qh_ctx_config"); return -1; }
int qh_host_alloc(void **p, size_t bytes, qmoe_err *err) { never("qh_host_alloc"); return -1; }
void qh_host_free(void *p) { never("qh_host_free"); }
int qh_layer_begin(qmoe_ctx *c, int layer, qmoe_err *err) { never("qh_layer_begin"); return -1; }
int qh_layer_slot(qmoe_ctx *c, int layer, int t, void **dst, size_t *bytes, int *on_host, qmoe_err *err) {
    never("qh_layer_slot");
    return -1;
}
int qh_fill_zero(void *dst, size_t bytes, int on_host, qmoe_err *err) { never("qh_fill_zero"); return -1; }
int qh_copy_to_slot(void *dst, const void *src, size_t bytes, int on_host, qmoe_err *err) {
    never("qh_copy_to_slot");
    return -1;
}
void qh_layer_end(qmoe_ctx *c, int layer, int has_bias, int has_norm) { never("qh_layer_end"); }
int qh_hc_config(qmoe_ctx *c, int layer, int *hc, int *lowrank, int *d, qmoe_err *err) {
    never("qh_hc_config");
    return -1;
}
int qh_hc_slot(qmoe_ctx *c, int layer, int t, void **dst, size_t *bytes, int *on_host, qmoe_err *err) {
    never("qh_hc_slot");
    return -1;
}
int qh_hc_begin(qmoe_ctx *c, int layer, qmoe_err *err) { never("qh_hc_begin"); return -1; }
void qh_hc_end(qmoe_ctx *c, int layer) { never("qh_hc_end"); }

static int open_dir(const char *dir) {
    qmoe_err err;
    qmoe_st *ix = NULL;
    if (qmoe_st_open(&ix, dir, &err)) {
        err.msg[sizeof(err.msg) - 1] = 0;
        for (char *m = err.msg; *m; m++) /* names from the file may hold any bytes */
            if ((unsigned char)*m < 0x20 || (unsigned char)*m >= 0x7f) *m = '?';
        printf("refused %s\n", err.msg);
        return 0;
    }
    const size_t n = qmoe_st_count(ix);
    for (size_t i = 0; i < n; i++) {
        const char *name = qmoe_st_name(ix, i);
        qmoe_st_tensor t;
        if (!name || !qmoe_st_find(ix, name, &t)) {
            fprintf(stderr, "indexed name %zu not found\n", i);
            return 1;
        }
        if (t.dtype < 0 || t.ndim < 0 || t.ndim > 8 || !qmoe_st_dtype_name(t.dtype)) {
            fprintf(stderr, "bad entry for %s\n", name);
            return 1;
        }
        unsigned char *buf = (unsigned char *)malloc(t.nbytes + 1);
        if (!buf) return 1;
        if (qmoe_st_read(ix, name, buf, (size_t)t.nbytes, &err)) {
            fprintf(stderr, "read of %s failed: %s\n", name, err.msg);
            free(buf);
            return 1;
        }
        if (t.nbytes > 0 && qmoe_st_read(ix, name, buf, (size_t)t.nbytes - 1, &err) == 0) {
            fprintf(stderr, "read of %s into a short buffer succeeded\n", name);
            free(buf);
            return 1;
        }
        free(buf);
    }
    qmoe_st_tensor t;
    if (qmoe_st_find(ix, "no.such.tensor", &t) || qmoe_st_name(ix, n) != NULL) return 1;
    qmoe_st_close(ix);
    printf("ok %zu\n", n);
    return 0;
}

static uint64_t rng_state;
static uint32_t rnd(uint32_t m) {
    rng_state = rng_state * 6364136223846793005ull + 1442695040888963407ull;
    return (uint32_t)(rng_state >> 33) % m;
}

static int cache_run(uint64_t seed, int ops) {
    rng_state = seed;
    static const int shapes[][3] = {{1, 8, 3}, {4, 64, 16}, {2, 512, 64}, {3, 5, 5}, {1, 300, 1}};
    for (size_t sh = 0; sh < sizeof(shapes) / sizeof(shapes[0]); sh++)
        for (int policy = 0; policy < 3; policy++) {
            const int parts = shapes[sh][0], items = shapes[sh][1], slots = shapes[sh][2];
            qmoe_xcache *c = NULL;
            qmoe_err err;
            if (qmoe_xcache_create(&c, parts, items, slots, policy, 1u << 20, &err)) {
                fprintf(stderr, "create failed: %s\n", err.msg);
                return 1;
            }
            int *pinned = (int *)calloc((size_t)parts * items, sizeof(int));
            for (int op = 0; op < ops; op++) {
                const int part = (int)rnd((uint32_t)parts + 1) - (rnd(50) == 0 ? 1 : 0);
                const int item = (int)rnd((uint32_t)items + 2) - 1;
                const int ok = part >= 0 && part < parts && item >= 0 && item < items;
                int ev = -1, r = -1, bad = 0;
                switch (rnd(7)) {
                case 0: r = qmoe_xcache_peek(c, part, item); break;
                case 1:
                case 2: r = qmoe_xcache_get(c, part, item); break;
                case 3: {
                    const int pin = rnd(8) == 0;
                    r = qmoe_xcache_put(c, part, item, pin, (int)rnd(2), &ev);
                    if (ok && ev >= 0 && (ev >= items || pinned[part * items + ev])) bad = 1;
                    if (ok && r >= 0 && pin) pinned[part * items + item] = 1;
                    break;
                }
                case 4:
                    qmoe_xcache_pin(c, part, item, 0);
                    if (ok) pinned[part * items + item] = 0;
                    break;
                case 5: qmoe_xcache_mark_hot(c, part, item, (int)rnd(2)); break;
                default:
                    if (rnd(20) == 0 && part >= 0 && part < parts) {
                        qmoe_xcache_clear(c, part);
                        memset(pinned + (size_t)part * items, 0, (size_t)items * sizeof(int));
                    }
                    break;
                }
                /* peek, get and put return a slot of the partition or -1 */
                if (r >= slots || r < -1 || (!ok && r != -1) || bad) {
                    fprintf(stderr, "shape %zu policy %d op %d: result %d (slots %d), evicted %d\n", sh,
                            policy, op, r, slots, ev);
                    free(pinned);
                    qmoe_xcache_destroy(c);
                    return 1;
                }
            }
            uint64_t cnt[4];
            qmoe_xcache_counts(c, cnt);
            free(pinned);
            qmoe_xcache_destroy(c);
        }
    printf("cache ok\n");
    return 0;
}

int main(int argc, char **argv) {
    if (argc == 4 && strcmp(argv[1], "--cache") == 0)
        return cache_run(strtoull(argv[2], NULL, 10), atoi(argv[3]));
    int rc = 0;
    for (int i = 1; i < argc; i++) rc |= open_dir(argv[i]);
    return rc;
}
