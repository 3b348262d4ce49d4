/*
 * qmoe_cache.c -- residency of routed experts in HBM expert slots when the
 * experts of a model do not all fit (host-pinned backing store, one slot
 * pool per layer).
 *
 * The policy restates the reference C port's expert cache (c/src/cache.c:
 * cache_get 187-204, cache_put 216-259, pick_victim 99-163), with two
 * departures that follow from slots instead of malloc'd values:
 *   - every entry has the same size (one expert), and a partition (layer)
 *     owns a fixed number of slots, so an insert evicts inside its own
 *     partition only -- the state the reference's partition fairness
 *     (cache.c:103-122, partitions = layers, model.c:1806) steers to once
 *     every layer is over its share;
 *   - recency is a logical clock (each get or put is one tick) instead of
 *     CLOCK_MONOTONIC nanoseconds, so two entries never tie on "touched".
 * Victim choice, as pick_victim: entries are visited from least to most
 * recently used, pinned ones skipped; a cold entry replaces a hot best
 * (and resets the best score to 0), a hot one never replaces a cold best;
 * otherwise LRU takes the oldest, LFU the lowest frequency, ADAPTIVE the
 * lowest (freq + 4*hot) / nbytes, ties to the older entry.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "qmoe_internal.h"

typedef struct {
    int item;   /* -1: free */
    int pinned, hot;
    uint64_t freq, touched;
    int prev, next; /* recency list of the partition (local slot indices) */
} xc_entry;

struct qmoe_xcache {
    int parts, items, slots, policy;
    uint64_t nbytes;
    int32_t *where; /* [parts * items] -> local slot or -1 */
    xc_entry *ent;  /* [parts * slots] */
    int *head, *tail, *nfree;
    uint64_t clock;
    uint64_t hits, misses, evictions, rejected;
};

static xc_entry *ent_of(qmoe_xcache *c, int part, int s) { return &c->ent[(size_t)part * c->slots + s]; }

static void unlink_slot(qmoe_xcache *c, int part, int s) {
    xc_entry *e = ent_of(c, part, s);
    if (e->prev >= 0) ent_of(c, part, e->prev)->next = e->next;
    else c->head[part] = e->next;
    if (e->next >= 0) ent_of(c, part, e->next)->prev = e->prev;
    else c->tail[part] = e->prev;
    e->prev = e->next = -1;
}

static void link_front(qmoe_xcache *c, int part, int s) {
    xc_entry *e = ent_of(c, part, s);
    e->prev = -1;
    e->next = c->head[part];
    if (c->head[part] >= 0) ent_of(c, part, c->head[part])->prev = s;
    c->head[part] = s;
    if (c->tail[part] < 0) c->tail[part] = s;
}

int qmoe_xcache_create(qmoe_xcache **out, int parts, int items, int slots, int policy,
                       uint64_t entry_bytes, qmoe_err *err) {
    if (!out || parts <= 0 || items <= 0 || slots <= 0 || slots > items || policy < 0 ||
        policy > QMOE_CACHE_ADAPTIVE || entry_bytes == 0) {
        if (err) snprintf(err->msg, sizeof(err->msg), "bad cache shape (parts %d, items %d, slots %d, policy %d)",
                          parts, items, slots, policy);
        return -1;
    }
    qmoe_xcache *c = (qmoe_xcache *)calloc(1, sizeof(qmoe_xcache));
    if (!c) goto oom;
    c->parts = parts;
    c->items = items;
    c->slots = slots;
    c->policy = policy;
    c->nbytes = entry_bytes;
    c->where = (int32_t *)malloc((size_t)parts * items * sizeof(int32_t));
    c->ent = (xc_entry *)calloc((size_t)parts * slots, sizeof(xc_entry));
    c->head = (int *)malloc((size_t)parts * sizeof(int));
    c->tail = (int *)malloc((size_t)parts * sizeof(int));
    c->nfree = (int *)malloc((size_t)parts * sizeof(int));
    if (!c->where || !c->ent || !c->head || !c->tail || !c->nfree) {
        qmoe_xcache_destroy(c);
        goto oom;
    }
    for (size_t i = 0; i < (size_t)parts * items; i++) c->where[i] = -1;
    for (size_t i = 0; i < (size_t)parts * slots; i++) {
        c->ent[i].item = -1;
        c->ent[i].prev = c->ent[i].next = -1;
    }
    for (int p = 0; p < parts; p++) {
        c->head[p] = c->tail[p] = -1;
        c->nfree[p] = slots;
    }
    *out = c;
    return 0;
oom:
    if (err) snprintf(err->msg, sizeof(err->msg), "out of host memory");
    return -1;
}

void qmoe_xcache_destroy(qmoe_xcache *c) {
    if (!c) return;
    free(c->where);
    free(c->ent);
    free(c->head);
    free(c->tail);
    free(c->nfree);
    free(c);
}

static int valid(const qmoe_xcache *c, int part, int item) {
    return c && part >= 0 && part < c->parts && item >= 0 && item < c->items;
}

int qmoe_xcache_peek(qmoe_xcache *c, int part, int item) {
    return valid(c, part, item) ? c->where[(size_t)part * c->items + item] : -1;
}

/* cache_get (cache.c:187-204): a hit counts, bumps freq and recency */
int qmoe_xcache_get(qmoe_xcache *c, int part, int item) {
    if (!valid(c, part, item)) return -1;
    const int s = c->where[(size_t)part * c->items + item];
    if (s < 0) {
        c->misses++;
        return -1;
    }
    xc_entry *e = ent_of(c, part, s);
    e->freq++;
    e->touched = ++c->clock;
    unlink_slot(c, part, s);
    link_front(c, part, s);
    c->hits++;
    return s;
}

/* pick_victim (cache.c:99-163) over one partition */
static int pick_victim(qmoe_xcache *c, int part) {
    int best = -1;
    double best_score = 0.0;
    uint64_t best_touched = 0;
    for (int s = c->tail[part]; s >= 0; s = ent_of(c, part, s)->prev) {
        const xc_entry *e = ent_of(c, part, s);
        if (e->pinned) continue;
        const xc_entry *b = best >= 0 ? ent_of(c, part, best) : NULL;
        if (b && !e->hot && b->hot) {
            best = s;
            best_score = 0.0;
            best_touched = e->touched;
            continue;
        }
        if (b && e->hot && !b->hot) continue;
        double score;
        if (c->policy == QMOE_CACHE_LRU) score = 0.0;
        else if (c->policy == QMOE_CACHE_LFU) score = (double)e->freq;
        else score = (double)(e->freq + (e->hot ? 4 : 0)) / (double)c->nbytes;
        int better;
        if (!b) better = 1;
        else if (c->policy == QMOE_CACHE_LRU) better = e->touched < best_touched;
        else better = score < best_score || (score == best_score && e->touched < best_touched);
        if (better) {
            best = s;
            best_score = score;
            best_touched = e->touched;
        }
    }
    return best;
}

/* cache_put (cache.c:216-259) for an item that is not resident: a free
 * slot if there is one, else the victim's.  Returns the slot, or -1 when
 * every slot is pinned (counted as rejected); *evicted = the evicted item
 * or -1. */
int qmoe_xcache_put(qmoe_xcache *c, int part, int item, int pin, int hot, int *evicted) {
    if (evicted) *evicted = -1;
    if (!valid(c, part, item)) return -1;
    int32_t *w = &c->where[(size_t)part * c->items + item];
    if (*w >= 0) { /* already resident: replace keeps pin/hot as cache_put does */
        xc_entry *e = ent_of(c, part, *w);
        e->pinned = pin || e->pinned;
        e->hot = hot || e->hot;
        e->freq = 1;
        e->touched = ++c->clock;
        unlink_slot(c, part, *w);
        link_front(c, part, *w);
        return *w;
    }
    int s = -1;
    if (c->nfree[part] > 0) {
        for (int i = 0; i < c->slots; i++)
            if (ent_of(c, part, i)->item < 0) {
                s = i;
                break;
            }
        c->nfree[part]--;
    } else {
        s = pick_victim(c, part);
        if (s < 0) {
            c->rejected++;
            return -1;
        }
        xc_entry *v = ent_of(c, part, s);
        if (evicted) *evicted = v->item;
        c->where[(size_t)part * c->items + v->item] = -1;
        unlink_slot(c, part, s);
        c->evictions++;
    }
    xc_entry *e = ent_of(c, part, s);
    e->item = item;
    e->pinned = pin;
    e->hot = hot;
    e->freq = 1;
    e->touched = ++c->clock;
    link_front(c, part, s);
    *w = s;
    return s;
}

int qmoe_xcache_pin(qmoe_xcache *c, int part, int item, int pinned) {
    const int s = qmoe_xcache_peek(c, part, item);
    if (s < 0) return 0;
    xc_entry *e = ent_of(c, part, s);
    const int changed = (e->pinned != 0) != (pinned != 0);
    e->pinned = pinned != 0;
    return changed;
}

int qmoe_xcache_mark_hot(qmoe_xcache *c, int part, int item, int hot) {
    const int s = qmoe_xcache_peek(c, part, item);
    if (s < 0) return 0;
    ent_of(c, part, s)->hot = hot != 0;
    return 1;
}

/* forget every entry of a partition (its weights were replaced) */
void qmoe_xcache_clear(qmoe_xcache *c, int part) {
    if (!c || part < 0 || part >= c->parts) return;
    for (int i = 0; i < c->items; i++) c->where[(size_t)part * c->items + i] = -1;
    for (int s = 0; s < c->slots; s++) {
        xc_entry *e = ent_of(c, part, s);
        memset(e, 0, sizeof(*e));
        e->item = -1;
        e->prev = e->next = -1;
    }
    c->head[part] = c->tail[part] = -1;
    c->nfree[part] = c->slots;
}

void qmoe_xcache_counts(const qmoe_xcache *c, uint64_t out[4]) {
    out[0] = c ? c->hits : 0;
    out[1] = c ? c->misses : 0;
    out[2] = c ? c->evictions : 0;
    out[3] = c ? c->rejected : 0;
}
