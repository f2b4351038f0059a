/*
 * si_kvpages.c -- paged KV bookkeeping and a multi-layer decode stack over
 * the MI355X C ABI.  Neither exists in the reference, which runs one layer
 * with one contiguous cache (qwen_one_layer.c:237-281); this is the next
 * step after a single layer: many sequences of unequal, growing length
 * decoding together through a stack of layers, each layer's K/V in its own
 * page pool, one page table shared by all layers (every layer holds the
 * same positions of a sequence).
 */
#define _GNU_SOURCE
#include "si_host.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

static void die(const char *message) {
    fprintf(stderr, "error: %s\n", message);
    exit(1);
}

static void check(int rc, const char *what) {
    if (rc != SI_OK) {
        fprintf(stderr, "error: %s: %s\n", what, si_last_error());
        exit(1);
    }
}

static void hip_check(hipError_t e, const char *what) {
    if (e != hipSuccess) {
        fprintf(stderr, "error: %s: %s\n", what, hipGetErrorString(e));
        exit(1);
    }
}

/* ------------------------------------------------------------------ */
/* page bookkeeping                                                    */
/* ------------------------------------------------------------------ */

struct si_kv_pages {
    int npages, page_size, max_seqs, max_pages;
    int *free_list; /* stack of free page ids */
    int nfree;
    int *table;     /* [max_seqs][max_pages] page ids (unused entries 0) */
    int *npg;       /* pages held per sequence, -1 = sequence slot unused */
    int *len;       /* positions per sequence */
};

si_kv_pages_t *si_kv_pages_create(int npages, int page_size, int max_seqs, int max_pages) {
    if (npages < 1 || page_size < 1 || (page_size & (page_size - 1)) || max_seqs < 1 ||
        max_pages < 1)
        die("si_kv_pages_create: bad sizes (page_size must be a power of two)");
    si_kv_pages_t *p = calloc(1, sizeof *p);
    if (!p) die("Out of memory");
    p->npages = npages;
    p->page_size = page_size;
    p->max_seqs = max_seqs;
    p->max_pages = max_pages;
    p->free_list = malloc(sizeof(int) * (size_t)npages);
    p->table = calloc((size_t)max_seqs * max_pages, sizeof(int));
    p->npg = malloc(sizeof(int) * (size_t)max_seqs);
    p->len = calloc((size_t)max_seqs, sizeof(int));
    if (!p->free_list || !p->table || !p->npg || !p->len) die("Out of memory");
    /* lowest ids on top of the stack: a fresh pool hands out 0, 1, 2, ... */
    for (int i = 0; i < npages; ++i) p->free_list[i] = npages - 1 - i;
    p->nfree = npages;
    for (int i = 0; i < max_seqs; ++i) p->npg[i] = -1;
    return p;
}

void si_kv_pages_destroy(si_kv_pages_t *p) {
    if (!p) return;
    free(p->free_list);
    free(p->table);
    free(p->npg);
    free(p->len);
    free(p);
}

static void check_seq(const si_kv_pages_t *p, int seq) {
    if (seq < 0 || seq >= p->max_seqs || p->npg[seq] < 0) die("si_kv_pages: unknown sequence");
}

int si_kv_seq_add(si_kv_pages_t *p) {
    for (int i = 0; i < p->max_seqs; ++i)
        if (p->npg[i] < 0) {
            p->npg[i] = 0;
            p->len[i] = 0;
            return i;
        }
    return -1;
}

int si_kv_seq_grow(si_kv_pages_t *p, int seq, int len) {
    check_seq(p, seq);
    if (len < p->len[seq]) die("si_kv_seq_grow: sequences only grow");
    const long long need = ((long long)len + p->page_size - 1) / p->page_size;
    if (need > p->max_pages || need - p->npg[seq] > p->nfree) return -1; /* nothing taken */
    int *row = p->table + (size_t)seq * p->max_pages;
    while (p->npg[seq] < need) row[p->npg[seq]++] = p->free_list[--p->nfree];
    p->len[seq] = len;
    return 0;
}

void si_kv_seq_free(si_kv_pages_t *p, int seq) {
    check_seq(p, seq);
    int *row = p->table + (size_t)seq * p->max_pages;
    /* returned in reverse order, so the next sequence reuses them in order */
    for (int i = p->npg[seq] - 1; i >= 0; --i) {
        p->free_list[p->nfree++] = row[i];
        row[i] = 0;
    }
    p->npg[seq] = -1;
    p->len[seq] = 0;
}

int si_kv_seq_len(const si_kv_pages_t *p, int seq) {
    check_seq(p, seq);
    return p->len[seq];
}

int si_kv_pages_free(const si_kv_pages_t *p) { return p->nfree; }

const int *si_kv_page_table(const si_kv_pages_t *p) { return p->table; }

/* ------------------------------------------------------------------ */
/* multi-layer decode stack                                            */
/* ------------------------------------------------------------------ */

struct si_stack {
    si_shape_t shape;
    int nlayers, max_seqs, max_ctx, page_size, npages;
    si_workspace_t *ws;
    si_layer_t **layers;
    uint16_t **kpool, **vpool;
    si_kv_pages_t *pages;
    int *dev_table; /* [max_seqs][max_pages], batch order of the last prepare */
    int *dev_ctx;   /* [max_seqs] */
    int *host_table, *host_ctx;
    float *act[2];  /* ping-pong activations between layers */
    int nseq;       /* rows of the last prepare */
    void *stream;   /* stream of the last si_stack_decode */
    int pending;    /* a decode was enqueued since the last prepare */
};

si_stack_t *si_stack_create(const si_shape_t *s, const si_layer_host_t *layers, int nlayers,
                            int max_seqs, int max_ctx, int npages, int page_size) {
    if (nlayers < 1 || max_seqs < 1 || max_ctx < 1) die("si_stack_create: bad sizes");
    si_stack_t *st = calloc(1, sizeof *st);
    if (!st) die("Out of memory");
    st->shape = *s;
    st->nlayers = nlayers;
    st->max_seqs = max_seqs;
    st->max_ctx = max_ctx;
    st->page_size = page_size;
    st->npages = npages;
    const int max_pages = (max_ctx + page_size - 1) / page_size;
    st->pages = si_kv_pages_create(npages, page_size, max_seqs, max_pages);
    check(si_workspace_create(s, max_seqs, max_ctx, &st->ws), "si_workspace_create");
    st->layers = calloc((size_t)nlayers, sizeof *st->layers);
    st->kpool = calloc((size_t)nlayers, sizeof *st->kpool);
    st->vpool = calloc((size_t)nlayers, sizeof *st->vpool);
    if (!st->layers || !st->kpool || !st->vpool) die("Out of memory");
    const size_t pool = (size_t)npages * page_size * s->kvheads * s->hdim * sizeof(uint16_t);
    for (int l = 0; l < nlayers; ++l) {
        check(si_layer_create_in(st->ws, &layers[l], &st->layers[l]), "si_layer_create_in");
        hip_check(hipMalloc((void **)&st->kpool[l], pool), "hipMalloc(K pool)");
        hip_check(hipMalloc((void **)&st->vpool[l], pool), "hipMalloc(V pool)");
    }
    hip_check(hipMalloc((void **)&st->dev_table, sizeof(int) * (size_t)max_seqs * max_pages),
              "hipMalloc(page table)");
    hip_check(hipMalloc((void **)&st->dev_ctx, sizeof(int) * (size_t)max_seqs), "hipMalloc");
    const size_t act = sizeof(float) * (size_t)max_seqs * s->hidden;
    hip_check(hipMalloc((void **)&st->act[0], act), "hipMalloc(activations)");
    hip_check(hipMalloc((void **)&st->act[1], act), "hipMalloc(activations)");
    st->host_table = calloc((size_t)max_seqs * max_pages, sizeof(int));
    st->host_ctx = calloc((size_t)max_seqs, sizeof(int));
    if (!st->host_table || !st->host_ctx) die("Out of memory");
    return st;
}

void si_stack_destroy(si_stack_t *st) {
    if (!st) return;
    for (int l = 0; l < st->nlayers; ++l) {
        si_layer_destroy(st->layers[l]);
        (void)hipFree(st->kpool[l]);
        (void)hipFree(st->vpool[l]);
    }
    si_workspace_destroy(st->ws);
    (void)hipFree(st->dev_table);
    (void)hipFree(st->dev_ctx);
    (void)hipFree(st->act[0]);
    (void)hipFree(st->act[1]);
    si_kv_pages_destroy(st->pages);
    free(st->layers);
    free(st->kpool);
    free(st->vpool);
    free(st->host_table);
    free(st->host_ctx);
    free(st);
}

si_kv_pages_t *si_stack_pages(si_stack_t *st) { return st->pages; }
uint16_t *si_stack_k_pool(si_stack_t *st, int layer) { return st->kpool[layer]; }
uint16_t *si_stack_v_pool(si_stack_t *st, int layer) { return st->vpool[layer]; }
si_layer_t *si_stack_layer(si_stack_t *st, int layer) { return st->layers[layer]; }
const int *si_stack_dev_table(const si_stack_t *st) { return st->dev_table; }
const int *si_stack_dev_ctx(const si_stack_t *st) { return st->dev_ctx; }
int si_stack_nseq(const si_stack_t *st) { return st->nseq; }

int si_stack_prepare(si_stack_t *st, const int *seqs, int nseq) {
    if (nseq < 1 || nseq > st->max_seqs) die("si_stack_prepare: nseq outside 1..max_seqs");
    /* the previous step's kernels read the device table and contexts this
     * call rewrites: wait for them */
    if (st->pending)
        hip_check(hipStreamSynchronize((hipStream_t)st->stream), "si_stack_prepare: wait");
    st->pending = 0;
    for (int i = 0; i < nseq; ++i)
        for (int j = 0; j < i; ++j)
            if (seqs[i] == seqs[j]) die("si_stack_prepare: a sequence appears twice");
    si_kv_pages_t *p = st->pages;
    for (int i = 0; i < nseq; ++i) {
        const int len = si_kv_seq_len(p, seqs[i]) + 1;
        if (len > st->max_ctx) die("si_stack_prepare: a sequence exceeds max_ctx");
        if (si_kv_seq_grow(p, seqs[i], len) != 0) {
            /* roll back this call's growth so the caller can preempt; the
             * device table and contexts still describe the previous step, so
             * no decode may run until a prepare succeeds */
            for (int j = 0; j < i; ++j) p->len[seqs[j]] -= 1;
            st->nseq = 0;
            return -1;
        }
    }
    for (int i = 0; i < nseq; ++i) {
        memcpy(st->host_table + (size_t)i * p->max_pages,
               p->table + (size_t)seqs[i] * p->max_pages, sizeof(int) * (size_t)p->max_pages);
        st->host_ctx[i] = p->len[seqs[i]];
    }
    hip_check(hipMemcpy(st->dev_table, st->host_table, sizeof(int) * (size_t)nseq * p->max_pages,
                        hipMemcpyHostToDevice), "upload page table");
    hip_check(hipMemcpy(st->dev_ctx, st->host_ctx, sizeof(int) * (size_t)nseq,
                        hipMemcpyHostToDevice), "upload contexts");
    st->nseq = nseq;
    return 0;
}

void si_stack_decode(si_stack_t *st, const float *x, float *out, int flags, void *stream) {
    if (st->nseq < 1) die("si_stack_decode: no si_stack_prepare call");
    int max_ctx = 1;
    for (int i = 0; i < st->nseq; ++i)
        if (st->host_ctx[i] > max_ctx) max_ctx = st->host_ctx[i];
    const float *in = x;
    for (int l = 0; l < st->nlayers; ++l) {
        float *o = l == st->nlayers - 1 ? out : st->act[l & 1];
        check(si_layer_decode_paged(st->layers[l], in, st->nseq, st->kpool[l], st->vpool[l],
                                    st->npages, st->page_size, st->dev_table,
                                    st->pages->max_pages, st->dev_ctx, max_ctx, max_ctx, o, flags,
                                    stream),
              "si_layer_decode_paged");
        in = o;
    }
    st->stream = stream;
    st->pending = 1;
}
