/*
 * pool.c — fork/join worker pool with dynamic chunk hand-out, the scheduling
 * model of threadpool.rs:97-160 (spin, then sleep).  Every output element is
 * produced by exactly one task, so results do not depend on the thread count.
 * TEST INFRASTRUCTURE ONLY (the oracle); see oracle.h.
 */
#include "oracle_internal.h"

#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>

struct or_pool {
    int n;
    pthread_t *th;
    pthread_mutex_t mu;
    pthread_cond_t cv;
    atomic_ulong epoch;
    atomic_int pending;
    atomic_int quit;
    /* current job */
    or_task_fn f;
    void *ctx;
    size_t total, grain;
    atomic_size_t next;
};

typedef struct {
    or_pool *p;
    int tid;
} worker_arg;

static void run_chunks(or_pool *p, int tid) {
    for (;;) {
        size_t s = atomic_fetch_add(&p->next, p->grain);
        if (s >= p->total) break;
        size_t e = s + p->grain < p->total ? s + p->grain : p->total;
        for (size_t i = s; i < e; i++) p->f(i, tid, p->ctx);
    }
}

static void *worker(void *a) {
    worker_arg *wa = (worker_arg *)a;
    or_pool *p = wa->p;
    int tid = wa->tid;
    free(wa);
    unsigned long seen = 0;
    for (;;) {
        unsigned long e;
        int spins = 0;
        while ((e = atomic_load(&p->epoch)) == seen && !atomic_load(&p->quit)) {
            if (++spins > 20000) {
                pthread_mutex_lock(&p->mu);
                while (atomic_load(&p->epoch) == seen && !atomic_load(&p->quit)) pthread_cond_wait(&p->cv, &p->mu);
                pthread_mutex_unlock(&p->mu);
                spins = 0;
            }
        }
        if (atomic_load(&p->quit)) return NULL;
        seen = e;
        run_chunks(p, tid);
        atomic_fetch_sub(&p->pending, 1);
    }
}

or_pool *or_pool_new(int n) {
    or_pool *p = (or_pool *)calloc(1, sizeof(or_pool));
    p->n = n < 1 ? 1 : n;
    pthread_mutex_init(&p->mu, NULL);
    pthread_cond_init(&p->cv, NULL);
    p->th = (pthread_t *)calloc((size_t)p->n, sizeof(pthread_t));
    for (int i = 1; i < p->n; i++) {
        worker_arg *a = (worker_arg *)malloc(sizeof(worker_arg));
        a->p = p;
        a->tid = i;
        pthread_create(&p->th[i], NULL, worker, a);
    }
    return p;
}

void or_pool_free(or_pool *p) {
    if (!p) return;
    atomic_store(&p->quit, 1);
    pthread_mutex_lock(&p->mu);
    pthread_cond_broadcast(&p->cv);
    pthread_mutex_unlock(&p->mu);
    for (int i = 1; i < p->n; i++) pthread_join(p->th[i], NULL);
    free(p->th);
    free(p);
}

int or_pool_threads(const or_pool *p) { return p->n; }

void or_pool_for(or_pool *p, size_t n, size_t grain, or_task_fn f, void *ctx) {
    if (grain < 1) grain = 1;
    if (n == 0) return;
    if (p->n == 1 || n <= grain) {
        for (size_t i = 0; i < n; i++) f(i, 0, ctx);
        return;
    }
    p->f = f;
    p->ctx = ctx;
    p->total = n;
    p->grain = grain;
    atomic_store(&p->next, 0);
    atomic_store(&p->pending, p->n - 1);
    pthread_mutex_lock(&p->mu);
    atomic_fetch_add(&p->epoch, 1);
    pthread_cond_broadcast(&p->cv);
    pthread_mutex_unlock(&p->mu);
    run_chunks(p, 0);
    while (atomic_load(&p->pending) != 0) {
    }
}
