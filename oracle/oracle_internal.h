/* oracle_internal.h — shared internals of the oracle (test infrastructure only). */
#ifndef RIE_ORACLE_INTERNAL_H
#define RIE_ORACLE_INTERNAL_H

#include "oracle.h"

typedef struct {
    const char *key;
    size_t key_len;
    uint32_t type;
    uint64_t u;
    int64_t i;
    double f;
    const char *str;
    size_t str_len;
    size_t arr_len;
    uint32_t arr_type;
} or_kv;

typedef struct {
    char name[96];
    uint32_t n_dims;
    uint64_t dims[4];
    int type;
    uint64_t offset, size;
    uint64_t rows, cols;
    const uint8_t *data;
} or_tensor;

typedef struct {
    or_kv *kv;
    size_t n_kv;
    or_tensor *tensors;
    size_t n_tensors;
    uint64_t data_start;
} or_gguf;

int or_gguf_parse(const uint8_t *p, size_t len, or_gguf *g, char *err, size_t err_len);
void or_gguf_free(or_gguf *g);
const or_kv *or_gguf_get(const or_gguf *g, const char *key);
const or_tensor *or_gguf_tensor(const or_gguf *g, const char *name);

/* parallel for: f(i, tid, ctx) for i in [0, n) with dynamic chunks of `grain` */
typedef void (*or_task_fn)(size_t i, int tid, void *ctx);
typedef struct or_pool or_pool;
or_pool *or_pool_new(int n_threads);
void or_pool_free(or_pool *p);
int or_pool_threads(const or_pool *p);
void or_pool_for(or_pool *p, size_t n, size_t grain, or_task_fn f, void *ctx);

#endif
