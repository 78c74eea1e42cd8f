/* paged_kv.c -- TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Restates BlockPool and PagedAttentionManager:
 *   include/core/page_attention.h:9-90, src/core/page_attention.cpp:25-216.
 * The manager's std::map<layer_id, LayerState> is a growable array keyed by
 * layer id with "created on first access" semantics, like operator[].
 */
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

struct or_block_pool {
    int32_t head_dim, n_kv_heads;
    int32_t num_blocks;     /* high-water mark of ids handed out */
    int32_t block_capacity; /* 0 = unbounded (page_attention.cpp:43) */
    size_t elem_size, block_bytes, buffer_bytes;
    uint8_t *buffer;
    int32_t *free_list;
    int32_t free_len, free_cap;
};

static void pool_init(or_block_pool *p, void *buffer, size_t buffer_bytes, int32_t capacity,
                      int32_t n_kv_heads, int32_t head_dim, size_t elem_size) {
    memset(p, 0, sizeof *p);
    p->block_capacity = capacity;
    p->n_kv_heads = n_kv_heads;
    p->head_dim = head_dim;
    p->elem_size = elem_size;
    p->buffer = (uint8_t *)buffer;
    p->buffer_bytes = buffer_bytes;
    /* page_attention.cpp:33 */
    p->block_bytes = (size_t)OR_PAGE_BLOCK_SIZE * (size_t)n_kv_heads * (size_t)head_dim * elem_size;
}

static void pool_push(or_block_pool *p, int32_t id) {
    if (p->free_len == p->free_cap) {
        p->free_cap = p->free_cap ? 2 * p->free_cap : 64;
        p->free_list = (int32_t *)realloc(p->free_list, (size_t)p->free_cap * sizeof(int32_t));
    }
    p->free_list[p->free_len++] = id;
}

or_block_pool *or_pool_create(void *buffer, size_t buffer_bytes, int32_t block_capacity,
                              int32_t n_kv_heads, int32_t head_dim, size_t elem_size) {
    or_block_pool *p = (or_block_pool *)malloc(sizeof *p);
    pool_init(p, buffer, buffer_bytes, block_capacity, n_kv_heads, head_dim, elem_size);
    return p;
}

void or_pool_destroy(or_block_pool *p) {
    if (!p) return;
    free(p->free_list);
    free(p);
}

/* BlockPool::alloc -- page_attention.cpp:37-46: pop the free-list back,
 * else hand out num_blocks++, else -1 at capacity. */
int32_t or_pool_alloc(or_block_pool *p) {
    if (p->free_len > 0) return p->free_list[--p->free_len];
    if (p->block_capacity > 0 && p->num_blocks >= p->block_capacity) return -1;
    return p->num_blocks++;
}

/* BlockPool::free -- :48-51: push back any id below the high-water mark */
void or_pool_free(or_block_pool *p, int32_t id) {
    if (id >= 0 && id < p->num_blocks) pool_push(p, id);
}

/* BlockPool::reset -- :53-57: free list = [0 .. num_blocks) */
void or_pool_reset(or_block_pool *p) {
    p->free_len = 0;
    for (int32_t i = 0; i < p->num_blocks; ++i) pool_push(p, i);
}

/* BlockPool::block_data -- :59-63 */
void *or_pool_block_data(const or_block_pool *p, int32_t id) {
    if (id < 0 || id >= p->num_blocks || !p->buffer) return NULL;
    return p->buffer + (size_t)id * p->block_bytes;
}

int32_t or_pool_num_blocks(const or_block_pool *p) { return p->num_blocks; }
int32_t or_pool_num_free(const or_block_pool *p) { return p->free_len; }

/* ------------------------------------------------------------------------- */

typedef struct {
    int32_t exists;
    int32_t layer_id;
    int32_t active;
    int32_t num_cached;
    int32_t n_kv_heads, head_dim, dtype;
    or_block_pool k_pool, v_pool;
    int32_t *k_ids, *v_ids; /* page_table: vector<PageEntry{k,v}> */
    int32_t n_pages, cap_pages;
} or_layer;

struct or_manager {
    int with_pool;
    or_layer *layers;
    int32_t n_layers;
};

static size_t dtype_size(int32_t dtype) {
    switch (dtype) {
        case OR_DTYPE_F32: return 4;
        case OR_DTYPE_F16: return 2;
        case OR_DTYPE_BF16: return 2;
        default: return 0;
    }
}

/* std::map operator[]: default-constructed LayerState on first access
 * (page_attention.h:57-66: active=false, num_cached=0, dtype=F32). */
static or_layer *get_layer(or_manager *m, int32_t layer_id) {
    for (int32_t i = 0; i < m->n_layers; ++i)
        if (m->layers[i].layer_id == layer_id) return &m->layers[i];
    m->layers = (or_layer *)realloc(m->layers, (size_t)(m->n_layers + 1) * sizeof(or_layer));
    or_layer *s = &m->layers[m->n_layers++];
    memset(s, 0, sizeof *s);
    s->exists = 1;
    s->layer_id = layer_id;
    s->dtype = OR_DTYPE_F32;
    return s;
}

static const or_layer *find_layer(const or_manager *m, int32_t layer_id) {
    for (int32_t i = 0; i < m->n_layers; ++i)
        if (m->layers[i].layer_id == layer_id) return &m->layers[i];
    return NULL;
}

static void table_push(or_layer *s, int32_t k, int32_t v) {
    if (s->n_pages == s->cap_pages) {
        s->cap_pages = s->cap_pages ? 2 * s->cap_pages : 64;
        s->k_ids = (int32_t *)realloc(s->k_ids, (size_t)s->cap_pages * sizeof(int32_t));
        s->v_ids = (int32_t *)realloc(s->v_ids, (size_t)s->cap_pages * sizeof(int32_t));
    }
    s->k_ids[s->n_pages] = k;
    s->v_ids[s->n_pages] = v;
    s->n_pages++;
}

or_manager *or_mgr_create(int with_pool) {
    or_manager *m = (or_manager *)calloc(1, sizeof *m);
    m->with_pool = with_pool;
    return m;
}

void or_mgr_destroy(or_manager *m) {
    if (!m) return;
    for (int32_t i = 0; i < m->n_layers; ++i) {
        or_layer *s = &m->layers[i];
        free(s->k_pool.free_list);
        free(s->v_pool.free_list);
        free(s->k_pool.buffer);
        free(s->v_pool.buffer);
        free(s->k_ids);
        free(s->v_ids);
    }
    free(m->layers);
    free(m);
}

/* init_layer -- page_attention.cpp:72-79 */
void or_mgr_init_layer(or_manager *m, int32_t layer, int32_t n_kv_heads, int32_t head_dim, int32_t dtype) {
    or_layer *s = get_layer(m, layer);
    s->n_kv_heads = n_kv_heads;
    s->head_dim = head_dim;
    s->dtype = dtype;
    s->active = 1;
    s->num_cached = 0;
}

/* reserve_layer -- :81-101.  Two pools of max_blocks * block_bytes from the
 * device kv_cache MemoryPool; here zeroed host memory (resource_cpu.cpp:43). */
void or_mgr_reserve_layer(or_manager *m, int32_t layer, int32_t max_blocks) {
    or_layer *s = get_layer(m, layer);
    if (!s->active || !m->with_pool) return;
    size_t es = dtype_size(s->dtype);
    size_t block_bytes = (size_t)OR_PAGE_BLOCK_SIZE * (size_t)s->n_kv_heads * (size_t)s->head_dim * es;
    size_t total = (size_t)max_blocks * block_bytes;
    free(s->k_pool.free_list);
    free(s->v_pool.free_list);
    free(s->k_pool.buffer);
    free(s->v_pool.buffer);
    void *kb = calloc(total ? total : 1, 1);
    void *vb = calloc(total ? total : 1, 1);
    pool_init(&s->k_pool, kb, total, max_blocks, s->n_kv_heads, s->head_dim, es);
    pool_init(&s->v_pool, vb, total, max_blocks, s->n_kv_heads, s->head_dim, es);
}

/* append_kv_pages -- :141-162.  At each page boundary allocate a K id and a V
 * id; a failed allocation breaks out of the loop, but num_cached still grows by
 * count (:161).  An entry is only pushed when the table is shorter than the
 * logical page (:157-158). */
void or_mgr_append_kv_pages(or_manager *m, int32_t layer, int32_t count) {
    or_layer *s = get_layer(m, layer);
    if (!s->active || count <= 0) return;
    for (int32_t p = 0; p < count; ++p) {
        int32_t g = s->num_cached + p;
        int32_t lb = g / OR_PAGE_BLOCK_SIZE;
        int32_t off = g % OR_PAGE_BLOCK_SIZE;
        if (off == 0) {
            int32_t k = or_pool_alloc(&s->k_pool);
            int32_t v = or_pool_alloc(&s->v_pool);
            if (k < 0 || v < 0) break;
            if (lb >= s->n_pages) table_push(s, k, v);
        }
    }
    s->num_cached += count;
}

/* append_kv_from_tensor -- :104-140.  K/V head-major [Hkv][S][D]; token p of
 * head h goes to page table[g/16], slot g%16, head h (page layout [16][Hkv][D]). */
void or_mgr_append_kv_from_tensor(or_manager *m, int32_t layer, const void *K, const void *V,
                                  int32_t n_kv_heads, int32_t seq_len, int32_t head_dim, int32_t dtype) {
    or_layer *s = get_layer(m, layer);
    if (!s->active || seq_len <= 0) return;
    int32_t prev = s->num_cached;
    size_t es = dtype_size(dtype);
    size_t row = (size_t)head_dim * es;
    size_t head_stride = (size_t)seq_len * (size_t)head_dim * es;
    or_mgr_append_kv_pages(m, layer, seq_len);
    for (int32_t p = 0; p < seq_len; ++p) {
        int32_t g = prev + p;
        int32_t lb = g / OR_PAGE_BLOCK_SIZE;
        int32_t off = g % OR_PAGE_BLOCK_SIZE;
        /* the reference indexes page_table[lb] unchecked (undefined once an
         * allocation failed); the restatement stops there instead. */
        if (lb >= s->n_pages) break;
        uint8_t *kb = (uint8_t *)or_pool_block_data(&s->k_pool, s->k_ids[lb]);
        uint8_t *vb = (uint8_t *)or_pool_block_data(&s->v_pool, s->v_ids[lb]);
        if (!kb || !vb) continue;
        uint8_t *kd = kb + (size_t)off * (size_t)n_kv_heads * row;
        uint8_t *vd = vb + (size_t)off * (size_t)n_kv_heads * row;
        for (int32_t h = 0; h < n_kv_heads; ++h) {
            memcpy(kd + (size_t)h * row, (const uint8_t *)K + (size_t)h * head_stride + (size_t)p * row, row);
            memcpy(vd + (size_t)h * row, (const uint8_t *)V + (size_t)h * head_stride + (size_t)p * row, row);
        }
    }
}

/* append_kv_from_pos -- :164-203.  The reference's loop over the positions
 * g = global_pos + p: at every g with g % 16 == 0 a block is taken from each
 * pool (the loop stops when one is exhausted) and entered into the table only
 * past its end, as append_kv_pages does; row p is written to page
 * table[g/16], slot g%16; at the end num_cached = max(num_cached,
 * global_pos + count).  Two departures, both where the reference has
 * undefined or wrong behaviour: the source row of head h is
 * K + (h*count + p)*D, head-major [Hkv][count][D] as append_kv_from_tensor
 * reads it (the reference reads K + p*D for every head, :195 and :198), and a
 * position whose page is not in the table stops the loop (the reference
 * indexes page_table[g/16] unchecked). */
void or_mgr_append_kv_from_pos(or_manager *m, int32_t layer, const void *K, const void *V, int32_t n_kv_heads,
                               int32_t head_dim, int32_t dtype, int32_t global_pos, int32_t count) {
    or_layer *s = get_layer(m, layer);
    if (!s->active) return;
    size_t es = dtype_size(dtype);
    size_t row = (size_t)head_dim * es;
    size_t head_stride = (size_t)(count > 0 ? count : 0) * row;
    for (int32_t p = 0; p < count; ++p) {
        int32_t g = global_pos + p;
        int32_t lb = g / OR_PAGE_BLOCK_SIZE;
        int32_t off = g % OR_PAGE_BLOCK_SIZE;
        if (off == 0) {
            int32_t k_id = or_pool_alloc(&s->k_pool);
            int32_t v_id = or_pool_alloc(&s->v_pool);
            if (k_id < 0 || v_id < 0) break;
            if (lb >= s->n_pages) table_push(s, k_id, v_id);
        }
        if (lb >= s->n_pages) break;
        uint8_t *kb = (uint8_t *)or_pool_block_data(&s->k_pool, s->k_ids[lb]);
        uint8_t *vb = (uint8_t *)or_pool_block_data(&s->v_pool, s->v_ids[lb]);
        if (!kb || !vb) continue;
        uint8_t *kd = kb + (size_t)off * (size_t)n_kv_heads * row;
        uint8_t *vd = vb + (size_t)off * (size_t)n_kv_heads * row;
        for (int32_t h = 0; h < n_kv_heads; ++h) {
            memcpy(kd + (size_t)h * row, (const uint8_t *)K + (size_t)h * head_stride + (size_t)p * row, row);
            memcpy(vd + (size_t)h * row, (const uint8_t *)V + (size_t)h * head_stride + (size_t)p * row, row);
        }
    }
    if (global_pos + count > s->num_cached) s->num_cached = global_pos + count;
}

/* reset -- :208-216 */
void or_mgr_reset(or_manager *m) {
    for (int32_t i = 0; i < m->n_layers; ++i) {
        or_layer *s = &m->layers[i];
        s->num_cached = 0;
        s->n_pages = 0;
        or_pool_reset(&s->k_pool);
        or_pool_reset(&s->v_pool);
    }
}

/* is_active -- page_attention.h:82-85 (does not create the layer) */
int or_mgr_is_active(const or_manager *m, int32_t layer) {
    const or_layer *s = find_layer(m, layer);
    return s && s->active;
}

int32_t or_mgr_num_cached(or_manager *m, int32_t layer) { return get_layer(m, layer)->num_cached; }
int32_t or_mgr_num_pages(or_manager *m, int32_t layer) { return get_layer(m, layer)->n_pages; }

int32_t or_mgr_get_page_table(or_manager *m, int32_t layer, int32_t *k_ids, int32_t *v_ids, int32_t cap) {
    or_layer *s = get_layer(m, layer);
    for (int32_t i = 0; i < s->n_pages && i < cap; ++i) {
        if (k_ids) k_ids[i] = s->k_ids[i];
        if (v_ids) v_ids[i] = s->v_ids[i];
    }
    return s->n_pages;
}

void or_mgr_set_page_table(or_manager *m, int32_t layer, const int32_t *k_ids, const int32_t *v_ids,
                           int32_t n, int32_t num_cached) {
    or_layer *s = get_layer(m, layer);
    s->n_pages = 0;
    for (int32_t i = 0; i < n; ++i) table_push(s, k_ids[i], v_ids[i]);
    s->num_cached = num_cached;
}

void *or_mgr_k_pool(or_manager *m, int32_t layer) { return get_layer(m, layer)->k_pool.buffer; }
void *or_mgr_v_pool(or_manager *m, int32_t layer) { return get_layer(m, layer)->v_pool.buffer; }

or_block_pool *or_mgr_pool(or_manager *m, int32_t layer, int which) {
    or_layer *s = get_layer(m, layer);
    return which ? &s->v_pool : &s->k_pool;
}

/* accessors used by attention.c */
int or__layer_view(or_manager *m, int32_t layer, int32_t *active, int32_t *num_cached, int32_t *n_pages,
                   const int32_t **k_ids, const int32_t **v_ids, or_block_pool **kp, or_block_pool **vp) {
    or_layer *s = get_layer(m, layer);
    *active = s->active;
    *num_cached = s->num_cached;
    *n_pages = s->n_pages;
    *k_ids = s->k_ids;
    *v_ids = s->v_ids;
    *kp = &s->k_pool;
    *vp = &s->v_pool;
    return 0;
}
