/*
 * compile_oracle.c — literal CPU restatement of the .gmdag DAG compiler rules.
 *
 * TEST INFRASTRUCTURE ONLY (see trace_oracle.c). It pins the product scene
 * compiler (navi_amd/csrc/scene_compiler.cpp), which must emit the same words
 * from the same dense grid.
 *
 * Restates projects/voxel-dag/src/compiler.cpp:
 *   float_to_half        :542-560  (kept as the optional "quirk" encoder)
 *   block_min_sdf        :563-577
 *   build_recursive      :579-659  (leaf, uniform collapse, void prune, dedup)
 *   dedup of leaves / internal nodes  :143-190 (exact structural match; the
 *                        hash only buckets candidates, so any hash gives the
 *                        same pool)
 *   compressToDAG        :661-674  (index 0 reserved, root copied to it)
 * The dense grid is [z][y][x] with index z*N*N + y*N + x, as at :483.
 *
 * The default fp16 encoder is IEEE 754 round-to-nearest-even (the reference's
 * :542-560 truncates and maps |d| < 2^-14, including 0, to +inf; that
 * behaviour is available with quirk_half = 1).
 *
 * Deliberately naive: block scans are recomputed at every level and the
 * dedup table is a plain linear-probe map. Use it on grids up to ~64^3.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* IEEE 754 binary32 -> binary16, round to nearest, ties to even. */
uint16_t oracle_float_to_half_rne(float f)
{
    uint32_t x;
    memcpy(&x, &f, sizeof x);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t expo = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (expo == 0xffu) {
        if (man == 0) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | (man >> 13)); /* quiet NaN */
    }
    const int e = (int)expo - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u); /* overflow -> inf */
    if (e <= 0) {
        /* subnormal half (or zero): value = m * 2^-24 */
        if (e < -10) return (uint16_t)sign; /* below half of the smallest subnormal */
        const uint32_t full = man | 0x800000u; /* 24-bit significand */
        const int shift = 14 - e;              /* bits dropped */
        uint32_t q = full >> shift;
        const uint32_t rem = full & ((1u << shift) - 1u);
        const uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (q & 1u))) q += 1;
        return (uint16_t)(sign | q); /* q may carry into the exponent: correct */
    }
    uint32_t q = ((uint32_t)e << 10) | (man >> 13);
    const uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1; /* may carry to inf: correct */
    return (uint16_t)(sign | q);
}

/* projects/voxel-dag/src/compiler.cpp:542-560, bug for bug (unsigned exponent). */
uint16_t oracle_float_to_half_quirk(float f)
{
    uint32_t i;
    memcpy(&i, &f, sizeof i);
    const uint32_t s = (i >> 16) & 0x00008000u;
    const uint32_t e = ((i >> 23) & 0x000000ffu) - (127u - 15u);
    uint32_t m = i & 0x007fffffu;
    if (e == 0u) { /* "e <= 0" on an unsigned value */
        m = (m | 0x00800000u) >> 1;
        return (uint16_t)(s | (m >> 13));
    } else if (e == 0xffu - (127u - 15u)) {
        if (m == 0) return (uint16_t)(s | 0x7c00u);
        return (uint16_t)(s | 0x7c00u | (m >> 13) | (m ? 1u : 0u));
    } else {
        if (e > 30u) return (uint16_t)(s | 0x7c00u);
        return (uint16_t)(s | (e << 10) | (m >> 13));
    }
}

typedef struct {
    uint64_t* w;
    size_t n, cap;
    int overflow;
} oc_pool;

typedef struct {
    uint32_t* slot; /* pool index + 1, 0 = empty */
    size_t cap;
} oc_map;

typedef struct {
    const float* grid;
    int N;
    float voxel;
    int quirk;
    oc_pool pool;
    oc_map map;
} oc_ctx;

static void oc_push(oc_pool* p, uint64_t v)
{
    if (p->n == p->cap) {
        size_t nc = p->cap ? p->cap * 2 : 1024;
        uint64_t* nw = (uint64_t*)realloc(p->w, nc * sizeof(uint64_t));
        if (!nw) {
            p->overflow = 1;
            return;
        }
        p->w = nw;
        p->cap = nc;
    }
    p->w[p->n++] = v;
}

static uint64_t oc_mix(uint64_t h)
{
    h ^= h >> 33;
    h *= 0xff51afd7ed558ccdull;
    h ^= h >> 33;
    h *= 0xc4ceb9fe1a85ec53ull;
    h ^= h >> 33;
    return h;
}

/* Key of a pool entry: the word itself for a leaf; mask and child list for an
 * internal node. */
static uint64_t oc_key_hash(uint64_t node, const uint32_t* kids, int nk)
{
    uint64_t h = oc_mix(node >> 55 | (node >> 63) << 8);
    if (node >> 63) return oc_mix(node);
    for (int i = 0; i < nk; ++i) h = oc_mix(h ^ ((uint64_t)kids[i] + 0x9e3779b97f4a7c15ull * (uint64_t)(i + 1)));
    return h;
}

static int oc_matches(const oc_pool* p, uint32_t idx, uint64_t node, const uint32_t* kids, int nk)
{
    const uint64_t cand = p->w[idx];
    if ((cand >> 63) != (node >> 63)) return 0;
    if (node >> 63) return cand == node;
    if (((cand >> 55) & 0xffu) != ((node >> 55) & 0xffu)) return 0;
    const uint32_t base = (uint32_t)(cand & 0xffffffffu);
    for (int i = 0; i < nk; ++i)
        if (p->w[base + (uint32_t)i] != (uint64_t)kids[i]) return 0;
    return 1;
}

static void oc_map_grow(oc_ctx* c);

static uint32_t oc_dedup(oc_ctx* c, uint64_t node, const uint32_t* kids, int nk)
{
    if ((c->pool.n + 9) * 2 > c->map.cap) oc_map_grow(c);
    const uint64_t h = oc_key_hash(node, kids, nk);
    size_t i = (size_t)(h & (c->map.cap - 1));
    while (c->map.slot[i]) {
        const uint32_t idx = c->map.slot[i] - 1;
        if (oc_matches(&c->pool, idx, node, kids, nk)) return idx;
        i = (i + 1) & (c->map.cap - 1);
    }
    const uint32_t at = (uint32_t)c->pool.n;
    if (node >> 63) {
        oc_push(&c->pool, node);
    } else {
        oc_push(&c->pool, 0); /* compiler.cpp:176-187: node, then its child table */
        const uint32_t start = (uint32_t)c->pool.n;
        for (int k = 0; k < nk; ++k) oc_push(&c->pool, (uint64_t)kids[k]);
        if (!c->pool.overflow) c->pool.w[at] = node | (uint64_t)start;
    }
    c->map.slot[i] = at + 1;
    return at;
}

static void oc_map_grow(oc_ctx* c)
{
    const size_t nc = c->map.cap ? c->map.cap * 2 : 4096;
    uint32_t* ns = (uint32_t*)calloc(nc, sizeof(uint32_t));
    /* rehash every node that owns a slot */
    for (size_t j = 0; j < c->map.cap; ++j) {
        const uint32_t v = c->map.slot[j];
        if (!v) continue;
        const uint32_t idx = v - 1;
        const uint64_t node = c->pool.w[idx];
        int nk = 0;
        const uint32_t* kids = NULL;
        uint32_t tmp[8];
        if (!(node >> 63)) {
            const uint32_t base = (uint32_t)(node & 0xffffffffu);
            const uint32_t mask = (uint32_t)((node >> 55) & 0xffu);
            for (int b = 0; b < 8; ++b)
                if (mask & (1u << b)) tmp[nk] = (uint32_t)c->pool.w[base + (uint32_t)nk], ++nk;
            kids = tmp;
        }
        /* an internal word's hash reads only its mask bits (node >> 55) */
        size_t i = (size_t)(oc_key_hash(node, kids, nk) & (nc - 1));
        while (ns[i]) i = (i + 1) & (nc - 1);
        ns[i] = v;
    }
    free(c->map.slot);
    c->map.slot = ns;
    c->map.cap = nc;
}

static float oc_at(const oc_ctx* c, int x, int y, int z)
{
    return c->grid[(size_t)z * c->N * c->N + (size_t)y * c->N + (size_t)x];
}

static uint16_t oc_half(const oc_ctx* c, float f)
{
    return c->quirk ? oracle_float_to_half_quirk(f) : oracle_float_to_half_rne(f);
}

/* compiler.cpp:563-577 */
static float oc_block_min(const oc_ctx* c, int x, int y, int z, int size)
{
    float m = 3.402823466e+38f;
    for (int bz = z; bz < z + size && bz < c->N; ++bz)
        for (int by = y; by < y + size && by < c->N; ++by)
            for (int bx = x; bx < x + size && bx < c->N; ++bx) {
                const float v = oc_at(c, bx, by, bz);
                if (v < m) m = v;
            }
    return m;
}

static uint64_t oc_leaf_word(const oc_ctx* c, float dist, int with_sem)
{
    const uint64_t sem = (with_sem && dist < c->voxel * 2.0f) ? 1u : 0u; /* :590, :615 */
    return (1ull << 63) | (sem << 16) | (uint64_t)oc_half(c, dist);
}

/* compiler.cpp:579-659 */
static uint32_t oc_build(oc_ctx* c, int x, int y, int z, int size)
{
    if (size == 1) return oc_dedup(c, oc_leaf_word(c, oc_at(c, x, y, z), 1), NULL, 0);

    const float first = oc_at(c, x, y, z); /* :600-622 */
    int uniform = 1;
    for (int bz = z; bz < z + size && bz < c->N && uniform; ++bz)
        for (int by = y; by < y + size && by < c->N && uniform; ++by)
            for (int bx = x; bx < x + size && bx < c->N && uniform; ++bx)
                if (fabsf(oc_at(c, bx, by, bz) - first) > 1e-6f) uniform = 0;
    if (uniform) return oc_dedup(c, oc_leaf_word(c, first, 1), NULL, 0);

    const int half = size / 2;
    const float extent = (float)half * c->voxel * 1.7321f; /* :626 */
    uint32_t kids[8];
    int nk = 0;
    uint32_t mask = 0;
    for (int i = 0; i < 8; ++i) { /* :631-648 */
        const int ox = (i & 1) ? half : 0, oy = (i & 2) ? half : 0, oz = (i & 4) ? half : 0;
        const float mn = oc_block_min(c, x + ox, y + oy, z + oz, half);
        if (mn > extent) continue;
        kids[nk++] = oc_build(c, x + ox, y + oy, z + oz, half);
        mask |= 1u << i;
    }
    if (mask == 0) { /* :650-656: far leaf, semantic 0 */
        const float mn = oc_block_min(c, x, y, z, size);
        return oc_dedup(c, (1ull << 63) | (uint64_t)oc_half(c, mn), NULL, 0);
    }
    return oc_dedup(c, (uint64_t)mask << 55, kids, nk);
}

/* compiler.cpp:661-674. Returns the word count; *out_words is malloc'd and
 * must be released with oracle_free. Returns 0 on allocation failure. */
uint64_t oracle_compile_dense(const float* grid, int32_t N, float voxel_size, int32_t quirk_half,
                              uint64_t** out_words)
{
    oc_ctx c;
    memset(&c, 0, sizeof c);
    c.grid = grid;
    c.N = N;
    c.voxel = voxel_size;
    c.quirk = quirk_half;
    oc_push(&c.pool, 0);
    const uint32_t root = oc_build(&c, 0, 0, 0, N);
    if (!c.pool.overflow) c.pool.w[0] = c.pool.w[root];
    free(c.map.slot);
    if (c.pool.overflow) {
        free(c.pool.w);
        *out_words = NULL;
        return 0;
    }
    *out_words = c.pool.w;
    return c.pool.n;
}

void oracle_free(void* p) { free(p); }

/* Batched encoders for the exhaustive tests. */
void oracle_half_encode(const float* in, int64_t n, int32_t quirk, uint16_t* out)
{
    for (int64_t i = 0; i < n; ++i)
        out[i] = quirk ? oracle_float_to_half_quirk(in[i]) : oracle_float_to_half_rne(in[i]);
}

float oracle_half_to_float(uint16_t h);

void oracle_half_decode(const uint16_t* in, int64_t n, float* out)
{
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_half_to_float(in[i]);
}
