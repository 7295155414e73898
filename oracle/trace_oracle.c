/*
 * trace_oracle.c — CPU restatement of torch-sdf's batched sphere tracer.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the parity checker for the HIP
 * tracer. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it; the product path never does.
 *
 * What it restates (reference paths relative to the seismael/navi checkout):
 *   constants            projects/torch-sdf/cpp_src/kernel.cuh:7-11, kernel.cu:9
 *   point_in_bounds*     kernel.cu:11-33
 *   load_dag_word        kernel.cu:35-41   (the LDS prefix copy is a cache of
 *                                           the same words, so it is dropped)
 *   decode_leaf_*        kernel.cu:43-52   (binary16 decoded from its IEEE 754
 *                                           definition, exact in binary32)
 *   distance_to_bounds_exit  kernel.cu:54-85
 *   query_dag_stackless  kernel.cu:88-200
 *   sphere_trace_kernel  kernel.cu:203-309
 *
 * Extensions the reference does not have, all off the default path:
 *   - hit_epsilon is an argument (reference: compile-time 0.01, kernel.cuh:7);
 *   - per-ray step count (loop iterations of kernel.cu:260-305) and the
 *     number of DAG words loaded (calls of load_dag_word at kernel.cu:137,198);
 *   - every word index is bounds-checked. The reference reads out of range
 *     (undefined behaviour); here such a ray stops at once and reports
 *     distance NaN, semantic 0 and fault flag 1 — the HIP kernels do the same.
 *
 * Floating point: p = o + t*d is evaluated as one fused multiply-add
 * (fmaf), every other operation is a single IEEE-754 binary32 operation with
 * round-to-nearest-even. Build with -ffp-contract=off and without fast-math.
 *
 * Parity pins (tests/test_oracle_*.py): the ten known-answer traces held by
 * projects/torch-sdf/tests/test_sphere_tracing.py:683-949, the exhaustive
 * binary16 decode against numpy's float16, hand-derived void-cell exits,
 * the closed-form slab distance of projects/contracts/.../oracle_box.py:115-160
 * and a cache-free brute-force march on random rays.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define OR_OUTSIDE_DOMAIN 1000.0f    /* kernel.cuh:8  kOutsideDomainDistance */
#define OR_DIR_EPS 1e-4f             /* kernel.cuh:9  kDirectionNormEpsilon */
#define OR_PREFIX_DEPTH 4            /* kernel.cuh:11 kTraversalCacheDepth */
#define OR_VOID_ADVANCE_EPS 1e-5f    /* kernel.cu:9   kVoidAdvanceEpsilon */
#define OR_MAX_DEPTH 32              /* kernel.cu:136 descent limit */

typedef struct {
    float lo[3];
    float hi[3];
} or_box;

/* Per-ray traversal caches, kernel.cu:236-247. */
typedef struct {
    uint32_t pre_ptr;
    or_box pre;
    int pre_valid;
    or_box vd;
    int vd_valid;
    or_box lf;
    float lf_dist;
    int32_t lf_sem;
    int lf_valid;
} or_cache;

/* Per-ray bookkeeping the reference does not keep. */
typedef struct {
    uint64_t words;
    int fault;
} or_count;

static int or_in_box(const float p[3], const or_box* b) /* kernel.cu:11-21 */
{
    return p[0] >= b->lo[0] && p[0] <= b->hi[0] &&
           p[1] >= b->lo[1] && p[1] <= b->hi[1] &&
           p[2] >= b->lo[2] && p[2] <= b->hi[2];
}

static int or_in_box_strict(const float p[3], const or_box* b) /* kernel.cu:23-33 */
{
    return p[0] > b->lo[0] && p[0] < b->hi[0] &&
           p[1] > b->lo[1] && p[1] < b->hi[1] &&
           p[2] > b->lo[2] && p[2] < b->hi[2];
}

/* IEEE 754 binary16 -> binary32 from the format's definition (kernel.cu:43-47
 * uses __half2float, an exact conversion). */
float oracle_half_to_float(uint16_t h)
{
    uint32_t sign = (uint32_t)(h >> 15) & 1u;
    uint32_t expo = (uint32_t)(h >> 10) & 0x1fu;
    uint32_t man = (uint32_t)h & 0x3ffu;
    uint32_t bits;
    float out;
    if (expo == 0) {
        /* zero or subnormal: man * 2^-24, exactly representable */
        out = ldexpf((float)man, -24);
        return sign ? -out : out;
    }
    if (expo == 31) {
        /* inf (man == 0) or NaN, payload kept in the high mantissa bits */
        bits = (sign << 31) | 0x7f800000u | (man << 13);
    } else {
        bits = (sign << 31) | ((expo - 15u + 127u) << 23) | (man << 13);
    }
    memcpy(&out, &bits, sizeof out);
    return out;
}

static int or_popcount8(uint32_t v)
{
    int c = 0;
    for (int i = 0; i < 8; ++i) c += (int)((v >> i) & 1u);
    return c;
}

/* kernel.cu:54-85 */
static float or_exit_distance(const float p[3], const float d[3], const or_box* b)
{
    float exit_t = OR_OUTSIDE_DOMAIN;
    for (int a = 0; a < 3; ++a) {
        if (d[a] > OR_DIR_EPS) {
            exit_t = fminf(exit_t, (b->hi[a] - p[a]) / d[a]);
        } else if (d[a] < -OR_DIR_EPS) {
            exit_t = fminf(exit_t, (b->lo[a] - p[a]) / d[a]);
        }
    }
    return fmaxf(exit_t, OR_VOID_ADVANCE_EPS);
}

static uint64_t or_load(const uint64_t* dag, uint64_t n_words, uint32_t idx, or_count* cnt)
{
    cnt->words += 1;
    if ((uint64_t)idx >= n_words) {
        cnt->fault = 1;
        return 0;
    }
    return dag[idx];
}

/* kernel.cu:88-200. Writes *out_dist / *out_sem only where the reference
 * does: after 32 levels without a leaf or void both stay untouched (stale). */
static void or_query(const uint64_t* dag, uint64_t n_words, const float p[3], const float d[3],
                     const or_box* dom, or_cache* c, float* out_dist, int32_t* out_sem,
                     or_count* cnt)
{
    if (!or_in_box(p, dom)) { /* :108-112 */
        *out_dist = OR_OUTSIDE_DOMAIN;
        *out_sem = 0;
        return;
    }
    if (c->lf_valid && or_in_box(p, &c->lf)) { /* :114-118 */
        *out_dist = c->lf_dist;
        *out_sem = c->lf_sem;
        return;
    }
    const int use_pre = c->pre_valid && or_in_box(p, &c->pre); /* :120-132 */
    uint32_t ptr = use_pre ? c->pre_ptr : 0u;
    or_box cur = use_pre ? c->pre : *dom;
    int depth = use_pre ? OR_PREFIX_DEPTH : 0;

    for (; depth < OR_MAX_DEPTH; ++depth) { /* :136-199 */
        const uint64_t node = or_load(dag, n_words, ptr, cnt);
        if (cnt->fault) return;
        if ((node >> 63) == 1u) { /* leaf :139-152 */
            c->lf = cur;
            c->lf_dist = oracle_half_to_float((uint16_t)(node & 0xffffu));
            c->lf_sem = (int32_t)((node >> 16) & 0xffffu);
            c->lf_valid = 1;
            *out_dist = c->lf_dist;
            *out_sem = c->lf_sem;
            return;
        }
        if (!use_pre && depth == OR_PREFIX_DEPTH) { /* :154-163 */
            c->pre_ptr = ptr;
            c->pre = cur;
            c->pre_valid = 1;
        }
        int octant = 0;
        for (int a = 0; a < 3; ++a) { /* :166-176 */
            const float mid = (cur.lo[a] + cur.hi[a]) * 0.5f;
            if (p[a] >= mid) {
                octant |= 1 << a;
                cur.lo[a] = mid;
            } else {
                cur.hi[a] = mid;
            }
        }
        const uint32_t mask = (uint32_t)((node >> 55) & 0xffu); /* :178 */
        if ((mask & (1u << octant)) == 0u) { /* void :179-190 */
            c->vd = cur;
            c->vd_valid = 1;
            *out_dist = or_exit_distance(p, d, &c->vd);
            *out_sem = 0;
            return;
        }
        const uint32_t child_base = (uint32_t)(node & 0xffffffffu); /* :192-198 */
        const uint32_t offset = (uint32_t)or_popcount8(mask & ((1u << octant) - 1u));
        ptr = (uint32_t)or_load(dag, n_words, child_base + offset, cnt);
        if (cnt->fault) return;
    }
}

/* One ray of kernel.cu:222-308. */
static void or_trace_one(const uint64_t* dag, uint64_t n_words, const float o[3], const float d[3],
                         int32_t max_steps, float max_distance, const or_box* dom, float hit_eps,
                         float* out_d, int32_t* out_s, int32_t* out_steps, uint64_t* out_words,
                         uint8_t* out_fault)
{
    or_cache c;
    memset(&c, 0, sizeof c);
    or_count cnt = {0, 0};
    float t = 0.0f;
    float dist = 0.0f;
    int32_t sem = 0;
    int32_t steps = 0;
    float rd = t;
    int32_t rs = 0;
    int done = 0;

    for (int32_t step = 0; step < max_steps; ++step) { /* :260-305 */
        steps = step + 1;
        float p[3];
        p[0] = fmaf(t, d[0], o[0]); /* :261-263, contracted to one fma */
        p[1] = fmaf(t, d[1], o[1]);
        p[2] = fmaf(t, d[2], o[2]);
        if (c.vd_valid && or_in_box_strict(p, &c.vd)) { /* :265-267 */
            dist = or_exit_distance(p, d, &c.vd);
            sem = 0;
        } else {
            or_query(dag, n_words, p, d, dom, &c, &dist, &sem, &cnt);
            if (cnt.fault) {
                rd = NAN;
                rs = 0;
                done = 1;
                break;
            }
        }
        if (sem != 0 && dist < hit_eps) { /* :297-301 */
            rd = t;
            rs = sem;
            done = 1;
            break;
        }
        t += dist; /* :302-304 */
        if (t > max_distance) break;
    }
    if (!done) { /* :307-308 */
        rd = t;
        rs = 0;
    }
    *out_d = rd;
    *out_s = rs;
    if (out_steps) *out_steps = steps;
    if (out_words) *out_words = cnt.words;
    if (out_fault) *out_fault = (uint8_t)cnt.fault;
}

/* Batched entry: rays [n_rays] with AoS origins/dirs [n_rays*3]. Optional
 * outputs may be NULL. n_threads <= 1 runs serially; otherwise OpenMP with
 * schedule(dynamic, 256) over rays. */
void oracle_trace(const uint64_t* dag, uint64_t n_words, const float* origins, const float* dirs,
                  int64_t n_rays, int32_t max_steps, float max_distance, const float* bbox_min,
                  const float* bbox_max, float hit_eps, float* out_d, int32_t* out_s,
                  int32_t* out_steps, uint64_t* out_words, uint8_t* out_fault, int32_t n_threads)
{
    or_box dom;
    for (int a = 0; a < 3; ++a) {
        dom.lo[a] = bbox_min[a];
        dom.hi[a] = bbox_max[a];
    }
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 256) num_threads(n_threads > 1 ? n_threads : 1) if (n_threads > 1)
#endif
    for (int64_t i = 0; i < n_rays; ++i) {
        or_trace_one(dag, n_words, origins + 3 * i, dirs + 3 * i, max_steps, max_distance, &dom,
                     hit_eps, out_d + i, out_s + i, out_steps ? out_steps + i : NULL,
                     out_words ? out_words + i : NULL, out_fault ? out_fault + i : NULL);
    }
}

/* Multi-scene batch: env e traces scene env_scene[e] of a concatenated word
 * pool (scene s occupies words [scene_base[s], scene_base[s]+scene_words[s]),
 * child pointers relative to its base). The reference equivalent is one
 * cast_rays call per scene over that scene's env subset
 * (projects/environment/.../sdfdag_backend.py:1215-1217,1897-1905). */
void oracle_trace_multi(const uint64_t* pool, const uint64_t* scene_base, const uint64_t* scene_words,
                        const float* scene_bounds /* [n_scenes][6] lo xyz, hi xyz */,
                        const int32_t* env_scene, int64_t n_envs, int64_t rays_per_env,
                        const float* origins, const float* dirs, int32_t max_steps,
                        float max_distance, float hit_eps, float* out_d, int32_t* out_s,
                        int32_t* out_steps, uint64_t* out_words, uint8_t* out_fault,
                        int32_t n_threads)
{
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 256) num_threads(n_threads > 1 ? n_threads : 1) if (n_threads > 1)
#endif
    for (int64_t i = 0; i < n_envs * rays_per_env; ++i) {
        const int32_t s = env_scene[i / rays_per_env];
        or_box dom;
        for (int a = 0; a < 3; ++a) {
            dom.lo[a] = scene_bounds[6 * s + a];
            dom.hi[a] = scene_bounds[6 * s + 3 + a];
        }
        or_trace_one(pool + scene_base[s], scene_words[s], origins + 3 * i, dirs + 3 * i, max_steps,
                     max_distance, &dom, hit_eps, out_d + i, out_s + i,
                     out_steps ? out_steps + i : NULL, out_words ? out_words + i : NULL,
                     out_fault ? out_fault + i : NULL);
    }
}

/* ---------------------------------------------------------------------------
 * Point-SDF query (collision / clearance). The reference has no such kernel;
 * the closest semantics are one fresh query_dag_stackless at a point
 * (kernel.cu:88-200) with no caches:
 *   outside the bounds (inclusive test, kernel.cu:108-112) -> (1000, 0, kind 0)
 *   leaf  -> (decoded fp16 distance, semantic, kind 1)
 *   void  -> (1.7321 * void cell side along x, 0, kind 2): the compiler prunes
 *            an octant only when every sample in it exceeds its diagonal
 *            half*voxel*1.7321 (projects/voxel-dag/src/compiler.cpp:626,639-643),
 *            so this is a clearance lower bound.
 *   descent limit reached -> (NaN, 0, kind 3); word index out of range ->
 *            (NaN, 0, kind 4).
 * Also reports the words loaded.
 * ------------------------------------------------------------------------- */
void oracle_point_query(const uint64_t* dag, uint64_t n_words, const float* points, int64_t n_points,
                        const float* bbox_min, const float* bbox_max, float* out_d,
                        int32_t* out_s, int32_t* out_kind, uint64_t* out_words)
{
    or_box dom;
    for (int a = 0; a < 3; ++a) {
        dom.lo[a] = bbox_min[a];
        dom.hi[a] = bbox_max[a];
    }
    for (int64_t i = 0; i < n_points; ++i) {
        const float* p = points + 3 * i;
        or_count cnt = {0, 0};
        float rd = NAN;
        int32_t rs = 0, kind = 3;
        if (!or_in_box(p, &dom)) {
            rd = OR_OUTSIDE_DOMAIN;
            kind = 0;
        } else {
            uint32_t ptr = 0;
            or_box cur = dom;
            for (int depth = 0; depth < OR_MAX_DEPTH; ++depth) {
                const uint64_t node = or_load(dag, n_words, ptr, &cnt);
                if (cnt.fault) break;
                if ((node >> 63) == 1u) {
                    rd = oracle_half_to_float((uint16_t)(node & 0xffffu));
                    rs = (int32_t)((node >> 16) & 0xffffu);
                    kind = 1;
                    break;
                }
                int octant = 0;
                for (int a = 0; a < 3; ++a) {
                    const float mid = (cur.lo[a] + cur.hi[a]) * 0.5f;
                    if (p[a] >= mid) {
                        octant |= 1 << a;
                        cur.lo[a] = mid;
                    } else {
                        cur.hi[a] = mid;
                    }
                }
                const uint32_t mask = (uint32_t)((node >> 55) & 0xffu);
                if ((mask & (1u << octant)) == 0u) {
                    rd = (cur.hi[0] - cur.lo[0]) * 1.7321f;
                    kind = 2;
                    break;
                }
                const uint32_t base = (uint32_t)(node & 0xffffffffu);
                const uint32_t off = (uint32_t)or_popcount8(mask & ((1u << octant) - 1u));
                ptr = (uint32_t)or_load(dag, n_words, base + off, &cnt);
                if (cnt.fault) break;
            }
            if (cnt.fault) {
                rd = NAN;
                rs = 0;
                kind = 4;
            }
        }
        out_d[i] = rd;
        out_s[i] = rs;
        out_kind[i] = kind;
        if (out_words) out_words[i] = cnt.words;
    }
}

/* ---------------------------------------------------------------------------
 * Cache-free march, used only to pin the cached march above. Every step does
 * a fresh descent from the root (the semantics of the reference's own
 * cache-free helper, projects/torch-sdf/tests/test_sphere_tracing.py:121-178,
 * extended with the void-cell exit distance of kernel.cu:179-190). Without
 * caches the result can differ from the cached march only when a sample lands
 * exactly on a face of a cached box (inclusive leaf/prefix tests, strict void
 * test, kernel.cu:114,120,265); *out_touch reports whether any sample lay on a
 * face of its freshly found leaf/void box or of that box's depth-4 ancestor.
 * ------------------------------------------------------------------------- */
static int or_on_face(const float p[3], const or_box* b)
{
    for (int a = 0; a < 3; ++a) {
        if (p[a] == b->lo[a] || p[a] == b->hi[a]) return 1;
    }
    return 0;
}

void oracle_trace_nocache(const uint64_t* dag, uint64_t n_words, const float* origins,
                          const float* dirs, int64_t n_rays, int32_t max_steps, float max_distance,
                          const float* bbox_min, const float* bbox_max, float hit_eps, float* out_d,
                          int32_t* out_s, int32_t* out_steps, uint8_t* out_touch)
{
    or_box dom;
    for (int a = 0; a < 3; ++a) {
        dom.lo[a] = bbox_min[a];
        dom.hi[a] = bbox_max[a];
    }
    for (int64_t i = 0; i < n_rays; ++i) {
        const float* o = origins + 3 * i;
        const float* d = dirs + 3 * i;
        float t = 0.0f, dist = 0.0f, rd = 0.0f;
        int32_t sem = 0, rs = 0, steps = 0;
        int touch = 0, done = 0;
        for (int32_t step = 0; step < max_steps; ++step) {
            steps = step + 1;
            float p[3] = {fmaf(t, d[0], o[0]), fmaf(t, d[1], o[1]), fmaf(t, d[2], o[2])};
            if (!or_in_box(p, &dom)) {
                dist = OR_OUTSIDE_DOMAIN;
                sem = 0;
            } else {
                uint32_t ptr = 0;
                or_box cur = dom;
                or_count cnt = {0, 0};
                int found = 0;
                for (int depth = 0; depth < OR_MAX_DEPTH && !found; ++depth) {
                    const uint64_t node = or_load(dag, n_words, ptr, &cnt);
                    if (cnt.fault) break;
                    if ((node >> 63) == 1u) {
                        dist = oracle_half_to_float((uint16_t)(node & 0xffffu));
                        sem = (int32_t)((node >> 16) & 0xffffu);
                        touch |= or_on_face(p, &cur);
                        found = 1;
                        break;
                    }
                    if (depth == OR_PREFIX_DEPTH) touch |= or_on_face(p, &cur);
                    int octant = 0;
                    for (int a = 0; a < 3; ++a) {
                        const float mid = (cur.lo[a] + cur.hi[a]) * 0.5f;
                        if (p[a] >= mid) {
                            octant |= 1 << a;
                            cur.lo[a] = mid;
                        } else {
                            cur.hi[a] = mid;
                        }
                    }
                    const uint32_t mask = (uint32_t)((node >> 55) & 0xffu);
                    if ((mask & (1u << octant)) == 0u) {
                        dist = or_exit_distance(p, d, &cur);
                        sem = 0;
                        touch |= or_on_face(p, &cur);
                        found = 1;
                        break;
                    }
                    const uint32_t base = (uint32_t)(node & 0xffffffffu);
                    const uint32_t off = (uint32_t)or_popcount8(mask & ((1u << octant) - 1u));
                    ptr = (uint32_t)or_load(dag, n_words, base + off, &cnt);
                    if (cnt.fault) break;
                }
                if (cnt.fault) {
                    rd = NAN;
                    rs = 0;
                    done = 1;
                    break;
                }
            }
            if (sem != 0 && dist < hit_eps) {
                rd = t;
                rs = sem;
                done = 1;
                break;
            }
            t += dist;
            if (t > max_distance) break;
        }
        if (!done) {
            rd = t;
            rs = 0;
        }
        out_d[i] = rd;
        out_s[i] = rs;
        if (out_steps) out_steps[i] = steps;
        if (out_touch) out_touch[i] = (uint8_t)touch;
    }
}
