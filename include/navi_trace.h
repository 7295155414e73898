/*
 * navi_trace.h — C ABI of the MI355X .gmdag sphere tracer (libnavi_trace.so).
 *
 * Plain pointers and sizes only: every device pointer is a HIP device address,
 * `stream` is a hipStream_t passed as void* (NULL = the null stream). The
 * tracing, query and post-pass entry points are asynchronous with respect to
 * the host and return 0 on success or a negative NAVI_E* code; the message of
 * the last failure on the calling thread is navi_last_error(). They allocate
 * nothing and never wait for the device once navi_device_init has run on the
 * current device (the record-layout tracers call it themselves on their first
 * launch on a device that lacks it). The host-memory helpers (navi_relayout,
 * navi_record_depth, navi_build_cell_table) run synchronously on the CPU.
 *
 * Reference interfaces (paths relative to the seismael/navi checkout) are cited
 * on each entry point.
 */
#ifndef NAVI_TRACE_H
#define NAVI_TRACE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NAVI_OK 0
#define NAVI_E_ARG (-1)     /* invalid argument (message says which) */
#define NAVI_E_LAUNCH (-2)  /* HIP launch or runtime failure */
#define NAVI_E_LAYOUT (-3)  /* DAG cannot be re-laid (see navi_scene_build) */
#define NAVI_E_NOMEM (-4)   /* device allocation failed (navi_device_init) */

/*
 * Per-device set-up (no reference counterpart: the reference kernel keeps no
 * state between launches, kernel.cu:311-326). On the current device,
 * allocates and clears the record-layout tracers' work-queue counters (64 KiB:
 * 4096 pairs of four words, kept until the process ends), creates the events
 * that guard the reserve pairs (below), and looks up the device's copy of
 * navi_trace_relaid_noalloc's static scratch; idempotent and thread-safe. Call
 * it where allocation and a device wait are acceptable (scene load), so that
 * no later launch on this device allocates or waits.
 *
 * Work-queue pairs: an eager launch uses its stream's pair (one per host
 * thread for hipStreamPerThread), kept for the life of the process; a launch
 * recorded into a graph gets a pair of its own, given back when that graph and
 * every executable graph instantiated from it are destroyed (executable graphs
 * of one capture share it: do not replay two of them at once). When the
 * 4032 table pairs are in use, an eager launch leases one of 64 reserve pairs,
 * free again once the launch has completed (an event recorded after it);
 * only when all of those are in flight does a launch run without a queue (the
 * general march on a static schedule, correct but slower).
 * navi_last_launch reports which case a launch met.
 */
int navi_device_init(void);

/* What the calling thread's last tracer launch enqueued (no reference
 * counterpart: the reference has one kernel, kernel.cu:311-326). */
typedef struct navi_launch_info {
    uint32_t kernels;      /* NAVI_KERNEL_* bits of the kernels enqueued */
    uint32_t queue;        /* NAVI_QUEUE_* kind of work-queue pair the launch used */
    int32_t pair;          /* index of that pair in the device's table, -1 for none / scratch */
    uint32_t fast_planes;  /* split-plane depth staged by trace_fast_kernel (0: not enqueued) */
    uint32_t planes;       /* split-plane depth staged by trace_relaid_kernel (0: none) */
    uint32_t staged;       /* 1 when finished rays are staged per tile in LDS */
    uint32_t waves;        /* waves of the tracing grid (trace_fast_kernel's when enqueued) */
    uint64_t n_rays;
} navi_launch_info;

/* navi_launch_info.kernels. trace_fast_kernel runs the fast march when every
 * scene of the launch qualifies (NAVI_SCENE_NONNEG_LEAVES, boxes below 2^100,
 * no record deeper than 30 levels; the device checks the scene table) and
 * otherwise hands the launch to trace_relaid_kernel, enqueued after it. */
#define NAVI_KERNEL_FAST 1u         /* trace_fast_kernel */
#define NAVI_KERNEL_FAST_WIDE 2u    /* ... in 1024-thread workgroups (two per CU) */
#define NAVI_KERNEL_COMBINED 4u     /* trace_relaid_kernel (both marches, seven waves per SIMD) */
#define NAVI_KERNEL_RAW 8u          /* the word-layout kernel (navi_cast_rays, navi_cast_rays_multi) */
/* navi_launch_info.queue */
#define NAVI_QUEUE_NONE 0u     /* no pair: static schedule, trace_fast_kernel not enqueued */
#define NAVI_QUEUE_STREAM 1u   /* the stream's pair */
#define NAVI_QUEUE_CAPTURE 2u  /* a pair of the graph being captured */
#define NAVI_QUEUE_LEASE 3u    /* a reserve pair leased for this launch */
#define NAVI_QUEUE_SCRATCH 4u  /* navi_trace_relaid_noalloc's static scratch */

/* Copies the calling thread's last launch's info into *info (zeroes when none). */
int navi_last_launch(navi_launch_info* info);

/* Hit threshold of the reference tracer (projects/torch-sdf/cpp_src/kernel.cuh:7). */
#define NAVI_DEFAULT_HIT_EPSILON 0.01f

/*
 * Trace n_rays rays through one DAG in the reference's own word layout.
 *
 * Replaces launch_sphere_trace_kernel (projects/torch-sdf/cpp_src/kernel.cuh:27-39,
 * kernel.cu:311-326) as called by cast_rays_forward
 * (projects/torch-sdf/cpp_src/bindings.cpp:43-110). Same arguments, plus:
 *   n_words      number of u64 words in `dag` (every load is bounds-checked;
 *                a ray whose descent leaves the array reports NaN / 0);
 *   n_rays       int64 (the reference narrows B*R to int, bindings.cpp:91);
 *   hit_epsilon  the reference's compile-time kHitEpsilon (pass 0.01f);
 *   out_steps    optional [n_rays] int32 march-loop iteration counts, or NULL;
 *   out_words    optional [n_rays] uint32 counts of DAG words the reference
 *                algorithm loads (load_dag_word calls, kernel.cu:137,198), or
 *                NULL (a separate, slower kernel instance when non-NULL);
 *   stream       the caller's current stream (the reference launches on the
 *                legacy default stream, kernel.cu:320).
 * origins/dirs are [n_rays][3] float32, out_distances [n_rays] float32,
 * out_semantics [n_rays] int32; every output element is written.
 */
int navi_cast_rays(const uint64_t* dag, uint64_t n_words, const float* origins, const float* dirs,
                   float* out_distances, int32_t* out_semantics, int64_t n_rays, int32_t max_steps,
                   float max_distance, const float bbox_min[3], const float bbox_max[3],
                   int32_t resolution, float hit_epsilon, int32_t* out_steps, uint32_t* out_words,
                   void* stream);

/* One resident scene of a multi-scene word pool (device memory, 40 bytes). */
typedef struct navi_scene_desc {
    uint64_t word_offset; /* first word of this scene's DAG in the pool */
    uint64_t n_words;     /* its word count; child pointers are relative to word_offset */
    float bbox_min[3];
    float bbox_max[3];
} navi_scene_desc;

/*
 * Trace n_envs * rays_per_env rays against several resident scenes in one
 * launch: env e traces scenes[env_scene[e]]. The reference holds one DAG per
 * call (projects/environment/src/navi_environment/backends/sdfdag_backend.py:
 * 1897-1905) and its equivalent of this call is one cast_rays per scene over
 * that scene's env subset (sdfdag_backend.py:1215-1217). `scenes` and
 * `env_scene` are device arrays; an env whose scene id is out of range
 * reports NaN / 0 / 0 steps. Outputs as in navi_cast_rays.
 */
int navi_cast_rays_multi(const uint64_t* pool, const navi_scene_desc* scenes, int32_t n_scenes,
                         const int32_t* env_scene, int64_t n_envs, int64_t rays_per_env,
                         const float* origins, const float* dirs, float* out_distances,
                         int32_t* out_semantics, int32_t max_steps, float max_distance,
                         float hit_epsilon, int32_t* out_steps, uint32_t* out_words, void* stream);

/*
 * Device layout (no reference counterpart; it replaces how the reference reads
 * its words, kernel.cu:35-41,137-198). Converts a DAG in the reference word
 * layout (host memory) into 32-byte records of eight u32 octant slots in
 * breadth-first order: 0x7fffffff void, 0x7ffffffe out-of-range child-table
 * word, 0x7ffffffd out-of-range child index (a fault only where the child is
 * examined, above the 32-level descent limit), 0xffff0000 | i a leaf of
 * semantic 0x7fff or above (entry i of the leaf table, navi_relayout_leaves),
 * other values with bit 31 set a leaf inlined (bits 30..16 semantic, 15..0
 * fp16 distance), else a record index. With out_records NULL only counts;
 * otherwise writes up to cap_records records. *root_slot is the root's slot
 * value (0 = record 0, or a leaf of a one-leaf DAG). n_levels_prefix
 * (optional, 8 entries) receives the number of records at depth <= l. When no
 * record lies deeper than 30 levels (navi_record_depth <= 30) every 0x7ffffffd
 * slot is written as 0x7ffffffe: it is examined above the descent limit,
 * where both fault. Returns NAVI_E_LAYOUT for DAGs with a reachable leaf of
 * semantic 0x7fff or above: convert those with navi_relayout_leaves.
 */
int navi_relayout(const uint64_t* words, uint64_t n_words, uint32_t* out_records, uint64_t cap_records,
                  uint64_t* n_records, uint32_t* root_slot, uint64_t* n_levels_prefix);

/*
 * navi_relayout with a leaf table for the leaves whose semantic does not fit
 * the inline slot's 15 bits (the format's field is 16 bits, docs/GMDAG.md:
 * 215,223): each distinct (semantic, distance) pair of semantic 0x7fff or
 * above gets one u32 entry (semantic << 16) | fp16 distance, in order of first
 * sight, and its leaves the slot 0xffff0000 | entry. *n_leaves receives the
 * entry count (0 for a DAG without such leaves); with out_leaves non-NULL the
 * entries are written (at most cap_leaves). At most 65536 entries per table
 * (NAVI_E_LAYOUT beyond). Several scenes in one record pool share one table:
 * concatenate the scenes' tables and add each scene's offset to the low 16
 * bits of its 0xffff0000 slots (the pool's table holds at most 65536 entries).
 */
int navi_relayout_leaves(const uint64_t* words, uint64_t n_words, uint32_t* out_records, uint64_t cap_records,
                         uint64_t* n_records, uint32_t* root_slot, uint64_t* n_levels_prefix,
                         uint32_t* out_leaves, uint32_t cap_leaves, uint32_t* n_leaves);

/* One resident scene in the device layout (device memory, 48 bytes). Several
 * scenes share one record pool: scene records are concatenated and every child
 * record slot (a slot value below 0x7ffffffd) is rebased to an absolute pool
 * index by adding the scene's rec_offset; root_slot is rec_offset for an
 * internal root, or the inlined leaf of a one-leaf DAG. */
typedef struct navi_relaid_scene {
    uint64_t rec_offset;  /* first record of this scene in the record pool */
    uint32_t n_records;
    uint32_t root_slot;
    float bbox_min[3];
    float bbox_max[3];
    uint32_t max_depth;   /* navi_record_depth of the scene's records as navi_relayout wrote
                             them; 0xffffffff if unknown */
    uint32_t flags;       /* NAVI_SCENE_* bits; 0 when unknown */
} navi_relaid_scene;

/* navi_relaid_scene.flags: no leaf slot of the scene's records (nor an inlined
 * root leaf) has its fp16 sign bit set, so distances never decrease along a
 * ray. When every scene of a launch has it (and its boxes are below 2^100),
 * the tracer skips the reference's void cache (kernel.cu:265-267), which then
 * only repeats what a fresh query finds. The tracer trusts the flag: set on a
 * scene with a negative leaf it gives wrong distances. Compute it with
 * navi_scene_flags. */
#define NAVI_SCENE_NONNEG_LEAVES 1u

/*
 * The NAVI_SCENE_* flags a scene's records support (no reference counterpart;
 * host memory): NAVI_SCENE_NONNEG_LEAVES when no leaf reachable from root_slot
 * (nor a root leaf) has its fp16 sign bit set, a table leaf's in `leaves`
 * (n_leaves entries; NULL and 0 for none). Pass the records and root_slot as
 * navi_build_cell_table takes them. Unreachable
 * records are not examined; out-of-range records and cycles end the walk
 * without error (the tracer reports those rays as faults).
 */
int navi_scene_flags(const uint32_t* records, uint64_t n_records, uint32_t root_slot, const uint32_t* leaves,
                     uint32_t n_leaves, uint32_t* flags);

/*
 * Depth of a scene's record graph (no reference counterpart; host memory):
 * the longest chain of internal records below root_slot (the root at depth
 * 0), or 0xffffffff when a cycle or an out-of-range record is reachable.
 * When every scene of a launch has max_depth <= 30 the tracer drops the
 * 32-level descent limit of kernel.cu:136, which such scenes never reach.
 */
int navi_record_depth(const uint32_t* records, uint64_t n_records, uint32_t root_slot, uint32_t* max_depth);

/*
 * Cell table of one scene (no reference counterpart; host memory in and out):
 * 8^depth u64 entries over the 2^depth x 2^depth x 2^depth grid of the cells
 * at that depth, depth in [4, 7]. Entry (iz << (2 * depth)) | (iy << depth) | ix
 * (the cell whose octant at level l has x bit (ix >> (depth - 1 - l)) & 1, y
 * and z likewise) = the slot a descent from the root meets within `depth`
 * levels (bits 31..0: a leaf, void or out-of-range slot, or the record of the
 * internal node at that depth) | its depth (bits 34..32; 0 for a one-leaf
 * DAG). Pass the scene's records and root_slot as the tracer sees them
 * (absolute record indices in a pool), so record slots in the table are
 * absolute too. The tracer's descents start at the table's depth: deeper
 * tables save record reads and cost 8x the memory per level (depth 6: 2 MiB
 * per scene, depth 7: 16 MiB).
 */
int navi_build_cell_table(const uint32_t* records, uint64_t n_records, uint32_t root_slot, int32_t depth,
                          uint64_t* out_table);

/*
 * Throughput tracer over the device layout: n_envs * rays_per_env rays, env e
 * traces scenes[env_scene ? env_scene[e] : 0] (at most 1024 scenes; `records`
 * holds n_records records with absolute child slots, see navi_relaid_scene;
 * cell_tables holds n_scenes cell tables of depth table_depth, 8^table_depth
 * entries each, scene s at s * 8^table_depth, from navi_build_cell_table).
 * Per-ray results are identical
 * to navi_cast_rays / navi_cast_rays_multi on the same DAG. env_order
 * (optional, a permutation of [0, n_envs); an entry outside that range is
 * skipped, its rays left unwritten) is the order envs are swept in — pass
 * envs grouped by scene, so resident scenes stream through the caches one at
 * a time, with the scenes of most steps per ray first: a launch lasts until
 * its slowest wave ends, so long rays should not start last. elevation_bins > 0 (a multiple of 8 dividing rays_per_env / 8)
 * declares the canonical az*El + el ray layout (projects/environment/src/
 * navi_environment/backends/sdfdag_backend.py:205-221) so rays are traced in
 * 8 x 8 angular tiles. Outputs as in navi_cast_rays.
 */
int navi_trace_relaid(const uint32_t* records, uint64_t n_records, const navi_relaid_scene* scenes,
                      int32_t n_scenes, const uint64_t* cell_tables, int32_t table_depth,
                      const int32_t* env_scene, const int32_t* env_order, int64_t n_envs,
                      int64_t rays_per_env, int32_t elevation_bins, const float* origins,
                      const float* dirs, float* out_distances, int32_t* out_semantics,
                      int32_t max_steps, float max_distance, float hit_epsilon, int32_t* out_steps,
                      void* stream);

/*
 * navi_trace_relaid for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. Same arguments and results as
 * navi_trace_relaid; it calls no hipMalloc, hipFree or allocating routine at
 * any time, not even on its first call on a device. Its work-queue counter
 * words live in a static device array of 256 bytes (each GPU the library runs
 * on holds its copy until the process ends), cleared by a small kernel on
 * `stream` before every launch; a launch needs three words whatever its size, so
 * the limits are navi_trace_relaid's (at most 2^30 rays, fewer than 2^27
 * records). Every call on one GPU shares those words: calls that overlap on one
 * GPU (concurrent streams, or graph replays running at once) race and may
 * leave rays unwritten; serialise them, or use navi_trace_relaid.
 */
int navi_trace_relaid_noalloc(const uint32_t* records, uint64_t n_records, const navi_relaid_scene* scenes,
                              int32_t n_scenes, const uint64_t* cell_tables, int32_t table_depth,
                              const int32_t* env_scene, const int32_t* env_order, int64_t n_envs,
                              int64_t rays_per_env, int32_t elevation_bins, const float* origins,
                              const float* dirs, float* out_distances, int32_t* out_semantics,
                              int32_t max_steps, float max_distance, float hit_epsilon, int32_t* out_steps,
                              void* stream);

/*
 * navi_trace_relaid with the rays generated in the kernel from per-env poses
 * (projects/environment/src/navi_environment/backends/sdfdag_backend.py:
 * 1300-1312 computes them with tensor ops and hands 24 bytes per ray to the
 * tracer): ray r of env e starts at env_pos[e] (3 floats) along
 * (x c + z s, y, (-x) s + z c), (x, y, z) = local_dirs[r] (rays_per_env x 3
 * floats, e.g. the az*El + el table of build_spherical_ray_directions,
 * :205-221) and (c, s) = env_rot[e] (cos and sin of the env's yaw). Each
 * product and sum is rounded on its own, as in the reference's eager tensor
 * code, so the rays are bit-identical to ones built that way from the same
 * cos / sin values. Everything else as navi_trace_relaid.
 */
int navi_trace_relaid_poses(const uint32_t* records, uint64_t n_records, const navi_relaid_scene* scenes,
                            int32_t n_scenes, const uint64_t* cell_tables, int32_t table_depth,
                            const int32_t* env_scene,
                            const int32_t* env_order, int64_t n_envs, int64_t rays_per_env,
                            int32_t elevation_bins, const float* local_dirs, const float* env_pos,
                            const float* env_rot, float* out_distances, int32_t* out_semantics,
                            int32_t max_steps, float max_distance, float hit_epsilon, int32_t* out_steps,
                            void* stream);

/* Element type of navi_relaid_launch.out_distances. The march accumulates in
 * float32 either way; a finished ray's distance is rounded to nearest even
 * (NaN as 0x7fc0 in bfloat16, a quiet NaN in float16). The reference's roadmap
 * item for this output: docs/FUTURE_HARDWARE_ROADMAP.md:140-222. */
#define NAVI_DIST_F32 0   /* float */
#define NAVI_DIST_BF16 1  /* bfloat16 (uint16 storage) */
#define NAVI_DIST_F16 2   /* IEEE binary16 */

/* Arguments of navi_trace_relaid_ex (device pointers unless noted). */
typedef struct navi_relaid_launch {
    const uint32_t* records;           /* record pool, as navi_trace_relaid */
    uint64_t n_records;
    const uint32_t* leaves;            /* the pool's leaf table (navi_relayout_leaves), or NULL */
    uint32_t n_leaves;                 /* its entries (0 for none) */
    const navi_relaid_scene* scenes;
    int32_t n_scenes;
    const uint64_t* cell_tables;
    int32_t table_depth;
    const int32_t* env_scene;          /* [n_envs] or NULL (scene 0) */
    const int32_t* env_order;          /* [n_envs] or NULL (in order) */
    int64_t n_envs;
    int64_t rays_per_env;
    int32_t elevation_bins;
    const float* origins;              /* [n_rays][3] explicit rays, or NULL with local_dirs */
    const float* dirs;
    const float* local_dirs;           /* rays from poses, as navi_trace_relaid_poses */
    const float* env_pos;
    const float* env_rot;
    void* out_distances;               /* [n_rays] of distance_dtype */
    int32_t* out_semantics;
    int32_t* out_steps;                /* or NULL */
    int32_t max_steps;
    float max_distance;
    float hit_epsilon;
    int32_t distance_dtype;            /* NAVI_DIST_* (0: float) */
} navi_relaid_launch;

/*
 * navi_trace_relaid / navi_trace_relaid_poses with every argument in one
 * struct (no reference counterpart), adding the leaf table for semantics of
 * 0x7fff and above (the format's 16-bit field, docs/GMDAG.md:215,223) and
 * distances as bfloat16 or float16 (distance_dtype).
 */
int navi_trace_relaid_ex(const navi_relaid_launch* launch, void* stream);

/*
 * Launch shape of the record-layout tracer (no reference counterpart: a tuning
 * knob of this library). Launches of at least `n_rays` rays whose scenes'
 * split planes fit two levels below the cell tables in 80 KiB of LDS run in
 * 1024-thread workgroups (two per CU); smaller launches, whose few workgroups
 * then spread over more CUs, in 256-thread ones. Results are identical either
 * way. Process-wide, thread-safe; takes effect from the next launch. Returns
 * the previous value (default 2^19).
 */
uint64_t navi_set_wide_min_rays(uint64_t n_rays);

/* Point-SDF queries (device pointers; see navi_point_query). */
typedef struct navi_point_queries {
    const uint32_t* records;           /* the record pool of navi_trace_relaid */
    uint64_t n_records;
    const navi_relaid_scene* scenes;
    int32_t n_scenes;
    const uint64_t* cell_tables;       /* cell tables as in navi_trace_relaid */
    int32_t table_depth;
    const int32_t* point_scene;        /* [n_points] scene ids, or NULL: scene 0 */
    const float* points;               /* [n_points][3] */
    int64_t n_points;
    float* out_distances;              /* [n_points] */
    int32_t* out_semantics;            /* [n_points] */
    int32_t* out_kind;                 /* [n_points] or NULL */
    const uint32_t* leaves;            /* the pool's leaf table (navi_relayout_leaves), or NULL */
    uint32_t n_leaves;                 /* its entries (0 for none) */
} navi_point_queries;

/*
 * Point-SDF queries (no reference kernel; the query of
 * projects/torch-sdf/cpp_src/kernel.cu:88-200 from the root, without caches)
 * over the device layout. Point i is looked up in scene point_scene[i].
 * Outputs per point: distance, semantic and, if out_kind is non-NULL, the
 * kind: 0 outside the scene box (1000, 0); 1 leaf (its fp16 distance and
 * semantic); 2 void cell (side along x times 1.7321: the compiler prunes an
 * octant only when every sample in it clears its half-diagonal,
 * projects/voxel-dag/src/compiler.cpp:626,639-643, so this is a clearance
 * lower bound; semantic 0); 3 the 32-level limit (NaN, 0); 4 out-of-range
 * data or an unknown scene id (NaN, 0).
 */
int navi_point_query(const navi_point_queries* queries, void* stream);

/* The observation post-pass (device pointers; see navi_observe). */
typedef struct navi_observation {
    const float* distances;            /* [n_envs][Az * El], flat index az * El + el */
    const int32_t* semantics;          /* [n_envs][Az * El]; needed for obs */
    int64_t n_envs;
    int32_t azimuth_bins, elevation_bins;
    float max_distance;
    float structure_band_min, structure_band_max;  /* reference defaults 1.5, 30 */
    float proximity_threshold;                     /* 2 */
    float collision_clearance;                     /* 0.15 */
    void* depth_f16;                   /* [n_envs][1][El][Az] IEEE binary16, or NULL */
    float* obs;                        /* [n_envs][3][Az][El]: depth, semantic, valid; or NULL */
    float* prev_depth;                 /* [n_envs][Az][El]: read, then overwritten by depth */
    float* delta;                      /* [n_envs][Az][El]: depth - prev_depth, or NULL */
    float* stats;                      /* [n_envs][5], or NULL */
    int32_t* collision;                /* [n_envs], or NULL */
} navi_observation;

/*
 * Observation post-pass in one launch (replaces the tensor code of
 * projects/environment/src/navi_environment/backends/sdfdag_backend.py:
 * 366-473, the collision test of :1340 and the observation stack and delta
 * of :1501-1526), optionally fused with point queries (as navi_point_query;
 * queries may be NULL, observation may be NULL for queries alone). Per env:
 * c = clamp(d, 0, max_distance) (NaN stays NaN); depth = clamp(log1p(c) /
 * log1p(max_distance), 0, 1); depth_f16 = depth transposed to (El, Az); obs =
 * (depth, float(semantic), float(isfinite(d))) in (Az, El) order; delta =
 * depth - prev_depth, or 0 for an env whose prev_depth sums below 1e-6 in
 * absolute value, after which prev_depth holds depth; stats = min c (NaN if
 * any is NaN), starvation ratio (c >= max_distance - 1e-3), proximity ratio
 * (finite and c <= proximity_threshold; 0 if that is <= 0), structure-band
 * ratio (finite and band_min <= c <= band_max; 0 unless band_max > band_min)
 * and forward structure ratio (the same over the first and last
 * max(1, Az / 6) azimuth bins); collision = min c < collision_clearance.
 * With neither obs nor delta asked for, depth_f16 comes from a log1p of
 * binary16 accuracy: within one binary16 ulp of the exact depth (as is the
 * fp16 of the float32 depth otherwise), not always the same bits as the
 * fp16 of the float32 depth.
 */
int navi_observe(const navi_observation* observation, const navi_point_queries* queries, void* stream);

/* Message of the last failure on the calling thread ("" if none). The
 * reference surfaces failures as c10::Error via TORCH_CHECK (bindings.cpp:57-89). */
const char* navi_last_error(void);

/* Library version, "major.minor.patch". */
const char* navi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* NAVI_TRACE_H */
