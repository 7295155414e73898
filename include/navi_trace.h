/*
 * navi_trace.h — C ABI of the MI355X .gmdag sphere tracer (libnavi_trace.so).
 *
 * Plain pointers and sizes only: every device pointer is a HIP device address,
 * `stream` is a hipStream_t passed as void* (NULL = the null stream). All
 * entry points are asynchronous with respect to the host, allocate nothing on
 * the call path, and return 0 on success or a negative NAVI_E* code; the
 * message of the last failure on the calling thread is navi_last_error().
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
#define NAVI_E_NOMEM (-4)   /* device allocation failed (scene build only) */

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
 *   stream       the caller's current stream (the reference launches on the
 *                legacy default stream, kernel.cu:320).
 * origins/dirs are [n_rays][3] float32, out_distances [n_rays] float32,
 * out_semantics [n_rays] int32; every output element is written.
 */
int navi_cast_rays(const uint64_t* dag, uint64_t n_words, const float* origins, const float* dirs,
                   float* out_distances, int32_t* out_semantics, int64_t n_rays, int32_t max_steps,
                   float max_distance, const float bbox_min[3], const float bbox_max[3],
                   int32_t resolution, float hit_epsilon, int32_t* out_steps, void* stream);

/* Message of the last failure on the calling thread ("" if none). The
 * reference surfaces failures as c10::Error via TORCH_CHECK (bindings.cpp:57-89). */
const char* navi_last_error(void);

/* Library version, "major.minor.patch". */
const char* navi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* NAVI_TRACE_H */
