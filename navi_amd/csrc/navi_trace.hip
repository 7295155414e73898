// navi_trace.hip — libnavi_trace.so: C-ABI entry points and the tracer kernel
// that walks the reference's own u64 word layout (the drop-in path).
//
// Reference semantics: projects/torch-sdf/cpp_src/kernel.cu:88-309 (paths relative
// to the seismael/navi checkout). The per-ray cache state machine (leaf cache,
// void cache, depth-4 prefix cache, with the reference's inclusive / strict box
// tests) is carried exactly, because the caches change results on box faces.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "navi_trace.h"
#include "trace_common.hpp"

namespace navi {

int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));  // errors.cpp
extern thread_local char g_last_error[512];                                          // errors.cpp

// Bounds-checked word load (kernel.cu:35-41 without the LDS copy, which only
// caches the same words). Out of range sets `fault`.
__device__ __forceinline__ uint64_t load_word(const uint64_t* __restrict__ dag, uint64_t n_words,
                                              uint32_t idx, bool& fault) {
    if (static_cast<uint64_t>(idx) >= n_words) {
        fault = true;
        return 0;
    }
    return dag[idx];
}

// Scene lookup for the raw-layout kernels: the single-scene entry point passes
// one descriptor by value; the multi-scene one reads env_scene[ray / R].
struct RawScene {
    const uint64_t* words;
    uint64_t n_words;
    Box dom;
    bool valid;
};

// One lane per ray; the loop body is kernel.cu:260-305 with query_dag_stackless
// (kernel.cu:88-200) inlined. kMulti: per-env scene table. kCount: also count
// the DAG words the reference algorithm loads (kernel.cu:137,198) per ray.
template <bool kMulti, bool kCount>
__global__ __launch_bounds__(256) void trace_raw_kernel(
    const uint64_t* __restrict__ pool, uint64_t n_words, Box dom0,
    const navi_scene_desc* __restrict__ scenes, int32_t n_scenes, const int32_t* __restrict__ env_scene,
    int64_t rays_per_env, const float* __restrict__ origins, const float* __restrict__ dirs,
    float* __restrict__ out_d, int32_t* __restrict__ out_s, int32_t* __restrict__ out_steps,
    uint32_t* __restrict__ out_words, int64_t n_rays, int32_t max_steps, float max_distance,
    float hit_eps) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n_rays) return;

    RawScene sc{pool, n_words, dom0, true};
    if constexpr (kMulti) {
        const int32_t s = env_scene[i / rays_per_env];
        if (s < 0 || s >= n_scenes) {
            sc.valid = false;
        } else {
            const navi_scene_desc d = scenes[s];
            sc.words = pool + d.word_offset;
            sc.n_words = d.n_words;
            sc.dom = Box{d.bbox_min[0], d.bbox_min[1], d.bbox_min[2], d.bbox_max[0], d.bbox_max[1], d.bbox_max[2]};
        }
    }
    const uint64_t* __restrict__ dag = sc.words;
    const Box dom = sc.dom;

    const float ox = origins[3 * i + 0], oy = origins[3 * i + 1], oz = origins[3 * i + 2];
    const float dx = dirs[3 * i + 0], dy = dirs[3 * i + 1], dz = dirs[3 * i + 2];

    float t = 0.0f, dist = 0.0f;
    int32_t sem = 0;
    // caches (kernel.cu:236-247)
    uint32_t pre_ptr = 0;
    Box pre = dom, vd = dom, lf = dom;
    bool pre_ok = false, vd_ok = false, lf_ok = false;
    float lf_dist = 0.0f;
    int32_t lf_sem = 0;
    bool fault = !sc.valid;
    bool hit = false;
    int32_t steps = 0;
    uint32_t words = 0;

    for (int32_t step = 0; step < max_steps && !fault; ++step) {
        steps = step + 1;
        const float px = __builtin_fmaf(t, dx, ox);
        const float py = __builtin_fmaf(t, dy, oy);
        const float pz = __builtin_fmaf(t, dz, oz);
        if (vd_ok && in_box_strict(px, py, pz, vd)) {  // kernel.cu:265-267
            dist = exit_distance(px, py, pz, dx, dy, dz, vd);
            sem = 0;
        } else if (!in_box(px, py, pz, dom)) {  // kernel.cu:108-112
            dist = kOutsideDomain;
            sem = 0;
        } else if (lf_ok && in_box(px, py, pz, lf)) {  // kernel.cu:114-118
            dist = lf_dist;
            sem = lf_sem;
        } else {
            const bool use_pre = pre_ok && in_box(px, py, pz, pre);  // kernel.cu:120-132
            uint32_t ptr = use_pre ? pre_ptr : 0u;
            Box cur = use_pre ? pre : dom;
            for (int depth = use_pre ? kPrefixDepth : 0; depth < kMaxDepth; ++depth) {
                if constexpr (kCount) ++words;
                const uint64_t node = load_word(dag, sc.n_words, ptr, fault);
                if (fault) break;
                if (node >> 63) {  // leaf, kernel.cu:139-152
                    lf = cur;
                    lf_dist = half_to_float(static_cast<uint32_t>(node));
                    lf_sem = static_cast<int32_t>((node >> 16) & 0xffffu);
                    lf_ok = true;
                    dist = lf_dist;
                    sem = lf_sem;
                    break;
                }
                if (!use_pre && depth == kPrefixDepth) {  // kernel.cu:154-163
                    pre_ptr = ptr;
                    pre = cur;
                    pre_ok = true;
                }
                const uint32_t oct = descend_octant(px, py, pz, cur);
                const uint32_t mask = static_cast<uint32_t>(node >> 55) & 0xffu;
                if (!(mask & (1u << oct))) {  // void, kernel.cu:179-190
                    vd = cur;
                    vd_ok = true;
                    dist = exit_distance(px, py, pz, dx, dy, dz, vd);
                    sem = 0;
                    break;
                }
                const uint32_t slot = static_cast<uint32_t>(node) +
                                      static_cast<uint32_t>(__builtin_popcount(mask & ((1u << oct) - 1u)));
                if constexpr (kCount) ++words;
                ptr = static_cast<uint32_t>(load_word(dag, sc.n_words, slot, fault));
                if (fault) break;
            }
            if (fault) break;
        }
        if (sem != 0 && dist < hit_eps) {  // kernel.cu:297-301
            hit = true;
            break;
        }
        t += dist;  // kernel.cu:302-304
        if (t > max_distance) break;
    }
    out_d[i] = fault ? __builtin_nanf("") : t;
    out_s[i] = (hit && !fault) ? sem : 0;
    if (out_steps) out_steps[i] = steps;
    if constexpr (kCount) out_words[i] = words;
}

}  // namespace navi

namespace navi {

extern thread_local navi_launch_info g_last_launch;  // trace_relaid.hip

int launch_raw(const uint64_t* pool, uint64_t n_words, Box dom, const navi_scene_desc* scenes,
               int32_t n_scenes, const int32_t* env_scene, int64_t rays_per_env, const float* origins,
               const float* dirs, float* out_d, int32_t* out_s, int32_t* out_steps, uint32_t* out_words,
               int64_t n_rays, int32_t max_steps, float max_distance, float hit_eps, void* stream) {
    const int threads = 256;
    const int64_t blocks = (n_rays + threads - 1) / threads;
    if (blocks > 0x7fffffff) return set_error(NAVI_E_ARG, "too many rays for one launch");
    g_last_launch = navi_launch_info{};
    g_last_launch.kernels = NAVI_KERNEL_RAW;
    g_last_launch.pair = -1;
    g_last_launch.n_rays = static_cast<uint64_t>(n_rays);
    g_last_launch.waves = static_cast<uint32_t>(blocks * (threads / 64));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid(static_cast<unsigned>(blocks)), block(threads);
    const bool multi = scenes != nullptr;
    const bool count = out_words != nullptr;
#define NAVI_LAUNCH_RAW(M, C)                                                                       \
    hipLaunchKernelGGL((trace_raw_kernel<M, C>), grid, block, 0, s, pool, n_words, dom, scenes,     \
                       n_scenes, env_scene, rays_per_env, origins, dirs, out_d, out_s, out_steps, \
                       out_words, n_rays, max_steps, max_distance, hit_eps)
    if (multi && count) NAVI_LAUNCH_RAW(true, true);
    else if (multi) NAVI_LAUNCH_RAW(true, false);
    else if (count) NAVI_LAUNCH_RAW(false, true);
    else NAVI_LAUNCH_RAW(false, false);
#undef NAVI_LAUNCH_RAW
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return set_error(NAVI_E_LAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
    return NAVI_OK;
}

}  // namespace navi

using namespace navi;

extern "C" {

int navi_cast_rays(const uint64_t* dag, uint64_t n_words, const float* origins, const float* dirs,
                   float* out_distances, int32_t* out_semantics, int64_t n_rays, int32_t max_steps,
                   float max_distance, const float bbox_min[3], const float bbox_max[3],
                   int32_t resolution, float hit_epsilon, int32_t* out_steps, uint32_t* out_words,
                   void* stream) {
    g_last_error[0] = '\0';
    // Same contract as bindings.cpp:83-86 and :10-21.
    if (max_steps <= 0) return set_error(NAVI_E_ARG, "max_steps must be a positive integer");
    if (!std::isfinite(max_distance) || !(max_distance > 0.0f))
        return set_error(NAVI_E_ARG, "max_distance must be a finite positive float");
    if (resolution <= 0) return set_error(NAVI_E_ARG, "resolution must be a positive integer");
    if (!bbox_min || !bbox_max) return set_error(NAVI_E_ARG, "bbox_min and bbox_max must each contain exactly 3 floats");
    for (int a = 0; a < 3; ++a) {
        if (!std::isfinite(bbox_min[a])) return set_error(NAVI_E_ARG, "bbox_min must contain only finite floats");
        if (!std::isfinite(bbox_max[a])) return set_error(NAVI_E_ARG, "bbox_max must contain only finite floats");
        if (!(bbox_min[a] < bbox_max[a]))
            return set_error(NAVI_E_ARG, "bbox_min entries must be strictly less than bbox_max entries");
    }
    if (n_rays < 0) return set_error(NAVI_E_ARG, "n_rays must be non-negative");
    if (n_words == 0 || !dag) return set_error(NAVI_E_ARG, "dag must hold at least one word");
    if (!(hit_epsilon == hit_epsilon)) return set_error(NAVI_E_ARG, "hit_epsilon must not be NaN");
    if (n_rays == 0) return NAVI_OK;
    if (!origins || !dirs || !out_distances || !out_semantics)
        return set_error(NAVI_E_ARG, "ray and output pointers must be non-null");

    const Box dom{bbox_min[0], bbox_min[1], bbox_min[2], bbox_max[0], bbox_max[1], bbox_max[2]};
    return launch_raw(dag, n_words, dom, nullptr, 0, nullptr, 1, origins, dirs, out_distances,
                      out_semantics, out_steps, out_words, n_rays, max_steps, max_distance, hit_epsilon,
                      stream);
}

int navi_cast_rays_multi(const uint64_t* pool, const navi_scene_desc* scenes, int32_t n_scenes,
                         const int32_t* env_scene, int64_t n_envs, int64_t rays_per_env,
                         const float* origins, const float* dirs, float* out_distances,
                         int32_t* out_semantics, int32_t max_steps, float max_distance,
                         float hit_epsilon, int32_t* out_steps, uint32_t* out_words, void* stream) {
    g_last_error[0] = '\0';
    if (max_steps <= 0) return set_error(NAVI_E_ARG, "max_steps must be a positive integer");
    if (!std::isfinite(max_distance) || !(max_distance > 0.0f))
        return set_error(NAVI_E_ARG, "max_distance must be a finite positive float");
    if (!(hit_epsilon == hit_epsilon)) return set_error(NAVI_E_ARG, "hit_epsilon must not be NaN");
    if (n_envs < 0 || rays_per_env < 0) return set_error(NAVI_E_ARG, "n_envs and rays_per_env must be non-negative");
    if (n_scenes <= 0 || !scenes || !pool || !env_scene) return set_error(NAVI_E_ARG, "scene table must be non-empty");
    const int64_t n_rays = n_envs * rays_per_env;
    if (n_rays == 0) return NAVI_OK;
    if (!origins || !dirs || !out_distances || !out_semantics)
        return set_error(NAVI_E_ARG, "ray and output pointers must be non-null");
    return launch_raw(pool, 0, Box{}, scenes, n_scenes, env_scene, rays_per_env, origins, dirs,
                      out_distances, out_semantics, out_steps, out_words, n_rays, max_steps,
                      max_distance, hit_epsilon, stream);
}

}  // extern "C"
