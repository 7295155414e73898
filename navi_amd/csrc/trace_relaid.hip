// trace_relaid.hip — the throughput tracer over the device record layout
// (relayout.cpp). Same per-ray results as the reference-layout kernel, which
// restates projects/torch-sdf/cpp_src/kernel.cu:88-309 (seismael/navi checkout).
//
// Execution model (CDNA4, wave64):
//   * persistent waves: the grid holds about as many waves as the chip keeps
//     resident; wave w walks 64-ray chunks w, w + W, w + 2W, ... of the work
//     order, so all waves sweep the batch front to back together;
//   * lane refill: a lane whose ray finished takes the next ray of its wave's
//     chunk sequence at once (ballot + prefix popcount), so a wave never idles
//     on a few long rays;
//   * if-if state machine: every loop iteration a lane either starts a march
//     step (caches answer most of them without memory traffic) or descends one
//     DAG level with a single 4-byte gather; lanes that finish a level or a
//     cached step in the same iteration are not held back by deeper ones;
//   * work order: envs in the order given (callers sort them by scene so the
//     resident scenes stream through L2 / MALL one or two at a time) and, when
//     the elevation count is a multiple of 8, 8 x 8 (az x el) tiles of the
//     canonical az*El + el ray layout, so a chunk's rays are angular
//     neighbours that share DAG nodes.
#include <hip/hip_runtime.h>

#include <cmath>

#include "navi_trace.h"
#include "trace_common.hpp"

namespace navi {

int set_error(int code, const char* fmt, ...);

constexpr uint32_t kSlotVoid = 0x7fffffffu;
constexpr uint32_t kSlotFault = 0x7ffffffeu;

struct RelaidParams {
    const uint32_t* __restrict__ records;
    const navi_relaid_scene* __restrict__ scenes;
    int32_t n_scenes;
    const int32_t* __restrict__ env_scene;  // null: every env uses scene 0
    const int32_t* __restrict__ env_order;  // null: identity
    int64_t n_envs;
    int64_t rays_per_env;
    int32_t tile_el;  // elevation bins when 8x8 tiling applies, else 0
    const float* __restrict__ origins;
    const float* __restrict__ dirs;
    float* __restrict__ out_d;
    int32_t* __restrict__ out_s;
    int32_t* __restrict__ out_steps;
    int32_t max_steps;
    float max_distance;
    float hit_eps;
    int64_t n_chunks;
};

// Work index q -> ray id (env * R + r).
__device__ __forceinline__ int64_t ray_of(const RelaidParams& P, int64_t q, int32_t& env_out) {
    const int64_t env_pos = q / P.rays_per_env;
    const int64_t qi = q - env_pos * P.rays_per_env;
    int64_t r = qi;
    if (P.tile_el > 0) {
        const int64_t tiles_el = P.tile_el >> 3;
        const int64_t tile = qi >> 6;
        const int64_t l = qi & 63;
        const int64_t ta = tile / tiles_el;
        const int64_t te = tile - ta * tiles_el;
        r = (ta * 8 + (l & 7)) * P.tile_el + te * 8 + (l >> 3);
    }
    const int32_t env = P.env_order ? P.env_order[env_pos] : static_cast<int32_t>(env_pos);
    env_out = env;
    return static_cast<int64_t>(env) * P.rays_per_env + r;
}

__device__ __forceinline__ float slot_dist(uint32_t s) { return half_to_float(s & 0xffffu); }
__device__ __forceinline__ int32_t slot_sem(uint32_t s) { return static_cast<int32_t>((s >> 16) & 0x7fffu); }

__global__ __launch_bounds__(256) void trace_relaid_kernel(RelaidParams P) {
    const uint32_t lane = threadIdx.x & 63u;
    const int64_t wave = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
    const int64_t n_waves = (static_cast<int64_t>(gridDim.x) * blockDim.x) >> 6;
    const int64_t n_rays = P.n_envs * P.rays_per_env;
    // this wave's chunks: wave, wave + n_waves, ...
    const int64_t my_chunks = wave < P.n_chunks ? (P.n_chunks - wave + n_waves - 1) / n_waves : 0;
    const int64_t seq_end = my_chunks * 64;
    int64_t seq_next = 0;  // wave-uniform
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));

    // per-lane ray state
    bool has_ray = false;
    int64_t ray = 0;
    float ox = 0.f, oy = 0.f, oz = 0.f, dx = 0.f, dy = 0.f, dz = 0.f;
    float t = 0.f, dist = 0.f, px = 0.f, py = 0.f, pz = 0.f;
    int32_t sem = 0, step = 0;
    const uint32_t* rec = P.records;
    uint32_t root_slot = 0, n_rec = 0;
    Box dom{}, lf{}, vd{}, pre{}, cur{};
    uint32_t lf_slot = 0, pre_rec = 0, cur_rec = 0;
    int32_t depth = 0;
    bool lf_ok = false, vd_ok = false, pre_ok = false, fresh = false, descending = false;

    while (true) {
        // ---- refill lanes without a ray from the wave's chunk sequence ----
        const uint64_t need = __ballot(!has_ray);
        if (need != 0ull && seq_next < seq_end) {
            if (!has_ray) {
                const int64_t s = seq_next + __popcll(need & lt_mask);
                if (s < seq_end) {
                    const int64_t q = (wave + (s >> 6) * n_waves) * 64 + (s & 63);
                    if (q < n_rays) {
                        int32_t env;
                        ray = ray_of(P, q, env);
                        const int32_t sc = P.env_scene ? P.env_scene[env] : 0;
                        ox = P.origins[3 * ray + 0];
                        oy = P.origins[3 * ray + 1];
                        oz = P.origins[3 * ray + 2];
                        dx = P.dirs[3 * ray + 0];
                        dy = P.dirs[3 * ray + 1];
                        dz = P.dirs[3 * ray + 2];
                        t = 0.f;
                        dist = 0.f;
                        sem = 0;
                        step = 0;
                        lf_ok = vd_ok = pre_ok = descending = false;
                        has_ray = true;
                        if (sc < 0 || sc >= P.n_scenes) {
                            // unknown scene: report like a fault, no steps
                            P.out_d[ray] = __builtin_nanf("");
                            P.out_s[ray] = 0;
                            if (P.out_steps) P.out_steps[ray] = 0;
                            has_ray = false;
                        } else {
                            const navi_relaid_scene d = P.scenes[sc];
                            rec = P.records + 8 * d.rec_offset;
                            root_slot = d.root_slot;
                            n_rec = d.n_records;
                            dom = Box{d.bbox_min[0], d.bbox_min[1], d.bbox_min[2],
                                      d.bbox_max[0], d.bbox_max[1], d.bbox_max[2]};
                        }
                    }
                }
            }
            seq_next += __popcll(need);
        }
        if (__ballot(has_ray) == 0ull) {
            if (seq_next >= seq_end) break;
            continue;
        }

        bool resolved = false, stale = false, fault = false;
        float rd = 0.f;
        int32_t rs = 0;

        // ---- start a march step (kernel.cu:260-269 and query :108-132) ----
        if (has_ray && !descending) {
            step += 1;
            px = __builtin_fmaf(t, dx, ox);
            py = __builtin_fmaf(t, dy, oy);
            pz = __builtin_fmaf(t, dz, oz);
            if (vd_ok && in_box_strict(px, py, pz, vd)) {
                rd = exit_distance(px, py, pz, dx, dy, dz, vd);
                resolved = true;
            } else if (!in_box(px, py, pz, dom)) {
                rd = kOutsideDomain;
                resolved = true;
            } else if (lf_ok && in_box(px, py, pz, lf)) {
                rd = slot_dist(lf_slot);
                rs = slot_sem(lf_slot);
                resolved = true;
            } else if (pre_ok && in_box(px, py, pz, pre)) {
                cur = pre;
                cur_rec = pre_rec;
                depth = kPrefixDepth;
                fresh = false;
                descending = true;
            } else if (root_slot & 0x80000000u) {  // the root itself is a leaf
                lf = dom;
                lf_slot = root_slot;
                lf_ok = true;
                rd = slot_dist(lf_slot);
                rs = slot_sem(lf_slot);
                resolved = true;
            } else {
                cur = dom;
                cur_rec = root_slot;
                depth = 0;
                fresh = true;
                descending = true;
            }
        }

        // ---- one descent level (kernel.cu:136-199) ----
        if (descending) {
            if (fresh && depth == kPrefixDepth) {
                pre = cur;
                pre_rec = cur_rec;
                pre_ok = true;
            }
            const uint32_t oct = descend_octant(px, py, pz, cur);
            // records come from navi_relayout; the bound keeps a corrupt table in memory
            const uint32_t slot = cur_rec < n_rec ? rec[8 * cur_rec + oct] : kSlotFault;
            if (slot == kSlotVoid) {
                vd = cur;
                vd_ok = true;
                rd = exit_distance(px, py, pz, dx, dy, dz, vd);
                resolved = true;
                descending = false;
            } else if (slot == kSlotFault) {
                fault = true;
                resolved = true;
                descending = false;
            } else if (slot & 0x80000000u) {
                // the reference examines this child at depth + 1 (< 32 required)
                if (depth + 1 < kMaxDepth) {
                    lf = cur;
                    lf_slot = slot;
                    lf_ok = true;
                    rd = slot_dist(slot);
                    rs = slot_sem(slot);
                } else {
                    stale = true;
                }
                resolved = true;
                descending = false;
            } else {
                depth += 1;
                cur_rec = slot;
                if (depth >= kMaxDepth) {  // 32 levels without leaf or void: stale
                    stale = true;
                    resolved = true;
                    descending = false;
                }
            }
        }

        // ---- finish the step (kernel.cu:297-308) ----
        if (resolved) {
            bool done = false;
            if (fault) {
                P.out_d[ray] = __builtin_nanf("");
                P.out_s[ray] = 0;
                done = true;
            } else {
                if (!stale) {
                    dist = rd;
                    sem = rs;
                }
                if (sem != 0 && dist < P.hit_eps) {
                    P.out_d[ray] = t;
                    P.out_s[ray] = sem;
                    done = true;
                } else {
                    t += dist;
                    if (t > P.max_distance || step >= P.max_steps) {
                        P.out_d[ray] = t;
                        P.out_s[ray] = 0;
                        done = true;
                    }
                }
            }
            if (done) {
                if (P.out_steps) P.out_steps[ray] = step;
                has_ray = false;
            }
        }
    }
}

int g_cu_count = 0;

int launch_relaid(const RelaidParams& base, hipStream_t stream) {
    RelaidParams P = base;
    const int64_t n_rays = P.n_envs * P.rays_per_env;
    P.n_chunks = (n_rays + 63) / 64;
    if (g_cu_count == 0) {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
        g_cu_count = cus;
    }
    const int threads = 256;
    const int64_t waves_wanted = P.n_chunks;
    const int64_t max_blocks = static_cast<int64_t>(g_cu_count) * 8;  // 32 waves per CU
    int64_t blocks = (waves_wanted + 3) / 4;
    if (blocks > max_blocks) blocks = max_blocks;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(trace_relaid_kernel, dim3(static_cast<unsigned>(blocks)), dim3(threads), 0, stream, P);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return set_error(NAVI_E_LAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
    return NAVI_OK;
}

}  // namespace navi

extern "C" int navi_trace_relaid(const uint32_t* records, const navi_relaid_scene* scenes, int32_t n_scenes,
                                 const int32_t* env_scene, const int32_t* env_order, int64_t n_envs,
                                 int64_t rays_per_env, int32_t elevation_bins, const float* origins,
                                 const float* dirs, float* out_distances, int32_t* out_semantics,
                                 int32_t max_steps, float max_distance, float hit_epsilon,
                                 int32_t* out_steps, void* stream) {
    using namespace navi;
    if (max_steps <= 0) return set_error(NAVI_E_ARG, "max_steps must be a positive integer");
    if (!std::isfinite(max_distance) || !(max_distance > 0.0f))
        return set_error(NAVI_E_ARG, "max_distance must be a finite positive float");
    if (!(hit_epsilon == hit_epsilon)) return set_error(NAVI_E_ARG, "hit_epsilon must not be NaN");
    if (n_envs < 0 || rays_per_env < 0) return set_error(NAVI_E_ARG, "n_envs and rays_per_env must be non-negative");
    if (n_scenes <= 0 || !scenes || !records) return set_error(NAVI_E_ARG, "scene table must be non-empty");
    if (n_envs * rays_per_env == 0) return NAVI_OK;
    if (!origins || !dirs || !out_distances || !out_semantics)
        return set_error(NAVI_E_ARG, "ray and output pointers must be non-null");
    RelaidParams P{};
    P.records = records;
    P.scenes = scenes;
    P.n_scenes = n_scenes;
    P.env_scene = env_scene;
    P.env_order = env_order;
    P.n_envs = n_envs;
    P.rays_per_env = rays_per_env;
    P.tile_el = (elevation_bins > 0 && elevation_bins % 8 == 0 && rays_per_env % (8LL * elevation_bins) == 0)
                    ? elevation_bins
                    : 0;
    P.origins = origins;
    P.dirs = dirs;
    P.out_d = out_distances;
    P.out_s = out_semantics;
    P.out_steps = out_steps;
    P.max_steps = max_steps;
    P.max_distance = max_distance;
    P.hit_eps = hit_epsilon;
    return launch_relaid(P, static_cast<hipStream_t>(stream));
}
