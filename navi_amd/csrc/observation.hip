// observation.hip — what the caller does with a trace, on the device: the
// observation post-pass (clamp, log-normalise, fp16 pack, per-env ratios and
// clearance, projects/environment/src/navi_environment/backends/
// sdfdag_backend.py:366-473 and :1340 of the seismael/navi checkout) and
// point-SDF queries over the device record layout, fused into one launch.
//
// Post-pass: one workgroup per env. The env's Az * El distances (flat index
// az * El + el) are read once, coalesced; every thread keeps counts and the
// minimum in registers, the workgroup reduces them through LDS, and thread 0
// writes the env's statistics. The fp16 depth is written transposed,
// (env, 1, El, Az), the layout the policy consumes.
//
// Point queries: one lane per point, a fresh descent with no caches (the
// query of kernel.cu:88-200 from the root): the cell table gives the first
// D levels, record reads the rest.
#include <hip/hip_runtime.h>

#include <cmath>

#include "navi_trace.h"
#include "trace_common.hpp"

// v_rcp_f32: within one ulp of the correctly rounded reciprocal
__device__ inline float navi_recip(float b) { return __builtin_amdgcn_rcpf(b); }
#define NAVI_MATH_FN __device__ inline
#include "log1p_nonneg.h"

namespace navi {

int set_error(int code, const char* fmt, ...);

namespace {

constexpr uint32_t kSlotVoid = 0x7fffffffu;
constexpr uint32_t kSlotFault = 0x7ffffffeu;
constexpr uint32_t kSlotBadChild = 0x7ffffffdu;
constexpr int kThreads = 512;
constexpr float kVoidClearance = 1.7321f;  // compiler.cpp:626,639-643: pruned octants clear half-diagonal

enum : int32_t { kKindOutside = 0, kKindLeaf = 1, kKindVoid = 2, kKindDepth = 3, kKindFault = 4 };

struct PostParams {
    navi_observation O;  // the post-pass (see include/navi_trace.h)
    int32_t n_envs;
    // The reference compares float32 tensors with Python floats and divides
    // by one: the host rounds max_distance - 1e-3 and log1p(max_distance),
    // evaluated in double, to float, as torch does with such scalars. torch
    // divides a float32 device tensor by such a scalar as a multiplication by
    // its float reciprocal: inv_log_denom = RN(1 / RN(log1p(max_distance))).
    float saturation, inv_log_denom;
    int32_t stage16;  // stage the transposed fp16 tile in LDS (n halves fit)
    // point queries
    const uint32_t* __restrict__ records;
    uint32_t n_records;
    const navi_relaid_scene* __restrict__ scenes;
    int32_t n_scenes;
    const uint64_t* __restrict__ cell_table;  // cell tables, 8^table_depth entries per scene
    uint32_t table_depth;
    const int32_t* __restrict__ point_scene;  // [n_points] or null (scene 0)
    const float* __restrict__ points;         // [n_points][3]
    int32_t n_points;
    float* __restrict__ point_d;
    int32_t* __restrict__ point_s;
    int32_t* __restrict__ point_kind;  // or null
    int32_t env_blocks;                // workgroups doing the post-pass; the rest do points
};

// kernel.cu:88-200 from the root at one point, no caches. Outside the domain:
// (1000, 0); leaf: its distance and semantic; void: the void cell's clearance
// bound, side * 1.7321; 32 levels without a result: NaN; out-of-range data: NaN.
__device__ void point_query(const PostParams& P, int32_t i) {
    const int32_t sc = P.point_scene ? P.point_scene[i] : 0;
    float d = __builtin_nanf("");
    int32_t s = 0, kind = kKindFault;
    if (sc >= 0 && sc < P.n_scenes) {
        const navi_relaid_scene S = P.scenes[sc];
        const float px = P.points[3 * i + 0], py = P.points[3 * i + 1], pz = P.points[3 * i + 2];
        const Box dom{S.bbox_min[0], S.bbox_min[1], S.bbox_min[2], S.bbox_max[0], S.bbox_max[1], S.bbox_max[2]};
        if (!in_box(px, py, pz, dom)) {
            d = kOutsideDomain;
            kind = kKindOutside;
        } else {
            Box cur = dom;
            uint32_t slot = S.root_slot;
            int32_t depth = 0;
            if (!(slot & 0x80000000u)) {
                const uint32_t D = P.table_depth;
                uint32_t jx = 0, jy = 0, jz = 0;
                for (uint32_t l = 0; l < D; ++l) {
                    const uint32_t oct = descend_octant(px, py, pz, cur);
                    jx = 2u * jx + (oct & 1u);
                    jy = 2u * jy + ((oct >> 1) & 1u);
                    jz = 2u * jz + (oct >> 2);
                }
                const uint64_t e = P.cell_table[((((uint32_t)sc << D | jz) << D | jy) << D) | jx];
                slot = static_cast<uint32_t>(e);
                depth = static_cast<int32_t>(e >> 32);
                if (depth < static_cast<int32_t>(D)) {
                    cur = dom;
                    for (int32_t l = 0; l < depth; ++l) {
                        const uint32_t b = D - 1u - static_cast<uint32_t>(l);
                        split_box(cur, ((jx >> b) & 1u) | (((jy >> b) & 1u) << 1) | (((jz >> b) & 1u) << 2));
                    }
                }
                while (slot < kSlotBadChild && depth < kMaxDepth) {
                    const uint32_t oct = descend_octant(px, py, pz, cur);
                    slot = P.records[8u * min(slot, P.n_records - 1u) + oct];
                    ++depth;
                }
            }
            if (slot & 0x80000000u) {
                if (depth < kMaxDepth) {
                    d = half_to_float(slot & 0xffffu);
                    s = static_cast<int32_t>((slot >> 16) & 0x7fffu);
                    kind = kKindLeaf;
                } else {
                    kind = kKindDepth;
                }
            } else if (slot == kSlotVoid) {
                d = (cur.x1 - cur.x0) * kVoidClearance;
                kind = kKindVoid;
            } else if (slot == kSlotFault || (slot == kSlotBadChild && depth < kMaxDepth)) {
                kind = kKindFault;
            } else {
                kind = kKindDepth;
            }
        }
    }
    P.point_d[i] = d;
    P.point_s[i] = s;
    if (P.point_kind) P.point_kind[i] = kind;
}

template <typename T>
__device__ T block_sum(T v, T* lds) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) lds[w] = v;
    __syncthreads();
    T r = 0;
    for (int k = 0; k < kThreads / 64; ++k) r += lds[k];
    return r;
}

// minimum over the workgroup of values that are not NaN
__device__ float block_min(float v, float* lds) {
    for (int off = 32; off > 0; off >>= 1) v = fminf(v, __shfl_xor(v, off));
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) lds[w] = v;
    __syncthreads();
    float r = lds[0];
    for (int k = 1; k < kThreads / 64; ++k) r = fminf(r, lds[k]);
    return r;
}

__global__ __launch_bounds__(kThreads) void observation_kernel(PostParams P) {
    if (static_cast<int32_t>(blockIdx.x) >= P.env_blocks) {
        const int32_t i = (static_cast<int32_t>(blockIdx.x) - P.env_blocks) * kThreads + threadIdx.x;
        if (i < P.n_points) point_query(P, i);
        return;
    }
    extern __shared__ _Float16 lds16[];  // the env's (El, Az) fp16 tile when staged
    __shared__ uint32_t lds_u[kThreads / 64];
    __shared__ float lds_f[kThreads / 64];
    const navi_observation& O = P.O;
    const int32_t e = blockIdx.x;
    const int32_t az = O.azimuth_bins, el = O.elevation_bins;
    const int32_t n = az * el;
    const int64_t base = static_cast<int64_t>(e) * n;
    const float* dist = O.distances + base;
    // sdfdag_backend.py:1510-1514: the delta is zero while the previous depth
    // sums (in absolute value) below 1e-6, i.e. before the first frame
    bool first = false;
    if (O.delta) {
        float acc = 0.0f;
        for (int32_t k = threadIdx.x; k < n; k += kThreads) acc += fabsf(O.prev_depth[base + k]);
        first = block_sum(acc, lds_f) < 1e-6f;
    }
    // sdfdag_backend.py:390: the first and last Az/6 azimuth bins (at least
    // one), i.e. flat indices k < fwd_lo and k >= fwd_hi
    const int32_t fwd = max(1, az / 6);
    const int32_t fwd_lo = fwd * el, fwd_hi = (az - fwd) * el;
    const bool band = O.structure_band_max > O.structure_band_min;
    uint32_t n_sat = 0, n_prox = 0, n_band = 0, n_fwd = 0, n_nan = 0;
    float mn = INFINITY;  // of the clamped values that are not NaN
    // Element k = a * El + r (azimuth bin a, elevation bin r) sits at t = r * Az + a
    // in the transposed fp16 depth. Counters use & rather than && so that
    // they stay branch-free.
    auto element = [&](int32_t k, int32_t t, float m) {
        const bool valid = isfinite(m);
        const bool nan = m != m;
        // torch.clamp(min=0, max=max_distance): both compares are false for NaN
        float c = m < 0.0f ? 0.0f : m;
        c = c > O.max_distance ? O.max_distance : c;
        mn = fminf(mn, c);
        n_nan += nan;
        n_sat += c >= P.saturation;
        n_prox += valid & (c <= O.proximity_threshold);
        const bool in_band = band & valid & (c >= O.structure_band_min) & (c <= O.structure_band_max);
        n_band += in_band;
        // an azimuth bin in both the first and the last Az/6 counts twice, as in torch.cat
        n_fwd += static_cast<uint32_t>(in_band & (k < fwd_lo)) + static_cast<uint32_t>(in_band & (k >= fwd_hi));
        // sdfdag_backend.py:441-443; c >= 0 here, so the log1p of non-negative
        // arguments applies (within one ulp of the exact log1p)
        const float q = nan ? c : fminf(fmaxf(navi_log1p_nonneg(c) * P.inv_log_denom, 0.0f), 1.0f);
        if (O.obs) {  // sdfdag_backend.py:1516-1524: stack(depth, semantic, valid), (Az, El) order
            float* ob = O.obs + 3 * base;
            ob[k] = q;
            ob[n + k] = static_cast<float>(O.semantics[base + k]);
            ob[2 * n + k] = valid ? 1.0f : 0.0f;
        }
        if (O.delta) {  // sdfdag_backend.py:1509-1515
            const float pv = O.prev_depth[base + k];
            O.delta[base + k] = first ? 0.0f : q - pv;
            O.prev_depth[base + k] = q;
        }
        if (O.depth_f16) {
            if (P.stage16) {
                lds16[t] = static_cast<_Float16>(q);
            } else {
                static_cast<_Float16*>(O.depth_f16)[base + t] = static_cast<_Float16>(q);
            }
        }
    };
    // kBatch coalesced loads in flight per thread before any is used. One
    // division per batch; then k advances by kThreads = da * El + dr, i.e. r by
    // dr and t by dr * Az + da, with a carry of one azimuth bin when r wraps.
    constexpr int32_t kBatch = 8;
    const int32_t da = kThreads / el, dr = kThreads - da * el;
    const int32_t dt = dr * az + da, wrap = 1 - el * az;
    for (int32_t k0 = threadIdx.x; k0 < n; k0 += kThreads * kBatch) {
        float m[kBatch];
#pragma unroll
        for (int32_t j = 0; j < kBatch; ++j) {
            const int32_t k = k0 + j * kThreads;
            m[j] = k < n ? dist[k] : 0.0f;
        }
        const int32_t a0 = k0 / el;
        int32_t r = k0 - a0 * el, t = r * az + a0;
#pragma unroll
        for (int32_t j = 0; j < kBatch; ++j) {
            const int32_t k = k0 + j * kThreads;
            if (k < n) element(k, t, m[j]);
            r += dr;
            t += dt;
            if (r >= el) {
                r -= el;
                t += wrap;
            }
            // keep the running (r, t): recomputing them from k costs integer multiplies
            asm volatile("" : "+v"(r), "+v"(t));
        }
    }
    if (O.depth_f16 && P.stage16) {
        __syncthreads();
        uint32_t* out = reinterpret_cast<uint32_t*>(static_cast<_Float16*>(O.depth_f16) + base);
        const uint32_t* src = reinterpret_cast<const uint32_t*>(lds16);
        for (int32_t k = threadIdx.x; k < n / 2; k += kThreads) out[k] = src[k];
    }
    n_sat = block_sum(n_sat, lds_u);
    n_prox = block_sum(n_prox, lds_u);
    n_band = block_sum(n_band, lds_u);
    n_fwd = block_sum(n_fwd, lds_u);
    n_nan = block_sum(n_nan, lds_u);
    mn = block_min(mn, lds_f);
    if (n_nan != 0) mn = __builtin_nanf("");  // torch.amin: NaN if any input is NaN
    if (threadIdx.x == 0) {
        const float fn = static_cast<float>(n);
        if (O.stats) {
            float* st = O.stats + 5 * static_cast<int64_t>(e);
            st[0] = mn;
            st[1] = static_cast<float>(n_sat) / fn;
            st[2] = O.proximity_threshold > 0.0f ? static_cast<float>(n_prox) / fn : 0.0f;
            st[3] = band ? static_cast<float>(n_band) / fn : 0.0f;
            st[4] = band ? static_cast<float>(n_fwd) / static_cast<float>(2 * fwd * el) : 0.0f;
        }
        if (O.collision) O.collision[e] = mn < O.collision_clearance ? 1 : 0;  // sdfdag_backend.py:1340
    }
}

int launch(const PostParams& P, hipStream_t stream) {
    const int64_t point_blocks = (static_cast<int64_t>(P.n_points) + kThreads - 1) / kThreads;
    const int64_t blocks = static_cast<int64_t>(P.env_blocks) + point_blocks;
    if (blocks == 0) return NAVI_OK;
    const size_t lds = P.stage16 ? static_cast<size_t>(P.O.azimuth_bins) * P.O.elevation_bins * 2 : 0;
    hipLaunchKernelGGL(observation_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), lds, stream, P);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return set_error(NAVI_E_LAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
    return NAVI_OK;
}

int points_setup(PostParams& P, const navi_point_queries* Q) {
    if (Q == nullptr || Q->n_points == 0) return NAVI_OK;
    if (Q->n_points < 0 || Q->n_points > (1LL << 30)) return set_error(NAVI_E_ARG, "n_points must be in [0, 2^30]");
    if (!Q->points || !Q->out_distances || !Q->out_semantics)
        return set_error(NAVI_E_ARG, "points and point outputs must be non-null");
    if (Q->n_scenes <= 0 || !Q->scenes || !Q->records || !Q->cell_tables)
        return set_error(NAVI_E_ARG, "scene table, records and cell_tables must be non-empty");
    if (Q->table_depth < 4 || Q->table_depth > 7) return set_error(NAVI_E_ARG, "table_depth must be in [4, 7]");
    if (Q->n_records > (1ull << 29)) return set_error(NAVI_E_ARG, "record pool exceeds 2^29 records");
    P.records = Q->records;
    P.n_records = static_cast<uint32_t>(Q->n_records);
    P.scenes = Q->scenes;
    P.n_scenes = Q->n_scenes;
    P.cell_table = Q->cell_tables;
    P.table_depth = static_cast<uint32_t>(Q->table_depth);
    P.point_scene = Q->point_scene;
    P.points = Q->points;
    P.n_points = static_cast<int32_t>(Q->n_points);
    P.point_d = Q->out_distances;
    P.point_s = Q->out_semantics;
    P.point_kind = Q->out_kind;
    return NAVI_OK;
}

}  // namespace
}  // namespace navi

extern "C" int navi_point_query(const navi_point_queries* queries, void* stream) {
    using namespace navi;
    PostParams P{};
    const int code = points_setup(P, queries);
    if (code != NAVI_OK || P.n_points == 0) return code;
    return launch(P, static_cast<hipStream_t>(stream));
}

extern "C" int navi_observe(const navi_observation* observation, const navi_point_queries* queries, void* stream) {
    using namespace navi;
    PostParams P{};
    if (observation != nullptr && observation->n_envs > 0) {
        const navi_observation& O = *observation;
        if (O.n_envs > 0x7fffffffLL) return set_error(NAVI_E_ARG, "n_envs must be below 2^31");
        if (O.azimuth_bins <= 0 || O.elevation_bins <= 0 ||
            static_cast<int64_t>(O.azimuth_bins) * O.elevation_bins > (1LL << 26))
            return set_error(NAVI_E_ARG, "azimuth_bins and elevation_bins must be positive, product <= 2^26");
        if (!std::isfinite(O.max_distance) || !(O.max_distance > 0.0f))
            return set_error(NAVI_E_ARG, "max_distance must be a finite positive float");
        if (!O.distances) return set_error(NAVI_E_ARG, "distances must be non-null");
        if (O.obs && !O.semantics) return set_error(NAVI_E_ARG, "obs needs semantics");
        if (O.delta && !O.prev_depth) return set_error(NAVI_E_ARG, "delta needs prev_depth");
        P.O = O;
        P.n_envs = static_cast<int32_t>(O.n_envs);
        P.env_blocks = P.n_envs;
        P.saturation = static_cast<float>(static_cast<double>(O.max_distance) - 1e-3);
        P.inv_log_denom = 1.0f / static_cast<float>(std::log1p(static_cast<double>(O.max_distance)));
        const int64_t n = static_cast<int64_t>(O.azimuth_bins) * O.elevation_bins;
        // a 48 KiB tile at most, and an even count for the 4-byte copy out
        P.stage16 = (O.depth_f16 != nullptr && n % 2 == 0 && n * 2 <= 48 * 1024) ? 1 : 0;
    }
    const int code = points_setup(P, queries);
    if (code != NAVI_OK) return code;
    return launch(P, static_cast<hipStream_t>(stream));
}
