// observation.hip — what the caller does with a trace, on the device: the
// observation post-pass (clamp, log-normalise, fp16 pack, per-env ratios and
// clearance, projects/environment/src/navi_environment/backends/
// sdfdag_backend.py:366-473 and :1340 of the seismael/navi checkout) and
// point-SDF queries over the device record layout, fused into one launch.
//
// Post-pass: one workgroup per env, compiled for the set of outputs asked for.
// The env's Az * El distances (flat index az * El + el) are read once,
// coalesced (16-byte loads when Az * El and El are multiples of 4); counts are
// wave ballots summed on the scalar unit, the minimum a per-lane register; one
// LDS exchange gives thread 0 the workgroup's totals for the env's statistics.
// The fp16 depth is written transposed, (env, 1, El, Az), the layout the policy
// consumes, through an LDS tile with an odd row pitch. The kernel moves
// 6 bytes per ray (4 read, 2 written) and is bound by HBM: every term of the
// per-element work is kept to what the scalar and vector units can issue in
// the time those bytes take, and all workgroups of a 1024-env launch are
// resident at once (8 waves per SIMD).
//
// Point queries: one lane per point, a fresh descent with no caches (the
// query of kernel.cu:88-200 from the root): the cell table gives the first
// D levels, record reads the rest. Up to 64 points per env ride in the env
// workgroups (lanes of their first wave, before the env's pass), so that a
// launch needs no workgroups beyond one per env; more points get workgroups of
// their own.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <type_traits>

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
    int32_t stage16;  // stage the transposed fp16 tile in LDS (Az even, the tile fits)
    int32_t pitch;    // the tile's row pitch in halves: El rounded up to odd
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
    int32_t point_blocks;              // workgroups answering point queries only; the rest do envs
    int32_t points_per_env;            // > 0: env workgroup e also answers points [e * ppe, (e + 1) * ppe)
    const uint32_t* __restrict__ leaves;  // leaf table (slots 0xffff0000 | i), or null
    uint32_t n_leaves;
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
                    // an inline leaf (15-bit semantic), or a leaf-table entry (16-bit;
                    // 0 past the table's end)
                    uint32_t w = slot & 0x7fffffffu;
                    if ((slot & 0xffff0000u) == 0xffff0000u)
                        w = (P.leaves != nullptr && (slot & 0xffffu) < P.n_leaves) ? P.leaves[slot & 0xffffu] : 0u;
                    d = half_to_float(w & 0xffffu);
                    s = static_cast<int32_t>(w >> 16);
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

// log1p(c) for finite c >= 0 (NaN propagates) to the accuracy of the binary16
// depth, for launches that write no float32 depth: log(1 + c) = log2(u) ln 2 +
// log(1 + e / u), u = RN(1 + c), e = c - (u - 1) the rounding error of 1 + c
// (exact). log(1 + e / u) is taken as e (2 - u) for u < 2 (e / u to a relative
// (u - 1)^2, on a term below 2^-24 / c of the result) and as 0 for u >= 2
// (below 2^-24 / ln 2 of the result). v_log_f32 is the hardware base-2
// logarithm, a quarter-rate instruction: this is about a third of the vector
// instructions of navi_log1p_nonneg. The depth rounded to binary16 is within
// one binary16 ulp of the exact value for every input (checked on the device
// for every float in [0, max_distance] against log1p in float64).
__device__ inline float depth16_log1p(float c) {
    const float u = 1.0f + c;
    const float e = c - (u - 1.0f);
    return fmaf(__builtin_amdgcn_logf(u), 0x1.62e430p-1f, e * fmaxf(2.0f - u, 0.0f));
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

// the wave's lanes for which b holds
__device__ inline uint64_t ballot(bool b) { return __builtin_amdgcn_ballot_w64(b); }
__device__ inline uint32_t popc(uint64_t m) { return static_cast<uint32_t>(__popcll(m)); }

// the lanes l of a wave with base + l < limit, for a base uniform over the wave
__device__ inline uint64_t lanes_below(int32_t base, int32_t limit) {
    const int32_t c = limit - base;
    return c <= 0 ? 0ull : c >= 64 ? ~0ull : (1ull << c) - 1ull;
}

constexpr int kRed = 6;  // per-wave partials: five counts and the minimum's bits

// The post-pass of one env. kObs / kDelta: the float32 observation stack and the
// delta depth are written; kF16: the fp16 depth is not written (0), written
// straight to its transposed place (1), or staged in the LDS tile (2).
//
// Element k = a * El + r (azimuth bin a, elevation bin r) belongs at t = r * Az + a
// of the transposed fp16 depth. Staged, it goes to tile[a * pitch + r]: the reads
// of dist are coalesced along k, so a wave's lanes write consecutive halves, and
// the copy-out reads, for consecutive t, halves pitch apart, which falls in
// distinct banks for every lane of a wave since pitch is odd. The counts are
// ballots: one compare per element on the vector unit, the masks of the forward
// sector and of the env's end computed on the scalar unit from the wave's first k.
template <bool kObs, bool kDelta, int kF16>
__device__ void observe_env(const PostParams& P, int32_t e, _Float16* tile, uint32_t* red) {
    const navi_observation& O = P.O;
    const int32_t az = O.azimuth_bins, el = O.elevation_bins;
    const int32_t n = az * el;
    const int64_t base = static_cast<int64_t>(e) * n;
    const float* dist = O.distances + base;
    const int32_t tid = static_cast<int32_t>(threadIdx.x);
    const int32_t wave0 = __builtin_amdgcn_readfirstlane(tid);  // the wave's first thread
    // sdfdag_backend.py:1510-1514: the delta is zero while the previous depth
    // sums (in absolute value) below 1e-6, i.e. before the first frame
    bool first = false;
    if constexpr (kDelta) {
        float acc = 0.0f;
        for (int32_t k = tid; k < n; k += kThreads) acc += fabsf(O.prev_depth[base + k]);
        first = block_sum(acc, reinterpret_cast<float*>(red)) < 1e-6f;
        __syncthreads();  // red is reused below
    }
    // sdfdag_backend.py:390: the first and last Az/6 azimuth bins (at least
    // one), i.e. flat indices k < fwd_lo and k >= fwd_hi
    const int32_t fwd = max(1, az / 6);
    const int32_t fwd_lo = fwd * el, fwd_hi = (az - fwd) * el;
    const bool band = O.structure_band_max > O.structure_band_min;
    const uint64_t band_lanes = band ? ~0ull : 0ull;
    const float maxd = O.max_distance, sat = P.saturation, prox = O.proximity_threshold;
    const float bmin = O.structure_band_min, bmax = O.structure_band_max;
    const float inv = P.inv_log_denom;
    const int32_t pitch = P.pitch;
    uint32_t n_sat = 0, n_prox = 0, n_band = 0, n_fwd = 0, n_nan = 0;
    float mn = INFINITY;  // of the clamped values; with a NaN input the result is NaN anyway
    int32_t b0 = 0;
    // Launches that write only the fp16 depth (and the statistics): 16-byte
    // loads, lane l holding elements 4l .. 4l + 3 of each 256-element run of
    // its wave. With El % 4 == 0 the four share an azimuth bin (one tile row,
    // consecutive columns) and the forward sector (its bounds are multiples of
    // El), so the row and column are advanced and the sector mask is formed
    // once per four elements.
    if constexpr (kF16 == 2 && !kObs && !kDelta) {
        if ((n & 3) == 0 && (el & 3) == 0 && fwd_lo <= fwd_hi && (reinterpret_cast<uintptr_t>(dist) & 15) == 0) {
            constexpr int32_t kVec = 3;  // 16-byte loads in flight per thread
            constexpr int32_t kStep4 = 4 * kThreads * kVec;
            const int32_t da4 = (4 * kThreads) / el, dr4 = 4 * kThreads - da4 * el;
            uint64_t nan_any = 0;
            auto element = [&](float x, uint64_t fwd_mask, int32_t at) {
                const uint64_t nan = ballot(x != x);
                const uint64_t valid = ballot(x - x == 0.0f);  // finite
                const float c = __builtin_amdgcn_fmed3f(x, 0.0f, maxd);
                mn = fminf(mn, c);
                nan_any |= nan;
                n_sat += popc(ballot(c >= sat) & ~nan);
                n_prox += popc(ballot(c <= prox) & valid);
                // with band_max <= band_min these counts are not reported
                const uint64_t in_band = ballot(c >= bmin) & ballot(c <= bmax) & valid;
                n_band += popc(in_band);
                n_fwd += popc(in_band & fwd_mask);
                float lq = depth16_log1p(c);
                asm volatile("" : "+v"(lq));  // computed for every lane: no branch around it
                const float q = x != x ? x : fminf(fmaxf(lq * inv, 0.0f), 1.0f);
                tile[at] = static_cast<_Float16>(q);
            };
            for (; b0 + kStep4 <= n; b0 += kStep4) {
                const float4* d4 = reinterpret_cast<const float4*>(dist + b0);
                float4 m[kVec];
#pragma unroll
                for (int32_t v = 0; v < kVec; ++v) m[v] = d4[tid + v * kThreads];
                const int32_t k4 = b0 + 4 * tid;
                int32_t a = k4 / el;
                int32_t r = k4 - a * el;
#pragma unroll
                for (int32_t v = 0; v < kVec; ++v) {
                    const int32_t kv = k4 + 4 * v * kThreads;
                    const uint64_t fwd_mask = ballot(kv < fwd_lo || kv >= fwd_hi);
                    const int32_t at = __umul24(a, pitch) + r;
                    element(m[v].x, fwd_mask, at);
                    element(m[v].y, fwd_mask, at + 1);
                    element(m[v].z, fwd_mask, at + 2);
                    element(m[v].w, fwd_mask, at + 3);
                    r += dr4;
                    a += da4;
                    if (r >= el) {
                        r -= el;
                        ++a;
                    }
                    asm volatile("" : "+v"(r), "+v"(a));
                }
            }
            n_nan = nan_any != 0 ? 1u : 0u;  // only whether any is NaN is used
        }
    }
    // The general pass (and what the 16-byte pass leaves): kBatch coalesced
    // loads in flight per thread before any is used. One division per batch;
    // then k advances by kThreads = da * El + dr, i.e. r by dr and a by da,
    // with a carry of one azimuth bin when r wraps.
    constexpr int32_t kBatch = 8;
    const int32_t da = kThreads / el, dr = kThreads - da * el;
    auto run = [&](auto tail, int32_t b0) {
        constexpr bool kTail = decltype(tail)::value;
        const int32_t k0 = b0 + tid;
        float m[kBatch];
#pragma unroll
        for (int32_t j = 0; j < kBatch; ++j) {
            const int32_t k = k0 + j * kThreads;
            m[j] = (!kTail || k < n) ? dist[k] : 0.0f;
        }
        int32_t a = k0 / el;
        int32_t r = k0 - a * el;
#pragma unroll
        for (int32_t j = 0; j < kBatch; ++j) {
            const int32_t k = k0 + j * kThreads;
            const int32_t kw = b0 + wave0 + j * kThreads;  // k of the wave's lane 0
            const uint64_t live = kTail ? lanes_below(kw, n) : ~0ull;
            const float x = m[j];
            // one compare per ballot, combined on the scalar unit
            const uint64_t nan = ballot(x != x) & live;
            const uint64_t valid = ballot(x - x == 0.0f) & live;  // finite
            // torch.clamp(min=0, max=max_distance); NaN lanes are excluded below
            // by their mask, so what the median gives them is never used
            const float c = __builtin_amdgcn_fmed3f(x, 0.0f, maxd);
            if (!kTail || k < n) mn = fminf(mn, c);
            n_nan += popc(nan);
            n_sat += popc(ballot(c >= sat) & live & ~nan);
            n_prox += popc(ballot(c <= prox) & valid);
            const uint64_t in_band = ballot(c >= bmin) & ballot(c <= bmax) & valid & band_lanes;
            n_band += popc(in_band);
            // an azimuth bin in both the first and the last Az/6 counts twice, as in torch.cat
            n_fwd += popc(in_band & lanes_below(kw, fwd_lo)) + popc(in_band & ~lanes_below(kw, fwd_hi));
            // sdfdag_backend.py:441-443; c >= 0 here, so the log1p of non-negative
            // arguments applies (within one ulp of the exact log1p, or of the
            // binary16 depth where only that is written)
            float q = 0.0f;
            if constexpr (kObs || kDelta || kF16 != 0) {
                float lq = (kObs || kDelta) ? navi_log1p_nonneg(c) : depth16_log1p(c);
                asm volatile("" : "+v"(lq));  // computed for every lane: no branch around it
                q = x != x ? x : fminf(fmaxf(lq * inv, 0.0f), 1.0f);
            }
            if (!kTail || k < n) {
                if constexpr (kObs) {  // sdfdag_backend.py:1516-1524: stack(depth, semantic, valid), (Az, El) order
                    float* ob = O.obs + 3 * base;
                    ob[k] = q;
                    ob[n + k] = static_cast<float>(O.semantics[base + k]);
                    ob[2 * n + k] = x - x == 0.0f ? 1.0f : 0.0f;
                }
                if constexpr (kDelta) {  // sdfdag_backend.py:1509-1515
                    const float pv = O.prev_depth[base + k];
                    O.delta[base + k] = first ? 0.0f : q - pv;
                    O.prev_depth[base + k] = q;
                }
                if constexpr (kF16 == 1)
                    static_cast<_Float16*>(O.depth_f16)[base + __umul24(r, az) + a] = static_cast<_Float16>(q);
                if constexpr (kF16 == 2) tile[__umul24(a, pitch) + r] = static_cast<_Float16>(q);
            }
            r += dr;
            a += da;
            if (r >= el) {
                r -= el;
                ++a;
            }
            // keep the running (a, r): recomputing them from k costs integer multiplies
            asm volatile("" : "+v"(r), "+v"(a));
        }
    };
    constexpr int32_t kStep = kThreads * kBatch;
    for (; b0 + kStep <= n; b0 += kStep) run(std::integral_constant<bool, false>{}, b0);
    if (b0 < n) run(std::integral_constant<bool, true>{}, b0);
    for (int off = 32; off > 0; off >>= 1) mn = fminf(mn, __shfl_xor(mn, off));
    const int32_t w = tid >> 6;
    if ((tid & 63) == 0) {
        uint32_t* o = red + kRed * w;
        o[0] = n_sat;
        o[1] = n_prox;
        o[2] = n_band;
        o[3] = n_fwd;
        o[4] = n_nan;
        o[5] = __float_as_uint(mn);
    }
    __syncthreads();
    if constexpr (kF16 == 2) {
        _Float16* const out16 = static_cast<_Float16*>(O.depth_f16) + base;
        const uint16_t* src = reinterpret_cast<const uint16_t*>(tile);
        if ((az & 3) == 0 && (reinterpret_cast<uintptr_t>(out16) & 7) == 0) {
            // Az % 4 == 0: halves t .. t + 3 (t = 4i) share r, at tile[a * pitch + r] and
            // pitch, 2 pitch, 3 pitch further; one 8-byte store per lane
            uint2* out = reinterpret_cast<uint2*>(out16);
            int32_t r = (4 * tid) / az;
            int32_t a = 4 * tid - r * az;
            const int32_t dr4 = (4 * kThreads) / az, da4 = 4 * kThreads - dr4 * az;
            for (int32_t i = tid; i < n / 4; i += kThreads) {
                const int32_t at = __umul24(a, pitch) + r;
                const uint32_t h0 = src[at], h1 = src[at + pitch], h2 = src[at + 2 * pitch], h3 = src[at + 3 * pitch];
                out[i] = make_uint2(h0 | (h1 << 16), h2 | (h3 << 16));
                r += dr4;
                a += da4;
                if (a >= az) {
                    a -= az;
                    ++r;
                }
            }
        } else {
            // Az is even: halves t and t + 1 share r, at tile[a * pitch + r] and pitch further
            uint32_t* out = reinterpret_cast<uint32_t*>(out16);
            int32_t r = (2 * tid) / az;
            int32_t a = 2 * tid - r * az;
            const int32_t dr2 = (2 * kThreads) / az, da2 = 2 * kThreads - dr2 * az;
            for (int32_t i = tid; i < n / 2; i += kThreads) {
                const int32_t at = __umul24(a, pitch) + r;
                out[i] = static_cast<uint32_t>(src[at]) | (static_cast<uint32_t>(src[at + pitch]) << 16);
                r += dr2;
                a += da2;
                if (a >= az) {
                    a -= az;
                    ++r;
                }
            }
        }
    }
    if (tid == 0) {
        uint32_t c[kRed - 1] = {0, 0, 0, 0, 0};
        float lo = INFINITY;
        for (int32_t v = 0; v < kThreads / 64; ++v) {
            for (int32_t j = 0; j < kRed - 1; ++j) c[j] += red[kRed * v + j];
            lo = fminf(lo, __uint_as_float(red[kRed * v + 5]));
        }
        if (c[4] != 0) lo = __builtin_nanf("");  // torch.amin: NaN if any input is NaN
        const float fn = static_cast<float>(n);
        if (O.stats) {
            float* st = O.stats + 5 * static_cast<int64_t>(e);
            st[0] = lo;
            st[1] = static_cast<float>(c[0]) / fn;
            st[2] = O.proximity_threshold > 0.0f ? static_cast<float>(c[1]) / fn : 0.0f;
            st[3] = band ? static_cast<float>(c[2]) / fn : 0.0f;
            st[4] = band ? static_cast<float>(c[3]) / static_cast<float>(2 * fwd * el) : 0.0f;
        }
        if (O.collision) O.collision[e] = lo < O.collision_clearance ? 1 : 0;  // sdfdag_backend.py:1340
    }
}

// Workgroups [0, point_blocks) answer point queries, one lane each; they come
// first so that their chains of dependent record reads start with the launch.
// The rest do the post-pass, one env each, the first wave's first
// points_per_env lanes answering that env's share of the points beforehand.
// Eight waves per SIMD: four 512-thread workgroups per CU, so that a launch of
// 1024 envs is resident at once.
template <bool kObs, bool kDelta, int kF16>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(8))) void observation_kernel(PostParams P) {
    if (static_cast<int32_t>(blockIdx.x) < P.point_blocks) {
        const int32_t i = static_cast<int32_t>(blockIdx.x) * kThreads + threadIdx.x;
        if (i < P.n_points) point_query(P, i);
        return;
    }
    const int32_t e = static_cast<int32_t>(blockIdx.x) - P.point_blocks;
    if (static_cast<int32_t>(threadIdx.x) < P.points_per_env) {
        const int64_t i = static_cast<int64_t>(e) * P.points_per_env + threadIdx.x;
        if (i < P.n_points) point_query(P, static_cast<int32_t>(i));
    }
    extern __shared__ _Float16 tile[];  // the env's fp16 tile when staged
    __shared__ uint32_t red[kRed * (kThreads / 64)];
    observe_env<kObs, kDelta, kF16>(P, e, tile, red);
}

template <bool kObs, bool kDelta, int kF16>
int launch_as(const PostParams& P, hipStream_t stream, unsigned blocks, size_t lds) {
    hipLaunchKernelGGL((observation_kernel<kObs, kDelta, kF16>), dim3(blocks), dim3(kThreads), lds, stream, P);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return set_error(NAVI_E_LAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
    return NAVI_OK;
}

template <bool kObs, bool kDelta>
int launch_f16(const PostParams& P, hipStream_t stream, unsigned blocks, size_t lds) {
    if (!P.O.depth_f16) return launch_as<kObs, kDelta, 0>(P, stream, blocks, lds);
    if (P.stage16) return launch_as<kObs, kDelta, 2>(P, stream, blocks, lds);
    return launch_as<kObs, kDelta, 1>(P, stream, blocks, lds);
}

int launch(PostParams& P, hipStream_t stream) {
    int64_t point_blocks = (static_cast<int64_t>(P.n_points) + kThreads - 1) / kThreads;
    P.points_per_env = 0;
    if (P.n_envs > 0 && P.n_points > 0 && static_cast<int64_t>(P.n_points) <= 64LL * P.n_envs) {
        // every env workgroup takes up to 64 points: no extra workgroups
        P.points_per_env = static_cast<int32_t>((static_cast<int64_t>(P.n_points) + P.n_envs - 1) / P.n_envs);
        point_blocks = 0;
    }
    const int64_t blocks = static_cast<int64_t>(P.n_envs) + point_blocks;
    if (blocks == 0) return NAVI_OK;
    P.point_blocks = static_cast<int32_t>(point_blocks);
    const size_t lds = P.stage16 ? static_cast<size_t>(P.O.azimuth_bins) * P.pitch * 2 : 0;
    const unsigned b = static_cast<unsigned>(blocks);
    if (P.O.obs) return P.O.delta ? launch_f16<true, true>(P, stream, b, lds) : launch_f16<true, false>(P, stream, b, lds);
    return P.O.delta ? launch_f16<false, true>(P, stream, b, lds) : launch_f16<false, false>(P, stream, b, lds);
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
    if (Q->n_leaves > 0 && !Q->leaves) return set_error(NAVI_E_ARG, "leaves must be non-null when n_leaves > 0");
    P.leaves = Q->n_leaves > 0 ? Q->leaves : nullptr;
    P.n_leaves = Q->n_leaves;
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
        P.saturation = static_cast<float>(static_cast<double>(O.max_distance) - 1e-3);
        P.inv_log_denom = 1.0f / static_cast<float>(std::log1p(static_cast<double>(O.max_distance)));
        // a 48 KiB tile at most, and an even Az for the 4-byte copy out
        P.pitch = O.elevation_bins | 1;
        P.stage16 = (O.depth_f16 != nullptr && O.azimuth_bins % 2 == 0 &&
                     static_cast<int64_t>(O.azimuth_bins) * P.pitch * 2 <= 48 * 1024) ? 1 : 0;
    }
    const int code = points_setup(P, queries);
    if (code != NAVI_OK) return code;
    return launch(P, static_cast<hipStream_t>(stream));
}
