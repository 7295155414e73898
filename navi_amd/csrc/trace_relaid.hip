// trace_relaid.hip — the throughput tracer over the device record layout
// (relayout.cpp). Per-ray results are identical to the reference-layout kernel,
// which restates projects/torch-sdf/cpp_src/kernel.cu:88-309 (seismael/navi
// checkout); tests compare both against the CPU oracle bit for bit.
//
// Execution model (CDNA4, wave64):
//   * two kernels: the fast march (monotone, tame, shallow scenes with split
//     planes, the library compiler's) alone in trace_fast_kernel at eight
//     waves per SIMD, in two 1024-thread workgroups per CU for launches of at
//     least 2^19 rays (planes up to two levels below the cell table) or eight
//     256-thread ones, everything in trace_relaid_kernel at seven; a launch
//     enqueues the first when its planes fit, the second after it (returning
//     at once when the first traced the launch), see launch_relaid;
//   * persistent waves: the grid holds as many workgroups as the chip keeps
//     resident; waves claim work units (128 rays = two 8 x 8 tiles, or one
//     tile for batches too small to fill the chip) from a counter pair of
//     the launch's stream (or of the graph node it was captured into), the
//     last wave rearming it; without a counter (all 4096 pairs in use) wave
//     w takes 64-ray chunks w, w + W, ...;
//   * lane refill: once 8 (fast march: 12) of 64 lanes have finished their rays, the idle lanes
//     take the next rays (ballot + mbcnt rank), so a wave never idles on a few
//     long rays;
//   * one march step per outer iteration for every lane: the void / domain /
//     leaf / prefix tests; a descent, from the root or the cached prefix
//     cell, locates its depth-D cell (split planes staged in LDS, or splits)
//     and reads one cell-table entry; then a per-lane loop reads one 4-byte
//     slot per level until every lane of the wave has its leaf / void cell;
//     then the step resolves with selects, and lanes whose step was a leaf
//     take one more step if the leaf cache answers it alone;
//   * work order: envs in the order given (callers sort them by scene so the
//     resident scenes stream through L2 / MALL one or two at a time, the
//     costliest scenes first so the launch ends on short rays) and, when
//     the elevation count is a multiple of 8, 8 x 8 (az x el) tiles of the
//     canonical az*El + el ray layout, so a wave's rays are angular
//     neighbours that share DAG nodes.
// Launch-wide facts checked once per workgroup remove work without changing
// results: `tame` scene boxes (coordinates below 2^100), `shallow` scenes (no
// record deeper than 30 levels) and split planes close to a uniform grid.
// Arithmetic: the void-cell exit divides (kernel.cu:54-85) use a per-ray
// correctly rounded reciprocal and one Markstein correction,
// q = fma(fma(-a*r, b, a), r, a*r), which equals the IEEE quotient a/b when
// r = RN(1/b) and nothing over/underflows. Only quotients of at least 1e-5
// can reach the result (the exit is clamped below at 1e-5), and for those,
// with |b| > 1e-4 and tame boxes, every intermediate is a normal number;
// other launches take the IEEE division. 32-bit work indexing with
// multiply-high division by the (uniform) rays-per-env and tile counts.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <map>
#include <mutex>
#include <thread>
#include <unordered_map>
#include <utility>
#include <vector>

#include "navi_trace.h"
#include "trace_common.hpp"

// Structured buffer loads (the index scaled by the resource's stride in the
// address unit): the LLVM intrinsics, which clang exposes only in their raw form.
extern "C" __device__ uint32_t navi_struct_load_b32(__amdgpu_buffer_rsrc_t rsrc, int32_t index, int32_t voffset,
                                                     int32_t soffset, int32_t aux)
    __asm("llvm.amdgcn.struct.ptr.buffer.load.i32");
typedef uint32_t navi_u32x2 __attribute__((ext_vector_type(2)));
extern "C" __device__ navi_u32x2 navi_struct_load_b64(__amdgpu_buffer_rsrc_t rsrc, int32_t index, int32_t voffset,
                                                       int32_t soffset, int32_t aux)
    __asm("llvm.amdgcn.struct.ptr.buffer.load.v2i32");

namespace navi {

int set_error(int code, const char* fmt, ...);

constexpr uint32_t kSlotVoid = 0x7fffffffu;
constexpr uint32_t kSlotFault = 0x7ffffffeu;     // child-table word out of range
constexpr uint32_t kSlotBadChild = 0x7ffffffdu;  // child index out of range; lowest terminal value

// Division by a runtime-invariant divisor d >= 1 (Granlund-Montgomery):
// n / d = (t + ((n - t) >> 1)) >> (l - 1), t = mulhi(n, m), for all 32-bit n.
struct FastDiv {
    uint32_t d, m, l;
};

inline FastDiv make_fastdiv(uint32_t d) {
    FastDiv f{d, 0u, 0u};
    if (d <= 1) return f;
    uint32_t l = 0;
    while ((1ull << l) < d) ++l;
    f.l = l;
    f.m = static_cast<uint32_t>(((1ull << 32) * ((1ull << l) - d)) / d + 1);
    return f;
}

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
    if (f.d <= 1) return n;
    const uint32_t t = __umulhi(n, f.m);
    return (t + ((n - t) >> 1)) >> (f.l - 1);
}

static_assert(sizeof(navi_relaid_scene) == 48, "navi_relaid_scene is 48 bytes");

struct RelaidParams {
    const uint32_t* __restrict__ records;
    uint32_t n_records;  // records in the pool (child slots are absolute indices)
    const navi_relaid_scene* __restrict__ scenes;
    int32_t n_scenes;
    const uint64_t* __restrict__ cell_table;  // cell tables, 8^cell_depth entries per scene
    uint32_t cell_depth;                      // D in [4, 7]: descents start at depth D
    const int32_t* __restrict__ env_scene;  // null: every env uses scene 0
    const int32_t* __restrict__ env_order;  // null: identity
    uint32_t n_rays;
    uint32_t n_envs;
    uint32_t rays_per_env;
    FastDiv div_rays;      // by rays_per_env
    uint32_t tile_el;      // elevation bins when 8x8 tiling applies, else 0
    FastDiv div_tiles_el;  // by tile_el / 8
    const float* __restrict__ origins;  // [n_rays][3], or null with local_dirs
    const float* __restrict__ dirs;
    // Ray generation from poses (when local_dirs is non-null): ray r of env e
    // starts at env_pos[e] along R_y(yaw_e) local_dirs[r], env_rot[e] = (cos, sin).
    const float* __restrict__ local_dirs;  // [rays_per_env][3]
    const float* __restrict__ env_pos;     // [n_envs][3]
    const float* __restrict__ env_rot;     // [n_envs][2]
    float* __restrict__ out_d;  // of dist_dtype elements
    int32_t* __restrict__ out_s;
    int32_t* __restrict__ out_steps;
    int32_t max_steps;
    float max_distance;
    float hit_eps;
    uint32_t n_chunks;
    uint32_t* __restrict__ queue;  // [next unit, finished waves], or null: static schedule
    uint32_t n_units;              // work units of unit_rays rays
    uint32_t unit_rays;            // 128 (2 tiles), or 64 for batches too small to fill the chip
    uint32_t small_tables;         // the cell tables span fewer than 2^32 bytes
    uint32_t dist_dtype;           // NAVI_DIST_*: out_d holds float, bfloat16 or float16
    uint32_t stage;                // finished rays staged per tile in LDS (fast march)
    uint32_t after_fast;           // launched after trace_fast_kernel: return if that one ran
    // leaf table of the leaves of semantic 0x7fff or above (slot 0xffff0000 | i
    // holds entry i: semantic << 16 | fp16 distance), or null; sem_bits is 16
    // with a table (the march then keeps leaf words without their slot bit),
    // else 15 (the inline slot's field)
    const uint32_t* __restrict__ leaves;
    uint32_t n_leaves;
    uint32_t sem_bits;
};

constexpr uint32_t kTableLeaf = 0xffff0000u;  // a leaf slot of the leaf table (low 16 bits: entry)

// The leaf word of a leaf slot with its slot bit cleared: semantic in bits
// 31..16 (16 bits), fp16 distance in 15..0; a table leaf's entry, 0 past the
// table's end (distance +0, semantic 0).
__device__ __forceinline__ uint32_t table_leaf_word(uint32_t slot, const uint32_t* leaves, uint32_t n_leaves) {
    if ((slot & kTableLeaf) != kTableLeaf) return slot & 0x7fffffffu;
    const uint32_t i = slot & 0xffffu;
    return i < n_leaves ? leaves[i] : 0u;
}

// Work index q -> ray id (env * R + r).
__device__ __forceinline__ uint32_t ray_of(const RelaidParams& P, uint32_t q, int32_t& env_out) {
    const uint32_t env_pos = fdiv(q, P.div_rays);
    const uint32_t qi = q - env_pos * P.rays_per_env;
    uint32_t r = qi;
    if (P.tile_el) {
        const uint32_t tile = qi >> 6;
        const uint32_t l = qi & 63u;
        const uint32_t ta = fdiv(tile, P.div_tiles_el);
        const uint32_t te = tile - ta * (P.tile_el >> 3);
        r = (ta * 8u + (l & 7u)) * P.tile_el + te * 8u + (l >> 3);
    }
    const int32_t env = P.env_order ? P.env_order[env_pos] : static_cast<int32_t>(env_pos);
    env_out = env;
    return static_cast<uint32_t>(env) * P.rays_per_env + r;
}

// a / b for the exit distance: Markstein-corrected product with r = RN(1/b);
// equal to the IEEE quotient when nothing over/underflows. NaN when r is.
__device__ __forceinline__ float markstein(float a, float b, float r) {
    const float q0 = a * r;
    const float e = __builtin_fmaf(-q0, b, a);
    return __builtin_fmaf(e, r, q0);
}

// A finished ray's distance into out_d[i] as the launch's element type:
// float, or rounded to nearest even to bfloat16 (NaN as 0x7fc0) or float16.
// Non-temporal: lines of these scattered stores do not stay in L2.
__device__ __forceinline__ void store_distance(const RelaidParams& P, uint32_t i, float t) {
    if (P.dist_dtype == NAVI_DIST_F32) {
        __builtin_nontemporal_store(t, &P.out_d[i]);
        return;
    }
    uint16_t h;
    if (P.dist_dtype == NAVI_DIST_BF16) {
        const uint32_t u = __float_as_uint(t);
        h = (t != t) ? static_cast<uint16_t>(0x7fc0u) : static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
    } else {
        h = __builtin_bit_cast(uint16_t, static_cast<_Float16>(t));
    }
    __builtin_nontemporal_store(h, reinterpret_cast<uint16_t*>(P.out_d) + i);
}

// LDS addresses as 32-bit byte offsets (the local address space) and back
typedef __attribute__((address_space(3))) uint32_t lds_u32;
__device__ __forceinline__ uint32_t lds_address(uint32_t* p) {
    return static_cast<uint32_t>(reinterpret_cast<size_t>((lds_u32*)p));
}
__device__ __forceinline__ lds_u32* lds_pointer(uint32_t addr) { return (lds_u32*)static_cast<size_t>(addr); }

// v with its sign flipped where d's sign bit is set (exact): a coordinate in
// the frame mirrored along each axis on which the ray moves towards -inf
__device__ __forceinline__ float mirror(float v, float d) {
    return __uint_as_float(__float_as_uint(v) ^ (__float_as_uint(d) & 0x80000000u));
}

// The face of [lo, hi] ahead of a ray moving along d, in the mirrored frame:
// hi where d's sign bit is clear, -lo where it is set.
__device__ __forceinline__ float ahead(float lo, float hi, float d) {
    return __float_as_int(d) < 0 ? -lo : hi;
}

constexpr uint32_t kRefillMin = 8;
constexpr uint32_t kLeafRun = 1;  // leaf-cache steps taken after a leaf step
// The fast march's: its step costs fewer operations, so a lane waits less on
// a wave's longer runs (measured on the 16-scene 1024^3 batch: 2 leaf-cache
// steps 1.5% faster than 1, refills at 12 idle lanes 1% faster than at 8).
constexpr uint32_t kLeafRunFast = 2;
constexpr uint32_t kRefillMinFast = 12;
// rays per dynamically claimed work unit (2 tiles): larger units leave more rays
// held by one wave when the queue runs dry, smaller ones cost more claims
constexpr uint32_t kUnitRays = 128;
constexpr uint32_t kSmallUnitRays = 64;  // one tile, for small batches
// Output staging of the fast march: each wave keeps two tiles (64 rays) in
// LDS slots, a finished ray's distance and semantic go to its tile's slot, and
// a slot is written out when a new tile takes it over (the slots alternate) or
// the wave ends: eight consecutive lanes then store eight consecutive rays,
// whole 32-byte sectors, where a finished ray's own store writes 4 bytes of a
// line that L2 has long evicted before the rest of its tile is done. A slot
// position whose semantic is kStageEmpty holds no result (semantics are
// 15-bit leaf values or 0).
constexpr uint32_t kStageSlots = 2;
constexpr uint32_t kStageWords = 128;  // per slot: 64 distances, then 64 semantics
constexpr uint32_t kStageEmpty = 0xffffffffu;
constexpr uint32_t kNoTile = 0xffffffffu;
// staging bytes of a workgroup of `threads` threads
__host__ __device__ constexpr size_t stage_lds(int threads) {
    return static_cast<size_t>(threads / 64) * kStageSlots * kStageWords * sizeof(uint32_t);
}
constexpr size_t kStageLds = stage_lds(256);

// A scene as the kernel reads it, staged in LDS once per workgroup so a lane
// keeps only its scene index in registers.
struct SceneLds {
    float x0, y0, z0, x1, y1, z1;
    uint32_t root;  // absolute record of the root, or the inlined root leaf
    uint32_t pad;
};
constexpr int32_t kMaxScenes = 1024;  // 32 KiB of LDS
// Split planes of the first P levels, per scene: the scales n / (hi - lo) of
// x, y and z and a pad float, the offsets -lo * scale - 0.25 of x, y and z and
// a pad float, then per axis the n + 1 planes P_0 = lo, ..., P_n = hi of the
// n = 2^P depth-P cells and a pad float, the scene's block rounded up to 16
// bytes. The general kernel stages the deepest P (at most 6, at most
// two levels above the cell table) whose scene table and planes fit kPlaneLds
// bytes (seven 256-thread workgroups, 7 waves per SIMD, within a CU's 160 KiB
// of LDS); failing that, the deepest that fits kPlaneLdsWide (five
// workgroups): measured, planes at 6 or 5 waves per SIMD beat none at 7 (90
// scenes: 13%, 110: 5%), a deeper P at 6 waves loses to a shallower one at 7,
// and planes at 4 waves lose to none.
constexpr size_t kPlaneLds = 22528;
constexpr size_t kPlaneLdsWide = 32512;
// The fast kernel's LDS per workgroup in its 256-thread shape: eight
// workgroups per CU (planes at most 6 levels, at most two above the table).
constexpr size_t kFastLds = 20480;
// The wide fast kernel: two 1024-thread workgroups per CU (eight waves per
// SIMD), each with half the CU's 160 KiB of LDS, room for split planes two
// levels below the cell table (the first two levels below the table then take
// their octants from the plane index: no midpoints, comparisons or selects).
constexpr int kWideThreads = 1024;
constexpr size_t kFastLdsWide = 81920;
// Launches of fewer rays take the 256-thread workgroups: a small batch's few
// workgroups then spread over more CUs (the wide grid holds as many waves, in
// a quarter of the workgroups). Measured: 786 K rays on one 512^3 scene 3%
// faster wide, 49 K rays 8% slower. navi_set_wide_min_rays changes it.
constexpr uint64_t kWideMinRays = 1u << 19;
std::atomic<uint64_t> g_wide_min_rays{kWideMinRays};
// Launches of fewer rays skip the 256-thread fast kernel: the combined kernel
// alone (its fast march at seven waves; such batches are bound by the latency
// of their rays' chains, not by occupancy) saves the second launch (64^3 box
// room 0.054 -> 0.053 ms, 49 K rays 0.111 -> 0.108 ms). With the default wide
// threshold every larger launch whose planes fit takes the wide shape; the
// 256-thread fast kernel serves launches between this and a raised one.
constexpr uint32_t kFastMinRays = 1u << 19;
__host__ __device__ constexpr uint32_t axis_stride(uint32_t depth) { return (1u << depth) + 2u; }
constexpr uint32_t kPlaneHeader = 8;  // floats before the planes: scales, pad, offsets, pad
__host__ __device__ constexpr uint32_t scene_stride(uint32_t depth) {
    return (kPlaneHeader + 3u * axis_stride(depth) + 3u) & ~3u;
}

// Split planes of every scene and axis for n = 2^P cells (pl[k] = P_k, then
// a pad float), with the per-axis scale and offset, computed by the whole
// workgroup: the nested midpoints level by level with the descent's own
// operations (kernel.cu:165-176), so cell boxes are the descent's boxes bit
// for bit. Returns (to every thread) whether they support the direct cell
// lookup of plane_cell: finite, each within 0.2 cell of the uniform grid, an
// accurate scale, and an offset below 2^14 in magnitude (so it is exact to
// 2^-10 cell).
template <int kPD>
__device__ bool stage_planes(const RelaidParams& P, float* lds_planes) {
    constexpr uint32_t kAxis = axis_stride(kPD);    // floats per axis
    constexpr uint32_t kScene = scene_stride(kPD);  // floats per scene
    constexpr uint32_t n = 1u << kPD;               // cells per axis
    const uint32_t pairs = 3u * static_cast<uint32_t>(P.n_scenes);
    int ok = 1;
    for (uint32_t i = threadIdx.x; i < pairs; i += blockDim.x) {
        const navi_relaid_scene& d = P.scenes[i / 3u];
        const uint32_t a = i % 3u;
        float* hdr = lds_planes + (i / 3u) * kScene;
        float* pl = hdr + kPlaneHeader + a * kAxis;
        const float lo = d.bbox_min[a], hi = d.bbox_max[a];
        pl[0] = lo;
        pl[n] = hi;
        pl[n + 1] = 0.0f;
        const float w = hi - lo;
        const float scale = static_cast<float>(n) / w;
        const float off = __builtin_fmaf(-lo, scale, -0.25f);
        const double cw = (static_cast<double>(hi) - static_cast<double>(lo)) / n;
        ok &= (w > 0.0f && w <= 0x1p127f && scale > 0.0f && scale <= 0x1p127f && cw > 0.0 &&
               fabs(static_cast<double>(scale) * cw - 1.0) <= 1e-6 && fabsf(off) <= 0x1p14f) ? 1 : 0;
        hdr[a] = scale;
        hdr[4 + a] = off;
        if (a == 0) hdr[3] = hdr[7] = 0.0f;
    }
    __syncthreads();
    // level by level: the midpoints of step-wide spans, `per` of them per axis
#pragma unroll 1
    for (uint32_t step = n; step > 1u; step >>= 1) {
        const uint32_t per = n / step;
#pragma unroll 1
        for (uint32_t i = threadIdx.x; i < pairs * per; i += blockDim.x) {
            const uint32_t pair = i / per;
            const uint32_t k = (i % per) * step;
            float* pl = lds_planes + (pair / 3u) * kScene + kPlaneHeader + (pair % 3u) * kAxis;
            pl[k + step / 2u] = (pl[k] + pl[k + step]) * 0.5f;
        }
        __syncthreads();
    }
#pragma unroll 1
    for (uint32_t i = threadIdx.x; i < pairs * (n + 1u); i += blockDim.x) {
        const uint32_t pair = i / (n + 1u);
        const uint32_t k = i % (n + 1u);
        const navi_relaid_scene& d = P.scenes[pair / 3u];
        const uint32_t a = pair % 3u;
        const float* pl = lds_planes + (pair / 3u) * kScene + kPlaneHeader + a * kAxis;
        const double lo = d.bbox_min[a], cw = (static_cast<double>(d.bbox_max[a]) - lo) / n;
        ok &= fabs(static_cast<double>(pl[k]) - (lo + k * cw)) <= 0.2 * cw ? 1 : 0;
    }
    return __syncthreads_and(ok) != 0;
}

// Depth-D cell of p along one axis from its planes (pl[k] = P_k, P_0 = lo),
// scale and offset, and the cell's bounds. With planes within 0.2 cell of
// uniform, an offset exact to 2^-10 cell and an accurate scale,
// u = p * scale + offset ~ (p - P_0) * scale - 0.25 lies within
// (j - 0.47, j + 0.97) for the cell j that holds p (P_j <= p < P_j+1, or
// j = n - 1 at p = P_n), so trunc(u) is j - 1 or j (0 when u < 0, where j is
// 0); capped at n - 2 it is still j - 1 or j, and one comparison with the
// next plane settles it.
__device__ __forceinline__ uint32_t plane_cell(float p, float off, float scale, const float* pl, uint32_t n, float& lo,
                                               float& hi) {
    const float u = __builtin_fmaf(p, scale, off);
    const uint32_t j0 = min(static_cast<uint32_t>(static_cast<int32_t>(u)), n - 2u);
    const float a = pl[j0], b = pl[j0 + 1], c = pl[j0 + 2];
    const bool up = p >= b;
    lo = up ? b : a;
    hi = up ? c : b;
    return j0 + (up ? 1u : 0u);
}

// kPD > 0: the scenes' split planes of the first kPD levels staged in LDS and
// kDepth the cell-table depth (kPD <= kDepth <= kPD + 2: a depth-kDepth cell is
// kDepth - kPD splits below its depth-kPD cell; in the fast march also
// kDepth < kPD: the table index is the plane index shifted right); kPD = 0: no
// planes, the table depth is P.cell_depth and cells come from splits.
// Wave-uniform work distribution of one wave: a static sequence of 64-ray
// chunks (wave, wave + n_waves, ...) without a queue, else work units claimed
// from the queue, `unit_used` rays of `unit` handed out so far.
struct Sched {
    uint32_t wave, n_waves, seq_end, seq_next, unit, unit_used;
    bool exhausted;
};

__device__ __forceinline__ Sched sched_init(const RelaidParams& P) {
    Sched S;
    S.wave = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    S.n_waves = (gridDim.x * blockDim.x) >> 6;
    const uint32_t my_chunks = S.wave < P.n_chunks ? (P.n_chunks - S.wave + S.n_waves - 1) / S.n_waves : 0u;
    S.seq_end = my_chunks * 64u;
    S.seq_next = 0;
    S.unit = 0;
    S.unit_used = P.unit_rays;
    S.exhausted = (P.queue == nullptr) ? (S.seq_end == 0) : false;
    return S;
}

// Work indices for the wave's idle lanes (`need`, n_need of them; `rank` =
// idle lanes below this one): this lane's index, or 0xffffffff for none.
template <bool kQueued = false>
__device__ __forceinline__ uint32_t claim(const RelaidParams& P, Sched& S, uint32_t n_need, uint32_t rank,
                                          uint32_t lane) {
    uint32_t q = 0xffffffffu;
    if (!kQueued && P.queue == nullptr) {
        const uint32_t sq = S.seq_next + rank;
        if (sq < S.seq_end) q = (S.wave + (sq >> 6) * S.n_waves) * 64u + (sq & 63u);
        S.seq_next += n_need;
        S.exhausted = S.seq_next >= S.seq_end;
    } else {
        const uint32_t avail = P.unit_rays - S.unit_used;
        if (rank < avail) q = S.unit * P.unit_rays + S.unit_used + rank;
        if (n_need > avail) {
            uint32_t claimed = 0;
            if (lane == 0) claimed = atomicAdd(P.queue, 1u);
            claimed = __builtin_amdgcn_readlane(claimed, 0);
            if (claimed < P.n_units) {
                if (rank >= avail) q = claimed * P.unit_rays + (rank - avail);
                S.unit = claimed;
                S.unit_used = n_need - avail;
            } else {
                S.exhausted = true;
                S.unit_used = P.unit_rays;
            }
        } else {
            S.unit_used += n_need;
        }
    }
    return q;
}

struct Float3 {
    float x, y, z;
};

// A ray as its march starts: id, scene, origin, direction and the exit
// reciprocals.
struct RayStart {
    uint32_t ray, scene;
    float ox, oy, oz, dx, dy, dz, rx, ry, rz;
};

// Loads the ray of work index q. Returns 1 for a ray to march, 0 for none
// (q beyond the batch, or an env_order entry outside [0, n_envs): skipped),
// and 2 for a ray of an unknown scene, already reported like a fault.
template <bool kPoses>
__device__ __forceinline__ int start_ray(const RelaidParams& P, uint32_t q, RayStart& R) {
    if (q >= P.n_rays) return 0;
    int32_t env = 0;
    R.ray = ray_of(P, q, env);
    if (static_cast<uint32_t>(env) >= P.n_envs) return 0;
    const int32_t sc = P.env_scene ? P.env_scene[env] : 0;
    if (kPoses) {
        // sdfdag_backend.py:1300-1312: origin = the env's position;
        // x' = x c + z s, y' = y, z' = (-x) s + z c, each product
        // and sum rounded on its own as in the eager tensor code
        const uint32_t r = R.ray - static_cast<uint32_t>(env) * P.rays_per_env;
        const float c = P.env_rot[2 * env], s = P.env_rot[2 * env + 1];
        const float lx = P.local_dirs[3 * r + 0];
        const float ly = P.local_dirs[3 * r + 1];
        const float lz = P.local_dirs[3 * r + 2];
        R.ox = P.env_pos[3 * env + 0];
        R.oy = P.env_pos[3 * env + 1];
        R.oz = P.env_pos[3 * env + 2];
        R.dx = lx * c + lz * s;
        R.dy = ly;
        R.dz = (-lx) * s + lz * c;
    } else {
        // one 12-byte load per vector (a wave's lanes then touch each cache
        // line of the AoS arrays once, not three times)
        const Float3 o = *reinterpret_cast<const Float3*>(P.origins + 3 * R.ray);
        const Float3 d = *reinterpret_cast<const Float3*>(P.dirs + 3 * R.ray);
        R.ox = o.x;
        R.oy = o.y;
        R.oz = o.z;
        R.dx = d.x;
        R.dy = d.y;
        R.dz = d.z;
    }
    // correctly rounded reciprocals (IEEE division) of the axes the exit uses
    // (|d| > 1e-4, kernel.cu:54-85); NaN marks the others, whose quotients
    // fminf then ignores
    R.rx = (R.dx > kDirEps || R.dx < -kDirEps) ? 1.0f / R.dx : __builtin_nanf("");
    R.ry = (R.dy > kDirEps || R.dy < -kDirEps) ? 1.0f / R.dy : __builtin_nanf("");
    R.rz = (R.dz > kDirEps || R.dz < -kDirEps) ? 1.0f / R.dz : __builtin_nanf("");
    if (sc < 0 || sc >= P.n_scenes) {
        // unknown scene: report like a fault, no steps
        store_distance(P, R.ray, __builtin_nanf(""));
        P.out_s[R.ray] = 0;
        if (P.out_steps) P.out_steps[R.ray] = 0;
        return 2;
    }
    R.scene = static_cast<uint32_t>(sc);
    return 1;
}

// The launch parameters as the kernel-argument segment holds them (the
// kernels' first argument). The march reads through this the fields only its
// rare paths need (refill, write-out): loads from that segment are invariant,
// so the compiler reloads them where they are used instead of keeping them in
// scalar registers across the loop (where they crowded out the step's own:
// 30 scalar registers spilled into vector-register lanes, one vector
// operation per read, four of them on every step for the table's resource).
__device__ __forceinline__ const RelaidParams& reload_params() {
    return *(const RelaidParams*)__builtin_amdgcn_kernarg_segment_ptr();  // address-space cast
}

// The fast march: launches whose scenes all have split planes in LDS, tame
// boxes, no record deeper than 30 levels and no negative leaf distance, with
// cell tables below 4 GiB (every scene the library's compiler writes) and a
// range below the outside-domain distance. Per ray the results are the general
// march's; it leaves out what such launches cannot meet: the void cache (it
// changes nothing in them, see the kernel), the depth counter (the 32-level
// limit never applies), the range checks of the exit quotients and of the
// leaf-run step (tame boxes) and the box faces behind the ray (below). The
// step's conditions are wave masks, so its path has no short-circuit branches,
// and the cell table is read through a buffer resource (32-bit offsets).
// kLeaves: the launch may have a leaf table (16-bit semantics), checked at run
// time; false compiles the table's handling out (the fast kernel's instances
// for launches without one: measured, the handling costs those 1.2%).
template <int kDepth, int kPD, bool kPoses, bool kQueued, bool kLeaves>
__device__ __forceinline__ void march_fast(const RelaidParams& P, const SceneLds* lds_scenes,
                                           const float* lds_planes, uint32_t* lds_stage) {
    static_assert(kPD >= 4 && kPD <= 8 && kDepth >= 4 && kDepth <= kPD + 2 && kDepth <= 7,
                  "planes of 4..8 levels, the table at most two levels below them");
    constexpr uint32_t D = kDepth;                    // the table depth
    constexpr uint32_t kAxis = axis_stride(kPD);      // floats per axis
    constexpr uint32_t kScene = scene_stride(kPD);    // floats per scene
    constexpr uint32_t kCells = 1u << kPD;            // cells per axis
    constexpr uint32_t kShP = kPD - kPrefixDepth;     // depth-kPD index >> kShP = depth-4 index
    // the cell indices a descent carries are at depth kJ: the table's when it
    // lies below the planes (splits in registers), else the planes' (the table
    // index is then the plane index shifted by kUp, and the levels between
    // the two take their octants from the plane index's bits)
    constexpr uint32_t kJ = D > kPD ? D : kPD;
    constexpr uint32_t kUp = kPD - (D < kPD ? D : kPD);
    constexpr uint32_t kShD = kJ - kPrefixDepth;      // depth-kJ index >> kShD = depth-4 index
    // the prefix cache's packed fields (a depth-kPD upper-face index is at most 2^kPD)
    constexpr uint32_t kFW = kPD >= 8 ? 10u : 8u;
    constexpr uint32_t kFMask = (1u << kFW) - 1u;
    constexpr uint32_t kOnes = 1u | (1u << kFW) | (1u << (2u * kFW));
    const uint32_t lane = threadIdx.x & 63u;
    // indexed by slot (4 bytes) and by table entry (8 bytes)
    const __amdgpu_buffer_rsrc_t records = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(P.records), static_cast<short>(4), static_cast<int>(P.n_records * 8u), 0x00020000);
    const __amdgpu_buffer_rsrc_t tables = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint64_t*>(P.cell_table), static_cast<short>(8),
        static_cast<int>(static_cast<uint32_t>(P.n_scenes) << (3u * D)), 0x00020000);
    Sched sched = sched_init(P);

    // per-lane ray state; the prefix cache as in the general march's plane
    // kernels (depth-kPD plane index of the cached cell's upper face per axis,
    // x | y << 8 | z << 16, all ones when nothing is cached)
    //
    // The samples are taken in a frame mirrored along each axis on which the
    // ray's direction has its sign bit set: q' = fma(t, |d|, o') with o' the
    // mirrored origin is -q there and q elsewhere, bit for bit (rounding is
    // symmetric), and the sample p itself is q' with the sign flipped back. In
    // these launches t never decreases (leaf distances are non-negative, void
    // and domain steps positive), so along each axis the samples move one way,
    // and a box that held an earlier sample can only be left through the faces
    // ahead of the ray: the leaf cache and the domain test keep those faces
    // alone (mirrored, so a sample is inside while q' <= face' on every axis).
    // The domain's faces behind the ray hold from the origin on; a ray whose
    // origin lies outside the domain gets NaN faces (never inside), and its
    // first step ends it, as any step outside does while the range is below
    // the outside-domain distance (the launch's condition for this march).
    uint32_t ray = 0, scene = 0, lf_slot = 0, pre_cell = 0xffffffffu;
    // the lane's scene in LDS: its split planes and first cell-table entry (set at a refill)
    const float* my_planes = lds_planes;
    uint32_t my_table = 0;
    float ox = 0.f, oy = 0.f, oz = 0.f, dx = 0.f, dy = 0.f, dz = 0.f, rx = 0.f, ry = 0.f, rz = 0.f;
    float t = 0.f;
    int32_t step = 0;
    // faces ahead (mirrored) of the cached leaf (NaN: none) and of the domain
    float lfx = __builtin_nanf(""), lfy = lfx, lfz = lfx, dmx = lfx, dmy = lfx, dmz = lfx;

    // ---- output staging: the wave's slots (kStageSlots tiles), their tiles
    // (uniform), and per lane the LDS byte address of its ray's distance in its
    // tile's slot, or 0 (the ray stores its own outputs; the staging area lies
    // above the scene table, never at address 0) ----
    const bool stage = P.stage != 0u;
    const bool out_steps = P.out_steps != nullptr;
    uint32_t tag = 0, ring = 0;
    uint32_t st0 = kNoTile, st1 = kNoTile;
    uint32_t* const my_stage = lds_stage + (threadIdx.x >> 6) * (kStageSlots * kStageWords);
    const uint32_t stage_addr = lds_address(my_stage);
    const uint32_t flush_pos = P.tile_el ? (((lane & 7u) << 3) | (lane >> 3)) : lane;
    // writes out slot k (tile `tile`) and empties it; every lane of the wave
    // takes one position, eight lanes per run of eight consecutive rays
    auto flush_slot = [&](uint32_t k, uint32_t tile) {
        uint32_t* sl = my_stage + k * kStageWords;
        const uint32_t sv = sl[64u + flush_pos];
        const uint32_t tv = sl[flush_pos];
        sl[64u + flush_pos] = kStageEmpty;
        if (sv != kStageEmpty) {
            const RelaidParams& RP = reload_params();
            int32_t env = 0;
            const uint32_t r = ray_of(RP, tile * 64u + flush_pos, env);
            store_distance(RP, r, __uint_as_float(tv));
            __builtin_nontemporal_store(static_cast<int32_t>(sv), &RP.out_s[r]);
        }
    };
    if (stage) {
#pragma unroll
        for (uint32_t k = 0; k < kStageSlots; ++k) my_stage[k * kStageWords + 64u + lane] = kStageEmpty;
    }

    // the wave's lanes without a ray as a wave mask (uniform); a lane reads its
    // own bit with an inverse ballot (the mask is the lane predicate itself):
    // a bool carried across iterations would cost a select and a compare
    // per ballot
    uint64_t need = ~0ull;
    // per axis the lanes whose direction has its sign bit set (the mirrored
    // axes), as wave masks read back with inverse ballots (set at a refill)
    uint64_t neg_x = 0, neg_y = 0, neg_z = 0;
    while (true) {
        // ---- refill idle lanes (as the general march) ----
        const uint32_t n_need = lane_count(need);
        if ((n_need >= kRefillMinFast || n_need == 64u) && !sched.exhausted) {
            const uint32_t rank = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(need >> 32),
                                                            __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(need), 0u));
            const RelaidParams& RP = reload_params();
            const uint32_t q = claim<kQueued>(RP, sched, n_need, rank, lane);
            RayStart R;
            bool fresh = false;
            if (__builtin_amdgcn_inverse_ballot_w64(need) && start_ray<kPoses>(RP, q, R) == 1) {
                fresh = true;
                ray = R.ray;
                scene = R.scene;
                ox = mirror(R.ox, R.dx);
                oy = mirror(R.oy, R.dy);
                oz = mirror(R.oz, R.dz);
                dx = R.dx;
                dy = R.dy;
                dz = R.dz;
                rx = R.rx;
                ry = R.ry;
                rz = R.rz;
                t = 0.f;
                step = 0;
                pre_cell = 0xffffffffu;
                my_planes = lds_planes + __umul24(scene, kScene);
                my_table = scene << (3u * D);
                const SceneLds& S = lds_scenes[scene];
                const Box dom{S.x0, S.y0, S.z0, S.x1, S.y1, S.z1};
                const float nan = __builtin_nanf("");
                const bool inside = in_box(R.ox, R.oy, R.oz, dom);
                dmx = inside ? ahead(dom.x0, dom.x1, dx) : nan;
                dmy = inside ? ahead(dom.y0, dom.y1, dy) : nan;
                dmz = inside ? ahead(dom.z0, dom.z1, dz) : nan;
                // a one-leaf DAG: its leaf is the domain (kernel.cu:139-152)
                const bool root_leaf = (S.root & 0x80000000u) != 0u;
                lfx = root_leaf ? dmx : nan;
                lfy = root_leaf ? dmy : nan;
                lfz = root_leaf ? dmz : nan;
                lf_slot = (kLeaves && RP.leaves != nullptr && root_leaf)
                              ? table_leaf_word(S.root, RP.leaves, RP.n_leaves)
                              : S.root;
            }
            const uint64_t started = wave_mask(fresh);
            neg_x = wave_mask(__float_as_int(dx) < 0);
            neg_y = wave_mask(__float_as_int(dy) < 0);
            neg_z = wave_mask(__float_as_int(dz) < 0);
            need &= ~started;
            if (stage) {
                // each tile among the fresh rays (at most two per refill) gets a
                // slot: the one holding it, else the ring's next, written out
                // first; rays of an evicted tile still marching store their own
                const uint32_t qtile = q >> 6;
                uint64_t todo = started;
                while (todo != 0ull) {
                    const uint32_t T = __builtin_amdgcn_readlane(qtile, static_cast<uint32_t>(__builtin_ctzll(todo)));
                    uint32_t k;
                    if (st0 == T) {
                        k = 0;
                    } else if (st1 == T) {
                        k = 1;
                    } else {
                        k = ring;
                        ring ^= 1u;
                        const uint32_t old = k == 0 ? st0 : st1;
                        if (old != kNoTile) {
                            flush_slot(k, old);
                            const bool evicted = tag - (stage_addr + k * kStageWords * 4u) < kStageWords * 4u;
                            tag = evicted ? 0u : tag;
                        }
                        st0 = k == 0 ? T : st0;
                        st1 = k == 1 ? T : st1;
                    }
                    const bool same = fresh && qtile == T;
                    tag = same ? stage_addr + k * kStageWords * 4u + (q & 63u) * 4u : tag;
                    todo &= ~wave_mask(same);
                }
            }
        }
        if (need == ~0ull) {
            if (sched.exhausted) break;
            continue;
        }

        // ---- start the step: domain and leaf-cache tests (kernel.cu:108-118) ----
        // The step's conditions are kept as wave masks: ballots of single
        // comparisons (free: a comparison writes its lane mask) combined on the
        // scalar unit, read back per lane with inverse ballots. A ballot of a
        // combined or carried bool would cost a select and a compare each.
        const uint64_t m_ray = ~need;
        ++step;  // a lane without a ray counts too: a refill resets its count
        const float qx = __builtin_fmaf(t, fabsf(dx), ox);
        const float qy = __builtin_fmaf(t, fabsf(dy), oy);
        const float qz = __builtin_fmaf(t, fabsf(dz), oz);
        const uint64_t m_dom = wave_mask(qx <= dmx) & wave_mask(qy <= dmy) & wave_mask(qz <= dmz);
        // (the leaf lies in the domain)
        const uint64_t m_hit_lf = wave_mask(qx <= lfx) & wave_mask(qy <= lfy) & wave_mask(qz <= lfz);
        const bool descending = lane_in(m_ray & m_dom & ~m_hit_lf);
        // the faces ahead (mirrored) of the box a descent ends in; lanes that do
        // not descend keep the void marker and faces at +inf, so their exit
        // quotients are NaN, the exit distance is the outside-domain distance
        // (fminf drops NaN), and a lane outside the domain takes that step as
        // a void step (a leaf-cache lane takes its leaf's distance first)
        constexpr float kInf = __builtin_inff();
        float hx = kInf, hy = kInf, hz = kInf;
        uint32_t slot = kSlotVoid;

        if (descending) {
            const float px = mirror(qx, dx), py = mirror(qy, dy), pz = mirror(qz, dz);
            Box cur;
            // ---- the depth-kPD cell from the split planes ----
            const float* hdr = my_planes;
            const float* plx = hdr + kPlaneHeader;
            const float* ply = plx + kAxis;
            const float* plz = ply + kAxis;
            const float4 scale = *reinterpret_cast<const float4*>(hdr);
            const float4 offs = *reinterpret_cast<const float4*>(hdr + 4);
            uint32_t jx = plane_cell(px, offs.x, scale.x, plx, kCells, cur.x0, cur.x1);
            uint32_t jy = plane_cell(py, offs.y, scale.y, ply, kCells, cur.y0, cur.y1);
            uint32_t jz = plane_cell(pz, offs.z, scale.z, plz, kCells, cur.z0, cur.z1);
            // the prefix cache matters only on an upper face of the cached
            // cell (kernel.cu:120-132); see the general march
            const uint32_t ux = pre_cell & kFMask, uy = (pre_cell >> kFW) & kFMask, uz = pre_cell >> (2u * kFW);
            const bool ex = jx == ux, ey = jy == uy, ez = jz == uz;
            const bool lx0 = px == cur.x0, ly0 = py == cur.y0, lz0 = pz == cur.z0;
            const bool fx = ex && lx0, fy = ey && ly0, fz = ez && lz0;
            bool use_pre = false;
            if (fx || fy || fz) {  // rare
                const bool ix = (jx >> kShP) + 1u == (ux >> kShP);
                const bool iy = (jy >> kShP) + 1u == (uy >> kShP);
                const bool iz = (jz >> kShP) + 1u == (uz >> kShP);
                use_pre = (fx || ix) && (fy || iy) && (fz || iz);
                if (use_pre) {
                    jx -= fx ? 1u : 0u;
                    jy -= fy ? 1u : 0u;
                    jz -= fz ? 1u : 0u;
                    const float lx = plx[jx], ly = ply[jy], lz = plz[jz];
                    cur.x1 = fx ? cur.x0 : cur.x1;
                    cur.y1 = fy ? cur.y0 : cur.y1;
                    cur.z1 = fz ? cur.z0 : cur.z1;
                    cur.x0 = fx ? lx : cur.x0;
                    cur.y0 = fy ? ly : cur.y0;
                    cur.z0 = fz ? lz : cur.z0;
                }
            }
            // ---- splits down to the table depth (kernel.cu:165-176) ----
#pragma unroll
            for (uint32_t l = kPD; l < D; ++l) {
                const float mx = (cur.x0 + cur.x1) * 0.5f;
                const float my = (cur.y0 + cur.y1) * 0.5f;
                const float mz = (cur.z0 + cur.z1) * 0.5f;
                const bool gx = px >= mx, gy = py >= my, gz = pz >= mz;
                cur.x0 = gx ? mx : cur.x0;
                cur.x1 = gx ? cur.x1 : mx;
                cur.y0 = gy ? my : cur.y0;
                cur.y1 = gy ? cur.y1 : my;
                cur.z0 = gz ? mz : cur.z0;
                cur.z1 = gz ? cur.z1 : mz;
                jx = append_bit(jx, gx);
                jy = append_bit(jy, gy);
                jz = append_bit(jz, gz);
            }
            // ---- one cell-table read: the slot D levels down, and its depth ----
            const navi_u32x2 e = navi_struct_load_b64(
                tables,
                static_cast<int32_t>(my_table | ((jz >> kUp) << (2u * D)) | ((jy >> kUp) << D) | (jx >> kUp)), 0,
                0, 0);
            slot = e[0];
            uint32_t depth = e[1];
            if (kPD <= D && depth < D) {
                // a leaf / void / fault above depth D: its box from the planes
                // down to depth kPD, splits below
                const uint32_t dp = min(depth, static_cast<uint32_t>(kPD));
                const uint32_t sh = D - dp;
                const uint32_t up = kPD - dp;
                const uint32_t w = 1u << up;
                const uint32_t kx = (jx >> sh) << up, ky = (jy >> sh) << up, kz = (jz >> sh) << up;
                cur = Box{plx[kx], ply[ky], plz[kz], plx[kx + w], ply[ky + w], plz[kz + w]};
                if (kDepth > kPD + 1) {  // depth can lie between kPD and D
#pragma unroll 1
                    for (uint32_t l = static_cast<uint32_t>(kPD); l < depth; ++l) {
                        const uint32_t b = D - 1u - l;
                        split_box(cur, ((jx >> b) & 1u) | (((jy >> b) & 1u) << 1) | (((jz >> b) & 1u) << 2));
                    }
                }
            }
            // kernel.cu:154-163: a fresh descent caches its depth-4 cell when the
            // path goes below depth 4 (prefix descents meeting the fresh
            // descent's cell re-save the cell they hold)
            const bool below4 = depth > kPrefixDepth;
            const bool at4 = depth == kPrefixDepth;
            const bool internal = slot < kSlotBadChild;
            const bool save = !use_pre && (below4 || (at4 && internal));
            // per axis ((j >> kShD) + 1) << kShP, on the three indices packed in
            // 8-bit fields (j < 128: no field carries into the next)
            constexpr uint32_t kLow = (1u << kShD) - 1u;
            constexpr uint32_t kKeep = (kFMask & ~kLow) * kOnes;
            const uint32_t packed = jx | (jy << kFW) | (jz << (2u * kFW));
            const uint32_t saved = ((packed & kKeep) >> (kShD - kShP)) + (1u << kShP) * kOnes;
            pre_cell = save ? saved : pre_cell;

            if constexpr (kPD > D) {
                static_assert((kFW == 8u || kFW == 10u) && kPD <= D + 2, "octant gather: 8- or 10-bit fields, bits 0-1");
                // ---- from the table down to depth kPD: the octants are the
                // plane index's bits (kernel.cu:165-176 picks the same ones:
                // the depth-kPD cell lies in the box each split leads to) ----
#pragma unroll
                for (uint32_t l = D; l < static_cast<uint32_t>(kPD); ++l) {
                    if (slot < kSlotBadChild) {  // an internal node at depth l
                        // the octant: bit b of each index field of `packed`, gathered
                        // by one 24-bit multiply (x to bit 22, y to 23, z to 24;
                        // every other product bit lies apart from those three)
                        const uint32_t b = kPD - 1u - l;  // 0 or 1 (the loop is unrolled)
                        const uint32_t kBits = kOnes << b;
                        const uint32_t kGather =
                            (1u << (22u - b)) | (1u << (23u - kFW - b)) | (1u << (24u - 2u * kFW - b));
                        const uint32_t oct = __builtin_amdgcn_ubfe(__umul24(packed & kBits, kGather), 22u, 3u);
                        slot = navi_struct_load_b32(records, static_cast<int32_t>((slot << 3) | oct), 0, 0, 0);
                        depth = l + 1u;
                    }
                }
                if (depth < static_cast<uint32_t>(kPD)) {
                    // a leaf / void / fault above depth kPD: its box from the planes
                    const uint32_t up = kPD - depth;
                    const uint32_t w = 1u << up;
                    const uint32_t kx = (jx >> up) << up, ky = (jy >> up) << up, kz = (jz >> up) << up;
                    cur = Box{plx[kx], ply[ky], plz[kz], plx[kx + w], ply[ky + w], plz[kz + w]};
                }
            }

            // ---- below depth kJ: one 4-byte slot per level (kernel.cu:136-199) ----
            // (at most 32 - kJ trips, see the general march)
            uint32_t cur_rec = slot;
            bool deeper = slot < kSlotBadChild;
            for (uint32_t trip = kJ; deeper && trip < static_cast<uint32_t>(kMaxDepth); ++trip) {
                slot = navi_struct_load_b32(records, static_cast<int32_t>(descend_index(px, py, pz, cur, cur_rec)), 0, 0, 0);
                cur_rec = slot;
                deeper = slot < kSlotBadChild;
            }
            hx = __builtin_amdgcn_inverse_ballot_w64(neg_x) ? -cur.x0 : cur.x1;
            hy = __builtin_amdgcn_inverse_ballot_w64(neg_y) ? -cur.y0 : cur.y1;
            hz = __builtin_amdgcn_inverse_ballot_w64(neg_z) ? -cur.z0 : cur.z1;
        }

        // ---- the query's outcome and the leaf cache ----
        const uint64_t m_new_leaf = wave_mask(static_cast<int32_t>(slot) < 0);
        const uint64_t m_leaf = m_hit_lf | m_new_leaf;
        const bool new_leaf = lane_in(m_new_leaf);
        lfx = new_leaf ? hx : lfx;
        lfy = new_leaf ? hy : lfy;
        lfz = new_leaf ? hz : lfz;
        lf_slot = new_leaf ? slot : lf_slot;
        if (kLeaves && P.leaves != nullptr) {  // uniform: the pool has a leaf table (16-bit semantics)
            const RelaidParams& RP = reload_params();
            if (new_leaf) lf_slot = table_leaf_word(slot, RP.leaves, RP.n_leaves);
        }

        // ---- finish the step (kernel.cu:54-85, 297-308) ----
        // The exit quotient (face - p) / d of the reference's face (hi when
        // d > 0, else lo) is (face' - q') / |d| bit for bit: where d's sign
        // bit is set both numerator and divisor are negated (and where
        // d = +0 the reciprocal is NaN, so which face is moot).
        const float nx = hx - qx, ny = hy - qy, nz = hz - qz;
        const float e = fminf(fminf(fminf(markstein(nx, fabsf(dx), fabsf(rx)), markstein(ny, fabsf(dy), fabsf(ry))),
                                    markstein(nz, fabsf(dz), fabsf(rz))),
                              kOutsideDomain);
        const float void_d = e > kVoidAdvanceEps ? e : kVoidAdvanceEps;  // fmaxf: e is never NaN
        const float leaf_d = half_to_float(lf_slot & 0xffffu);
        const int32_t leaf_s =
            static_cast<int32_t>(kLeaves ? __builtin_amdgcn_ubfe(lf_slot, 16u, P.sem_bits) : (lf_slot >> 16) & 0x7fffu);
        // the step's distance: the void's exit, the leaf's, the outside-domain
        // step, or NaN after a fault (so t becomes NaN); a ray's semantic is its
        // leaf's when the step hits and 0 whenever it ends otherwise, so only
        // the step that ends a ray needs it (void, outside and fault steps never
        // hit: their semantic is 0)
        // (inverse ballots are convergent: read them outside the conditional
        // expression, which then stays a chain of selects)
        const bool on_leaf = lane_in(m_leaf);
        const float dist = on_leaf ? leaf_d : (slot == kSlotVoid ? void_d : __builtin_nanf(""));
        const uint64_t m_hit = m_leaf & wave_mask(leaf_s != 0) & wave_mask(dist < P.hit_eps);
        const float t_next = t + dist;
        uint64_t m_fin = m_ray & (wave_mask(slot == kSlotFault) | m_hit | wave_mask(t_next > P.max_distance) |
                                  wave_mask(step >= P.max_steps));
        t = lane_in(m_ray & ~m_hit) ? t_next : t;

        // ---- one more step if the leaf cache answers it alone ----
        // (within the leaf box neither the void cache nor the domain test can
        // fire for tame boxes; it repeats the leaf's distance, so it cannot hit)
        uint64_t m_run = m_ray & ~m_fin & m_leaf;
#pragma unroll
        for (uint32_t k = 0; k < kLeafRunFast; ++k) {
            const float ux = __builtin_fmaf(t, fabsf(dx), ox);
            const float uy = __builtin_fmaf(t, fabsf(dy), oy);
            const float uz = __builtin_fmaf(t, fabsf(dz), oz);
            m_run &= wave_mask(ux <= lfx) & wave_mask(uy <= lfy) & wave_mask(uz <= lfz);
            step = add_lane_bit(step, m_run);
            t = lane_in(m_run) ? t + dist : t;
            const uint64_t m_fin2 = m_run & (wave_mask(t > P.max_distance) | wave_mask(step >= P.max_steps));
            m_fin |= m_fin2;
            m_run &= ~m_fin2;
        }
        need |= m_fin;
        if (lane_in(m_fin)) {
            const int32_t sem = lane_in(m_hit) ? leaf_s : 0;
            if (tag != 0u) {
                lds_u32* e = lds_pointer(tag);
                e[0] = __float_as_uint(t);
                e[64] = static_cast<uint32_t>(sem);
            } else {
                const RelaidParams& RP = reload_params();
                store_distance(RP, ray, t);
                __builtin_nontemporal_store(sem, &RP.out_s[ray]);
            }
            if (out_steps) {
                const RelaidParams& RP = reload_params();
                RP.out_steps[ray] = step;
            }
        }
    }
    if (stage) {
        if (st0 != kNoTile) flush_slot(0, st0);
        if (st1 != kNoTile) flush_slot(1, st1);
    }
}

// The march of one launch (everything after the workgroup's set-up). kFast:
// the launch has split planes and tame, shallow, monotone scenes (no void
// cache, no depth counter, no range checks); the flags are then compile-time
// constants, and everything the other launches need is compiled out.
template <int kDepth, int kPD, bool kPoses, bool kFast>
__device__ __forceinline__ void march(const RelaidParams& P, SceneLds* lds_scenes, float* lds_planes, int tame,
                                      int shallow, int planes, bool void_cache) {
    constexpr bool kPlanes = kPD > 0;
    if (kFast) {
        tame = 1;
        shallow = 1;
        planes = 1;
        void_cache = false;
    }
    const uint32_t D = kPlanes ? static_cast<uint32_t>(kDepth) : P.cell_depth;  // the table depth
    constexpr uint32_t kAxis = kPlanes ? axis_stride(kPD) : 0u;    // floats per axis
    constexpr uint32_t kScene = kPlanes ? scene_stride(kPD) : 0u;  // floats per scene
    constexpr uint32_t kCells = kPlanes ? (1u << kPD) : 0u;        // cells per axis
    const uint32_t lane = threadIdx.x & 63u;
    // The record pool as a buffer resource indexed by slot (stride 4 bytes): the
    // hardware scales the index and bounds every read by the pool's size (at
    // most 2^27 records, 2^30 slots; an out-of-range read returns 0). Dword 3 =
    // 0x00020000: 32-bit data format, as gfx9 buffers need.
    const __amdgpu_buffer_rsrc_t records = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(P.records), static_cast<short>(4), static_cast<int>(P.n_records * 8u), 0x00020000);
    Sched sched = sched_init(P);

    // per-lane ray state
    bool has_ray = false;
    uint32_t ray = 0;
    float ox = 0.f, oy = 0.f, oz = 0.f, dx = 0.f, dy = 0.f, dz = 0.f, rx = 0.f, ry = 0.f, rz = 0.f;
    float t = 0.f, dist = 0.f;
    int32_t sem = 0, step = 0;
    uint32_t scene = 0;  // this ray's scene (an index into lds_scenes)
    Box lf{}, vd{};
    // The prefix cache (kernel.cu:120-132, 154-163). The plane kernels keep
    // the cached depth-4 cell as the depth-kPD plane index of its upper face
    // per axis, x | y << 8 | z << 16, all ones when nothing is cached, and no
    // box: the plane lookup of p decides in integers. Otherwise the cell's
    // depth-4 indices x | y << 4 | z << 8 (valid with pre_ok), with its box
    // kept (kDepth = 0) or rebuilt by four splits (planes switched off for
    // the launch).
    Box pre{};
    uint32_t lf_slot = 0;
    uint32_t pre_cell = 0;
    bool lf_ok = false, vd_ok = false, pre_ok = false;

    while (true) {
        // ---- refill lanes without a ray from the wave's chunk sequence ----
        // Refill once an eighth of the wave is idle (or all of it): the refill
        // block costs the whole wave, idle lanes only their own slot.
        const uint64_t need = wave_mask(!has_ray);
        const uint32_t n_need = lane_count(need);
        if ((n_need >= kRefillMin || n_need == 64u) && !sched.exhausted) {
            // idle lanes below this one (mbcnt: set bits of `need` under the lane)
            const uint32_t rank = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(need >> 32),
                                                            __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(need), 0u));
            const RelaidParams& RP = reload_params();
            const uint32_t q = claim(RP, sched, n_need, rank, lane);
            RayStart R;
            if (!has_ray && start_ray<kPoses>(RP, q, R) == 1) {
                ray = R.ray;
                scene = R.scene;
                ox = R.ox;
                oy = R.oy;
                oz = R.oz;
                dx = R.dx;
                dy = R.dy;
                dz = R.dz;
                rx = R.rx;
                ry = R.ry;
                rz = R.rz;
                t = 0.f;
                dist = 0.f;
                sem = 0;
                step = 0;
                lf_ok = vd_ok = pre_ok = false;
                pre_cell = 0xffffffffu;
                has_ray = true;
                // A one-leaf DAG answers every in-domain query with that leaf
                // and the domain box (kernel.cu:139-152 at depth 0): prime the
                // leaf cache with it, which gives the same results as the
                // first query would.
                const SceneLds& S = lds_scenes[scene];
                if (S.root & 0x80000000u) {
                    lf = Box{S.x0, S.y0, S.z0, S.x1, S.y1, S.z1};
                    lf_slot = RP.leaves != nullptr ? table_leaf_word(S.root, RP.leaves, RP.n_leaves) : S.root;
                    lf_ok = true;
                }
            }
        }
        if (wave_mask(has_ray) == 0ull) {
            if (sched.exhausted) break;
            continue;
        }

        // ---- start the march step (kernel.cu:260-269, query :108-132) ----
        // Everything below is written with selects, and the descent loop
        // touches only cur / cur_rec / depth (plus the prefix save), so the
        // cache boxes stay in fixed registers.
        step += has_ray ? 1 : 0;
        const SceneLds& S = lds_scenes[scene];
        const Box dom{S.x0, S.y0, S.z0, S.x1, S.y1, S.z1};
        const float px = __builtin_fmaf(t, dx, ox);
        const float py = __builtin_fmaf(t, dy, oy);
        const float pz = __builtin_fmaf(t, dz, oz);
        // the cache tests in the reference's order, as exclusive outcomes:
        // void cache (kernel.cu:265-267), outside the domain (:108-112), leaf
        // cache (:114-118); one-leaf scenes always end here
        const bool hit_vd = void_cache && vd_ok && in_box_strict(px, py, pz, vd);
        const bool outside = !hit_vd && !in_box(px, py, pz, dom);
        const bool hit_lf = !hit_vd && !outside && lf_ok && in_box(px, py, pz, lf);
        bool descending = has_ray && !(hit_vd || outside || hit_lf);
        Box cur = dom;
        uint32_t cur_rec = 0;
        int32_t depth = kPrefixDepth;
        uint32_t slot = 0;

        // ---- every descent: locate the depth-D cell, one cell-table read ----
        // The cell table holds what D record reads from the root would meet
        // (navi_build_cell_table). A fresh descent (kernel.cu:133-135) meets
        // the cell that holds p by the >= rule of kernel.cu:165-176. A
        // descent from the cached prefix cell (:120-132) meets the same cell,
        // except on the prefix cell's upper faces, which the inclusive cache
        // test admits: there it meets the cell's last sub-cell, one below the
        // cell past the face. The cell comes from the split planes when the
        // scenes allow it, else from splits done here; either way its box is
        // the descent's box bit for bit.
        if (descending) {
            // the scene's scales and planes of x, y, z
            const float* hdr = lds_planes + __umul24(scene, kScene);
            const float* plx = hdr + kPlaneHeader;
            const float* ply = plx + kAxis;
            const float* plz = ply + kAxis;
            uint32_t jx = 0, jy = 0, jz = 0;
            bool use_pre;
            if (kPlanes && planes) {
                const float4 scale = *reinterpret_cast<const float4*>(hdr);
                const float4 offs = *reinterpret_cast<const float4*>(hdr + 4);
                jx = plane_cell(px, offs.x, scale.x, plx, kCells, cur.x0, cur.x1);
                jy = plane_cell(py, offs.y, scale.y, ply, kCells, cur.y0, cur.y1);
                jz = plane_cell(pz, offs.z, scale.z, plz, kCells, cur.z0, cur.z1);
                // The prefix cell holds p, faces included (kernel.cu:120-132),
                // when per axis p's cell lies in it or p is on its upper face,
                // where p's cell starts (p == its lower plane; the domain's
                // upper face is inside: there p's cell is the last one). A
                // descent from it meets the cell a fresh descent meets (the
                // saved prefix is then the one already cached), except when p
                // is on an upper face: only then does the prefix matter.
                constexpr uint32_t sh = kPD - kPrefixDepth;
                const uint32_t ux = pre_cell & 0xffu, uy = (pre_cell >> 8) & 0xffu, uz = pre_cell >> 16;
                const bool fx = jx == ux && px == cur.x0;
                const bool fy = jy == uy && py == cur.y0;
                const bool fz = jz == uz && pz == cur.z0;
                use_pre = (fx || fy || fz) && (fx || (jx >> sh) + 1u == (ux >> sh)) &&
                          (fy || (jy >> sh) + 1u == (uy >> sh)) && (fz || (jz >> sh) + 1u == (uz >> sh));
                // on an upper face the descent from the prefix cell stays in it
                if (use_pre) {  // rare
                    jx -= fx ? 1u : 0u;
                    jy -= fy ? 1u : 0u;
                    jz -= fz ? 1u : 0u;
                    const float lx = plx[jx], ly = ply[jy], lz = plz[jz];
                    cur.x1 = fx ? cur.x0 : cur.x1;
                    cur.y1 = fy ? cur.y0 : cur.y1;
                    cur.z1 = fz ? cur.z0 : cur.z1;
                    cur.x0 = fx ? lx : cur.x0;
                    cur.y0 = fy ? ly : cur.y0;
                    cur.z0 = fz ? lz : cur.z0;
                }
#pragma unroll
                for (int l = static_cast<int>(kPD); l < kDepth; ++l) {
                    const float mx = (cur.x0 + cur.x1) * 0.5f;
                    const float my = (cur.y0 + cur.y1) * 0.5f;
                    const float mz = (cur.z0 + cur.z1) * 0.5f;
                    const bool gx = px >= mx, gy = py >= my, gz = pz >= mz;
                    cur.x0 = gx ? mx : cur.x0;
                    cur.x1 = gx ? cur.x1 : mx;
                    cur.y0 = gy ? my : cur.y0;
                    cur.y1 = gy ? cur.y1 : my;
                    cur.z0 = gz ? mz : cur.z0;
                    cur.z1 = gz ? cur.z1 : mz;
                    jx = append_bit(jx, gx);
                    jy = append_bit(jy, gy);
                    jz = append_bit(jz, gz);
                }
            } else {
                if (kPlanes) {  // planes off for this launch: rebuild the prefix box
                    // (also without a prefix, so that no box lives across steps)
                    pre = dom;
                    for (int l = 0; l < kPrefixDepth; ++l) {
                        const uint32_t b = static_cast<uint32_t>(kPrefixDepth - 1 - l);
                        split_box(pre, ((pre_cell >> b) & 1u) | (((pre_cell >> (4u + b)) & 1u) << 1) |
                                           (((pre_cell >> (8u + b)) & 1u) << 2));
                    }
                }
                use_pre = pre_ok && in_box(px, py, pz, pre);
                // a prefix descent starts from the cached cell, a fresh one
                // from the domain, four levels up
                cur.x0 = use_pre ? pre.x0 : dom.x0;
                cur.y0 = use_pre ? pre.y0 : dom.y0;
                cur.z0 = use_pre ? pre.z0 : dom.z0;
                cur.x1 = use_pre ? pre.x1 : dom.x1;
                cur.y1 = use_pre ? pre.y1 : dom.y1;
                cur.z1 = use_pre ? pre.z1 : dom.z1;
                jx = use_pre ? (pre_cell & 15u) : 0u;
                jy = use_pre ? ((pre_cell >> 4) & 15u) : 0u;
                jz = use_pre ? (pre_cell >> 8) : 0u;
#pragma unroll
                for (int l = 0; l < kPrefixDepth; ++l) {  // fresh lanes only
                    const float mx = (cur.x0 + cur.x1) * 0.5f;
                    const float my = (cur.y0 + cur.y1) * 0.5f;
                    const float mz = (cur.z0 + cur.z1) * 0.5f;
                    const bool gx = px >= mx, gy = py >= my, gz = pz >= mz;
                    const bool sx = !use_pre, ux = sx && gx, uy = sx && gy, uz = sx && gz;
                    cur.x0 = ux ? mx : cur.x0;
                    cur.x1 = (sx && !gx) ? mx : cur.x1;
                    cur.y0 = uy ? my : cur.y0;
                    cur.y1 = (sx && !gy) ? my : cur.y1;
                    cur.z0 = uz ? mz : cur.z0;
                    cur.z1 = (sx && !gz) ? mz : cur.z1;
                    jx = sx ? append_bit(jx, gx) : jx;
                    jy = sx ? append_bit(jy, gy) : jy;
                    jz = sx ? append_bit(jz, gz) : jz;
                }
#pragma unroll 1
                for (uint32_t l = kPrefixDepth; l < D; ++l) {
                    const float mx = (cur.x0 + cur.x1) * 0.5f;
                    const float my = (cur.y0 + cur.y1) * 0.5f;
                    const float mz = (cur.z0 + cur.z1) * 0.5f;
                    const bool gx = px >= mx, gy = py >= my, gz = pz >= mz;
                    cur.x0 = gx ? mx : cur.x0;
                    cur.x1 = gx ? cur.x1 : mx;
                    cur.y0 = gy ? my : cur.y0;
                    cur.y1 = gy ? cur.y1 : my;
                    cur.z0 = gz ? mz : cur.z0;
                    cur.z1 = gz ? cur.z1 : mz;
                    jx = append_bit(jx, gx);
                    jy = append_bit(jy, gy);
                    jz = append_bit(jz, gz);
                }
            }
            const uint64_t e = P.cell_table[(((scene << D | jz) << D | jy) << D) | jx];
            slot = static_cast<uint32_t>(e);
            depth = static_cast<int32_t>(e >> 32);
            if (depth < static_cast<int32_t>(D)) {
                // leaf / void / fault above depth D: its box is the one after
                // `depth` splits
                if (kPlanes && planes) {
                    // the planes give the box down to depth kPD, splits the rest
                    const uint32_t dp = min(static_cast<uint32_t>(depth), static_cast<uint32_t>(kPD));
                    const uint32_t sh = D - dp;
                    const uint32_t up = kPD - dp;
                    const uint32_t w = 1u << up;
                    const uint32_t kx = (jx >> sh) << up, ky = (jy >> sh) << up, kz = (jz >> sh) << up;
                    cur = Box{plx[kx], ply[ky], plz[kz], plx[kx + w], ply[ky + w], plz[kz + w]};
                    if (kDepth > kPD + 1) {  // depth can lie between kPD and D
#pragma unroll 1
                        for (uint32_t l = static_cast<uint32_t>(kPD); l < static_cast<uint32_t>(depth); ++l) {
                            const uint32_t b = D - 1u - l;
                            split_box(cur, ((jx >> b) & 1u) | (((jy >> b) & 1u) << 1) | (((jz >> b) & 1u) << 2));
                        }
                    }
                } else {
                    cur = dom;
#pragma unroll 1
                    for (int32_t l = 0; l < depth; ++l) {
                        const uint32_t b = D - 1u - static_cast<uint32_t>(l);
                        split_box(cur, ((jx >> b) & 1u) | (((jy >> b) & 1u) << 1) | (((jz >> b) & 1u) << 2));
                    }
                }
            }
            // kernel.cu:154-163: a fresh descent caches the depth-4 node when it
            // is internal, i.e. when the path goes below depth 4; the cell is
            // the depth-4 ancestor of the depth-D cell. (The plane kernels
            // re-save the cached cell on the prefix descents that meet the
            // fresh descent's cell: the same value.)
            const bool save = !use_pre && (depth > kPrefixDepth || (depth == kPrefixDepth && slot < kSlotBadChild));
            if (save) {
                const uint32_t sh = D - kPrefixDepth;
                const uint32_t kx = jx >> sh, ky = jy >> sh, kz = jz >> sh;
                if (!kPlanes) {
                    pre = dom;
                    for (int l = 0; l < kPrefixDepth; ++l) {
                        const uint32_t b = static_cast<uint32_t>(kPrefixDepth - 1 - l);
                        split_box(pre, ((kx >> b) & 1u) | (((ky >> b) & 1u) << 1) | (((kz >> b) & 1u) << 2));
                    }
                }
                if (kPlanes && planes) {
                    constexpr uint32_t up = kPlanes ? kPD - kPrefixDepth : 0u;
                    pre_cell = ((kx + 1u) << up) | (((ky + 1u) << up) << 8) | (((kz + 1u) << up) << 16);
                } else {
                    pre_cell = kx | (ky << 4) | (kz << 8);
                }
                pre_ok = true;
            }
            cur_rec = slot;
            descending = slot < kSlotBadChild;  // an internal node at depth D
        }

        // ---- descend below depth D, one 4-byte gather per level (kernel.cu:136-199) ----
        // A per-lane loop: lanes that found their leaf / void leave it and are
        // masked off; the wave runs it as long as its deepest descent.
        // Child slots from navi_relayout are always in range; the buffer
        // resource's bound only keeps a corrupt caller-built pool inside its
        // allocation (a read past it returns 0).
        if (shallow) {
            // A shallow scene's slots all lie at depth <= 31, at most 31 - D
            // reads below the table; the wave-uniform bound of 32 - D trips
            // only matters for a pool whose max_depth understates it (a cycle
            // behind a zeroed descriptor), which then ends like the 32-level
            // limit (stale result) instead of looping.
            for (uint32_t trip = D; descending && trip < static_cast<uint32_t>(kMaxDepth); ++trip) {
                slot = navi_struct_load_b32(records, static_cast<int32_t>(descend_index(px, py, pz, cur, cur_rec)), 0, 0, 0);
                cur_rec = slot;  // read again only while internal
                descending = slot < kSlotBadChild;
            }
            descending = false;
        } else {
            while (descending) {
                slot = navi_struct_load_b32(records, static_cast<int32_t>(descend_index(px, py, pz, cur, cur_rec)), 0, 0, 0);
                depth += 1;
                cur_rec = slot;
                descending = slot < kSlotBadChild && depth < kMaxDepth;
            }
            // a bad child index faults only where the reference examines the
            // child, above the 32-level limit; at depth 32 the result is stale
            slot = (slot == kSlotBadChild && depth < kMaxDepth) ? kSlotFault : slot;
        }

        // ---- classify the query result and update the caches ----
        // Lanes that did not descend keep slot == 0 (an internal slot), so the
        // descent outcomes below are false for them. (The shallow loop leaves
        // `depth` at the table's value, <= D <= 7: below the limit, as every
        // slot of a shallow scene is. Shallow scenes carry no bad-child slots:
        // navi_relayout and the cell table turn them into faults, which they
        // are at every depth < 32.)
        const bool new_leaf = (slot & 0x80000000u) != 0u && depth < kMaxDepth;  // examined at depth < 32
        const bool new_void = slot == kSlotVoid;
        const bool is_void = hit_vd || new_void;
        const bool is_leaf = hit_lf || new_leaf;
        const bool is_fault = slot == kSlotFault;
        if (void_cache) {
            vd.x0 = new_void ? cur.x0 : vd.x0;
            vd.y0 = new_void ? cur.y0 : vd.y0;
            vd.z0 = new_void ? cur.z0 : vd.z0;
            vd.x1 = new_void ? cur.x1 : vd.x1;
            vd.y1 = new_void ? cur.y1 : vd.y1;
            vd.z1 = new_void ? cur.z1 : vd.z1;
            vd_ok = vd_ok || new_void;
        }
        lf.x0 = new_leaf ? cur.x0 : lf.x0;
        lf.y0 = new_leaf ? cur.y0 : lf.y0;
        lf.z0 = new_leaf ? cur.z0 : lf.z0;
        lf.x1 = new_leaf ? cur.x1 : lf.x1;
        lf.y1 = new_leaf ? cur.y1 : lf.y1;
        lf.z1 = new_leaf ? cur.z1 : lf.z1;
        lf_slot = new_leaf ? slot : lf_slot;
        if (P.leaves != nullptr) {  // uniform: the pool has a leaf table (16-bit semantics)
            const RelaidParams& RP = reload_params();
            if (new_leaf) lf_slot = table_leaf_word(slot, RP.leaves, RP.n_leaves);
        }
        lf_ok = lf_ok || new_leaf;

        // ---- finish the step (kernel.cu:297-308) ----
        // kernel.cu:54-85 on the void box, branch-free: the face per axis is
        // fixed by the direction's sign; axes with |d| <= 1e-4 have a NaN
        // reciprocal and drop out of the minimum.
        // (without the void cache every void step found its cell just now)
        float nx, ny, nz;
        if (void_cache) {
            nx = (dx > 0.f ? vd.x1 : vd.x0) - px;
            ny = (dy > 0.f ? vd.y1 : vd.y0) - py;
            nz = (dz > 0.f ? vd.z1 : vd.z0) - pz;
        } else {
            nx = (dx > 0.f ? cur.x1 : cur.x0) - px;
            ny = (dy > 0.f ? cur.y1 : cur.y0) - py;
            nz = (dz > 0.f ? cur.z1 : cur.z0) - pz;
        }
        float e;
        if (tame) {
            e = fminf(fminf(fminf(markstein(nx, dx, rx), markstein(ny, dy, ry)), markstein(nz, dz, rz)),
                      kOutsideDomain);
        } else {
            e = kOutsideDomain;
            e = rx == rx ? fminf(e, nx / dx) : e;
            e = ry == ry ? fminf(e, ny / dy) : e;
            e = rz == rz ? fminf(e, nz / dz) : e;
        }
        const float void_d = fmaxf(e, kVoidAdvanceEps);
        const float leaf_d = half_to_float(lf_slot & 0xffffu);
        const int32_t leaf_s = static_cast<int32_t>(__builtin_amdgcn_ubfe(lf_slot, 16u, P.sem_bits));
        // stale (32 levels without leaf or void): dist / sem keep their values
        dist = is_void ? void_d : (is_leaf ? leaf_d : (outside ? kOutsideDomain : dist));
        sem = is_void ? 0 : (is_leaf ? leaf_s : (outside ? 0 : sem));
        const bool hit = !is_fault && sem != 0 && dist < P.hit_eps;
        const float t_next = t + dist;
        // a finished ray reports t (NaN after a fault) and its semantic if it
        // hit, else 0 (kernel.cu:297-308); the one write is after the leaf run
        bool finish = has_ray && (is_fault || hit || t_next > P.max_distance || step >= P.max_steps);
        t = (has_ray && !hit) ? t_next : t;
        t = (finish && is_fault) ? __builtin_nanf("") : t;
        sem = (finish && !hit) ? 0 : sem;
        has_ray = has_ray && !finish;

        // ---- further steps answered by the leaf cache alone ----
        // After a leaf step that neither hit nor ended the ray, the next point
        // often stays in the same leaf box; such a step (kernel.cu:260-305
        // with the void-cache, domain and leaf-cache tests of :265-267 and
        // :108-118 in that order) repeats the distance and semantic just
        // used, so it cannot hit. Up to kLeafRun of them are taken here per
        // lane, far cheaper than a full step; the first point that leaves the
        // box is left to the next full step, which recomputes it.
        // With tame boxes the first two tests cannot fire inside the leaf
        // box: it lies within the domain, and the cached void cell is another
        // terminal cell of the same tree, so the two differ on a split plane
        // with the leaf box on its closed side and the void interior strictly
        // on the other.
        bool run = has_ray && is_leaf;
        for (uint32_t k = 0; k < kLeafRun && run; ++k) {
            const float qx = __builtin_fmaf(t, dx, ox);
            const float qy = __builtin_fmaf(t, dy, oy);
            const float qz = __builtin_fmaf(t, dz, oz);
            run = in_box(qx, qy, qz, lf);
            if (!tame) {
                const Box dm{S.x0, S.y0, S.z0, S.x1, S.y1, S.z1};
                run = run && !(vd_ok && in_box_strict(qx, qy, qz, vd)) && in_box(qx, qy, qz, dm);
            }
            if (run) {
                step += 1;
                t = t + dist;
                if (t > P.max_distance || step >= P.max_steps) {
                    finish = true;
                    sem = 0;
                    has_ray = false;
                    run = false;
                }
            }
        }
        if (finish) {
            const RelaidParams& RP = reload_params();
            store_distance(RP, ray, t);
            __builtin_nontemporal_store(sem, &RP.out_s[ray]);
            if (RP.out_steps) RP.out_steps[ray] = step;
        }
    }
}

// A workgroup's set-up: the scene table (and with kPD > 0 the split planes of
// kPD levels) staged in LDS, and the launch-wide conditions, the same in every
// workgroup.
struct LaunchConds {
    int tame, shallow, planes;
    bool void_cache;
};

template <int kPD>
__device__ LaunchConds stage_scenes(const RelaidParams& P, SceneLds* lds_scenes, float* lds_planes) {
    constexpr bool kPlanes = kPD > 0;
    // `tame`: every scene box has coordinates below 2^100 in magnitude, so
    // lo + hi never overflows, every split plane lies within its box, each
    // descent box lies within its parent and the domain, and exit quotients
    // (numerators below 2^101, divisors above 1e-4) stay far from overflow.
    // `shallow`: no record of any scene lies deeper than 30 levels, so every
    // slot a descent reads is at depth <= 31 and the 32-level limit of
    // kernel.cu:136 never applies. `monotone`: no scene has a negative leaf
    // distance, so t never decreases along a ray.
    int tame = 1, shallow = 1, monotone = 1;
    for (int32_t i = threadIdx.x; i < P.n_scenes; i += blockDim.x) {
        const navi_relaid_scene d = P.scenes[i];
        lds_scenes[i] = SceneLds{d.bbox_min[0], d.bbox_min[1], d.bbox_min[2],
                                 d.bbox_max[0], d.bbox_max[1], d.bbox_max[2], d.root_slot, 0u};
        for (int a = 0; a < 3; ++a)
            tame &= (fabsf(d.bbox_min[a]) < 0x1p100f && fabsf(d.bbox_max[a]) < 0x1p100f) ? 1 : 0;
        shallow &= d.max_depth <= static_cast<uint32_t>(kMaxDepth - 2) ? 1 : 0;
        monotone &= (d.flags & NAVI_SCENE_NONNEG_LEAVES) ? 1 : 0;
    }
    LaunchConds c;
    c.tame = __syncthreads_and(tame);
    c.shallow = __syncthreads_and(shallow);
    // The void cache (kernel.cu:265-267) changes nothing in tame, monotone
    // launches: a point strictly inside the cached void cell lies in the
    // closed box of no other terminal cell (tame boxes nest), so the leaf
    // cache misses and a query meets that cell again, with the same exit
    // distance. Along a ray whose t never decreases the samples inside the
    // open cell are consecutive, right after the step that found it, so the
    // prefix cache then holds that cell's depth-4 ancestor (when it is deeper
    // than 4; else the query stops above depth 4 and saves nothing) and the
    // query leaves every cache as it was. Such launches skip the void cache.
    c.void_cache = !(c.tame && __syncthreads_and(monotone));
    // `planes`: every scene's depth-D cells can be located from its planes
    int planes = 0;
    if constexpr (kPlanes) planes = stage_planes<kPD>(P, lds_planes) ? 1 : 0;
    c.planes = planes;
    return c;
}

// Whether a launch takes the fast march (every workgroup reaches the same answer).
__device__ __forceinline__ bool fast_applies(const RelaidParams& P, const LaunchConds& c) {
    return c.planes && c.tame && c.shallow && !c.void_cache && P.small_tables && P.max_distance < kOutsideDomain;
}

// The last wave to finish rearms the queue for the next launch on this
// stream: every other wave has made its final claim before counting itself.
__device__ __forceinline__ void rearm_queue(const RelaidParams& P) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t n_waves = (gridDim.x * blockDim.x) >> 6;
    if (P.queue != nullptr && lane == 0) {
        if (atomicAdd(P.queue + 1, 1u) == n_waves - 1u) {
            atomicExch(P.queue, 0u);
            atomicExch(P.queue + 1, 0u);
        }
    }
}

// The fast march in a kernel of its own, at eight waves per SIMD (64 vector
// registers; the general march needs 72, and six waves instead of seven cost
// the fast march 8% where eight gain it 5%). Launched first when its planes
// fit one of its two shapes and the launch has a work queue; it records in the
// queue's third word whether the fast march applied and returns at once when
// it does not (the general kernel, launched next, then traces the launch).
template <int kDepth, int kPD, bool kPoses, int kThreads, bool kLeaves>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(8))) void trace_fast_kernel(RelaidParams P) {
    static_assert(kPD >= 4 && kPD <= 8 && kDepth >= 4 && kDepth <= kPD + 2 && kDepth <= 7,
                  "planes of 4..8 levels, the table at most two levels below them");
    extern __shared__ SceneLds lds_scenes[];
    float* const lds_planes = reinterpret_cast<float*>(lds_scenes + P.n_scenes);
    const LaunchConds c = stage_scenes<kPD>(P, lds_scenes, lds_planes);
    const bool fast = fast_applies(P, c);
    if (blockIdx.x == 0 && threadIdx.x == 0) P.queue[2] = fast ? 1u : 0u;
    if (!fast) return;
    march_fast<kDepth, kPD, kPoses, true, kLeaves>(P, lds_scenes, lds_planes,
                                             reinterpret_cast<uint32_t*>(lds_planes + P.n_scenes * scene_stride(kPD)));
    rearm_queue(P);
}

// Both marches, at seven waves per SIMD: the fast march where it applies (for
// launches whose planes fit neither of the fast kernel's shapes), else
// the general one. Launched after trace_fast_kernel (after_fast), it returns at
// once when that one traced the launch.
template <int kDepth, int kPD, bool kPoses>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(7))) void trace_relaid_kernel(RelaidParams P) {
    constexpr bool kPlanes = kPD > 0;
    static_assert(!kPlanes || (kPD >= 4 && kPD <= 6 && kDepth >= kPD && kDepth <= kPD + 2 && kDepth <= 7),
                  "planes of 4..6 levels, the table at most two levels below them");
    if (P.after_fast && __hip_atomic_load(P.queue + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u) return;
    extern __shared__ SceneLds lds_scenes[];
    float* const lds_planes = reinterpret_cast<float*>(lds_scenes + P.n_scenes);
    const LaunchConds c = stage_scenes<kPD>(P, lds_scenes, lds_planes);
    if constexpr (kPlanes) {
        if (fast_applies(P, c))
            march_fast<kDepth, kPD, kPoses, false, true>(
                P, lds_scenes, lds_planes, reinterpret_cast<uint32_t*>(lds_planes + P.n_scenes * scene_stride(kPD)));
        else
            march<kDepth, kPD, kPoses, false>(P, lds_scenes, lds_planes, c.tame, c.shallow, c.planes, c.void_cache);
    } else {
        march<kDepth, kPD, kPoses, false>(P, lds_scenes, lds_planes, c.tame, c.shallow, c.planes, c.void_cache);
    }
    rearm_queue(P);
}

// Resident waves the chip holds for this kernel: the persistent grid is sized
// to exactly that, so no wave waits for a slot and the sweep has no second,
// partly empty round.
// (per device, kernel variant and LDS size of the launch; guarded by g_queue_mu).
std::map<std::pair<std::pair<int, int>, size_t>, int> g_grid_blocks;

// Work-queue counters: [next unit, finished waves, the fast kernel traced the
// launch, unused] in one 64 KiB device buffer per device, allocated and zeroed
// by navi_device_init (the third word is written by each fast kernel before the
// general kernel after it reads it; "pair" below means these four words).
// * An eager launch uses the pair of its (stream, thread for
//   hipStreamPerThread): launches on one stream run in order, so the pair is
//   never used by two launches at once, and the kernel's last wave rearms it
//   for the next.
// * A launch recorded into a graph gets a pair of its own (a graph may be
//   replayed on any stream, and two launches of one capture may run at once),
//   cleared by a small kernel node before the tracer on every replay. A HIP
//   user object retained by the graph gives the pair back when the graph and
//   the executable graphs made from it are destroyed.
// * When the table's pairs are all taken, an eager launch leases one of the
//   reserve pairs: one whose event (recorded after its last launch) has
//   completed, cleared before the launch. A launch finds no pair (and takes the
//   static schedule) only while every reserve pair is in flight, or while a
//   stream captures on a device that was never initialised (no allocation
//   inside a capture).
constexpr int kQueueSlots = 4096;
constexpr int kQueueWords = 4;
constexpr int kLeasePairs = 64;                          // the table's last pairs
constexpr int kTablePairs = kQueueSlots - kLeasePairs;  // streams and captures
std::mutex g_queue_mu;
struct DeviceQueues {
    uint32_t* mem = nullptr;
    int used = 0;                                    // table pairs handed out, [0, kTablePairs)
    std::vector<int> free_pairs;                     // given back by destroyed graphs
    std::map<std::pair<void*, size_t>, int> slot;   // (stream, thread) -> pair
    hipEvent_t lease_event[kLeasePairs] = {};
    uint8_t lease_busy[kLeasePairs] = {};            // 1: being set up by a launch (event not yet recorded)
    uint8_t lease_used[kLeasePairs] = {};            // an event has been recorded after a launch
    int lease_next = 0;
};
std::unordered_map<int, DeviceQueues> g_queues;

// The calling thread's last launch (navi_last_launch).
thread_local navi_launch_info g_last_launch = {};

// Allocates the current device's counters and lease events if it has none
// (g_queue_mu held).
int init_device_locked(int dev) {
    DeviceQueues& q = g_queues[dev];
    if (q.mem != nullptr) return NAVI_OK;
    void* p = nullptr;
    if (hipMalloc(&p, kQueueSlots * kQueueWords * sizeof(uint32_t)) != hipSuccess)
        return set_error(NAVI_E_NOMEM, "work-queue counters: hipMalloc failed on device %d", dev);
    if (hipMemset(p, 0, kQueueSlots * kQueueWords * sizeof(uint32_t)) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess) {
        (void)hipFree(p);
        return set_error(NAVI_E_LAUNCH, "work-queue counters: clearing failed on device %d", dev);
    }
    for (int i = 0; i < kLeasePairs; ++i) {
        if (hipEventCreateWithFlags(&q.lease_event[i], hipEventDisableTiming) != hipSuccess) {
            for (int k = 0; k < i; ++k) (void)hipEventDestroy(q.lease_event[k]);
            (void)hipFree(p);
            return set_error(NAVI_E_LAUNCH, "work-queue counters: hipEventCreate failed on device %d", dev);
        }
    }
    q.mem = static_cast<uint32_t*>(p);
    return NAVI_OK;
}

// A capture's pair, handed back by the destructor of the user object the
// captured graph retains.
struct CapturePair {
    int dev, pair;
};
void release_capture_pair(void* p) {
    CapturePair* cp = static_cast<CapturePair*>(p);
    {
        std::lock_guard<std::mutex> lock(g_queue_mu);
        g_queues[cp->dev].free_pairs.push_back(cp->pair);
    }
    delete cp;
}

// The pair a launch on `stream` uses: its counter words (null for none), its
// NAVI_QUEUE_* kind and table index; a leased pair's lease index in *lease.
struct QueueChoice {
    uint32_t* words = nullptr;
    uint32_t kind = NAVI_QUEUE_NONE;
    int pair = -1;
    int lease = -1;
    int dev = 0;
};

QueueChoice queue_for(hipStream_t stream) {
    QueueChoice c;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return c;
    c.dev = dev;
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &status) != hipSuccess) status = hipStreamCaptureStatusNone;
    const bool capturing = status != hipStreamCaptureStatusNone;
    {
        std::lock_guard<std::mutex> lock(g_queue_mu);
        DeviceQueues& q = g_queues[dev];
        if (q.mem == nullptr && (capturing || init_device_locked(dev) != NAVI_OK)) return c;
        if (capturing) {
            if (!q.free_pairs.empty()) {
                c.pair = q.free_pairs.back();
                q.free_pairs.pop_back();
            } else if (q.used < kTablePairs) {
                c.pair = q.used++;
            } else {
                return c;
            }
            c.kind = NAVI_QUEUE_CAPTURE;
        } else {
            const size_t thread =
                stream == hipStreamPerThread ? std::hash<std::thread::id>{}(std::this_thread::get_id()) : 0;
            const auto key = std::make_pair(static_cast<void*>(stream), thread);
            auto it = q.slot.find(key);
            if (it == q.slot.end() && q.used < kTablePairs) it = q.slot.emplace(key, q.used++).first;
            if (it != q.slot.end()) {
                c.pair = it->second;
                c.kind = NAVI_QUEUE_STREAM;
            } else {
                // lease a reserve pair whose last launch has completed
                for (int k = 0; k < kLeasePairs && c.lease < 0; ++k) {
                    const int i = (q.lease_next + k) % kLeasePairs;
                    if (q.lease_busy[i]) continue;
                    if (q.lease_used[i] && hipEventQuery(q.lease_event[i]) != hipSuccess) continue;
                    c.lease = i;
                }
                if (c.lease < 0) return c;
                q.lease_busy[c.lease] = 1;
                q.lease_next = (c.lease + 1) % kLeasePairs;
                c.pair = kTablePairs + c.lease;
                c.kind = NAVI_QUEUE_LEASE;
            }
        }
        c.words = q.mem + kQueueWords * c.pair;
    }
    if (c.kind == NAVI_QUEUE_CAPTURE) {
        // tie the pair to the graph being captured (outside the lock: HIP may
        // run destructors, which take it); on failure the pair stays taken
        hipGraph_t graph = nullptr;
        unsigned long long id = 0;
        hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
        hipUserObject_t obj = nullptr;
        CapturePair* cp = new CapturePair{dev, c.pair};
        if (hipStreamGetCaptureInfo_v2(stream, &st, &id, &graph, nullptr, nullptr) == hipSuccess && graph != nullptr &&
            hipUserObjectCreate(&obj, cp, release_capture_pair, 1, hipUserObjectNoDestructorSync) == hipSuccess) {
            (void)hipGraphRetainUserObject(graph, obj, 1, hipGraphUserObjectMove);
        } else {
            delete cp;
        }
    }
    return c;
}

// After a leased launch was enqueued: record its event (the pair is free again
// once it completes).
void finish_lease(const QueueChoice& c, hipStream_t stream) {
    if (c.kind != NAVI_QUEUE_LEASE) return;
    std::lock_guard<std::mutex> lock(g_queue_mu);
    DeviceQueues& q = g_queues[c.dev];
    q.lease_used[c.lease] = hipEventRecord(q.lease_event[c.lease], stream) == hipSuccess ? 1 : 0;
    q.lease_busy[c.lease] = q.lease_used[c.lease] ? 0 : 1;  // a failed record keeps the pair out of use
}

// Scratch of navi_trace_relaid_noalloc: one set of work-queue counter words per device
// in a static device array (each GPU the library runs on holds its own copy
// until the process ends). Host code never uses the array's name as an
// address: navi_device_init (or the entry point's first call on a device)
// looks up the device's copy with hipGetSymbolAddress and keeps the pointer.
constexpr int kScratchWords = 64;  // 256 bytes; a launch uses words 0 to 2
constexpr int kMaxDevices = 64;
uint32_t* g_scratch_ptr[kMaxDevices] = {};  // guarded by g_queue_mu

}  // namespace navi

static __device__ __align__(256) uint32_t scratch[navi::kScratchWords];

namespace navi {

// The current device's copy of `scratch` into *out (g_queue_mu held; dev current).
int scratch_locked(int dev, uint32_t** out) {
    if (dev < 0 || dev >= kMaxDevices)
        return set_error(NAVI_E_ARG, "device %d is beyond the %d devices the scratch table holds", dev, kMaxDevices);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (err != hipSuccess || ptr == nullptr)
            return set_error(NAVI_E_LAUNCH, "scratch: hipGetSymbolAddress failed on device %d: %s", dev,
                             hipGetErrorString(err));
        g_scratch_ptr[dev] = static_cast<uint32_t*>(ptr);
    }
    *out = g_scratch_ptr[dev];
    return NAVI_OK;
}

// Zeroes the counter words before a launch that shares them (a kernel node, never a
// memset node, so the launch can be captured into a graph).
__global__ void clear_queue_kernel(uint32_t* queue) {
    if (threadIdx.x < 3) queue[threadIdx.x] = 0u;
}

// Grid blocks of a persistent launch of `kernel` with `lds` bytes per workgroup:
// the workgroups the chip holds at once (cached per device, variant and LDS).
int resident_blocks(void (*kernel)(RelaidParams), int variant, size_t lds, bool keep, int threads) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = 0;
    const auto key = std::make_pair(std::make_pair(dev, variant), lds);
    {
        std::lock_guard<std::mutex> lock(g_queue_mu);
        auto it = g_grid_blocks.find(key);
        if (it != g_grid_blocks.end()) return it->second;
    }
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, lds) != hipSuccess || per_cu <= 0)
        per_cu = 1;
    const int blocks = cus * per_cu;
    if (keep) {  // the no-allocation entry point keeps no host table entry either
        std::lock_guard<std::mutex> lock(g_queue_mu);
        g_grid_blocks[key] = blocks;
    }
    return blocks;
}

// Sizes the work units and the grid of one persistent launch and enqueues it;
// *waves receives the grid's waves.
int enqueue_relaid(void (*kernel)(RelaidParams), RelaidParams P, int variant, size_t lds, bool keep,
                   hipStream_t stream, int threads = 256, uint32_t* waves = nullptr) {
    const int grid_blocks = resident_blocks(kernel, variant, lds, keep, threads);
    const int waves_per_block = threads / 64;
    // Small batches: one-tile units, so that more waves get work (a launch
    // wants several units per resident wave to balance the long rays).
    P.unit_rays = kUnitRays;
    if (static_cast<int64_t>(P.n_rays) < static_cast<int64_t>(kUnitRays) * 4 * waves_per_block * grid_blocks)
        P.unit_rays = kSmallUnitRays;
    P.n_units = (P.n_rays + P.unit_rays - 1u) / P.unit_rays;
    int64_t blocks = (static_cast<int64_t>(P.n_chunks) + waves_per_block - 1) / waves_per_block;
    if (blocks > grid_blocks) blocks = grid_blocks;
    if (blocks < 1) blocks = 1;
    if (waves) *waves = static_cast<uint32_t>(blocks) * static_cast<uint32_t>(waves_per_block);
    hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(blocks)), dim3(threads), lds, stream, P);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return set_error(NAVI_E_LAUNCH, "kernel launch failed: %s", hipGetErrorString(err));
    return NAVI_OK;
}

// The deepest split-plane depth P <= min(D, 6), at most two levels above the
// table, whose planes and scene table fit `budget` bytes; 0 if none does.
int plane_depth_for(int32_t n_scenes, uint32_t D, size_t budget) {
    for (int p = D < 6 ? static_cast<int>(D) : 6; p >= 4 && p + 2 >= static_cast<int>(D); --p)
        if (static_cast<size_t>(n_scenes) * (sizeof(SceneLds) + scene_stride(p) * sizeof(float)) <= budget) return p;
    return 0;
}

// The deepest split-plane depth P in [max(4, D - 2), min(D + 2, 8)] whose
// planes and scene table fit `budget` bytes; 0 if none does.
int plane_depth_wide(int32_t n_scenes, uint32_t D, size_t budget) {
    const int lo = D > 6 ? static_cast<int>(D) - 2 : 4;
    for (int p = D + 2 < 8 ? static_cast<int>(D) + 2 : 8; p >= lo; --p)
        if (static_cast<size_t>(n_scenes) * (sizeof(SceneLds) + scene_stride(p) * sizeof(float)) <= budget) return p;
    return 0;
}

// queue: the counter words to use (no_alloc), or null to take the stream's.
// A launch whose planes fit kFastLdsWide or kFastLds (and that has a queue, a
// range below the outside-domain distance and small tables) enqueues trace_fast_kernel, then
// trace_relaid_kernel with after_fast, which returns at once when the fast
// kernel traced it (every other launch: trace_relaid_kernel alone).
int launch_relaid_queued(RelaidParams P, hipStream_t stream, uint32_t* scratch_queue, navi_launch_info& info);

int launch_relaid(RelaidParams P, hipStream_t stream, uint32_t* scratch_queue = nullptr) {
    navi_launch_info info = {};
    info.n_rays = P.n_rays;
    QueueChoice c;
    if (scratch_queue != nullptr) {
        c.words = scratch_queue;
        c.kind = NAVI_QUEUE_SCRATCH;
    } else {
        c = queue_for(stream);
    }
    info.queue = c.kind;
    info.pair = c.pair;
    const int code = launch_relaid_queued(P, stream, c.words, info);
    finish_lease(c, stream);  // also after a failed launch: the lease's event then completes at once
    g_last_launch = info;
    return code;
}

// The launch with its counter words `queue` (null: static schedule).
int launch_relaid_queued(RelaidParams P, hipStream_t stream, uint32_t* queue, navi_launch_info& info) {
    const bool no_alloc = info.queue == NAVI_QUEUE_SCRATCH;
    P.n_chunks = (P.n_rays + 63u) / 64u;
    P.queue = queue;
    const uint32_t D = P.cell_depth;
    P.small_tables = (static_cast<uint64_t>(P.n_scenes) << (3u * D + 3u)) < (1ull << 32) ? 1u : 0u;
    const bool poses = P.local_dirs != nullptr;
    const bool leaves = P.leaves != nullptr;
    // counters another launch may have used: cleared first (a kernel node,
    // never a memset node, so the launch can be captured into a graph)
    if (P.queue != nullptr && info.queue != NAVI_QUEUE_STREAM)
        hipLaunchKernelGGL(clear_queue_kernel, dim3(1), dim3(64), 0, stream, P.queue);

    // the fast kernel: for large launches planes up to two levels below the
    // table in two 1024-thread workgroups per CU, else planes that fit eight
    // 256-thread workgroups
    P.after_fast = 0u;
    if (P.queue != nullptr && P.small_tables && P.max_distance < kOutsideDomain) {
        RelaidParams F = P;
        void (*fast)(RelaidParams) = nullptr;
        size_t lds = 0;
        int threads = kWideThreads;
        int variant = 0;
        const bool wide = F.n_rays >= g_wide_min_rays.load(std::memory_order_relaxed);
        const int pw = wide ? plane_depth_wide(F.n_scenes, D, kFastLdsWide) : 0;
        if (pw != 0) {
            lds = static_cast<size_t>(F.n_scenes) * (sizeof(SceneLds) + scene_stride(pw) * sizeof(float));
            F.stage = (F.out_steps == nullptr && lds + stage_lds(kWideThreads) <= kFastLdsWide) ? 1u : 0u;
            if (F.stage) lds += stage_lds(kWideThreads);
#define NAVI_FAST(d, p)                                                                                       \
    (leaves ? (poses ? trace_fast_kernel<d, p, true, kWideThreads, true> : trace_fast_kernel<d, p, false, kWideThreads, true>) \
            : (poses ? trace_fast_kernel<d, p, true, kWideThreads, false>                                        \
                     : trace_fast_kernel<d, p, false, kWideThreads, false>))
            switch (pw * 8 + static_cast<int>(D)) {
                case 4 * 8 + 4: fast = NAVI_FAST(4, 4); break;
                case 5 * 8 + 4: fast = NAVI_FAST(4, 5); break;
                case 6 * 8 + 4: fast = NAVI_FAST(4, 6); break;
                case 4 * 8 + 5: fast = NAVI_FAST(5, 4); break;
                case 5 * 8 + 5: fast = NAVI_FAST(5, 5); break;
                case 6 * 8 + 5: fast = NAVI_FAST(5, 6); break;
                case 7 * 8 + 5: fast = NAVI_FAST(5, 7); break;
                case 4 * 8 + 6: fast = NAVI_FAST(6, 4); break;
                case 5 * 8 + 6: fast = NAVI_FAST(6, 5); break;
                case 6 * 8 + 6: fast = NAVI_FAST(6, 6); break;
                case 7 * 8 + 6: fast = NAVI_FAST(6, 7); break;
                case 8 * 8 + 6: fast = NAVI_FAST(6, 8); break;
                case 5 * 8 + 7: fast = NAVI_FAST(7, 5); break;
                case 6 * 8 + 7: fast = NAVI_FAST(7, 6); break;
                case 7 * 8 + 7: fast = NAVI_FAST(7, 7); break;
                case 8 * 8 + 7: fast = NAVI_FAST(7, 8); break;
                default: break;
            }
#undef NAVI_FAST
            variant = 2 * (pw * 8 + static_cast<int>(D)) + static_cast<int>(poses) + 2048 + (leaves ? 4096 : 0);
        }
        // (the 256-thread shape has no instances for leaf tables: such launches take the combined kernel)
        const int pf = (fast == nullptr && !leaves && F.n_rays >= kFastMinRays) ? plane_depth_for(F.n_scenes, D, kFastLds)
                                                                                : 0;
        if (pf != 0) {
            threads = 256;
            lds = static_cast<size_t>(F.n_scenes) * (sizeof(SceneLds) + scene_stride(pf) * sizeof(float));
            F.stage = (F.out_steps == nullptr && lds + kStageLds <= kFastLds) ? 1u : 0u;
            if (F.stage) lds += kStageLds;
#define NAVI_FAST(d, p) (poses ? trace_fast_kernel<d, p, true, 256, false> : trace_fast_kernel<d, p, false, 256, false>)
            switch (pf * 8 + static_cast<int>(D)) {
                case 4 * 8 + 4: fast = NAVI_FAST(4, 4); break;
                case 4 * 8 + 5: fast = NAVI_FAST(5, 4); break;
                case 4 * 8 + 6: fast = NAVI_FAST(6, 4); break;
                case 5 * 8 + 5: fast = NAVI_FAST(5, 5); break;
                case 5 * 8 + 6: fast = NAVI_FAST(6, 5); break;
                case 5 * 8 + 7: fast = NAVI_FAST(7, 5); break;
                case 6 * 8 + 6: fast = NAVI_FAST(6, 6); break;
                case 6 * 8 + 7: fast = NAVI_FAST(7, 6); break;
                default: break;
            }
#undef NAVI_FAST
            variant = 2 * (pf * 8 + static_cast<int>(D)) + static_cast<int>(poses) + 1024;
        }
        if (fast != nullptr) {
            const int code = enqueue_relaid(fast, F, variant, lds, !no_alloc, stream, threads, &info.waves);
            if (code != NAVI_OK) return code;
            P.after_fast = 1u;
            info.kernels |= NAVI_KERNEL_FAST | (threads == kWideThreads ? NAVI_KERNEL_FAST_WIDE : 0u);
            info.fast_planes = static_cast<uint32_t>(pw != 0 ? pw : pf);
            info.staged = F.stage;
        }
    }

    // both marches at seven waves: planes fitting kPlaneLds, else kPlaneLdsWide
    int pd = plane_depth_for(P.n_scenes, D, kPlaneLds);
    if (pd == 0) pd = plane_depth_for(P.n_scenes, D, kPlaneLdsWide);
    size_t lds = static_cast<size_t>(P.n_scenes) * (sizeof(SceneLds) + (pd ? scene_stride(pd) * sizeof(float) : 0));
    // output staging where it fits the budget the planes were sized for (and
    // no step counts are asked for: those are stored per ray)
    P.stage = (pd != 0 && P.out_steps == nullptr && lds + kStageLds <= (lds <= kPlaneLds ? kPlaneLds : kPlaneLdsWide))
                  ? 1u : 0u;
    if (P.stage) lds += kStageLds;
    void (*kernel)(RelaidParams) = nullptr;
#define NAVI_RELAID(d, p) (poses ? trace_relaid_kernel<d, p, true> : trace_relaid_kernel<d, p, false>)
    switch (pd * 8 + static_cast<int>(D)) {
        case 4 * 8 + 4: kernel = NAVI_RELAID(4, 4); break;
        case 4 * 8 + 5: kernel = NAVI_RELAID(5, 4); break;
        case 4 * 8 + 6: kernel = NAVI_RELAID(6, 4); break;
        case 5 * 8 + 5: kernel = NAVI_RELAID(5, 5); break;
        case 5 * 8 + 6: kernel = NAVI_RELAID(6, 5); break;
        case 5 * 8 + 7: kernel = NAVI_RELAID(7, 5); break;
        case 6 * 8 + 6: kernel = NAVI_RELAID(6, 6); break;
        case 6 * 8 + 7: kernel = NAVI_RELAID(7, 6); break;
        default: kernel = NAVI_RELAID(0, 0); break;
    }
#undef NAVI_RELAID
    info.kernels |= NAVI_KERNEL_COMBINED;
    info.planes = static_cast<uint32_t>(pd);
    if (!P.after_fast) info.staged = P.stage;
    return enqueue_relaid(kernel, P, 2 * (pd * 8 + static_cast<int>(D)) + static_cast<int>(poses), lds, !no_alloc,
                          stream, 256, P.after_fast ? nullptr : &info.waves);
}

}  // namespace navi

namespace navi {

// Arguments shared by the two relaid entry points.
int relaid_setup(RelaidParams& P, const uint32_t* records, uint64_t n_records, const navi_relaid_scene* scenes,
                 int32_t n_scenes, const uint64_t* cell_tables, int32_t table_depth, const int32_t* env_scene,
                 const int32_t* env_order, int64_t n_envs, int64_t rays_per_env, int32_t elevation_bins,
                 float* out_distances, int32_t* out_semantics, int32_t max_steps, float max_distance,
                 float hit_epsilon, int32_t* out_steps) {
    if (max_steps <= 0) return set_error(NAVI_E_ARG, "max_steps must be a positive integer");
    if (!std::isfinite(max_distance) || !(max_distance > 0.0f))
        return set_error(NAVI_E_ARG, "max_distance must be a finite positive float");
    if (!(hit_epsilon == hit_epsilon)) return set_error(NAVI_E_ARG, "hit_epsilon must not be NaN");
    if (n_envs < 0 || rays_per_env < 0) return set_error(NAVI_E_ARG, "n_envs and rays_per_env must be non-negative");
    if (n_scenes <= 0 || !scenes || !records) return set_error(NAVI_E_ARG, "scene table must be non-empty");
    if (!cell_tables) return set_error(NAVI_E_ARG, "cell_tables is required (navi_build_cell_table)");
    if (table_depth < 4 || table_depth > 7) return set_error(NAVI_E_ARG, "table_depth must be in [4, 7]");
    if (n_scenes > kMaxScenes) return set_error(NAVI_E_ARG, "navi_trace_relaid takes at most 1024 scenes");
    // the pool is read through a buffer resource whose size field (bytes) is
    // 32-bit: 2^27 records would wrap it to 0
    if (n_records >= (1ull << 27)) return set_error(NAVI_E_ARG, "record pool must hold fewer than 2^27 records (4 GiB)");
    if (rays_per_env > (1LL << 30) || (rays_per_env > 0 && n_envs > (1LL << 30) / rays_per_env))
        return set_error(NAVI_E_ARG, "navi_trace_relaid handles at most 2^30 rays per launch");
    // 32-bit work indexing: every ray index times 3, plus 2, fits in uint32
    const int64_t n_rays = n_envs * rays_per_env;
    if (n_rays > 0 && (!out_distances || !out_semantics))
        return set_error(NAVI_E_ARG, "output pointers must be non-null");
    P = RelaidParams{};
    P.records = records;
    P.n_records = static_cast<uint32_t>(n_records);
    P.scenes = scenes;
    P.n_scenes = n_scenes;
    P.cell_table = cell_tables;
    P.cell_depth = static_cast<uint32_t>(table_depth);
    P.env_scene = env_scene;
    P.env_order = env_order;
    P.n_rays = static_cast<uint32_t>(n_rays);
    P.n_envs = static_cast<uint32_t>(n_envs);
    P.rays_per_env = static_cast<uint32_t>(rays_per_env);
    P.div_rays = make_fastdiv(P.rays_per_env);
    P.tile_el = (elevation_bins > 0 && elevation_bins % 8 == 0 && rays_per_env % (8LL * elevation_bins) == 0)
                    ? static_cast<uint32_t>(elevation_bins)
                    : 0u;
    P.div_tiles_el = make_fastdiv(P.tile_el ? P.tile_el / 8u : 1u);
    P.out_d = out_distances;
    P.out_s = out_semantics;
    P.out_steps = out_steps;
    P.max_steps = max_steps;
    P.max_distance = max_distance;
    P.hit_eps = hit_epsilon;
    P.sem_bits = 15u;
    return NAVI_OK;
}

}  // namespace navi

extern "C" int navi_device_init(void) {
    using namespace navi;
    int dev = 0;
    const hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return set_error(NAVI_E_LAUNCH, "no HIP device: %s", hipGetErrorString(err));
    std::lock_guard<std::mutex> lock(g_queue_mu);
    uint32_t* ptr = nullptr;
    const int code = scratch_locked(dev, &ptr);
    if (code != NAVI_OK) return code;
    return init_device_locked(dev);
}

extern "C" uint64_t navi_set_wide_min_rays(uint64_t n_rays) { return navi::g_wide_min_rays.exchange(n_rays); }

extern "C" int navi_last_launch(navi_launch_info* info) {
    if (!info) return navi::set_error(NAVI_E_ARG, "info must be non-null");
    *info = navi::g_last_launch;
    return NAVI_OK;
}

extern "C" int navi_trace_relaid_ex(const navi_relaid_launch* L, void* stream) {
    using namespace navi;
    if (!L) return set_error(NAVI_E_ARG, "launch must be non-null");
    RelaidParams P;
    const int code = relaid_setup(P, L->records, L->n_records, L->scenes, L->n_scenes, L->cell_tables, L->table_depth,
                                  L->env_scene, L->env_order, L->n_envs, L->rays_per_env, L->elevation_bins,
                                  static_cast<float*>(L->out_distances), L->out_semantics, L->max_steps,
                                  L->max_distance, L->hit_epsilon, L->out_steps);
    if (code != NAVI_OK) return code;
    if (L->distance_dtype != NAVI_DIST_F32 && L->distance_dtype != NAVI_DIST_BF16 && L->distance_dtype != NAVI_DIST_F16)
        return set_error(NAVI_E_ARG, "distance_dtype must be NAVI_DIST_F32, NAVI_DIST_BF16 or NAVI_DIST_F16");
    if (P.n_rays == 0) return NAVI_OK;
    P.dist_dtype = static_cast<uint32_t>(L->distance_dtype);
    if (L->local_dirs) {
        if (!L->env_pos || !L->env_rot) return set_error(NAVI_E_ARG, "env_pos and env_rot must be non-null");
        P.local_dirs = L->local_dirs;
        P.env_pos = L->env_pos;
        P.env_rot = L->env_rot;
    } else {
        if (!L->origins || !L->dirs) return set_error(NAVI_E_ARG, "origins and dirs (or local_dirs) must be non-null");
        P.origins = L->origins;
        P.dirs = L->dirs;
    }
    if (L->n_leaves > 0) {
        if (!L->leaves) return set_error(NAVI_E_ARG, "leaves must be non-null when n_leaves > 0");
        if (L->n_leaves > 0x10000u) return set_error(NAVI_E_ARG, "a leaf table holds at most 65536 entries");
        P.leaves = L->leaves;
        P.n_leaves = L->n_leaves;
        P.sem_bits = 16u;
    }
    return launch_relaid(P, static_cast<hipStream_t>(stream));
}


extern "C" int navi_trace_relaid_noalloc(const uint32_t* records, uint64_t n_records,
                                         const navi_relaid_scene* scenes, int32_t n_scenes,
                                         const uint64_t* cell_tables, int32_t table_depth,
                                         const int32_t* env_scene, const int32_t* env_order, int64_t n_envs,
                                         int64_t rays_per_env, int32_t elevation_bins, const float* origins,
                                         const float* dirs, float* out_distances, int32_t* out_semantics,
                                         int32_t max_steps, float max_distance, float hit_epsilon,
                                         int32_t* out_steps, void* stream) {
    using namespace navi;
    RelaidParams P;
    const int code = relaid_setup(P, records, n_records, scenes, n_scenes, cell_tables, table_depth, env_scene,
                                  env_order, n_envs, rays_per_env, elevation_bins, out_distances, out_semantics,
                                  max_steps, max_distance, hit_epsilon, out_steps);
    if (code != NAVI_OK || P.n_rays == 0) return code;
    if (!origins || !dirs) return set_error(NAVI_E_ARG, "ray and output pointers must be non-null");
    P.origins = origins;
    P.dirs = dirs;
    int dev = 0;
    const hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return set_error(NAVI_E_LAUNCH, "no HIP device: %s", hipGetErrorString(err));
    uint32_t* queue = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_queue_mu);
        const int sc = scratch_locked(dev, &queue);
        if (sc != NAVI_OK) return sc;
    }
    return launch_relaid(P, static_cast<hipStream_t>(stream), queue);
}

extern "C" int navi_trace_relaid(const uint32_t* records, uint64_t n_records, const navi_relaid_scene* scenes,
                                 int32_t n_scenes, const uint64_t* cell_tables, int32_t table_depth,
                                 const int32_t* env_scene, const int32_t* env_order, int64_t n_envs,
                                 int64_t rays_per_env, int32_t elevation_bins, const float* origins,
                                 const float* dirs, float* out_distances, int32_t* out_semantics,
                                 int32_t max_steps, float max_distance, float hit_epsilon,
                                 int32_t* out_steps, void* stream) {
    using namespace navi;
    RelaidParams P;
    const int code = relaid_setup(P, records, n_records, scenes, n_scenes, cell_tables, table_depth, env_scene,
                                  env_order, n_envs, rays_per_env, elevation_bins, out_distances, out_semantics,
                                  max_steps, max_distance, hit_epsilon, out_steps);
    if (code != NAVI_OK || P.n_rays == 0) return code;
    if (!origins || !dirs) return set_error(NAVI_E_ARG, "ray and output pointers must be non-null");
    P.origins = origins;
    P.dirs = dirs;
    return launch_relaid(P, static_cast<hipStream_t>(stream));
}

extern "C" int navi_trace_relaid_poses(const uint32_t* records, uint64_t n_records,
                                       const navi_relaid_scene* scenes, int32_t n_scenes,
                                       const uint64_t* cell_tables, int32_t table_depth,
                                       const int32_t* env_scene,
                                       const int32_t* env_order, int64_t n_envs, int64_t rays_per_env,
                                       int32_t elevation_bins, const float* local_dirs, const float* env_pos,
                                       const float* env_rot, float* out_distances, int32_t* out_semantics,
                                       int32_t max_steps, float max_distance, float hit_epsilon,
                                       int32_t* out_steps, void* stream) {
    using namespace navi;
    RelaidParams P;
    const int code = relaid_setup(P, records, n_records, scenes, n_scenes, cell_tables, table_depth, env_scene,
                                  env_order, n_envs, rays_per_env, elevation_bins, out_distances, out_semantics,
                                  max_steps, max_distance, hit_epsilon, out_steps);
    if (code != NAVI_OK || P.n_rays == 0) return code;
    if (!local_dirs || !env_pos || !env_rot)
        return set_error(NAVI_E_ARG, "local_dirs, env_pos and env_rot must be non-null");
    P.local_dirs = local_dirs;
    P.env_pos = env_pos;
    P.env_rot = env_rot;
    return launch_relaid(P, static_cast<hipStream_t>(stream));
}
