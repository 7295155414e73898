// scene_compiler.cpp — libnavi_scene.so: procedural scene -> .gmdag DAG words.
//
// The input format of the tracer is produced by the reference's voxel-dag
// compiler (projects/voxel-dag/src/compiler.cpp, paths relative to the
// seismael/navi checkout). This is a host-side compiler for procedural scenes
// that emits words under the same rules:
//   - samples on voxel corners bmin + i*voxel, dense index z*N*N + y*N + x
//     (compiler.cpp:474-483);
//   - build_recursive (compiler.cpp:579-659): size-1 leaf with semantic
//     d < 2*voxel; uniform collapse when every sample is within 1e-6 of the
//     block's first sample; an octant is void when its minimum sample exceeds
//     half*voxel*1.7321; an all-void node becomes a far leaf (semantic 0);
//   - exact structural dedup of leaves and internal nodes, post-order pool,
//     index 0 reserved and overwritten with the root (compiler.cpp:143-190,
//     661-674);
//   - fp16 distances rounded to nearest even (the reference's float_to_half,
//     compiler.cpp:542-560, truncates and maps |d| < 2^-14 to +inf; it is
//     available as quirk_half = 1).
//
// What differs from the reference is only how the samples are obtained. The
// scene is a union of analytic primitives and each sample is the truncated
// unsigned CSG distance min(|min_i s_i(p)|, trunc). The grid is never
// materialised: an octree over 8^3-voxel bricks classifies each primitive per
// region by a 1-Lipschitz interval bound on its exact SDF, so a brick is
// evaluated only where some primitive surface lies within the truncation
// distance; every other brick is the constant `trunc`. Block minima / maxima
// for the build rules come from a min/max pyramid over bricks (and scans inside
// a brick), which gives the same decisions as the reference's block scans
// because IEEE subtraction is monotone.
#include <omp.h>
#include <stdint.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

namespace {

enum PrimType : int { kSphere = 0, kSolidBox = 1, kRoomInterior = 2 };

struct Prim {
    int type;
    double a[6];
};

// Exact signed distance of one primitive (negative inside the solid).
inline double box_sdf(const double p[3], const double lo[3], const double hi[3]) {
    double q[3], out2 = 0.0, inside = -1e300;
    for (int k = 0; k < 3; ++k) {
        const double c = 0.5 * (lo[k] + hi[k]);
        const double h = 0.5 * (hi[k] - lo[k]);
        q[k] = std::fabs(p[k] - c) - h;
        const double m = q[k] > 0.0 ? q[k] : 0.0;
        out2 += m * m;
        inside = q[k] > inside ? q[k] : inside;
    }
    return std::sqrt(out2) + (inside < 0.0 ? inside : 0.0);
}

inline double prim_sdf(const Prim& pr, const double p[3]) {
    switch (pr.type) {
        case kSphere: {
            const double dx = p[0] - pr.a[0], dy = p[1] - pr.a[1], dz = p[2] - pr.a[2];
            return std::sqrt(dx * dx + dy * dy + dz * dz) - pr.a[3];
        }
        case kSolidBox:
            return box_sdf(p, pr.a, pr.a + 3);
        default:  // room interior is free space: the solid is the complement
            return -box_sdf(p, pr.a, pr.a + 3);
    }
}

constexpr int kBrick = 8;

struct Scene {
    std::vector<Prim> prims;
    double bmin[3];
    double voxel;
    int N;
    double trunc;
};

inline void sample_point(const Scene& s, int x, int y, int z, double p[3]) {
    p[0] = s.bmin[0] + x * s.voxel;
    p[1] = s.bmin[1] + y * s.voxel;
    p[2] = s.bmin[2] + z * s.voxel;
}

inline float sample_value(const Scene& s, const std::vector<int>& active, const double p[3]) {
    double m = 1e300;
    for (int i : active) m = std::min(m, prim_sdf(s.prims[i], p));
    const double v = std::min(std::fabs(m), s.trunc);
    return static_cast<float>(v);
}

// Sparse grid: per brick, either the constant `trunc` or 512 evaluated samples.
struct SparseGrid {
    int N = 0, nb = 0;  // voxels per axis, bricks per axis
    float trunc = 0.f;
    std::vector<int32_t> brick_id;  // nb^3, -1 = constant trunc
    std::vector<float> data;        // active bricks * 512, [z][y][x] inside the brick
    // min/max pyramid over bricks; level 0 = bricks, level L has nb>>L per axis
    std::vector<std::vector<float>> pmin, pmax;

    inline float at(int x, int y, int z) const {
        const int b = brick_id[((size_t)(z / kBrick) * nb + (y / kBrick)) * nb + (x / kBrick)];
        if (b < 0) return trunc;
        return data[(size_t)b * 512 + ((z % kBrick) * kBrick + (y % kBrick)) * kBrick + (x % kBrick)];
    }
};

// Octree over bricks: collect bricks with a primitive surface within trunc.
struct Classifier {
    const Scene& s;
    std::vector<std::pair<int, std::vector<int>>> active_bricks;  // (linear brick, prims)
    int nb;

    Classifier(const Scene& sc, int nbricks) : s(sc), nb(nbricks) {}

    void visit(int bx, int by, int bz, int bsize, const std::vector<int>& cand) {
        // region of samples covered: voxel indices [b*K, (b+bsize)*K - 1]
        const int lo_i[3] = {bx * kBrick, by * kBrick, bz * kBrick};
        const int hi_i[3] = {std::min((bx + bsize) * kBrick, s.N) - 1,
                             std::min((by + bsize) * kBrick, s.N) - 1,
                             std::min((bz + bsize) * kBrick, s.N) - 1};
        if (lo_i[0] >= s.N || lo_i[1] >= s.N || lo_i[2] >= s.N) return;
        double c[3], r2 = 0.0;
        for (int k = 0; k < 3; ++k) {
            const double a = s.bmin[k] + lo_i[k] * s.voxel;
            const double b = s.bmin[k] + hi_i[k] * s.voxel;
            c[k] = 0.5 * (a + b);
            r2 += 0.25 * (b - a) * (b - a);
        }
        const double R = std::sqrt(r2) * (1.0 + 1e-12) + 1e-9;
        std::vector<int> keep;
        keep.reserve(cand.size());
        for (int i : cand) {
            const double v = prim_sdf(s.prims[i], c);  // 1-Lipschitz: v - R <= s(p) <= v + R
            if (v + R <= -s.trunc) return;             // inside a solid deeper than trunc: all trunc
            if (v - R >= s.trunc) continue;            // surface farther than trunc
            keep.push_back(i);
        }
        if (keep.empty()) return;
        if (bsize == 1) {
            active_bricks.emplace_back((bz * nb + by) * nb + bx, std::move(keep));
            return;
        }
        const int h = bsize / 2;
        for (int o = 0; o < 8; ++o)
            visit(bx + ((o & 1) ? h : 0), by + ((o & 2) ? h : 0), bz + ((o & 4) ? h : 0), h, keep);
    }
};

void build_sparse(const Scene& s, SparseGrid& g, int threads) {
    g.N = s.N;
    g.nb = (s.N + kBrick - 1) / kBrick;
    g.trunc = static_cast<float>(std::min(s.trunc, 3.0e38));
    int top = 1;
    while (top < g.nb) top *= 2;
    Classifier cl(s, g.nb);
    std::vector<int> all(s.prims.size());
    for (size_t i = 0; i < all.size(); ++i) all[i] = (int)i;
    cl.visit(0, 0, 0, top, all);
    std::sort(cl.active_bricks.begin(), cl.active_bricks.end(),
              [](const auto& a, const auto& b) { return a.first < b.first; });
    g.brick_id.assign((size_t)g.nb * g.nb * g.nb, -1);
    const size_t na = cl.active_bricks.size();
    g.data.assign(na * 512, 0.f);
    for (size_t k = 0; k < na; ++k) g.brick_id[cl.active_bricks[k].first] = (int32_t)k;

    std::vector<float> bmin_v(g.brick_id.size(), g.trunc), bmax_v(g.brick_id.size(), g.trunc);
#pragma omp parallel for schedule(dynamic, 16) num_threads(threads)
    for (long long k = 0; k < (long long)na; ++k) {
        const int lin = cl.active_bricks[k].first;
        const std::vector<int>& act = cl.active_bricks[k].second;
        const int bx = lin % g.nb, by = (lin / g.nb) % g.nb, bz = lin / (g.nb * g.nb);
        float mn = 3.4e38f, mx = -3.4e38f;
        for (int z = 0; z < kBrick; ++z)
            for (int y = 0; y < kBrick; ++y)
                for (int x = 0; x < kBrick; ++x) {
                    const int gx = bx * kBrick + x, gy = by * kBrick + y, gz = bz * kBrick + z;
                    float v = g.trunc;
                    if (gx < s.N && gy < s.N && gz < s.N) {
                        double p[3];
                        sample_point(s, gx, gy, gz, p);
                        v = sample_value(s, act, p);
                        mn = std::min(mn, v);
                        mx = std::max(mx, v);
                    }
                    g.data[(size_t)k * 512 + (z * kBrick + y) * kBrick + x] = v;
                }
        bmin_v[lin] = mn;
        bmax_v[lin] = mx;
    }
    // pyramid
    g.pmin.clear();
    g.pmax.clear();
    g.pmin.push_back(std::move(bmin_v));
    g.pmax.push_back(std::move(bmax_v));
    int n = g.nb;
    while (n > 1) {
        const int m = (n + 1) / 2;
        std::vector<float> a((size_t)m * m * m), b((size_t)m * m * m);
        const auto& pa = g.pmin.back();
        const auto& pb = g.pmax.back();
        for (int z = 0; z < m; ++z)
            for (int y = 0; y < m; ++y)
                for (int x = 0; x < m; ++x) {
                    float mn = 3.4e38f, mx = -3.4e38f;
                    for (int o = 0; o < 8; ++o) {
                        const int cx = 2 * x + (o & 1), cy = 2 * y + ((o >> 1) & 1), cz = 2 * z + (o >> 2);
                        if (cx >= n || cy >= n || cz >= n) continue;
                        const size_t li = ((size_t)cz * n + cy) * n + cx;
                        mn = std::min(mn, pa[li]);
                        mx = std::max(mx, pb[li]);
                    }
                    a[((size_t)z * m + y) * m + x] = mn;
                    b[((size_t)z * m + y) * m + x] = mx;
                }
        g.pmin.push_back(std::move(a));
        g.pmax.push_back(std::move(b));
        n = m;
    }
}

// Min and max of samples in the block [x, x+size)^3 clipped to N.
void block_minmax(const SparseGrid& g, int x, int y, int z, int size, float& mn, float& mx) {
    if (size >= kBrick && x % kBrick == 0 && y % kBrick == 0 && z % kBrick == 0) {
        int lvl = 0, s = size / kBrick;
        while (s > 1) {
            s >>= 1;
            ++lvl;
        }
        // ceil-halving per level matches the pyramid's extent
        int m = g.nb;
        for (int k = 0; k < lvl; ++k) m = (m + 1) / 2;
        const int bx = (x / kBrick) >> lvl, by = (y / kBrick) >> lvl, bz = (z / kBrick) >> lvl;
        const size_t li = ((size_t)bz * m + by) * m + bx;
        mn = g.pmin[lvl][li];
        mx = g.pmax[lvl][li];
        return;
    }
    mn = 3.4e38f;
    mx = -3.4e38f;
    const int x1 = std::min(x + size, g.N), y1 = std::min(y + size, g.N), z1 = std::min(z + size, g.N);
    for (int bz = z; bz < z1; ++bz)
        for (int by = y; by < y1; ++by)
            for (int bx = x; bx < x1; ++bx) {
                const float v = g.at(bx, by, bz);
                mn = std::min(mn, v);
                mx = std::max(mx, v);
            }
}

uint16_t half_rne(float f) {
    uint32_t x;
    std::memcpy(&x, &f, sizeof x);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t expo = (x >> 23) & 0xffu;
    const uint32_t man = x & 0x7fffffu;
    if (expo == 0xffu) return (uint16_t)(sign | (man ? (0x7e00u | (man >> 13)) : 0x7c00u));
    const int e = (int)expo - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        const uint32_t full = man | 0x800000u;
        const int shift = 14 - e;
        uint32_t q = full >> shift;
        const uint32_t rem = full & ((1u << shift) - 1u);
        const uint32_t hw = 1u << (shift - 1);
        if (rem > hw || (rem == hw && (q & 1u))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((uint32_t)e << 10) | (man >> 13);
    const uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
}

uint16_t half_quirk(float f) {  // compiler.cpp:542-560
    uint32_t i;
    std::memcpy(&i, &f, sizeof i);
    const uint32_t s = (i >> 16) & 0x8000u;
    const uint32_t e = ((i >> 23) & 0xffu) - (127u - 15u);
    uint32_t m = i & 0x7fffffu;
    if (e == 0u) {
        m = (m | 0x800000u) >> 1;
        return (uint16_t)(s | (m >> 13));
    } else if (e == 0xffu - (127u - 15u)) {
        if (m == 0) return (uint16_t)(s | 0x7c00u);
        return (uint16_t)(s | 0x7c00u | (m >> 13) | (m ? 1u : 0u));
    }
    if (e > 30u) return (uint16_t)(s | 0x7c00u);
    return (uint16_t)(s | (e << 10) | (m >> 13));
}

// Structural dedup table (open addressing over pool indices).
struct DagBuilder {
    std::vector<uint64_t> pool;
    std::vector<uint32_t> slots;  // pool index + 1
    size_t mask = 0;
    float voxel;
    bool quirk;

    static inline uint64_t mix(uint64_t h) {
        h ^= h >> 33;
        h *= 0xff51afd7ed558ccdull;
        h ^= h >> 33;
        h *= 0xc4ceb9fe1a85ec53ull;
        h ^= h >> 33;
        return h;
    }
    static uint64_t key_hash(uint64_t node, const uint32_t* kids, int nk) {
        if (node >> 63) return mix(node);
        uint64_t h = mix(node >> 55);
        for (int i = 0; i < nk; ++i) h = mix(h ^ ((uint64_t)kids[i] + 0x9e3779b97f4a7c15ull * (uint64_t)(i + 1)));
        return h;
    }
    bool matches(uint32_t idx, uint64_t node, const uint32_t* kids, int nk) const {
        const uint64_t c = pool[idx];
        if ((c >> 63) != (node >> 63)) return false;
        if (node >> 63) return c == node;
        if (((c >> 55) & 0xffu) != ((node >> 55) & 0xffu)) return false;
        const uint32_t base = (uint32_t)c;
        for (int i = 0; i < nk; ++i)
            if (pool[base + i] != kids[i]) return false;
        return true;
    }
    void grow() {
        const size_t cap = slots.empty() ? (1u << 16) : slots.size() * 2;
        std::vector<uint32_t> ns(cap, 0);
        const size_t m = cap - 1;
        for (uint32_t v : slots) {
            if (!v) continue;
            const uint64_t node = pool[v - 1];
            uint32_t kids[8];
            int nk = 0;
            if (!(node >> 63)) {
                const uint32_t base = (uint32_t)node;
                const int cnt = __builtin_popcount((uint32_t)(node >> 55) & 0xffu);
                for (int i = 0; i < cnt; ++i) kids[nk++] = (uint32_t)pool[base + i];
            }
            size_t i = key_hash(node, kids, nk) & m;
            while (ns[i]) i = (i + 1) & m;
            ns[i] = v;
        }
        slots.swap(ns);
        mask = m;
    }
    uint32_t dedup(uint64_t node, const uint32_t* kids, int nk) {
        if ((pool.size() + 9) * 2 > slots.size()) grow();
        size_t i = key_hash(node, kids, nk) & mask;
        while (slots[i]) {
            const uint32_t idx = slots[i] - 1;
            if (matches(idx, node, kids, nk)) return idx;
            i = (i + 1) & mask;
        }
        const uint32_t at = (uint32_t)pool.size();
        if (node >> 63) {
            pool.push_back(node);
        } else {
            pool.push_back(0);
            const uint32_t start = (uint32_t)pool.size();
            for (int k = 0; k < nk; ++k) pool.push_back(kids[k]);
            pool[at] = node | start;
        }
        slots[i] = at + 1;
        return at;
    }
    uint16_t h(float f) const { return quirk ? half_quirk(f) : half_rne(f); }
    uint64_t leaf(float d, bool with_sem) const {
        const uint64_t sem = (with_sem && d < voxel * 2.0f) ? 1u : 0u;
        return (1ull << 63) | (sem << 16) | (uint64_t)h(d);
    }
};

// Value source: either a dense grid or the sparse brick grid.
struct DenseSrc {
    const float* g;
    int N;
    inline float at(int x, int y, int z) const { return g[((size_t)z * N + y) * N + x]; }
    void minmax(int x, int y, int z, int size, float& mn, float& mx) const {
        mn = 3.4e38f;
        mx = -3.4e38f;
        const int x1 = std::min(x + size, N), y1 = std::min(y + size, N), z1 = std::min(z + size, N);
        for (int bz = z; bz < z1; ++bz)
            for (int by = y; by < y1; ++by)
                for (int bx = x; bx < x1; ++bx) {
                    const float v = at(bx, by, bz);
                    mn = std::min(mn, v);
                    mx = std::max(mx, v);
                }
    }
};

struct SparseSrc {
    const SparseGrid& g;
    inline float at(int x, int y, int z) const { return g.at(x, y, z); }
    void minmax(int x, int y, int z, int size, float& mn, float& mx) const {
        block_minmax(g, x, y, z, size, mn, mx);
    }
};

// compiler.cpp:579-659 with block scans answered by min/max queries.
template <class Src>
uint32_t build(DagBuilder& b, const Src& src, int N, int x, int y, int z, int size) {
    if (size == 1) return b.dedup(b.leaf(src.at(x, y, z), true), nullptr, 0);
    const float first = src.at(x, y, z);
    {
        float mn, mx;
        src.minmax(x, y, z, size, mn, mx);
        if (!(std::fabs(mx - first) > 1e-6f) && !(std::fabs(mn - first) > 1e-6f))
            return b.dedup(b.leaf(first, true), nullptr, 0);
    }
    const int half = size / 2;
    const float extent = static_cast<float>(half) * b.voxel * 1.7321f;
    uint32_t kids[8];
    int nk = 0;
    uint32_t mask = 0;
    for (int i = 0; i < 8; ++i) {
        const int ox = (i & 1) ? half : 0, oy = (i & 2) ? half : 0, oz = (i & 4) ? half : 0;
        if (x + ox >= N || y + oy >= N || z + oz >= N) {
            // an octant entirely past the grid has no samples: its minimum is
            // FLT_MAX (compiler.cpp:567-576), which exceeds any extent
            continue;
        }
        float mn, mx;
        src.minmax(x + ox, y + oy, z + oz, half, mn, mx);
        if (mn > extent) continue;
        kids[nk++] = build(b, src, N, x + ox, y + oy, z + oz, half);
        mask |= 1u << i;
    }
    if (mask == 0) {
        float mn, mx;
        src.minmax(x, y, z, size, mn, mx);
        return b.dedup((1ull << 63) | (uint64_t)b.h(mn), nullptr, 0);
    }
    return b.dedup((uint64_t)mask << 55, kids, nk);
}

thread_local char g_err[256] = "";

template <class Src>
uint64_t compile_words(const Src& src, int N, float voxel, int quirk, uint64_t** out) {
    DagBuilder b;
    b.voxel = voxel;
    b.quirk = quirk != 0;
    b.pool.reserve(1 << 16);
    b.pool.push_back(0);
    const uint32_t root = build(b, src, N, 0, 0, 0, N);
    b.pool[0] = b.pool[root];
    uint64_t* mem = static_cast<uint64_t*>(std::malloc(b.pool.size() * sizeof(uint64_t)));
    if (!mem) {
        std::snprintf(g_err, sizeof g_err, "out of host memory for %zu words", b.pool.size());
        return 0;
    }
    std::memcpy(mem, b.pool.data(), b.pool.size() * sizeof(uint64_t));
    *out = mem;
    return b.pool.size();
}

bool parse_scene(const double* prims, int32_t n_prims, const double bmin[3], double voxel, int32_t res,
                 double trunc, Scene& s) {
    if (res <= 0 || !(voxel > 0.0) || !(trunc > 0.0) || n_prims < 0) {
        std::snprintf(g_err, sizeof g_err, "invalid scene parameters");
        return false;
    }
    s.prims.resize(n_prims);
    for (int i = 0; i < n_prims; ++i) {
        s.prims[i].type = static_cast<int>(prims[7 * i]);
        if (s.prims[i].type < 0 || s.prims[i].type > 2) {
            std::snprintf(g_err, sizeof g_err, "unknown primitive type %d", s.prims[i].type);
            return false;
        }
        for (int k = 0; k < 6; ++k) s.prims[i].a[k] = prims[7 * i + 1 + k];
    }
    for (int k = 0; k < 3; ++k) s.bmin[k] = bmin[k];
    s.voxel = voxel;
    s.N = res;
    s.trunc = trunc;
    return true;
}

}  // namespace

extern "C" {

const char* navi_scene_last_error(void) { return g_err; }

void navi_scene_free(void* p) { std::free(p); }

// Dense samples of a procedural scene, [z][y][x] float32 (tests and small grids).
// prims: n_prims rows of 7 doubles (type, 6 parameters):
//   type 0 sphere (cx, cy, cz, r, -, -), 1 solid box (lo xyz, hi xyz),
//   2 room interior (lo xyz, hi xyz; the solid is everything outside the box).
int navi_scene_sample_dense(const double* prims, int32_t n_prims, const double* bmin, double voxel,
                            int32_t res, double trunc, float* out, int32_t threads) {
    Scene s;
    if (!parse_scene(prims, n_prims, bmin, voxel, res, trunc, s)) return -1;
    std::vector<int> all(s.prims.size());
    for (size_t i = 0; i < all.size(); ++i) all[i] = (int)i;
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
    for (int z = 0; z < res; ++z)
        for (int y = 0; y < res; ++y)
            for (int x = 0; x < res; ++x) {
                double p[3];
                sample_point(s, x, y, z, p);
                out[((size_t)z * res + y) * res + x] = sample_value(s, all, p);
            }
    return 0;
}

// DAG words of a dense grid (same rules as the procedural path).
uint64_t navi_dag_compile_dense(const float* grid, int32_t res, float voxel_size, int32_t quirk_half,
                                uint64_t** out_words) {
    DenseSrc src{grid, res};
    return compile_words(src, res, voxel_size, quirk_half, out_words);
}

// DAG words of a procedural scene without materialising the grid.
// voxel_size_f32 is the header's float voxel (used by the build rules);
// sample positions use the double `voxel`. Returns the word count (0 = error).
uint64_t navi_scene_compile(const double* prims, int32_t n_prims, const double* bmin, double voxel,
                            int32_t res, double trunc, float voxel_size_f32, int32_t quirk_half,
                            int32_t threads, uint64_t** out_words, uint64_t* out_active_bricks) {
    Scene s;
    if (!parse_scene(prims, n_prims, bmin, voxel, res, trunc, s)) return 0;
    SparseGrid g;
    build_sparse(s, g, threads > 0 ? threads : 1);
    if (out_active_bricks) *out_active_bricks = g.data.size() / 512;
    SparseSrc src{g};
    return compile_words(src, res, voxel_size_f32, quirk_half, out_words);
}

}  // extern "C"
