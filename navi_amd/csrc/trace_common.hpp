// trace_common.hpp — device-side pieces shared by the tracer kernels.
//
// Semantics follow projects/torch-sdf/cpp_src/kernel.cu (paths relative to the
// seismael/navi checkout); each helper cites the lines it restates. Every
// floating-point operation is a single IEEE-754 binary32 operation: the library
// is built with -ffp-contract=off and the one contraction the reference build
// makes (p = o + t*d, kernel.cu:261-263) is written as an explicit fma.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace navi {

constexpr float kOutsideDomain = 1000.0f;   // kernel.cuh:8
constexpr float kDirEps = 1e-4f;            // kernel.cuh:9
constexpr int kPrefixDepth = 4;             // kernel.cuh:11
constexpr float kVoidAdvanceEps = 1e-5f;    // kernel.cu:9
constexpr int kMaxDepth = 32;               // kernel.cu:136

struct Box {
    float x0, y0, z0, x1, y1, z1;
};

// kernel.cu:11-21 (inclusive)
__device__ __forceinline__ bool in_box(float px, float py, float pz, const Box& b) {
    return px >= b.x0 && px <= b.x1 && py >= b.y0 && py <= b.y1 && pz >= b.z0 && pz <= b.z1;
}

// kernel.cu:23-33 (strict)
__device__ __forceinline__ bool in_box_strict(float px, float py, float pz, const Box& b) {
    return px > b.x0 && px < b.x1 && py > b.y0 && py < b.y1 && pz > b.z0 && pz < b.z1;
}

// kernel.cu:43-47: binary16 -> binary32 (exact; v_cvt_f32_f16 keeps f16 denormals).
__device__ __forceinline__ float half_to_float(uint32_t bits) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits & 0xffffu)));
}

// kernel.cu:54-85
__device__ __forceinline__ float exit_distance(float px, float py, float pz, float dx, float dy,
                                               float dz, const Box& b) {
    float t = kOutsideDomain;
    if (dx > kDirEps) {
        t = fminf(t, (b.x1 - px) / dx);
    } else if (dx < -kDirEps) {
        t = fminf(t, (b.x0 - px) / dx);
    }
    if (dy > kDirEps) {
        t = fminf(t, (b.y1 - py) / dy);
    } else if (dy < -kDirEps) {
        t = fminf(t, (b.y0 - py) / dy);
    }
    if (dz > kDirEps) {
        t = fminf(t, (b.z1 - pz) / dz);
    } else if (dz < -kDirEps) {
        t = fminf(t, (b.z0 - pz) / dz);
    }
    return fmaxf(t, kVoidAdvanceEps);
}

// kernel.cu:165-176: split `cur` at its midpoint toward p; returns the octant.
__device__ __forceinline__ uint32_t descend_octant(float px, float py, float pz, Box& cur) {
    const float mx = (cur.x0 + cur.x1) * 0.5f;
    const float my = (cur.y0 + cur.y1) * 0.5f;
    const float mz = (cur.z0 + cur.z1) * 0.5f;
    uint32_t oct = 0;
    if (px >= mx) { oct |= 1u; cur.x0 = mx; } else { cur.x1 = mx; }
    if (py >= my) { oct |= 2u; cur.y0 = my; } else { cur.y1 = my; }
    if (pz >= mz) { oct |= 4u; cur.z0 = mz; } else { cur.z1 = mz; }
    return oct;
}

// The wave's lanes for which b holds. (HIP's __ballot takes an int and compares
// it with 0, which costs a select and a compare for a bool that lives as a lane
// mask, e.g. across loop iterations.)
__device__ __forceinline__ uint64_t wave_mask(bool b) { return __builtin_amdgcn_ballot_w64(b); }

// set bits of a wave mask, as a 32-bit count (two scalar bit counts; a 64-bit
// count would be compared on the vector unit)
__device__ __forceinline__ uint32_t lane_count(uint64_t m) {
    return static_cast<uint32_t>(__builtin_popcount(static_cast<uint32_t>(m))) +
           static_cast<uint32_t>(__builtin_popcount(static_cast<uint32_t>(m >> 32)));
}

// i * 2 + b in one add-with-carry, the comparison's lane mask as carry-in
// (the compiler spends two operations, a select and a shift-or).
__device__ __forceinline__ uint32_t append_bit(uint32_t i, bool b) {
    const uint64_t mask = wave_mask(b);  // this lane's bit is b; inactive lanes are ignored
    uint32_t r;
    uint64_t carry_out;
    asm("v_addc_co_u32_e64 %0, %1, %2, %2, %3" : "=v"(r), "=s"(carry_out) : "v"(i), "s"(mask));
    return r;
}

// This lane's bit of a wave mask (the mask itself is the lane predicate).
__device__ __forceinline__ bool lane_in(uint64_t mask) { return __builtin_amdgcn_inverse_ballot_w64(mask); }

// i + (this lane's bit of mask): one add-with-carry, the mask as carry-in.
// The mask is wave-uniform; reading it through readfirstlane keeps it in
// scalar registers for the asm operand even where the compiler cannot prove
// that (free where it can).
__device__ __forceinline__ int32_t add_lane_bit(int32_t i, uint64_t mask) {
    // (the builtin returns int: widen through uint32_t, not by sign extension)
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(mask >> 32)));
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(mask)));
    const uint64_t m = (static_cast<uint64_t>(hi) << 32) | lo;
    int32_t r;
    uint64_t carry_out;
    asm("v_addc_co_u32_e64 %0, %1, %2, 0, %3" : "=v"(r), "=s"(carry_out) : "v"(i), "s"(m));
    return r;
}

// descend_octant fused with slot addressing: returns base * 8 + octant, the
// octant's z, y and x bits appended in that order (one add-with-carry each).
__device__ __forceinline__ uint32_t descend_index(float px, float py, float pz, Box& cur, uint32_t base) {
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
    uint32_t i = append_bit(base, gz);
    i = append_bit(i, gy);
    return append_bit(i, gx);
}

// One split of descend_octant toward a known octant.
__device__ __forceinline__ void split_box(Box& cur, uint32_t oct) {
    const float mx = (cur.x0 + cur.x1) * 0.5f;
    const float my = (cur.y0 + cur.y1) * 0.5f;
    const float mz = (cur.z0 + cur.z1) * 0.5f;
    if (oct & 1u) { cur.x0 = mx; } else { cur.x1 = mx; }
    if (oct & 2u) { cur.y0 = my; } else { cur.y1 = my; }
    if (oct & 4u) { cur.z0 = mz; } else { cur.z1 = mz; }
}

}  // namespace navi
