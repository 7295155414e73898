// relayout.cpp — host-side conversion of the reference DAG word layout into the
// tracer's device layout (part of libnavi_trace.so).
//
// Reference layout (docs/GMDAG.md:161-228, projects/torch-sdf/cpp_src/kernel.cu:
// 137-198 of the seismael/navi checkout): u64 words; a leaf has bit 63 set, its
// semantic in bits 31..16 and an fp16 distance in bits 15..0; an internal node
// has a child mask in bits 62..55 and a child-table base in bits 31..0, the
// table holding popcount(mask) words whose low 32 bits index the child.
// Descending one level costs two dependent loads (node, then table slot).
//
// Device layout: one 32-byte record per reachable internal node, records in
// breadth-first order from the root (so the top levels are a contiguous
// prefix), each holding eight u32 slots indexed by octant:
//   0x7fffffff             void octant (mask bit clear)
//   0x7ffffffe             the child-table word lies past the array: the
//                          reference reads out of range at this level
//   0x7ffffffd             the child index lies past the array: the reference
//                          reads out of range when it examines the child
//                          (only below the 32-level limit of kernel.cu:136)
//   0xffff0000 | i         leaf whose semantic is 0x7fff or above (the format's
//                          field is 16 bits, docs/GMDAG.md:215,223): entry i of
//                          a leaf table of u32 (semantic << 16) | fp16 distance
//   bit 31 set             leaf inlined: bits 30..16 semantic (below 0x7fff),
//                          15..0 fp16 distance
//   otherwise              index of the child's record
// Descending one level is one 4-byte load at record*8 + octant, and a leaf
// costs no load of its own (one more for a table leaf). Traversal semantics
// are unchanged: the tracer's caches key on boxes, which depend only on the
// tree shape.
//
// Not representable (NAVI_E_LAYOUT; use the reference-layout kernel): more
// than 0x7ffffffc internal nodes, more than 65536 distinct (semantic,
// distance) pairs of semantic 0x7fff or above, or any such leaf when the
// caller gives no leaf table (navi_relayout).
#include <stdint.h>

#include <cstring>
#include <unordered_map>
#include <vector>

#include "navi_trace.h"

namespace navi {
int set_error(int code, const char* fmt, ...);
}

namespace {

constexpr uint32_t kSlotVoid = 0x7fffffffu;
constexpr uint32_t kSlotFault = 0x7ffffffeu;
constexpr uint32_t kSlotBadChild = 0x7ffffffdu;  // lowest terminal slot value
constexpr uint32_t kUnassigned = 0xffffffffu;
constexpr uint32_t kTableLeaf = 0xffff0000u;  // a leaf slot whose semantic field is all ones
constexpr uint32_t kMaxTableLeaves = 0x10000u;

// The leaf table being built: distinct (semantic << 16 | distance) words of
// semantic 0x7fff or above, in order of first sight; null when the caller
// gives none.
struct LeafTable {
    std::vector<uint32_t> words;
    std::unordered_map<uint32_t, uint32_t> index;
};

// Slot value of a leaf word (bit 63 set), or false when it needs a leaf table
// that is absent or full.
inline bool leaf_slot(uint64_t node, LeafTable* leaves, uint32_t& out) {
    const uint32_t sem = static_cast<uint32_t>(node >> 16) & 0xffffu;
    const uint32_t dist = static_cast<uint32_t>(node & 0xffffu);
    if (sem < 0x7fffu) {
        out = 0x80000000u | (sem << 16) | dist;
        return true;
    }
    if (leaves == nullptr) return false;
    const uint32_t word = (sem << 16) | dist;
    auto it = leaves->index.find(word);
    if (it == leaves->index.end()) {
        if (leaves->words.size() >= kMaxTableLeaves) return false;
        it = leaves->index.emplace(word, static_cast<uint32_t>(leaves->words.size())).first;
        leaves->words.push_back(word);
    }
    out = kTableLeaf | it->second;
    return true;
}

// Slot value for a child word index, assigning record ids on first sight.
inline bool child_slot(const uint64_t* w, uint64_t n, uint32_t idx, std::vector<uint32_t>& rec_of,
                       std::vector<uint32_t>& queue, LeafTable* leaves, uint32_t& out) {
    if (static_cast<uint64_t>(idx) >= n) {
        out = kSlotBadChild;
        return true;
    }
    const uint64_t node = w[idx];
    if (node >> 63) return leaf_slot(node, leaves, out);
    if (rec_of[idx] == kUnassigned) {
        if (queue.size() >= kSlotBadChild) return false;
        rec_of[idx] = static_cast<uint32_t>(queue.size());
        queue.push_back(idx);
    }
    out = rec_of[idx];
    return true;
}

}  // namespace

namespace {

// Longest chain of internal records below `root` (the root at 0), or
// 0xffffffff when a cycle or an out-of-range record is reachable.
// Iterative depth-first search, O(records + slots).
uint32_t longest_chain(const uint32_t* records, uint64_t n_records, uint32_t root) {
    if (root >= kSlotBadChild) return 0;  // one-leaf DAG (or a void / fault root slot)
    if (root >= n_records) return 0xffffffffu;
    // height[r]: longest chain of records below r (0 = no internal child);
    // kOpen marks a record on the current path (a revisit means a cycle).
    constexpr uint32_t kUnseen = 0xffffffffu, kOpen = 0xfffffffeu;
    std::vector<uint32_t> height(n_records, kUnseen);
    struct Frame {
        uint32_t rec;
        uint32_t next;  // next octant to visit
        uint32_t best;
    };
    std::vector<Frame> stack;
    stack.push_back({root, 0u, 0u});
    height[root] = kOpen;
    while (!stack.empty()) {
        Frame& f = stack.back();
        if (f.next == 8u) {
            height[f.rec] = f.best;
            const uint32_t h = f.best;
            stack.pop_back();
            if (!stack.empty() && h + 1u > stack.back().best) stack.back().best = h + 1u;
            continue;
        }
        const uint32_t slot = records[8ull * f.rec + f.next++];
        if (slot >= kSlotBadChild) continue;  // leaf, void or fault slot
        if (slot >= n_records) return 0xffffffffu;
        const uint32_t h = height[slot];
        if (h == kOpen) return 0xffffffffu;
        if (h == kUnseen) {
            height[slot] = kOpen;
            stack.push_back({slot, 0u, 0u});
        } else if (h + 1u > f.best) {
            f.best = h + 1u;
        }
    }
    return height[root];
}

}  // namespace

namespace {

int relayout(const uint64_t* words, uint64_t n_words, uint32_t* out_records, uint64_t cap_records,
             uint64_t* n_records, uint32_t* root_slot, uint64_t* n_levels_prefix, LeafTable* leaves) {
    using navi::set_error;
    if (!words || n_words == 0) return set_error(NAVI_E_ARG, "dag must hold at least one word");
    if (!n_records || !root_slot) return set_error(NAVI_E_ARG, "n_records and root_slot are required");
    const uint64_t root = words[0];
    if (root >> 63) {  // a one-leaf DAG: no records
        if (!leaf_slot(root, leaves, *root_slot))
            return set_error(NAVI_E_LAYOUT, "leaf semantic %u needs a leaf table",
                             static_cast<uint32_t>(root >> 16) & 0xffffu);
        *n_records = 0;
        if (n_levels_prefix) std::memset(n_levels_prefix, 0, 8 * sizeof(uint64_t));
        return NAVI_OK;
    }
    std::vector<uint32_t> rec_of(n_words, kUnassigned);
    std::vector<uint32_t> queue;
    queue.reserve(1024);
    rec_of[0] = 0;
    queue.push_back(0);
    *root_slot = 0;
    // breadth-first: record r's children are assigned ids in octant order
    size_t level_end = 1;
    int level = 0;
    if (n_levels_prefix) std::memset(n_levels_prefix, 0, 8 * sizeof(uint64_t));
    for (size_t r = 0; r < queue.size(); ++r) {
        if (r == level_end) {
            if (n_levels_prefix && level < 8) n_levels_prefix[level] = level_end;
            ++level;
            level_end = queue.size();
        }
        const uint64_t node = words[queue[r]];
        const uint32_t mask = static_cast<uint32_t>(node >> 55) & 0xffu;
        const uint32_t base = static_cast<uint32_t>(node);
        uint32_t slots[8];
        uint32_t k = 0;
        for (uint32_t oct = 0; oct < 8; ++oct) {
            if (!(mask & (1u << oct))) {
                slots[oct] = kSlotVoid;
                continue;
            }
            const uint32_t tab = base + k;  // uint32 arithmetic, as kernel.cu:197
            ++k;
            if (static_cast<uint64_t>(tab) >= n_words) {
                slots[oct] = kSlotFault;
                continue;
            }
            const uint32_t child = static_cast<uint32_t>(words[tab]);
            if (!child_slot(words, n_words, child, rec_of, queue, leaves, slots[oct]))
                return set_error(NAVI_E_LAYOUT, leaves ? "DAG not representable in the device layout (more than "
                                                         "65536 distinct leaves of semantic 0x7fff or above, or "
                                                         "too many nodes)"
                                                       : "DAG not representable in the device layout (a leaf "
                                                         "semantic of 0x7fff or above needs a leaf table, "
                                                         "navi_relayout_leaves; or too many nodes)");
        }
        if (out_records) {
            if (r >= cap_records) return set_error(NAVI_E_ARG, "record buffer too small");
            std::memcpy(out_records + 8 * r, slots, sizeof slots);
        }
    }
    if (n_levels_prefix) {
        for (int l = level; l < 8; ++l) n_levels_prefix[l] = queue.size();
    }
    *n_records = queue.size();
    // When no record lies deeper than 30 levels every slot is examined above
    // the 32-level limit, where a bad child index faults like a bad table word.
    if (out_records && longest_chain(out_records, queue.size(), 0u) <= 30u) {
        for (size_t k = 0; k < 8 * queue.size(); ++k)
            if (out_records[k] == kSlotBadChild) out_records[k] = kSlotFault;
    }
    return NAVI_OK;
}

}  // namespace

extern "C" int navi_relayout(const uint64_t* words, uint64_t n_words, uint32_t* out_records,
                             uint64_t cap_records, uint64_t* n_records, uint32_t* root_slot,
                             uint64_t* n_levels_prefix) {
    return relayout(words, n_words, out_records, cap_records, n_records, root_slot, n_levels_prefix, nullptr);
}

extern "C" int navi_relayout_leaves(const uint64_t* words, uint64_t n_words, uint32_t* out_records,
                                    uint64_t cap_records, uint64_t* n_records, uint32_t* root_slot,
                                    uint64_t* n_levels_prefix, uint32_t* out_leaves, uint32_t cap_leaves,
                                    uint32_t* n_leaves) {
    using navi::set_error;
    if (!n_leaves) return set_error(NAVI_E_ARG, "n_leaves is required");
    LeafTable leaves;
    const int code = relayout(words, n_words, out_records, cap_records, n_records, root_slot, n_levels_prefix,
                              &leaves);
    if (code != NAVI_OK) return code;
    *n_leaves = static_cast<uint32_t>(leaves.words.size());
    if (out_leaves) {
        if (leaves.words.size() > cap_leaves) return set_error(NAVI_E_ARG, "leaf table buffer too small");
        if (!leaves.words.empty()) std::memcpy(out_leaves, leaves.words.data(), leaves.words.size() * 4);
    }
    return NAVI_OK;
}

// The NAVI_SCENE_* flags the records reachable from root_slot support: an
// iterative walk over the internal records (each visited once; out-of-range
// records end their branch) that looks at every leaf slot's fp16 sign bit,
// in the leaf table for a table leaf.
extern "C" int navi_scene_flags(const uint32_t* records, uint64_t n_records, uint32_t root_slot,
                                const uint32_t* leaves, uint32_t n_leaves, uint32_t* flags) {
    using navi::set_error;
    if (!flags || (!records && n_records) || (!leaves && n_leaves)) return set_error(NAVI_E_ARG, "null argument");
    bool negative = false;
    auto leaf_negative = [&](uint32_t slot) {
        uint32_t word = slot;
        if ((slot & kTableLeaf) == kTableLeaf) {
            const uint32_t i = slot & 0xffffu;
            if (i >= n_leaves) return false;  // the tracer reads 0 there: distance +0
            word = leaves[i];
        }
        return ((word >> 15) & 1u) != 0u;
    };
    if (root_slot & 0x80000000u) {
        negative = leaf_negative(root_slot);
    } else if (root_slot < n_records) {
        std::vector<uint8_t> seen(n_records, 0);
        std::vector<uint32_t> stack{root_slot};
        seen[root_slot] = 1;
        while (!stack.empty() && !negative) {
            const uint32_t r = stack.back();
            stack.pop_back();
            for (uint32_t oct = 0; oct < 8u; ++oct) {
                const uint32_t slot = records[8ull * r + oct];
                if (slot & 0x80000000u) {
                    negative = negative || leaf_negative(slot);
                } else if (slot < kSlotBadChild && slot < n_records && !seen[slot]) {
                    seen[slot] = 1;
                    stack.push_back(slot);
                }
            }
        }
    }
    *flags = negative ? 0u : NAVI_SCENE_NONNEG_LEAVES;
    return NAVI_OK;
}

namespace {

// Cells of the block a slot covers at depth d: a terminal slot (leaf, void,
// fault, bad child) above depth D, or the slot met at depth D, fills its
// (2^(D-d))^3 cells; an internal slot above depth D recurses into its
// octants (x bit 0, y bit 1, z bit 2: the upper half along an axis holds the
// points >= the midpoint, kernel.cu:165-176).
void fill_cells(const uint32_t* records, uint64_t n_records, uint32_t slot, uint32_t d, uint32_t D,
                uint32_t x0, uint32_t y0, uint32_t z0, uint64_t* out) {
    if (d == D || slot >= kSlotBadChild) {
        // a bad child index examined above depth 32 is a fault
        const uint32_t s = slot == kSlotBadChild ? kSlotFault : slot;
        const uint64_t v = static_cast<uint64_t>(s) | (static_cast<uint64_t>(d) << 32);
        const uint32_t w = 1u << (D - d);
        for (uint32_t z = z0; z < z0 + w; ++z)
            for (uint32_t y = y0; y < y0 + w; ++y) {
                uint64_t* row = out + ((static_cast<uint64_t>(z) << D | y) << D);
                for (uint32_t x = x0; x < x0 + w; ++x) row[x] = v;
            }
        return;
    }
    const uint32_t half = 1u << (D - d - 1);
    for (uint32_t oct = 0; oct < 8u; ++oct) {
        const uint32_t child = static_cast<uint64_t>(slot) < n_records ? records[8ull * slot + oct] : kSlotFault;
        fill_cells(records, n_records, child, d + 1, D, x0 + (oct & 1u) * half, y0 + ((oct >> 1) & 1u) * half,
                   z0 + (oct >> 2) * half, out);
    }
}

}  // namespace

// Cell table: what a descent from the root reaches within the first D
// levels (kernel.cu:136-199 stops at a leaf or void cell). The depth-D cells
// form a 2^D x 2^D x 2^D grid; entry (iz << 2D) | (iy << D) | ix holds, for the
// cell whose octant at depth l has x bit (ix >> (D - 1 - l)) & 1 (y, z
// likewise), the slot met and, in bits 32..34, its depth d: a leaf / void /
// fault slot at d <= D, or the record of the internal node at d = D. Only
// octant bits are involved, so a tracer that locates the cell itself and
// reads one entry follows the same path as D record reads; the depth-4 node
// on that path (the prefix cache of kernel.cu:154-163) is internal exactly
// when d > 4, or d = 4 and the slot is a record. A one-leaf DAG maps every
// entry to its root leaf at depth 0.
extern "C" int navi_build_cell_table(const uint32_t* records, uint64_t n_records, uint32_t root_slot,
                                     int32_t depth, uint64_t* out_table) {
    using navi::set_error;
    if (!out_table || (!records && n_records)) return set_error(NAVI_E_ARG, "null argument");
    if (depth < 4 || depth > 7) return set_error(NAVI_E_ARG, "table depth must be in [4, 7]");
    fill_cells(records, n_records, root_slot, 0u, static_cast<uint32_t>(depth), 0u, 0u, 0u, out_table);
    return NAVI_OK;
}

// Longest chain of internal records below the root, in levels: the deepest
// record reachable from root_slot sits at that depth (the root at 0). Records
// hold record slots as indices into `records` (a pool). *max_depth is
// 0xffffffff when a cycle or an out-of-range record is reachable, where the
// descent limit of kernel.cu:136 decides results.
extern "C" int navi_record_depth(const uint32_t* records, uint64_t n_records, uint32_t root_slot,
                                 uint32_t* max_depth) {
    using navi::set_error;
    if (!max_depth || (!records && n_records)) return set_error(NAVI_E_ARG, "null argument");
    *max_depth = longest_chain(records, n_records, root_slot);
    return NAVI_OK;
}
