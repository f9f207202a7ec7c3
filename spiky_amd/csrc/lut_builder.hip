// lut_builder.hip -- host-side receptive-field index builder.
//
// Replaces, for the LUT layers, the reference's spatial growth engine
// (spiky_cuda/synapse_growth/synapse_growth.cu:16-445, kernel
// synapse_growth_kernels_logic.proto:69-374) as driven by the Python helpers
// Conv2DSynapseGrowthHelper / RandomRectanglesSynapseGrowthHelper /
// GivenRectanglesSynapseGrowthHelper (src/spiky/util/synapse_growth.py).
//
// A source neuron at (x, y, z) connects to every target neuron whose
// coordinates lie inside the cuboid [x+x1, x+x2] x [y+y1, y+y2] x [z+z1, z+z2],
// the bounds evaluated in fp32 exactly as the reference does
// (synapse_growth_kernels_logic.proto:229-256: a target is rejected if it is
// below the lower or above the upper bound).  With connection probability
// p == 1 the result is deterministic: targets of a source in ascending id
// order, sources in ascending id order.  p < 1 keeps a target when a
// splitmix64 hash of (seed, source id, target id) falls below p; that draw has
// no counterpart in the reference (whose generator is cuRAND) and is stable
// across runs only.
#include "../../include/spiky_lut.h"

#include <algorithm>
#include <cstring>
#include <numeric>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

}  // namespace

extern "C" int spiky_grow_cuboid(uint32_t n_src, const int32_t *src_ids, const float *src_xyz,
                                 uint32_t n_tgt, const int32_t *tgt_ids, const float *tgt_xyz,
                                 const float *cuboid, float p, uint64_t seed,
                                 uint32_t max_per_source, int64_t *out_offsets,
                                 int32_t *out_targets, uint64_t capacity, uint64_t *out_total) {
    if (!src_ids || !src_xyz || !tgt_ids || !tgt_xyz || !cuboid || !out_offsets || !out_total)
        return SPIKY_VALUE_ERROR;
    if (!(p > 0.0f && p <= 1.0f)) return SPIKY_VALUE_ERROR;
    // sources in ascending id order
    std::vector<uint32_t> sorder(n_src);
    std::iota(sorder.begin(), sorder.end(), 0u);
    std::stable_sort(sorder.begin(), sorder.end(),
                     [&](uint32_t a, uint32_t b) { return src_ids[a] < src_ids[b]; });
    // targets sorted along x for a range search
    std::vector<uint32_t> torder(n_tgt);
    std::iota(torder.begin(), torder.end(), 0u);
    std::stable_sort(torder.begin(), torder.end(),
                     [&](uint32_t a, uint32_t b) { return tgt_xyz[3 * a] < tgt_xyz[3 * b]; });
    std::vector<float> tx(n_tgt);
    for (uint32_t i = 0; i < n_tgt; i++) tx[i] = tgt_xyz[3 * torder[i]];
    const uint64_t p_threshold = (p >= 1.0f) ? ~0ull : (uint64_t)((double)p * 18446744073709551615.0);
    uint64_t total = 0;
    std::vector<int32_t> found;
    out_offsets[0] = 0;
    for (uint32_t si = 0; si < n_src; si++) {
        const uint32_t s = sorder[si];
        const float sx = src_xyz[3 * s], sy = src_xyz[3 * s + 1], sz = src_xyz[3 * s + 2];
        const float lx = sx + cuboid[0], ly = sy + cuboid[1], lz = sz + cuboid[2];
        const float hx = sx + cuboid[3], hy = sy + cuboid[4], hz = sz + cuboid[5];
        found.clear();
        auto it = std::lower_bound(tx.begin(), tx.end(), lx);
        for (size_t k = (size_t)(it - tx.begin()); k < tx.size() && !(tx[k] > hx); k++) {
            const uint32_t t = torder[k];
            const float ty = tgt_xyz[3 * t + 1], tz = tgt_xyz[3 * t + 2];
            if (ty < ly || ty > hy || tz < lz || tz > hz) continue;
            if (p < 1.0f) {
                const uint64_t h = splitmix64(seed ^ splitmix64(((uint64_t)(uint32_t)src_ids[s] << 32) |
                                                                (uint32_t)tgt_ids[t]));
                if (h > p_threshold) continue;
            }
            found.push_back(tgt_ids[t]);
        }
        std::sort(found.begin(), found.end());
        found.erase(std::unique(found.begin(), found.end()), found.end());
        if (max_per_source > 0 && found.size() > max_per_source) found.resize(max_per_source);
        if (out_targets) {
            if (total + found.size() > capacity) return SPIKY_VALUE_ERROR;
            std::memcpy(out_targets + total, found.data(), found.size() * sizeof(int32_t));
        }
        total += found.size();
        out_offsets[si + 1] = (int64_t)total;
    }
    *out_total = total;
    return SPIKY_OK;
}
