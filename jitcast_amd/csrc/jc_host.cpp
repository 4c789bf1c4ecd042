// Host-side mirrors of the reference's per-call layout work for the attention stages: the live
// mask, the row order that makes groups contiguous and the per-row group bounds. The reference
// computes these in Java on every forward call before uploading them (ModelLayout.java:70-116,
// Chronos2Forward.java:147-194, 475-489; TimestralForward.java:614-629).
#include <cmath>
#include <cstdint>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "../../include/jitcast_hip.h"

namespace jc {
int host_fail(int code, const char* fmt, ...);
}

extern "C" {

int jc_c2_live(const float* window, int rows, int nc, int patch, int reg, int h, int32_t* live) {
    if (rows < 0 || nc < 0 || patch < 1 || (reg != 0 && reg != 1) || h < 1 || (rows > 0 && (!window || !live)))
        return jc::host_fail(JC_EINVAL, "jc_c2_live: bad arguments (rows=%d nc=%d patch=%d reg=%d h=%d)", rows, nc,
                             patch, reg, h);
    const int n = nc + reg + h;
    for (int i = 0; i < rows; i++) {
        const float* w = window + (size_t)i * nc * patch;
        for (int p = 0; p < nc; p++) {
            int any = 0;
            for (int s = p * patch; s < (p + 1) * patch; s++) any |= !std::isnan(w[s]);
            live[(size_t)i * n + p] = any;
        }
        for (int p = nc; p < n; p++) live[(size_t)i * n + p] = 1;
    }
    return JC_OK;
}

int jc_c2_group_order(const int32_t* group, int rows, int32_t* order, int* identity) {
    if (rows < 0 || (rows > 0 && (!group || !order)))
        return jc::host_fail(JC_EINVAL, "jc_c2_group_order: bad arguments (rows=%d)", rows);
    // groups in order of first appearance, rows in order within a group
    std::vector<int32_t> ids;
    std::unordered_map<int32_t, std::vector<int32_t>> members;
    for (int i = 0; i < rows; i++) {
        auto it = members.find(group[i]);
        if (it == members.end()) {
            ids.push_back(group[i]);
            members[group[i]] = {i};
        } else {
            it->second.push_back(i);
        }
    }
    int k = 0, same = 1;
    for (int32_t id : ids)
        for (int32_t r : members[id]) {
            same &= r == k;
            order[k++] = r;
        }
    if (identity) *identity = same;
    return JC_OK;
}

int jc_c2_group_bounds(const int32_t* group, int rows, int32_t* start, int32_t* end) {
    if (rows < 0 || (rows > 0 && (!group || !start || !end)))
        return jc::host_fail(JC_EINVAL, "jc_c2_group_bounds: bad arguments (rows=%d)", rows);
    std::unordered_set<int32_t> seen;
    for (int i = 0; i < rows;) {
        if (!seen.insert(group[i]).second)
            return jc::host_fail(JC_EINVAL, "jc_c2_group_bounds: rows of group %d are not contiguous", group[i]);
        int e = i;
        while (e < rows && group[e] == group[i]) e++;
        for (int k = i; k < e; k++) {
            start[k] = i;
            end[k] = e;
        }
        i = e;
    }
    return JC_OK;
}

}  // extern "C"
