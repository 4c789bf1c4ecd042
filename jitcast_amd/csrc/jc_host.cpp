// Host-side mirrors of the reference's per-call layout work for the attention stages: the live
// mask, the row order that makes groups contiguous and the per-row group bounds. The reference
// computes these in Java on every forward call before uploading them (ModelLayout.java:70-116,
// Chronos2Forward.java:147-194, 475-489; TimestralForward.java:614-629).
#include <algorithm>
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

// BlockLayout.of (J/timestral/BlockLayout.java:77-148) and position() (203-207): the per-block
// layout the Timestral attention kernels consume.
int jc_ts_block_layout(const uint8_t* observed, const uint8_t* future_observed, const int32_t* group,
                       const int32_t* role, int rows, int t, int patch, int h, int covariate_enabled,
                       int attend_missing, int block_size, int* enc_out, int* covariates_out, int32_t* key_valid,
                       int32_t* known, int32_t* pos) {
    const char* W = "jc_ts_block_layout";
    if (rows < 0 || t < 0 || patch < 1 || !enc_out || !covariates_out ||
        (rows > 0 && (!observed || !group || !key_valid || !known || !pos)))
        return jc::host_fail(JC_EINVAL, "%s: bad arguments (rows=%d t=%d patch=%d)", W, rows, t, patch);
    if (t % patch != 0)
        return jc::host_fail(JC_EINVAL, "%s: context length %d is not a multiple of the patch size %d", W, t, patch);
    if (h < 1) return jc::host_fail(JC_EINVAL, "%s: horizon patches must be >= 1, got %d", W, h);
    bool cov = false;
    if (role && covariate_enabled)
        for (int i = 0; i < rows; i++) cov |= role[i] != 0;
    if (cov && h > block_size)
        return jc::host_fail(JC_EINVAL, "%s: a block with covariates decodes at most %d patches, got %d", W,
                             block_size, h);
    const int ll = t / patch;
    const int enc = cov ? ll + h : ll;
    const int n = enc + h;
    // the window's observation mask: the context, plus (with covariates) the known-future steps
    auto obs = [&](int i, int s) -> bool {
        if (s < t) return observed[(size_t)i * t + s] != 0;
        return future_observed && future_observed[(size_t)i * h * patch + (s - t)] != 0;
    };
    std::vector<int> first_obs(rows, enc);
    for (int i = 0; i < rows; i++) {
        bool started = false;
        for (int p = 0; p < enc; p++) {
            bool any = false;
            for (int s = p * patch; s < (p + 1) * patch; s++) any |= obs(i, s);
            if (any && first_obs[i] == enc) first_obs[i] = p;
            started |= any;
            key_valid[(size_t)i * enc + p] = (attend_missing ? started : any) ? 1 : 0;
        }
    }
    // the first patch any row of the series observes (0 if none does)
    std::unordered_map<int32_t, int> group_first;
    for (int i = 0; i < rows; i++) {
        auto it = group_first.find(group[i]);
        if (it == group_first.end())
            group_first[group[i]] = first_obs[i];
        else
            it->second = std::min(it->second, first_obs[i]);
    }
    for (int i = 0; i < rows; i++) {
        int f = group_first[group[i]];
        f = f == enc ? 0 : f;
        known[i] = (cov && role[i] == 2) ? 1 : 0;
        for (int k = 0; k < n; k++) {
            const int p = k < enc ? k : ll + k - enc;
            pos[(size_t)i * n + k] = p - f + enc;  // the table row of jc_ts_rope_table
        }
    }
    *enc_out = enc;
    *covariates_out = cov ? 1 : 0;
    return JC_OK;
}

}  // extern "C"
