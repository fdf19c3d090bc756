// Broadcast elementwise operands as collapsed strided views: the output's
// axes merged wherever every operand's strides allow, unit axes dropped, so
// a launch sees at most kMaxRank independent axes (and most see one).
#pragma once

#include "hip_common.h"

namespace chelis {

constexpr int kMaxRank = 4;

struct Shape {
    int32_t rank;
    int64_t ext[kMaxRank];
};

// Collapse adjacent output axes wherever every operand's strides allow it
// (stride[a] == stride[a+1] * ext[a+1]), dropping unit axes.
inline bool collapse(const chelis_gpu_tensor *out, const chelis_gpu_tensor *const *ins, int n_in, Shape *sh,
                     int64_t (*st)[kMaxRank]) {
    int64_t ext[16];
    int64_t s[CHELIS_FUSED_MAX_INPUTS][16];
    int r = 0;
    for (int a = 0; a < out->rank; ++a) {
        if (out->shape[a] == 1) continue;
        ext[r] = out->shape[a];
        // an extent-1 operand axis broadcasts: it never advances
        for (int k = 0; k < n_in; ++k) s[k][r] = ins[k]->shape[a] == 1 ? 0 : ins[k]->strides[a];
        ++r;
    }
    // merge from the innermost axis outward
    int64_t mext[16];
    int64_t ms[CHELIS_FUSED_MAX_INPUTS][16];
    int m = 0;
    for (int a = 0; a < r; ++a) {
        if (m > 0) {
            bool ok = true;
            for (int k = 0; k < n_in && ok; ++k) ok = ms[k][m - 1] == s[k][a] * ext[a];
            if (ok) {
                mext[m - 1] *= ext[a];
                for (int k = 0; k < n_in; ++k) ms[k][m - 1] = s[k][a];
                continue;
            }
        }
        mext[m] = ext[a];
        for (int k = 0; k < n_in; ++k) ms[k][m] = s[k][a];
        ++m;
    }
    if (m > kMaxRank) return false;
    sh->rank = m;
    for (int a = 0; a < m; ++a) sh->ext[a] = mext[a];
    for (int k = 0; k < n_in; ++k)
        for (int a = 0; a < kMaxRank; ++a) st[k][a] = a < m ? ms[k][a] : 0;
    return true;
}

}  // namespace chelis
