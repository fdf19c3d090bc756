// Launch-shape arithmetic shared by every launcher (host code only, so it
// is also compiled and checked on its own by the CPU tests).
#pragma once

#include <cstdint>

namespace chelis {

// HIP bounds one launch's work-items per grid dimension (blocks x threads)
// below 2^32. Launchers whose kernels cover their work with a grid-stride
// loop cap their grid; the others refuse a larger launch through
// grid_fits with a clear error instead of a failed launch.
constexpr int64_t kGridItems = int64_t(1) << 32;
inline bool grid_fits(int64_t blocks, int64_t threads) {
    return blocks >= 0 && threads > 0 && blocks <= (kGridItems - 1) / threads;
}
// ceil(work / per_block), at least 1, saturated at 2^32 - 1 (which never
// grid_fits a block of more than one thread)
inline unsigned grid_for(int64_t work, int per_block) {
    int64_t g = (work + per_block - 1) / per_block;
    if (g < 1) g = 1;
    return (unsigned)(g > 0xffffffffLL ? 0xffffffffLL : g);
}

}  // namespace chelis
