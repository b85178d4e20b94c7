// Launch geometry shared by the attention kernels and their host launchers.
//
// A launch covers `total` logical work items (item x head).  The grid is
// rounded up to a multiple of the 8 XCDs, and workgroup `bid` runs logical
// item xcd_logical(bid, grid): the dispatcher hands workgroups to the XCDs
// round-robin (bid % 8), so consecutive logical items -- items of one head
// whose key windows overlap -- land on the same XCD and share its L2.  The
// map is a bijection on [0, grid); a workgroup whose logical item is
// >= total returns before touching memory.
//
// Plain C++ (no HIP types) so that the host test suite compiles this header
// with g++ and checks the arithmetic without a GPU.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define HIER_HD __host__ __device__
#else
#define HIER_HD
#endif

namespace hier {

constexpr int kXcds = 8;

// Workgroups launched for `total` logical items (0 for none).
HIER_HD inline constexpr int64_t xcd_grid(int64_t total) {
  return total <= 0 ? 0 : (total + kXcds - 1) / kXcds * kXcds;
}

// Largest `total` a launch accepts: the grid and every logical index must fit
// a positive int.
constexpr int64_t kMaxLaunchItems = (1ll << 31) - 2 * kXcds;

// Logical item of workgroup `bid` in a grid of `grid` workgroups
// (grid % kXcds == 0).
HIER_HD inline constexpr int xcd_logical(int bid, int grid) {
  return (bid % kXcds) * (grid / kXcds) + bid / kXcds;
}

}  // namespace hier
