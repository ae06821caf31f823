// Grid shape and index width of the generated elementwise kernels
// (ew_jit.cpp).  Header-only so host tests can check the width rule.
#pragma once

#include <cstdint>

namespace mfx {

constexpr int kEwThreads = 256;              // threads per workgroup
constexpr int64_t kEwMaxBlocks = 1LL << 20;  // grid cap; larger jobs stride

// Workgroups launched for `work_items` chunks.
constexpr int64_t ew_blocks(int64_t work_items) {
  const int64_t b = (work_items + kEwThreads - 1) / kEwThreads;
  return b < 1 ? 1 : (b > kEwMaxBlocks ? kEwMaxBlocks : b);
}

// True when the grid-stride loop needs 64-bit indices.  The loop variable
// reaches at most (work_items - 1) + blocks * kEwThreads before its exit
// test, which must not pass INT32_MAX.
constexpr bool ew_needs_wide_index(int64_t work_items) {
  return (work_items - 1) + ew_blocks(work_items) * kEwThreads > INT32_MAX;
}

}  // namespace mfx
