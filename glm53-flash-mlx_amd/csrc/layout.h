// Weight layout conversion (bank import / export).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace glm53 {

struct RelayoutArgs {
  const uint8_t* src;     // matrices of `rows` x `cols` E4M3 codes, layout from_log2
  uint8_t* dst;           // same shape, layout to_log2 (no overlap with src)
  int64_t rows, cols;     // rows * cols % 16 == 0; cols % 128 == 0 unless both layouts are row-major
  int64_t matrices;
  int64_t matrix_stride;  // bytes between consecutive matrices (in src and dst)
  int from_log2, to_log2; // row-group sizes (common.h; 0 = row-major)
};

hipError_t launch_relayout(const RelayoutArgs& a, hipStream_t st);

}  // namespace glm53
