// Re-lay of E4M3 expert matrices between the row-major checkpoint layout
// (packed.py:782-850 of the reference: expert-major [E, rows, cols]) and the
// row-group layout the kernels stream (common.h): a one-time copy at bank
// import, HBM-bound (every byte read once and written once).
#include "common.h"
#include "layout.h"

namespace glm53 {

typedef uint32_t relayout_u32x4 __attribute__((ext_vector_type(4)));

// One thread per 16-byte piece of the destination, in destination order, so
// the stores of a wavefront cover 1 KB contiguously; 16 consecutive columns
// of one 128-column block are contiguous in every layout, so the piece is
// one 16-byte load from the source (8 lanes read a row's 128-byte line of a
// K block when the source is row-major).
__global__ __launch_bounds__(256) void relayout_kernel(RelayoutArgs a) {
  const int64_t pieces_per_matrix = a.rows * a.cols / 16;
  const int64_t p = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (p >= pieces_per_matrix * a.matrices) return;
  const int64_t m = p / pieces_per_matrix;
  const int64_t o = (p - m * pieces_per_matrix) * 16;  // byte offset in the destination matrix
  // (row, column) of that byte under the destination layout
  const int gt = a.to_log2;
  const int64_t group_bytes = a.cols << gt;
  const int64_t grp = o / group_bytes;
  const int64_t rem = o - grp * group_bytes;
  const int64_t block_bytes = int64_t{128} << gt;
  const int64_t kb = rem / block_bytes;
  const int64_t in_block = rem - kb * block_bytes;
  const int64_t row = (grp << gt) + (in_block >> 7);
  const int64_t col = (kb << 7) + (in_block & 127);
  const int64_t src_off = group_row_base(row, a.cols, a.from_log2) + group_col(col, a.from_log2);
  const uint8_t* src = a.src + m * a.matrix_stride + src_off;
  uint8_t* dst = a.dst + m * a.matrix_stride + o;
  *reinterpret_cast<relayout_u32x4*>(dst) =
      __builtin_nontemporal_load(reinterpret_cast<const relayout_u32x4*>(src));
}

hipError_t launch_relayout(const RelayoutArgs& a, hipStream_t st) {
  const int64_t pieces = a.rows * a.cols / 16 * a.matrices;
  if (pieces == 0) return hipSuccess;
  const int64_t blocks = (pieces + 255) / 256;
  hipLaunchKernelGGL(relayout_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace glm53
