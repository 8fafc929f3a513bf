// Synthetic weight generation (benchmarks and device-side test inputs).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace glm53 {

struct SynthFp8Args {
  uint8_t* codes;   // [rows, cols] E4M3 per matrix
  float* scale;     // [ceil(rows/128), ceil(cols/128)] per matrix
  int64_t rows, cols;
  uint64_t seed;    // matrix b uses stream_key(seed, b)
  float std;
  int64_t batch;            // matrices
  int64_t codes_stride;     // bytes between matrices
  int64_t scale_stride;     // floats between matrices
  int group_log2;           // code layout: row groups of 2^group_log2 rows (common.h; 0 = row-major)
};

hipError_t launch_synth_fp8(const SynthFp8Args& a, hipStream_t st);
hipError_t launch_synth_f32(float* out, int64_t n, uint64_t seed, float std, float lo, float hi, int uniform,
                            hipStream_t st);
hipError_t launch_synth_bf16(uint16_t* out, int64_t n, uint64_t seed, float std, hipStream_t st);
hipError_t launch_probe_read(const uint8_t* buf, int64_t bytes, uint32_t* sink, int blocks, hipStream_t st);
hipError_t launch_synth_step_input(uint16_t* out, int64_t n, uint64_t seed, float std, uint32_t* counter,
                                   hipStream_t st);

}  // namespace glm53
