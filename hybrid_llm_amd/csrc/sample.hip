// Token sampling over fp32 logits [rows, V].
//
// Greedy: first index of the maximum per row, i.e. torch.argmax semantics as
// used by sample_standalone.py:5609-5610 (NaN counts as the maximum, the
// lowest index wins among equal values).
#include "common.hpp"
#include "abi_util.hpp"

namespace llmy {

// One 1024-thread workgroup per row; each thread keeps the best packed
// (value, index) key of its strided slice (loads unrolled 8 deep so the row
// streams with many loads in flight), then waves and the block reduce.
__global__ __launch_bounds__(1024) void argmax_rows_kernel(const float* __restrict__ logits,
                                                           int V, int32_t* __restrict__ out) {
  __shared__ uint64_t part[16];
  const float* row = logits + static_cast<size_t>(blockIdx.x) * V;
  uint64_t best = 0ull;
  for (int base = 0; base < V; base += 8 * 1024) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = base + u * 1024 + threadIdx.x;
      v[u] = i < V ? row[i] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = base + u * 1024 + threadIdx.x;
      if (i < V) {
        const uint64_t key = value_index_key(v[u], static_cast<uint32_t>(i));
        best = key > best ? key : best;
      }
    }
  }
  best = wave_max_u64(best);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = part[0];
    for (int w = 1; w < 16; ++w) b = part[w] > b ? part[w] : b;
    out[blockIdx.x] = static_cast<int32_t>(key_index(b));
  }
}

}  // namespace llmy

using namespace llmy;

extern "C" int32_t llmy_sample_argmax_f32(const float* logits, int32_t rows, int32_t V,
                                          int32_t* out, void* stream) {
  LLMY_REQUIRE(rows >= 0 && V > 0);
  if (rows == 0) return 0;
  LLMY_REQUIRE(logits && out);
  hipLaunchKernelGGL(argmax_rows_kernel, dim3(rows), dim3(1024), 0, as_stream(stream), logits, V,
                     out);
  return launch_status();
}
