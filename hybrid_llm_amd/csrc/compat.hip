// The reference C ABI's two fp32 operator hooks, with their exact signatures,
// so sample_standalone.py binds them unchanged (argtypes at
// sample_standalone.py:2499-2508):
//
//   llmy_moe_selected_fp32  one-token sparse MoE over the selected experts
//                           (llmy_cuda/include/llmy.h:80-88; caller
//                           sample_standalone.py:3001-3075)
//   llmy_mhc_sinkhorn4      out-of-place Sinkhorn over [matrices, 4, 4]
//                           (llmy_cuda/include/llmy.h:74-78; caller
//                           sample_standalone.py:2544-2587)
//
// Both return cudaErrorInvalidValue (1) for null pointers or non-positive
// sizes before any launch (llmy_cuda/src/llmy.cpp:216-217,230-233), else the
// launch status.
#include "common.hpp"
#include "abi_util.hpp"

namespace llmy {

// ---------------------------------------------------------------------------
// Selected-expert MoE, fp32 weights (one token).
//   activation[j, h]   = silu(gate_up[e_j, h] . x) * (gate_up[e_j, H + h] . x)
//   route_output[j, d] = prob[j] * (down[e_j, d] . activation[j])
//   out[d]             = sum_j route_output[j, d]   (j ascending)
// with e_j = idx[j].  A route whose id lies outside [0, E) contributes zeros
// (its activation and route_output rows are written as 0).  Both GEMVs stream
// fp32 weight rows: one wavefront per row, 16-byte loads when rows are
// 16-byte aligned, a DPP wave reduction, 4 wavefronts per workgroup.

__device__ __forceinline__ float row_dot(const float* __restrict__ w, const float* __restrict__ v,
                                         int n, bool vec4) {
  const int lane = threadIdx.x & (kWave - 1);
  float acc = 0.f;
  if (vec4) {
    const float4* w4 = reinterpret_cast<const float4*>(w);
    const float4* v4 = reinterpret_cast<const float4*>(v);
    for (int i = lane; i < n / 4; i += kWave) {
      const float4 a = w4[i], b = v4[i];
      acc += a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
    }
  } else {
    for (int i = lane; i < n; i += kWave) acc += w[i] * v[i];
  }
  return wave_sum(acc);
}

__global__ __launch_bounds__(256) void moe_sel_gate_up_kernel(
    const float* __restrict__ x, const int64_t* __restrict__ idx,
    const float* __restrict__ gate_up, float* __restrict__ activation, int D, int H, int E, int k,
    bool vec4) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);  // over k * H
  if (row >= k * H) return;
  const int j = row / H, h = row - j * H;
  const int64_t e = idx[j];
  float a = 0.f;
  if (e >= 0 && e < E) {
    const float* wg = gate_up + (static_cast<size_t>(e) * 2 * H + h) * D;
    const float g = row_dot(wg, x, D, vec4);
    const float u = row_dot(wg + static_cast<size_t>(H) * D, x, D, vec4);
    a = siluf_(g) * u;
  }
  if ((threadIdx.x & (kWave - 1)) == 0) activation[row] = a;
}

__global__ __launch_bounds__(256) void moe_sel_down_kernel(
    const int64_t* __restrict__ idx, const float* __restrict__ prob,
    const float* __restrict__ down, const float* __restrict__ activation,
    float* __restrict__ route_output, float* __restrict__ out, int D, int H, int E, int k,
    bool vec4) {
  const int d = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (d >= D) return;
  const bool lead = (threadIdx.x & (kWave - 1)) == 0;
  float sum = 0.f;
  for (int j = 0; j < k; ++j) {
    const int64_t e = idx[j];
    float r = 0.f;
    if (e >= 0 && e < E) {
      const float* wd = down + (static_cast<size_t>(e) * D + d) * H;
      r = prob[j] * row_dot(wd, activation + static_cast<size_t>(j) * H, H, vec4);
    }
    if (lead) route_output[static_cast<size_t>(j) * D + d] = r;
    sum += r;
  }
  if (lead) out[d] = sum;
}

// ---------------------------------------------------------------------------
// Sinkhorn over 4x4 matrices in the log domain, as the PyTorch path of
// sample_standalone.py:2582-2586: each iteration subtracts every row's
// logsumexp, then every column's; the result is exp of the final matrix
// (iterations == 0 gives exp(input)).  One thread per matrix, the 16 values
// in registers.

__device__ __forceinline__ float lse4(float a, float b, float c, float d) {
  const float m = fmaxf(fmaxf(a, b), fmaxf(c, d));
  if (m == -INFINITY) return -INFINITY;
  return m + logf(expf(a - m) + expf(b - m) + expf(c - m) + expf(d - m));
}

__global__ __launch_bounds__(256) void sinkhorn4_kernel(const float* __restrict__ in,
                                                        float* __restrict__ out, int matrices,
                                                        int iterations) {
  const int m = blockIdx.x * blockDim.x + threadIdx.x;
  if (m >= matrices) return;
  const float* src = in + static_cast<size_t>(m) * 16;
  float a[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) a[i] = src[i];
  for (int it = 0; it < iterations; ++it) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float l = lse4(a[4 * r], a[4 * r + 1], a[4 * r + 2], a[4 * r + 3]);
#pragma unroll
      for (int c = 0; c < 4; ++c) a[4 * r + c] -= l;
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float l = lse4(a[c], a[4 + c], a[8 + c], a[12 + c]);
#pragma unroll
      for (int r = 0; r < 4; ++r) a[4 * r + c] -= l;
    }
  }
  float* dst = out + static_cast<size_t>(m) * 16;
#pragma unroll
  for (int i = 0; i < 16; ++i) dst[i] = expf(a[i]);
}

}  // namespace llmy

using namespace llmy;

extern "C" int32_t llmy_moe_selected_fp32(const float* x, const int64_t* idx, const float* prob,
                                          const float* gate_up, const float* down,
                                          float* activation, float* route_output, float* out,
                                          int32_t D, int32_t H, int32_t E, int32_t k,
                                          void* stream) {
  LLMY_REQUIRE(x && idx && prob && gate_up && down && activation && route_output && out);
  LLMY_REQUIRE(D > 0 && H > 0 && E > 0 && k > 0);
  LLMY_REQUIRE(static_cast<int64_t>(k) * H < (1ll << 31) && static_cast<int64_t>(k) * D < (1ll << 31));
  const bool vec4 = D % 4 == 0 && H % 4 == 0 && aligned(x, 16) && aligned(gate_up, 16) &&
                    aligned(down, 16) && aligned(activation, 16);
  hipStream_t s = as_stream(stream);
  const int rows = k * H;
  hipLaunchKernelGGL(moe_sel_gate_up_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, x, idx,
                     gate_up, activation, D, H, E, k, vec4);
  hipLaunchKernelGGL(moe_sel_down_kernel, dim3((D + 3) / 4), dim3(256), 0, s, idx, prob, down,
                     activation, route_output, out, D, H, E, k, vec4);
  return launch_status();
}

extern "C" int32_t llmy_mhc_sinkhorn4(const float* input, float* output, int32_t matrices,
                                      int32_t iterations, void* stream) {
  LLMY_REQUIRE(input && output && matrices > 0 && iterations >= 0);
  hipLaunchKernelGGL(sinkhorn4_kernel, dim3((matrices + 255) / 256), dim3(256), 0,
                     as_stream(stream), input, output, matrices, iterations);
  return launch_status();
}
