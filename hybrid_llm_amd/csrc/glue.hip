// Elementwise / row-wise glue of the block stack: RMSNorm, embedding gather,
// and the GDN causal depthwise conv gate.
#include "common.hpp"
#include "abi_util.hpp"

namespace llmy {

// out[m] = bf16(x[m] * rsqrt(mean(x[m]^2) + eps) * w)  (model/layers/norms.py:13-16,
// fp32 variance).  One wavefront per row, float4 loads.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ x,
                                                      const float* __restrict__ w,
                                                      uint16_t* __restrict__ out, int M, int D,
                                                      float eps) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= M) return;
  const float* xr = x + static_cast<long long>(row) * D;
  float ss = 0.f;
  for (int d = lane * 4; d < D; d += 256) {
    const float4 v = *reinterpret_cast<const float4*>(xr + d);
    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  }
  const float r = rsqrtf(wave_sum(ss) / static_cast<float>(D) + eps);
  uint16_t* orow = out + static_cast<long long>(row) * D;
  for (int d = lane * 4; d < D; d += 256) {
    const float4 v = *reinterpret_cast<const float4*>(xr + d);
    const float4 wv = *reinterpret_cast<const float4*>(w + d);
    *reinterpret_cast<uint2*>(orow + d) = make_uint2(pack_bf2(v.x * r * wv.x, v.y * r * wv.y),
                                                     pack_bf2(v.z * r * wv.z, v.w * r * wv.w));
  }
}

// x[b] = float(E[tok[b]])  (model/model.py:386 embed_tokens; tied LM head).
__global__ __launch_bounds__(256) void embed_kernel(const int32_t* __restrict__ tokens,
                                                    const uint16_t* __restrict__ table,
                                                    float* __restrict__ x, int B, int D, int V) {
  const int b = blockIdx.x;
  int tok = tokens[b];
  tok = tok < 0 ? 0 : (tok >= V ? V - 1 : tok);
  const uint16_t* src = table + static_cast<long long>(tok) * D;
  float* dst = x + static_cast<long long>(b) * D;
  for (int d = threadIdx.x; d < D; d += 256) dst[d] = bf2f(src[d]);
}

// Causal depthwise conv gate of the GDN block for one new token
// (model/layers/gated_deltanet.py:257-268 with conv_history): window =
// [hist[0..K-2], h]; conv[d] = sum_j w[d, j] * window[j][d]; out = sigmoid(conv);
// hist <- window[1..K-1].  Each thread owns one (b, d), so the in-place shift
// has no cross-thread hazard.
template <int KC>
__global__ __launch_bounds__(256) void gdn_conv_kernel(const uint16_t* __restrict__ h,
                                                       uint16_t* __restrict__ hist,
                                                       const float* __restrict__ w,
                                                       float* __restrict__ out, int B, int D) {
  const long long i = blockIdx.x * 256ll + threadIdx.x;
  if (i >= static_cast<long long>(B) * D) return;
  const int b = static_cast<int>(i / D);
  const int d = static_cast<int>(i % D);
  uint16_t win[KC];
  uint16_t* hb = hist + static_cast<long long>(b) * (KC - 1) * D + d;
#pragma unroll
  for (int j = 0; j < KC - 1; ++j) win[j] = hb[static_cast<long long>(j) * D];
  win[KC - 1] = h[i];
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < KC; ++j) acc = fmaf(w[d * KC + j], bf2f(win[j]), acc);
  out[i] = sigmoidf_(acc);
#pragma unroll
  for (int j = 0; j < KC - 1; ++j) hb[static_cast<long long>(j) * D] = win[j + 1];
}

}  // namespace llmy

using namespace llmy;

extern "C" int32_t llmy_rmsnorm_f32_bf16(const float* x, const float* w, llmy_bf16* out,
                                         int32_t M, int32_t D, float eps, void* stream) {
  LLMY_REQUIRE(M >= 0 && D > 0 && D % 4 == 0);
  if (M == 0) return 0;
  LLMY_REQUIRE(x && w && out);
  LLMY_REQUIRE(aligned(x, 16) && aligned(w, 16) && aligned(out, 8));
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((M + 3) / 4), dim3(256), 0, as_stream(stream), x, w,
                     out, M, D, eps);
  return launch_status();
}

extern "C" int32_t llmy_embed_bf16(const int32_t* tokens, const llmy_bf16* table, float* x,
                                   int32_t B, int32_t D, int32_t V, void* stream) {
  LLMY_REQUIRE(B >= 0 && D > 0 && V > 0);
  if (B == 0) return 0;
  LLMY_REQUIRE(tokens && table && x);
  hipLaunchKernelGGL(embed_kernel, dim3(B), dim3(256), 0, as_stream(stream), tokens, table, x, B,
                     D, V);
  return launch_status();
}

extern "C" int32_t llmy_gdn_conv_gate(const llmy_bf16* h, llmy_bf16* hist, const float* w,
                                      float* out, int32_t B, int32_t D, int32_t kernel,
                                      void* stream) {
  LLMY_REQUIRE(B >= 0 && D > 0 && kernel == 4);
  if (B == 0) return 0;
  LLMY_REQUIRE(h && hist && w && out);
  const long long n = static_cast<long long>(B) * D;
  hipLaunchKernelGGL(gdn_conv_kernel<4>, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256),
                     0, as_stream(stream), h, hist, w, out, B, D);
  return launch_status();
}
