// Multi-stream hyper-connections (mHC, model/layers/mhc.py:156-231) around the
// block's sublayers (model/model.py:119-126,177-264): the residual of a token is
// S streams X [S, D] fp32.  Per sublayer
//
//   maps:  f = RMSNorm(X.flatten()) (weight map_norm, eps = fp32 epsilon),
//          raw = theta f  [2S + S^2]   (a GEMM of the caller: llmy_linear_bf16),
//          pre = sigmoid(a0 raw[0:S] + pre_bias),
//          post = 2 sigmoid(a1 raw[S:2S] + post_bias),
//          R = Sinkhorn(a2 raw[2S:] + res_bias)  (log domain, rows then columns)
//   read:  h = RMSNorm_block(LayerNorm(sum_s pre_s X_s))        (the sublayer input)
//   write: X_i += sigmoid(gating) scale_i * (sum_j R_ij X_j + post_i U)
//
// where U is the sublayer's output.  The streams start as E[token] + seed_s
// (model.py:442-444).  One workgroup per token row; the S x S Sinkhorn runs on
// S * S lanes of wavefront 0 with row and column log-sum-exps as xor shuffles.
#include <algorithm>

#include "common.hpp"
#include "abi_util.hpp"

namespace llmy {

namespace {

// Block-wide sum over 256 threads (4 wavefronts), fixed order.
__device__ __forceinline__ float block_sum4(float v, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_sum(v);
  __syncthreads();  // red free from a previous use
  if (lane == 0) red[wave] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// log-sum-exp over a group of G lanes (G a power of two) whose lane ids
// differ only in the bits STRIDE .. STRIDE * G / 2 (xor offsets); torch's
// max-shifted form: max + log(sum exp(x - max)).
template <int G, int STRIDE>
__device__ __forceinline__ float group_lse(float x) {
  float mx = x;
#pragma unroll
  for (int o = STRIDE; o < STRIDE * G; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
  float s = expf(x - mx);
#pragma unroll
  for (int o = STRIDE; o < STRIDE * G; o <<= 1) s += __shfl_xor(s, o, kWave);
  return mx + logf(s);
}

}  // namespace

// streams[m, s, :] = E[tokens[m], :] + seed[s, :]
__global__ __launch_bounds__(256) void mhc_embed_kernel(const int32_t* __restrict__ tokens,
                                                        const uint16_t* __restrict__ table,
                                                        const float* __restrict__ seed,
                                                        float* __restrict__ streams, int S, int D,
                                                        int V) {
  const int m = blockIdx.x;
  int tok = tokens[m];
  tok = tok < 0 ? 0 : (tok >= V ? V - 1 : tok);
  const uint16_t* e = table + static_cast<long long>(tok) * D;
  float* x = streams + static_cast<long long>(m) * S * D;
  for (int i = threadIdx.x; i < S * D; i += 256) {
    const int d = i % D;
    x[i] = bf2f(e[d]) + seed[i];
  }
}

template <int S>
__global__ __launch_bounds__(256) void mhc_read_kernel(
    const float* __restrict__ X, const float* __restrict__ raw, long long raw_ld,
    const float* __restrict__ pre_bias, const float* __restrict__ post_bias,
    const float* __restrict__ res_bias, const float* __restrict__ alpha, int iterations,
    const float* __restrict__ ln_w, const float* __restrict__ ln_b, float ln_eps,
    const float* __restrict__ norm_w, float norm_eps, float* __restrict__ maps,
    uint16_t* __restrict__ h, int D) {
  constexpr int SS = S * S;
  __shared__ float pre_s[S];
  __shared__ float red[4];
  const int m = blockIdx.x;
  const int t = threadIdx.x;
  const float* r = raw + static_cast<long long>(m) * raw_ld;
  if (t < 64) {
    // lanes l < S*S: R[l / S][l % S]; lanes l < S also make pre_l and post_l
    const int l = t;
    float x = l < SS ? alpha[2] * r[2 * S + l] + res_bias[l] : 0.f;
    for (int it = 0; it < iterations; ++it) {
      x -= group_lse<S, 1>(x);  // rows: lanes i S + j, j = 0 .. S-1
      x -= group_lse<S, S>(x);  // columns: lanes i S + j, i = 0 .. S-1
    }
    float* mp = maps + static_cast<long long>(m) * (S + SS);
    if (l < SS) mp[S + l] = expf(x);
    if (l < S) {
      pre_s[l] = sigmoidf_(alpha[0] * r[l] + pre_bias[l]);
      mp[l] = 2.f * sigmoidf_(alpha[1] * r[S + l] + post_bias[l]);
    }
  }
  __syncthreads();
  float pre[S];
#pragma unroll
  for (int s = 0; s < S; ++s) pre[s] = pre_s[s];
  const float* xr = X + static_cast<long long>(m) * S * D;
  // read: v = sum_s pre_s X_s (this thread's float4 groups of d)
  constexpr int MAXG = 4;  // D <= 4096
  float4 v[MAXG];
  float sum = 0.f;
#pragma unroll
  for (int gI = 0; gI < MAXG; ++gI) {
    const int d = 4 * (t + 256 * gI);
    v[gI] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (d < D) {
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const float4 xs = *reinterpret_cast<const float4*>(xr + static_cast<long long>(s) * D + d);
        v[gI].x = fmaf(pre[s], xs.x, v[gI].x);
        v[gI].y = fmaf(pre[s], xs.y, v[gI].y);
        v[gI].z = fmaf(pre[s], xs.z, v[gI].z);
        v[gI].w = fmaf(pre[s], xs.w, v[gI].w);
      }
      sum += (v[gI].x + v[gI].y) + (v[gI].z + v[gI].w);
    }
  }
  // LayerNorm (biased variance, two passes)
  const float mean = block_sum4(sum, red) / static_cast<float>(D);
  float sq = 0.f;
#pragma unroll
  for (int gI = 0; gI < MAXG; ++gI) {
    const int d = 4 * (t + 256 * gI);
    if (d < D) {
      const float a0 = v[gI].x - mean, a1 = v[gI].y - mean, a2 = v[gI].z - mean,
                  a3 = v[gI].w - mean;
      sq += (a0 * a0 + a1 * a1) + (a2 * a2 + a3 * a3);
    }
  }
  const float rstd = rsqrtf(block_sum4(sq, red) / static_cast<float>(D) + ln_eps);
  float ss = 0.f;
#pragma unroll
  for (int gI = 0; gI < MAXG; ++gI) {
    const int d = 4 * (t + 256 * gI);
    if (d < D) {
      const float4 w = *reinterpret_cast<const float4*>(ln_w + d);
      const float4 b = *reinterpret_cast<const float4*>(ln_b + d);
      v[gI].x = (v[gI].x - mean) * rstd * w.x + b.x;
      v[gI].y = (v[gI].y - mean) * rstd * w.y + b.y;
      v[gI].z = (v[gI].z - mean) * rstd * w.z + b.z;
      v[gI].w = (v[gI].w - mean) * rstd * w.w + b.w;
      ss += (v[gI].x * v[gI].x + v[gI].y * v[gI].y) + (v[gI].z * v[gI].z + v[gI].w * v[gI].w);
    }
  }
  // the sublayer's RMSNorm, bf16 out
  const float rn = rsqrtf(block_sum4(ss, red) / static_cast<float>(D) + norm_eps);
  uint16_t* hr = h + static_cast<long long>(m) * D;
#pragma unroll
  for (int gI = 0; gI < MAXG; ++gI) {
    const int d = 4 * (t + 256 * gI);
    if (d < D) {
      const float4 w = *reinterpret_cast<const float4*>(norm_w + d);
      *reinterpret_cast<uint2*>(hr + d) =
          make_uint2(pack_bf2(v[gI].x * rn * w.x, v[gI].y * rn * w.y),
                     pack_bf2(v[gI].z * rn * w.z, v[gI].w * rn * w.w));
    }
  }
}

template <int S>
__global__ __launch_bounds__(256) void mhc_write_kernel(float* __restrict__ X,
                                                        const float* __restrict__ U,
                                                        long long u_ld,
                                                        const float* __restrict__ maps,
                                                        const float* __restrict__ scale,
                                                        const float* __restrict__ gating_logit,
                                                        int D) {
  constexpr int SS = S * S;
  const int m = blockIdx.x;
  const float* mp = maps + static_cast<long long>(m) * (S + SS);
  float post[S], R[SS];
#pragma unroll
  for (int i = 0; i < S; ++i) post[i] = mp[i];
#pragma unroll
  for (int i = 0; i < SS; ++i) R[i] = mp[S + i];
  const float g = sigmoidf_(gating_logit[0]);
  float* xr = X + static_cast<long long>(m) * S * D;
  const float* ur = U + static_cast<long long>(m) * u_ld;
  for (int d = 4 * threadIdx.x; d < D; d += 1024) {
    float4 xs[S];
#pragma unroll
    for (int s = 0; s < S; ++s)
      xs[s] = *reinterpret_cast<const float4*>(xr + static_cast<long long>(s) * D + d);
    const float4 u = *reinterpret_cast<const float4*>(ur + d);
#pragma unroll
    for (int i = 0; i < S; ++i) {
      float4 acc = make_float4(post[i] * u.x, post[i] * u.y, post[i] * u.z, post[i] * u.w);
      float4 mix = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int j = 0; j < S; ++j) {
        mix.x = fmaf(R[i * S + j], xs[j].x, mix.x);
        mix.y = fmaf(R[i * S + j], xs[j].y, mix.y);
        mix.z = fmaf(R[i * S + j], xs[j].z, mix.z);
        mix.w = fmaf(R[i * S + j], xs[j].w, mix.w);
      }
      acc.x += mix.x;
      acc.y += mix.y;
      acc.z += mix.z;
      acc.w += mix.w;
      const float4 sc = *reinterpret_cast<const float4*>(scale + static_cast<long long>(i) * D + d);
      float4 o;
      o.x = xs[i].x + g * (acc.x * sc.x);
      o.y = xs[i].y + g * (acc.y * sc.y);
      o.z = xs[i].z + g * (acc.z * sc.z);
      o.w = xs[i].w + g * (acc.w * sc.w);
      *reinterpret_cast<float4*>(xr + static_cast<long long>(i) * D + d) = o;
    }
  }
}

__global__ __launch_bounds__(256) void f32_to_bf16_kernel(const float* __restrict__ x,
                                                          uint16_t* __restrict__ out,
                                                          long long n4) {
  for (long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x; i < n4;
       i += static_cast<long long>(gridDim.x) * 256) {
    const float4 v = reinterpret_cast<const float4*>(x)[i];
    reinterpret_cast<uint2*>(out)[i] = make_uint2(pack_bf2(v.x, v.y), pack_bf2(v.z, v.w));
  }
}

// out[r, k] = k < K ? x[r * K + k] : 0 for k < Kp: a GEMM operand whose input
// width is zero-padded to the kernels' multiple of 256, one 32-bit word
// (two bf16) per thread (K, Kp even).
__global__ __launch_bounds__(256) void pad_cols_kernel(const uint32_t* __restrict__ x,
                                                       uint32_t* __restrict__ out, long long rows,
                                                       int K2, int Kp2) {
  const long long n = rows * Kp2;
  for (long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += static_cast<long long>(gridDim.x) * 256) {
    const long long r = i / Kp2;
    const int c = static_cast<int>(i - r * Kp2);
    out[i] = c < K2 ? x[r * K2 + c] : 0u;
  }
}

}  // namespace llmy

using namespace llmy;

extern "C" int32_t llmy_mhc_embed(const int32_t* tokens, const llmy_bf16* table,
                                  const float* seed, float* streams, int32_t M, int32_t S,
                                  int32_t D, int32_t V, void* stream) {
  LLMY_REQUIRE(M >= 0 && S >= 1 && D > 0 && V > 0);
  if (M == 0) return 0;
  LLMY_REQUIRE(tokens && table && seed && streams);
  hipLaunchKernelGGL(mhc_embed_kernel, dim3(M), dim3(256), 0, as_stream(stream), tokens, table,
                     seed, streams, S, D, V);
  return launch_status();
}

extern "C" int32_t llmy_mhc_read(const float* streams, const float* raw, int64_t raw_ld,
                                 const float* pre_bias, const float* post_bias,
                                 const float* res_bias, const float* alpha, int32_t iterations,
                                 const float* ln_w, const float* ln_b, float ln_eps,
                                 const float* norm_w, float norm_eps, float* maps, llmy_bf16* h,
                                 int32_t M, int32_t S, int32_t D, void* stream) {
  LLMY_REQUIRE(M >= 0 && (S == 2 || S == 4) && D > 0 && D % 4 == 0 && D <= 4096);
  LLMY_REQUIRE(iterations >= 0 && raw_ld >= 2 * S + S * S);
  if (M == 0) return 0;
  LLMY_REQUIRE(streams && raw && pre_bias && post_bias && res_bias && alpha && ln_w && ln_b &&
               norm_w && maps && h);
  LLMY_REQUIRE(aligned(streams, 16) && aligned(ln_w, 16) && aligned(ln_b, 16) &&
               aligned(norm_w, 16) && aligned(h, 8));
  const hipStream_t s = as_stream(stream);
  if (S == 4)
    hipLaunchKernelGGL(mhc_read_kernel<4>, dim3(M), dim3(256), 0, s, streams, raw, raw_ld,
                       pre_bias, post_bias, res_bias, alpha, iterations, ln_w, ln_b, ln_eps,
                       norm_w, norm_eps, maps, h, D);
  else
    hipLaunchKernelGGL(mhc_read_kernel<2>, dim3(M), dim3(256), 0, s, streams, raw, raw_ld,
                       pre_bias, post_bias, res_bias, alpha, iterations, ln_w, ln_b, ln_eps,
                       norm_w, norm_eps, maps, h, D);
  return launch_status();
}

extern "C" int32_t llmy_mhc_write(float* streams, const float* update, int64_t update_ld,
                                  const float* maps, const float* scale,
                                  const float* gating_logit, int32_t M, int32_t S, int32_t D,
                                  void* stream) {
  LLMY_REQUIRE(M >= 0 && (S == 2 || S == 4) && D > 0 && D % 4 == 0 && update_ld >= D);
  if (M == 0) return 0;
  LLMY_REQUIRE(streams && update && maps && scale && gating_logit);
  LLMY_REQUIRE(aligned(streams, 16) && aligned(update, 16) && aligned(scale, 16) &&
               update_ld % 4 == 0);
  const hipStream_t s = as_stream(stream);
  if (S == 4)
    hipLaunchKernelGGL(mhc_write_kernel<4>, dim3(M), dim3(256), 0, s, streams, update, update_ld,
                       maps, scale, gating_logit, D);
  else
    hipLaunchKernelGGL(mhc_write_kernel<2>, dim3(M), dim3(256), 0, s, streams, update, update_ld,
                       maps, scale, gating_logit, D);
  return launch_status();
}

extern "C" int32_t llmy_f32_to_bf16(const float* x, llmy_bf16* out, int64_t n, void* stream) {
  LLMY_REQUIRE(n >= 0 && n % 4 == 0);
  if (n == 0) return 0;
  LLMY_REQUIRE(x && out && aligned(x, 16) && aligned(out, 8));
  const long long n4 = n / 4;
  const unsigned blocks = static_cast<unsigned>(std::min<long long>((n4 + 255) / 256, 8192));
  hipLaunchKernelGGL(f32_to_bf16_kernel, dim3(blocks), dim3(256), 0, as_stream(stream), x, out,
                     n4);
  return launch_status();
}

extern "C" int32_t llmy_pad_cols_bf16(const llmy_bf16* x, llmy_bf16* out, int32_t rows,
                                      int32_t K, int32_t Kp, void* stream) {
  LLMY_REQUIRE(rows >= 0 && K > 0 && K <= Kp && K % 2 == 0 && Kp % 2 == 0);
  if (rows == 0) return 0;
  LLMY_REQUIRE(x && out && aligned(x, 4) && aligned(out, 4));
  const long long n = static_cast<long long>(rows) * (Kp / 2);
  const unsigned blocks = static_cast<unsigned>(std::min<long long>((n + 255) / 256, 8192));
  hipLaunchKernelGGL(pad_cols_kernel, dim3(blocks), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const uint32_t*>(x), reinterpret_cast<uint32_t*>(out),
                     static_cast<long long>(rows), K / 2, Kp / 2);
  return launch_status();
}
