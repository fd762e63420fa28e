// Context-aware MoE router, local-context branch (model/layers/context_router.py:
// 59-76 for a sequence, :94-137 for one decode token; model/layers/mla_memory.py:
// 23-48 for the latent channel and its causal box mean):
//
//   local_t = RMSNorm(h_t; router.norm)                       (fp32)
//   lat_t   = LayerNorm(W_down . local_t; ln_w, ln_b, 1e-5)     (latent_dim L)
//   ctx_t   = mean(lat_s : max(0, t-W+1) <= s <= t)            (W = local_context)
//   c_t     = W_co . (W_lco . ctx_t)                           (local_context_out, context_out)
//   route_t = local_t + sigmoid(g) * c_t;  logits_t = W_r . route_t
//
// then the usual top-k + softmax over the logits.  The window mean is the same
// rule for a prompt (the box filter of MLALatentMemory.forward) and for a
// decode token (the mean over the rolling history plus the current latent in
// forward_step): each sequence keeps a ring of its last W latents, slot
// pos % W, and a token's mean covers the min(pos + 1, W) latents up to it.
//
// Three launches here; the two wide projections go through the bf16 linear
// entry (the window kernel writes ctx_t in bf16 for it) and the top-k through
// the logits entry of router.hip:
//   ctx_latent_kernel   h (bf16) -> local (fp32), lat (fp32)
//   ctx_window_kernel   lat, ring, pos -> ctx (bf16); ring updated
//   ctx_logits_kernel   local, c, g, W_r -> logits (fp32)
#include <cmath>

#include "abi_util.hpp"
#include "common.hpp"

namespace llmy {

namespace {

constexpr int kCtxTokens = 8;     // tokens per workgroup of the latent kernel
constexpr int kCtxMaxLatent = 512;

// One workgroup of 4 wavefronts per kCtxTokens tokens.  Wave w normalises
// tokens w and w+4 (lanes split D), then computes latent outputs w, w+4, ...
// for all the workgroup's tokens (one W_down row load per output, one wave
// reduction per token), then LayerNorms tokens w and w+4.
template <int NCH>
__global__ __launch_bounds__(256) void ctx_latent_kernel(
    const uint16_t* __restrict__ h, const float* __restrict__ norm_w,
    const float* __restrict__ w_down, const float* __restrict__ ln_w,
    const float* __restrict__ ln_b, float* __restrict__ local, float* __restrict__ lat, int rows,
    int L, float eps, float ln_eps) {
  constexpr int D = 256 * NCH;
  __shared__ float s_local[kCtxTokens][D];
  __shared__ float s_lat[kCtxTokens][kCtxMaxLatent];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const long long r0 = static_cast<long long>(blockIdx.x) * kCtxTokens;
  const int nt = static_cast<int>(min(static_cast<long long>(kCtxTokens), rows - r0));

  for (int j = wave; j < nt; j += 4) {
    const long long r = r0 + j;
    float v[NCH][4];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const uint2 p = *reinterpret_cast<const uint2*>(h + r * D + 4 * lane + 256 * c);
      v[c][0] = __uint_as_float(p.x << 16);
      v[c][1] = __uint_as_float(p.x & 0xffff0000u);
      v[c][2] = __uint_as_float(p.y << 16);
      v[c][3] = __uint_as_float(p.y & 0xffff0000u);
#pragma unroll
      for (int q = 0; q < 4; ++q) ss += v[c][q] * v[c][q];
    }
    const float rr = rsqrtf(wave_sum(ss) / static_cast<float>(D) + eps);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int d = 4 * lane + 256 * c;
      const float4 w = *reinterpret_cast<const float4*>(norm_w + d);
      const float4 o = make_float4(v[c][0] * rr * w.x, v[c][1] * rr * w.y, v[c][2] * rr * w.z,
                                   v[c][3] * rr * w.w);
      *reinterpret_cast<float4*>(&s_local[j][d]) = o;
      *reinterpret_cast<float4*>(local + r * D + d) = o;
    }
  }
  __syncthreads();

  for (int l = wave; l < L; l += 4) {
    float4 wv[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      wv[c] = *reinterpret_cast<const float4*>(w_down + static_cast<long long>(l) * D +
                                               4 * lane + 256 * c);
    for (int j = 0; j < nt; ++j) {
      float acc = 0.f;
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const float4 x = *reinterpret_cast<const float4*>(&s_local[j][4 * lane + 256 * c]);
        acc += wv[c].x * x.x + wv[c].y * x.y + wv[c].z * x.z + wv[c].w * x.w;
      }
      const float s = wave_sum(acc);
      if (lane == 0) s_lat[j][l] = s;
    }
  }
  __syncthreads();

  const int per = L / kWave;  // latent values per lane (L % 64 == 0)
  for (int j = wave; j < nt; j += 4) {
    float sum = 0.f;
    for (int q = 0; q < per; ++q) sum += s_lat[j][lane + kWave * q];
    const float mean = wave_sum(sum) / static_cast<float>(L);
    float var = 0.f;
    for (int q = 0; q < per; ++q) {
      const float d = s_lat[j][lane + kWave * q] - mean;
      var += d * d;
    }
    const float rs = rsqrtf(wave_sum(var) / static_cast<float>(L) + ln_eps);
    float* out = lat + (r0 + j) * L;
    for (int q = 0; q < per; ++q) {
      const int i = lane + kWave * q;
      out[i] = (s_lat[j][i] - mean) * rs * ln_w[i] + ln_b[i];
    }
  }
}

// One thread per (sequence, latent channel): the window sum runs in fp64, so
// the mean of every token equals the mean of its window up to fp32 rounding
// however long the prompt.  Tokens of sequence b sit at absolute positions
// pos[b] + t; the ring holds the last W latents of each sequence (slot p % W).
__global__ __launch_bounds__(64) void ctx_window_kernel(
    const float* __restrict__ lat, float* __restrict__ ring, const int32_t* __restrict__ pos,
    uint16_t* __restrict__ ctx, int T, int W, int L) {
  const int b = blockIdx.y;
  const int l = blockIdx.x * kWave + threadIdx.x;
  if (l >= L) return;
  const long long p0 = pos ? max(pos[b], 0) : 0;
  float* rg = ring + static_cast<long long>(b) * W * L + l;
  double s = 0.0;
  const int n0 = static_cast<int>(min(p0, static_cast<long long>(W)));
  for (int i = 0; i < n0; ++i) s += rg[static_cast<long long>(i) * L];
  for (int t = 0; t < T; ++t) {
    const long long a = p0 + t;
    const long long slot = a % W;
    const long long row = static_cast<long long>(b) * T + t;
    const float v = lat[row * L + l];
    if (a >= W) s -= rg[slot * L];
    rg[slot * L] = v;
    s += v;
    const double n = static_cast<double>(min(a + 1, static_cast<long long>(W)));
    ctx[row * L + l] = f2bf(static_cast<float>(s / n));
  }
}

// One workgroup per token: route = local + sigmoid(g) * c in registers, then
// wave w computes the logits of experts w, w+4, ... (lanes split D).
template <int NCH>
__global__ __launch_bounds__(256) void ctx_logits_kernel(
    const float* __restrict__ local, const float* __restrict__ c, const float* __restrict__ g,
    const float* __restrict__ w_router, float* __restrict__ logits, int E) {
  constexpr int D = 256 * NCH;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const long long t = blockIdx.x;
  const float sg = 1.f / (1.f + expf(-g[0]));
  float4 r[NCH];
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch) {
    const int d = 4 * lane + 256 * ch;
    const float4 a = *reinterpret_cast<const float4*>(local + t * D + d);
    const float4 b = *reinterpret_cast<const float4*>(c + t * D + d);
    r[ch] = make_float4(fmaf(sg, b.x, a.x), fmaf(sg, b.y, a.y), fmaf(sg, b.z, a.z),
                        fmaf(sg, b.w, a.w));
  }
  for (int e = wave; e < E; e += 4) {
    float acc = 0.f;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
      const float4 w = *reinterpret_cast<const float4*>(w_router + static_cast<long long>(e) * D +
                                                        4 * lane + 256 * ch);
      acc += w.x * r[ch].x + w.y * r[ch].y + w.z * r[ch].z + w.w * r[ch].w;
    }
    const float s = wave_sum(acc);
    if (lane == 0) logits[t * E + e] = s;
  }
}

}  // namespace

}  // namespace llmy

using namespace llmy;

extern "C" int32_t llmy_router_context_latent_f32(const llmy_bf16* h, const float* norm_w,
                                                  const float* w_down, const float* ln_w,
                                                  const float* ln_b, float* local, float* lat,
                                                  int32_t rows, int32_t D, int32_t L, float eps,
                                                  float ln_eps, void* stream) {
  LLMY_REQUIRE(rows >= 0 && (D == 256 || D == 512 || D == 768 || D == 1024));
  LLMY_REQUIRE(L > 0 && L % kWave == 0 && L <= kCtxMaxLatent);
  if (rows == 0) return 0;
  LLMY_REQUIRE(h && norm_w && w_down && ln_w && ln_b && local && lat);
  LLMY_REQUIRE(aligned(h, 8) && aligned(norm_w, 16) && aligned(w_down, 16) && aligned(local, 16));
  const dim3 grid((rows + kCtxTokens - 1) / kCtxTokens);
  const hipStream_t s = as_stream(stream);
  const uint16_t* hh = reinterpret_cast<const uint16_t*>(h);
  switch (D / 256) {
    case 1: hipLaunchKernelGGL(ctx_latent_kernel<1>, grid, dim3(256), 0, s, hh, norm_w, w_down, ln_w, ln_b, local, lat, rows, L, eps, ln_eps); break;
    case 2: hipLaunchKernelGGL(ctx_latent_kernel<2>, grid, dim3(256), 0, s, hh, norm_w, w_down, ln_w, ln_b, local, lat, rows, L, eps, ln_eps); break;
    case 3: hipLaunchKernelGGL(ctx_latent_kernel<3>, grid, dim3(256), 0, s, hh, norm_w, w_down, ln_w, ln_b, local, lat, rows, L, eps, ln_eps); break;
    default: hipLaunchKernelGGL(ctx_latent_kernel<4>, grid, dim3(256), 0, s, hh, norm_w, w_down, ln_w, ln_b, local, lat, rows, L, eps, ln_eps); break;
  }
  return launch_status();
}

extern "C" int32_t llmy_router_context_window(const float* lat, float* ring, const int32_t* pos,
                                              llmy_bf16* ctx, int32_t B, int32_t T, int32_t W,
                                              int32_t L, void* stream) {
  LLMY_REQUIRE(B >= 0 && T >= 0 && W > 0 && L > 0 && B <= 65535);
  if (B == 0 || T == 0) return 0;
  LLMY_REQUIRE(lat && ring && ctx);
  hipLaunchKernelGGL(ctx_window_kernel, dim3((L + kWave - 1) / kWave, B), dim3(kWave), 0,
                     as_stream(stream), lat, ring, pos, reinterpret_cast<uint16_t*>(ctx), T, W, L);
  return launch_status();
}

extern "C" int32_t llmy_router_context_logits_f32(const float* local, const float* c,
                                                  const float* route_gate, const float* w_router,
                                                  float* logits, int32_t rows, int32_t D,
                                                  int32_t E, void* stream) {
  LLMY_REQUIRE(rows >= 0 && (D == 256 || D == 512 || D == 768 || D == 1024) && E > 0 && E <= 1024);
  if (rows == 0) return 0;
  LLMY_REQUIRE(local && c && route_gate && w_router && logits);
  LLMY_REQUIRE(aligned(local, 16) && aligned(c, 16) && aligned(w_router, 16));
  const hipStream_t s = as_stream(stream);
  switch (D / 256) {
    case 1: hipLaunchKernelGGL(ctx_logits_kernel<1>, dim3(rows), dim3(256), 0, s, local, c, route_gate, w_router, logits, E); break;
    case 2: hipLaunchKernelGGL(ctx_logits_kernel<2>, dim3(rows), dim3(256), 0, s, local, c, route_gate, w_router, logits, E); break;
    case 3: hipLaunchKernelGGL(ctx_logits_kernel<3>, dim3(rows), dim3(256), 0, s, local, c, route_gate, w_router, logits, E); break;
    default: hipLaunchKernelGGL(ctx_logits_kernel<4>, dim3(rows), dim3(256), 0, s, local, c, route_gate, w_router, logits, E); break;
  }
  return launch_status();
}

// ---------------------------------------------------------------- global branch
// The context-aware router's global branch (context_router.py:66-68,126-127;
// mla_memory.py:52-90; the native twin router_hca_latent_attention,
// llmy_cuda/src/model.cpp:972-1062): multi-head attention of the router's
// query over latents of the HCA block's compressed summaries, whose keys and
// values the caller projects once per summary.

namespace llmy {

// out[r] = bf16(LayerNorm(x[r]) * w + b), biased variance (nn.LayerNorm).
__global__ __launch_bounds__(256) void layernorm_kernel(const float* __restrict__ x,
                                                        const float* __restrict__ w,
                                                        const float* __restrict__ bias,
                                                        uint16_t* __restrict__ out, int L,
                                                        float eps) {
  __shared__ float red[4];
  const int r = blockIdx.x;
  const float* xr = x + static_cast<int64_t>(r) * L;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  auto block_sum = [&](float v) {
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
  };
  float s = 0.f;
  for (int i = threadIdx.x; i < L; i += 256) s += xr[i];
  const float mean = block_sum(s) / static_cast<float>(L);
  float q = 0.f;
  for (int i = threadIdx.x; i < L; i += 256) {
    const float d = xr[i] - mean;
    q += d * d;
  }
  const float inv = 1.0f / sqrtf(block_sum(q) / static_cast<float>(L) + eps);
  for (int i = threadIdx.x; i < L; i += 256)
    out[static_cast<int64_t>(r) * L + i] = f2bf((xr[i] - mean) * inv * w[i] + bias[i]);
}

// Workgroup = (query row, head).  Query row r = b * T + t sits at position
// pos[b] (pos NULL: t); slot j of row b is visible when 1 <= tag <= that + 1.
__global__ __launch_bounds__(256) void latent_attn_kernel(
    const uint16_t* __restrict__ q, int64_t q_ld, const uint16_t* __restrict__ keys,
    const uint16_t* __restrict__ vals, const int32_t* __restrict__ tag,
    const int32_t* __restrict__ pos, uint16_t* __restrict__ out, int64_t out_ld, int T, int C,
    int heads, int hd, float scale_log2) {
  extern __shared__ float sc[];
  __shared__ float red[4];
  const int h = blockIdx.x % heads;
  const int r = blockIdx.x / heads;
  const int b = r / T;
  const int qp = pos ? pos[b] : r - b * T;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int W = heads * hd;
  const uint16_t* qh = q + static_cast<int64_t>(r) * q_ld + h * hd;
  for (int j = threadIdx.x; j < C; j += 256) {
    const int tg = tag[static_cast<int64_t>(b) * C + j];
    float s = -INFINITY;
    if (tg >= 1 && tg <= qp + 1) {
      const uint16_t* kr = keys + (static_cast<int64_t>(b) * C + j) * W + h * hd;
      float dot = 0.f;
      for (int e = 0; e < hd; e += 8) {
        float a[8], c[8];
        unpack8(*reinterpret_cast<const uint4*>(qh + e), a);
        unpack8(*reinterpret_cast<const uint4*>(kr + e), c);
#pragma unroll
        for (int i = 0; i < 8; ++i) dot = fmaf(a[i], c[i], dot);
      }
      s = dot * scale_log2;
    }
    sc[j] = s;
  }
  float m = -INFINITY;
  for (int j = threadIdx.x; j < C; j += 256) m = fmaxf(m, sc[j]);
  m = wave_max(m);
  __syncthreads();
  if (lane == 0) red[wave] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float sum = 0.f;
  if (m != -INFINITY)
    for (int j = threadIdx.x; j < C; j += 256) sum += exp2_fast(sc[j] - m);
  sum = wave_sum(sum);
  __syncthreads();
  if (lane == 0) red[wave] = sum;
  __syncthreads();
  sum = (red[0] + red[1]) + (red[2] + red[3]);
  const float inv = (m != -INFINITY && sum > 0.f) ? 1.0f / sum : 0.f;
  for (int j = threadIdx.x; j < C; j += 256) sc[j] = inv > 0.f ? exp2_fast(sc[j] - m) * inv : 0.f;
  __syncthreads();
  for (int d = threadIdx.x; d < hd; d += 256) {
    float acc = 0.f;
    for (int j = 0; j < C; ++j) {
      const float p = sc[j];
      if (p == 0.f) continue;
      acc = fmaf(p, bf2f(vals[(static_cast<int64_t>(b) * C + j) * W + h * hd + d]), acc);
    }
    out[static_cast<int64_t>(r) * out_ld + h * hd + d] = f2bf(acc);
  }
}

}  // namespace llmy

extern "C" int32_t llmy_layernorm_f32_bf16(const float* x, const float* w, const float* b,
                                           llmy_bf16* out, int32_t rows, int32_t L, float eps,
                                           void* stream) {
  LLMY_REQUIRE(rows >= 0 && L > 0);
  if (rows == 0) return 0;
  LLMY_REQUIRE(x && w && b && out);
  hipLaunchKernelGGL(layernorm_kernel, dim3(rows), dim3(256), 0, as_stream(stream), x, w, b,
                     out, L, eps);
  return launch_status();
}

extern "C" int32_t llmy_latent_attn_bf16(const llmy_bf16* q, int64_t q_ld, const llmy_bf16* keys,
                                         const llmy_bf16* vals, const int32_t* tag,
                                         const int32_t* pos, llmy_bf16* out, int64_t out_ld,
                                         int32_t B, int32_t T, int32_t C, int32_t heads,
                                         int32_t head_dim, float scale, void* stream) {
  LLMY_REQUIRE(B >= 0 && T >= 1 && C >= 1 && C <= 16384 && heads > 0 && head_dim > 0 &&
               head_dim % 8 == 0);
  if (B == 0) return 0;
  const int64_t W = static_cast<int64_t>(heads) * head_dim;
  LLMY_REQUIRE(q && keys && vals && tag && out && q_ld >= W && q_ld % 8 == 0 && out_ld >= W);
  LLMY_REQUIRE(aligned(q, 16) && aligned(keys, 16));
  LLMY_REQUIRE(static_cast<int64_t>(B) * T * heads < (1ll << 31));
  hipLaunchKernelGGL(latent_attn_kernel, dim3(B * T * heads), dim3(256),
                     static_cast<size_t>(C) * 4, as_stream(stream), q, q_ld, keys, vals, tag, pos,
                     out, out_ld, T, C, heads, head_dim, scale * 1.4426950408889634f);
  return launch_status();
}
