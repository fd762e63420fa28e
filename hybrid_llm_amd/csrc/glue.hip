// Elementwise / row-wise glue of the block stack: RMSNorm, embedding gather,
// and the GDN causal depthwise conv gate.
#include "common.hpp"
#include "abi_util.hpp"

#include <algorithm>
#include <cmath>

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

// Row-wise RMSNorm of an fp32 row held by one wavefront as NCH float4 chunks
// (element 4*lane + 256*c + j), written as bf16.
template <int NCH>
__device__ __forceinline__ void norm_row_store(const float4* v, const float* __restrict__ w,
                                               uint16_t* __restrict__ out, int lane, float eps) {
  constexpr int D = NCH * 256;
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) ss += v[c].x * v[c].x + v[c].y * v[c].y + v[c].z * v[c].z + v[c].w * v[c].w;
  const float r = rsqrtf(wave_sum(ss) / static_cast<float>(D) + eps);
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int d = 4 * lane + 256 * c;
    const float4 wv = *reinterpret_cast<const float4*>(w + d);
    *reinterpret_cast<uint2*>(out + d) =
        make_uint2(pack_bf2(v[c].x * r * wv.x, v[c].y * r * wv.y),
                   pack_bf2(v[c].z * r * wv.z, v[c].w * r * wv.w));
  }
}

// x[b] = float(table[tok[b]]); h[b] = bf16(RMSNorm(x[b]) * w).  One wave per row.
template <int NCH>
__global__ __launch_bounds__(256) void embed_norm_kernel(const int32_t* __restrict__ tokens,
                                                         const uint16_t* __restrict__ table,
                                                         const float* __restrict__ w,
                                                         float* __restrict__ x,
                                                         uint16_t* __restrict__ h, int B, int V,
                                                         float eps) {
  constexpr int D = NCH * 256;
  const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (b >= B) return;
  int tok = tokens[b];
  tok = tok < 0 ? 0 : (tok >= V ? V - 1 : tok);
  const uint16_t* src = table + static_cast<long long>(tok) * D;
  float* xr = x + static_cast<long long>(b) * D;
  float4 v[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int d = 4 * lane + 256 * c;
    const uint2 raw = *reinterpret_cast<const uint2*>(src + d);
    v[c] = make_float4(__uint_as_float(raw.x << 16), __uint_as_float(raw.x & 0xffff0000u),
                       __uint_as_float(raw.y << 16), __uint_as_float(raw.y & 0xffff0000u));
    *reinterpret_cast<float4*>(xr + d) = v[c];
  }
  norm_row_store<NCH>(v, w, h + static_cast<long long>(b) * D, lane, eps);
}

// MoE combine fused with the next RMSNorm: x[t] += sum_j y[route_pos[t*k+j]]
// (j ascending), then h[t] = bf16(RMSNorm(x[t]) * w) (skipped when w is null).
// One wave per row.  Routes are taken in groups of KG, and each group's route
// indices, y rows (with x and the norm weight in the first group) are
// requested together: a runtime loop over k waits on each load in turn.
constexpr int kCombineGroup = 2;
template <int NCH>
__global__ __launch_bounds__(256) void combine_norm_kernel(const float* __restrict__ y,
                                                           const int32_t* __restrict__ route_pos,
                                                           const float* __restrict__ w,
                                                           float* __restrict__ x,
                                                           uint16_t* __restrict__ h, int T, int k,
                                                           float eps) {
  constexpr int D = NCH * 256;
  constexpr int KG = kCombineGroup;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (t >= T) return;
  float* xr = x + static_cast<long long>(t) * D;
  float4 v[NCH], wv[NCH], s[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) s[c] = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int j0 = 0; j0 < k; j0 += KG) {
    int p[KG];
#pragma unroll
    for (int j = 0; j < KG; ++j) {
      const int jj = min(j0 + j, k - 1);  // past k: repeats the last route, not added
      p[j] = route_pos ? min(max(route_pos[t * k + jj], 0), T * k - 1) : t * k + jj;
    }
    float4 yv[KG][NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int d = 4 * lane + 256 * c;
#pragma unroll
      for (int j = 0; j < KG; ++j)
        yv[j][c] = *reinterpret_cast<const float4*>(y + static_cast<long long>(p[j]) * D + d);
      if (j0 == 0) {
        v[c] = *reinterpret_cast<const float4*>(xr + d);
        if (w != nullptr) wv[c] = *reinterpret_cast<const float4*>(w + d);
      }
    }
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
#pragma unroll
      for (int j = 0; j < KG; ++j) {
        if (j0 + j < k) {
          s[c].x += yv[j][c].x; s[c].y += yv[j][c].y; s[c].z += yv[j][c].z; s[c].w += yv[j][c].w;
        }
      }
    }
  }
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    v[c].x += s[c].x; v[c].y += s[c].y; v[c].z += s[c].z; v[c].w += s[c].w;
    *reinterpret_cast<float4*>(xr + 4 * lane + 256 * c) = v[c];
  }
  if (w == nullptr) return;
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) ss += v[c].x * v[c].x + v[c].y * v[c].y + v[c].z * v[c].z + v[c].w * v[c].w;
  const float r = rsqrtf(wave_sum(ss) / static_cast<float>(D) + eps);
  uint16_t* out = h + static_cast<long long>(t) * D;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int d = 4 * lane + 256 * c;
    *reinterpret_cast<uint2*>(out + d) =
        make_uint2(pack_bf2(v[c].x * r * wv[c].x, v[c].y * r * wv[c].y),
                   pack_bf2(v[c].z * r * wv[c].z, v[c].w * r * wv[c].w));
  }
}

// Shared experts as always-on routes: ids/gates [T, k] of the router become
// [T, k + S] with routes k .. k+S-1 of every token going to experts
// E .. E+S-1 (the shared experts, stacked after the routed ones) with gate
// g = 1/sqrt(S) (model/layers/moe.py:185-199).
__global__ __launch_bounds__(256) void append_shared_kernel(const int32_t* __restrict__ idx,
                                                            const float* __restrict__ gates,
                                                            int32_t* __restrict__ idx_out,
                                                            float* __restrict__ gates_out, int T,
                                                            int k, int E, int S, float g) {
  const int kx = k + S;
  const long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<long long>(T) * kx) return;
  const int t = static_cast<int>(i / kx), j = static_cast<int>(i - static_cast<long long>(t) * kx);
  idx_out[i] = j < k ? idx[t * k + j] : E + (j - k);
  gates_out[i] = j < k ? gates[t * k + j] : g;
}

// Zero row b of a [rows, row_bytes] buffer where mask[b] != 0 (the per-row
// state reset of model/recurrent_state.py:213-225).  A kernel rather than a
// memory set, so a captured graph may hold it.  V = 16-byte or 4-byte words.
template <typename V>
__global__ __launch_bounds__(256) void zero_rows_kernel(V* __restrict__ base, long long words,
                                                        const int32_t* __restrict__ mask) {
  const int b = blockIdx.y;
  if (mask[b] == 0) return;
  V* row = base + static_cast<long long>(b) * words;
  const V z{};
  for (long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x; i < words;
       i += static_cast<long long>(gridDim.x) * 256)
    row[i] = z;
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

#define LLMY_NCH_SWITCH(D, MACRO)      \
  switch (D) {                         \
    case 256: MACRO(1); break;         \
    case 512: MACRO(2); break;         \
    case 1024: MACRO(4); break;        \
    default: MACRO(8); break;          \
  }

extern "C" int32_t llmy_embed_norm_bf16(const int32_t* tokens, const llmy_bf16* table,
                                        const float* w, float* x, llmy_bf16* h, int32_t B,
                                        int32_t D, int32_t V, float eps, void* stream) {
  LLMY_REQUIRE(B >= 0 && V > 0 && (D == 256 || D == 512 || D == 1024 || D == 2048));
  if (B == 0) return 0;
  LLMY_REQUIRE(tokens && table && w && x && h);
  LLMY_REQUIRE(aligned(table, 8) && aligned(w, 16) && aligned(x, 16) && aligned(h, 8));
  const hipStream_t s = as_stream(stream);
#define LLMY_EMBED(N)                                                                        \
  hipLaunchKernelGGL(embed_norm_kernel<N>, dim3((B + 3) / 4), dim3(256), 0, s, tokens, table, \
                     w, x, h, B, V, eps)
  LLMY_NCH_SWITCH(D, LLMY_EMBED)
#undef LLMY_EMBED
  return launch_status();
}

extern "C" int32_t llmy_moe_combine_norm(const float* y, const int32_t* route_pos,
                                         const float* w, float* x, llmy_bf16* h, int32_t T,
                                         int32_t D, int32_t k, float eps, void* stream) {
  LLMY_REQUIRE(T >= 0 && k > 0 && (D == 256 || D == 512 || D == 1024 || D == 2048));
  if (T == 0) return 0;
  LLMY_REQUIRE(y && x && (w == nullptr || h != nullptr));
  LLMY_REQUIRE(aligned(y, 16) && aligned(x, 16) && (w == nullptr || (aligned(w, 16) && aligned(h, 8))));
  const hipStream_t s = as_stream(stream);
#define LLMY_COMBINE(N)                                                                        \
  hipLaunchKernelGGL(combine_norm_kernel<N>, dim3((T + 3) / 4), dim3(256), 0, s, y, route_pos, \
                     w, x, h, T, k, eps)
  LLMY_NCH_SWITCH(D, LLMY_COMBINE)
#undef LLMY_COMBINE
  return launch_status();
}

extern "C" int32_t llmy_moe_append_shared(const int32_t* idx, const float* gates, int32_t* idx_out,
                                          float* gates_out, int32_t T, int32_t k, int32_t E,
                                          int32_t S, void* stream) {
  LLMY_REQUIRE(T >= 0 && k > 0 && E > 0 && S > 0 && static_cast<long long>(T) * (k + S) < (1ll << 31));
  if (T == 0) return 0;
  LLMY_REQUIRE(idx && gates && idx_out && gates_out);
  const long long n = static_cast<long long>(T) * (k + S);
  hipLaunchKernelGGL(append_shared_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256),
                     0, as_stream(stream), idx, gates, idx_out, gates_out, T, k, E, S,
                     1.0f / std::sqrt(static_cast<float>(S)));
  return launch_status();
}

extern "C" int32_t llmy_zero_rows(void* base, int64_t row_bytes, int32_t rows,
                                  const int32_t* mask, void* stream) {
  LLMY_REQUIRE(rows >= 0 && row_bytes >= 0 && row_bytes % 4 == 0 && rows <= 65535);
  if (rows == 0 || row_bytes == 0) return 0;
  LLMY_REQUIRE(base && mask);
  const bool wide = row_bytes % 16 == 0 && aligned(base, 16);
  const long long words = wide ? row_bytes / 16 : row_bytes / 4;
  const unsigned gx = static_cast<unsigned>(std::min<long long>((words + 255) / 256, 64));
  if (wide)
    hipLaunchKernelGGL(zero_rows_kernel<uint4>, dim3(gx, rows), dim3(256), 0, as_stream(stream),
                       static_cast<uint4*>(base), words, mask);
  else
    hipLaunchKernelGGL(zero_rows_kernel<uint32_t>, dim3(gx, rows), dim3(256), 0,
                       as_stream(stream), static_cast<uint32_t*>(base), words, mask);
  return launch_status();
}
