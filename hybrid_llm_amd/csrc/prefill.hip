// Sequence-level glue for the batched prefill of the hybrid block stack:
// everything between the projection GEMMs and the sequence kernels
// (banded attention prefill, chunked GDN) that the one-token decode kernels
// do per step.  All four are elementwise or per-row and HBM-bound.
//
//   * llmy_kv_cache_fill_bf16: the attention layer's K/V of a prompt into the
//     ring cache [B, H, W, hd] that decode continues from (slot = pos % W);
//     only the last min(T, W) positions are kept, as hca.py:119-128 keeps the
//     last `local_window` history rows.
//   * llmy_gdn_prefill_prep_f32: per (token, head) L2 normalisation of q and
//     k (clamp 1e-12), beta = sigmoid(b + bias), g = sigmoid(decay_logit)
//     (gated_deltanet.py:124-132), read from the fp32 projection row
//     [q | k | v | gate | beta] and written in the chunked scan's layouts.
//   * llmy_gdn_gate_bf16: output gate o * sigmoid(gate) in bf16
//     (gated_deltanet.py:176,247: the scan output is rounded to the activation
//     dtype, then multiplied by the gate).
//   * llmy_gdn_conv_gate_prefill: the causal depthwise conv gate over a whole
//     sequence with the carried history (gated_deltanet.py:254-269), leaving
//     the last K-1 inputs as the new history.
#include "common.hpp"
#include "abi_util.hpp"

namespace llmy {

// One thread per 16-byte chunk of one (b, h, kept position) row of K and V.
__global__ __launch_bounds__(256) void kv_fill_kernel(const uint16_t* __restrict__ k,
                                                      const uint16_t* __restrict__ v,
                                                      long long ld, uint16_t* __restrict__ kc,
                                                      uint16_t* __restrict__ vc, int B, int T,
                                                      int H, int hd, int W, int kept) {
  const int cpr = hd / 8;  // chunks per head row
  const long long n = static_cast<long long>(B) * kept * H * cpr;
  const long long i = blockIdx.x * 256ll + threadIdx.x;
  if (i >= n) return;
  const int c = static_cast<int>(i % cpr);
  long long r = i / cpr;
  const int h = static_cast<int>(r % H);
  r /= H;
  const int j = static_cast<int>(r % kept);
  const int b = static_cast<int>(r / kept);
  const int t = T - kept + j;
  const long long src = (static_cast<long long>(b) * T + t) * ld + h * hd + 8 * c;
  const long long dst = ((static_cast<long long>(b) * H + h) * W + (t % W)) * hd + 8 * c;
  *reinterpret_cast<uint4*>(kc + dst) = *reinterpret_cast<const uint4*>(k + src);
  *reinterpret_cast<uint4*>(vc + dst) = *reinterpret_cast<const uint4*>(v + src);
}

// One workgroup of 4 wavefronts per token row; wavefront w takes heads
// w, w + 4, ...  For each head the lanes hold q and k (DK/64 values each),
// reduce the squared norms across the wavefront and store the normalised
// rows in bf16; v is rounded to bf16; lane 0 writes beta and g.
template <int DK>
__global__ __launch_bounds__(256) void gdn_prep_kernel(
    const float* __restrict__ proj, long long ld, const float* __restrict__ beta_bias,
    const float* __restrict__ decay_logit, uint16_t* __restrict__ q, uint16_t* __restrict__ k,
    uint16_t* __restrict__ v, float* __restrict__ beta, float* __restrict__ g, int H, int DV) {
  constexpr int NV = (DK + 63) / 64;
  const long long row = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const float* src = proj + row * ld;
  const int HK = H * DK, HV = H * DV;
  for (int h = wave; h < H; h += 4) {
    float qv[NV], kv[NV];
    float sq = 0.f, sk = 0.f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int d = lane + 64 * i;
      qv[i] = d < DK ? src[h * DK + d] : 0.f;
      kv[i] = d < DK ? src[HK + h * DK + d] : 0.f;
      sq = fmaf(qv[i], qv[i], sq);
      sk = fmaf(kv[i], kv[i], sk);
    }
    const float rq = rsqrtf(fmaxf(wave_sum(sq), 1e-12f));
    const float rk = rsqrtf(fmaxf(wave_sum(sk), 1e-12f));
    const long long qo = (row * H + h) * DK;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const int d = lane + 64 * i;
      if (d < DK) {
        q[qo + d] = f2bf(qv[i] * rq);
        k[qo + d] = f2bf(kv[i] * rk);
      }
    }
    const long long vo = (row * H + h) * DV;
    for (int d = lane; d < DV; d += 64) v[vo + d] = f2bf(src[2 * HK + h * DV + d]);
    if (lane == 0) {
      beta[row * H + h] = sigmoidf_(src[2 * HK + 2 * HV + h] + beta_bias[h]);
      g[row * H + h] = sigmoidf_(decay_logit[h]);
    }
  }
}

// out[r, j] = bf16(o[r, j] * sigmoid(gate[r, j])), 8 elements per thread;
// the gate logits are the fp32 projection row at column gate_off + j.
__global__ __launch_bounds__(256) void gdn_gate_kernel(const uint16_t* __restrict__ o,
                                                       const float* __restrict__ proj,
                                                       long long ld, int gate_off, int HV,
                                                       uint16_t* __restrict__ out, long long R) {
  const int cpr = HV / 8;
  const long long i = blockIdx.x * 256ll + threadIdx.x;
  if (i >= R * cpr) return;
  const long long r = i / cpr;
  const int j = static_cast<int>(i % cpr) * 8;
  float of[8];
  unpack8(*reinterpret_cast<const uint4*>(o + r * HV + j), of);
  const float* gp = proj + r * ld + gate_off + j;
  const float4 g0 = *reinterpret_cast<const float4*>(gp);
  const float4 g1 = *reinterpret_cast<const float4*>(gp + 4);
  const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
  uint32_t pk[4];
#pragma unroll
  for (int e = 0; e < 4; ++e)
    pk[e] = pack_bf2(of[2 * e] * sigmoidf_(gv[2 * e]), of[2 * e + 1] * sigmoidf_(gv[2 * e + 1]));
  *reinterpret_cast<uint4*>(out + r * HV + j) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
}

// Causal depthwise conv gate over a sequence.  Thread (b, time block, d)
// computes kConvSpan consecutive outputs of channel d from a register window
// of the last KC inputs; the window of the first block starts from the
// carried history.  Only the first block's thread rewrites the history of
// (b, d) — after reading it — so no thread reads a history another writes.
// With resets [B, T] (gated_deltanet.py:56-78: taps do not cross a reset),
// a tap at position p counts for token t only if no reset lies in (p, t];
// history taps only if none lies in [0, t].  The new history is then what a
// token-by-token pass would leave: the last KC - 1 inputs, zero where they
// precede the last reset.
constexpr int kConvSpan = 16;

template <int KC>
__global__ __launch_bounds__(256) void gdn_conv_prefill_kernel(const uint16_t* __restrict__ h,
                                                               uint16_t* __restrict__ hist,
                                                               const float* __restrict__ w,
                                                               const int32_t* __restrict__ reset,
                                                               float* __restrict__ out, int B,
                                                               int T, int D) {
  const int nblk = (T + kConvSpan - 1) / kConvSpan;
  const long long i = blockIdx.x * 256ll + threadIdx.x;
  if (i >= static_cast<long long>(B) * nblk * D) return;
  const int d = static_cast<int>(i % D);
  const long long r = i / D;
  const int tb = static_cast<int>(r % nblk);
  const int b = static_cast<int>(r / nblk);
  const int t0 = tb * kConvSpan;
  const uint16_t* hb = h + static_cast<long long>(b) * T * D + d;
  uint16_t* hs = hist + static_cast<long long>(b) * (KC - 1) * D + d;
  float wt[KC];
#pragma unroll
  for (int j = 0; j < KC; ++j) wt[j] = w[d * KC + j];
  // win[j] = input at position t - (KC - 1) + j; positions < 0 come from the history.
  uint16_t win[KC];
#pragma unroll
  for (int j = 0; j < KC - 1; ++j) {
    const int p = t0 - (KC - 1) + j;
    win[j + 1] = p >= 0 ? hb[static_cast<long long>(p) * D] : hs[static_cast<long long>(j) * D];
  }
  const int t1 = min(t0 + kConvSpan, T);
  // first position a tap may read (the last reset so far; -KC: none, history valid)
  const int32_t* rb = reset ? reset + static_cast<long long>(b) * T : nullptr;
  int vstart = -KC;
  if (rb) {
    for (int p = max(0, t0 - (KC - 1)); p < t0; ++p)
      if (rb[p] != 0) vstart = p;
  }
  for (int t = t0; t < t1; ++t) {
#pragma unroll
    for (int j = 0; j < KC - 1; ++j) win[j] = win[j + 1];
    win[KC - 1] = hb[static_cast<long long>(t) * D];
    if (rb && rb[t] != 0) vstart = t;
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < KC; ++j)
      acc = t - (KC - 1) + j >= vstart ? fmaf(wt[j], bf2f(win[j]), acc) : acc;
    out[(static_cast<long long>(b) * T + t) * D + d] = sigmoidf_(acc);
  }
  if (tb == 0) {
    // New history = the last KC - 1 entries of [old history, h[0 .. T-1]].
    // When this block reached T its window already holds them (including
    // old history entries for T < KC - 1); otherwise T > kConvSpan > KC - 1
    // and they are all inputs.
    int last = -KC;  // the last reset of the sequence (inputs before it are not kept)
    if (rb) {
      for (int p = max(0, T - (KC - 1)); p < T; ++p)
        if (rb[p] != 0) last = p;
    }
#pragma unroll
    for (int j = 0; j < KC - 1; ++j) {
      const uint16_t hv = t1 == T ? win[j + 1] : hb[static_cast<long long>(T - (KC - 1) + j) * D];
      hs[static_cast<long long>(j) * D] = T - (KC - 1) + j >= last ? hv : 0;
    }
  }
}

}  // namespace llmy

using namespace llmy;

extern "C" int32_t llmy_kv_cache_fill_bf16(const llmy_bf16* k, const llmy_bf16* v, int64_t ld,
                                           llmy_bf16* k_cache, llmy_bf16* v_cache, int32_t B,
                                           int32_t T, int32_t H, int32_t head_dim, int32_t W,
                                           void* stream) {
  LLMY_REQUIRE(B >= 0 && T >= 0 && H > 0 && W > 0 && head_dim > 0 && head_dim % 8 == 0);
  if (B == 0 || T == 0) return 0;
  LLMY_REQUIRE(k && v && k_cache && v_cache);
  LLMY_REQUIRE(ld >= static_cast<int64_t>(H) * head_dim && ld % 8 == 0);
  LLMY_REQUIRE(aligned(k, 16) && aligned(v, 16) && aligned(k_cache, 16) && aligned(v_cache, 16));
  const int kept = T < W ? T : W;
  const long long n = static_cast<long long>(B) * kept * H * (head_dim / 8);
  LLMY_REQUIRE((n + 255) / 256 < (1ll << 31));
  hipLaunchKernelGGL(kv_fill_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                     as_stream(stream), k, v, static_cast<long long>(ld), k_cache, v_cache, B, T,
                     H, head_dim, W, kept);
  return launch_status();
}

extern "C" int32_t llmy_gdn_prefill_prep_f32(const float* proj, int64_t ld,
                                             const float* beta_bias, const float* decay_logit,
                                             llmy_bf16* q, llmy_bf16* k, llmy_bf16* v,
                                             float* beta, float* g, int32_t rows, int32_t H,
                                             int32_t dk, int32_t dv, void* stream) {
  LLMY_REQUIRE(rows >= 0 && H > 0 && (dk == 64 || dk == 128 || dk == 256) && dv > 0);
  if (rows == 0) return 0;
  LLMY_REQUIRE(proj && beta_bias && decay_logit && q && k && v && beta && g);
  LLMY_REQUIRE(ld >= static_cast<int64_t>(H) * (2 * dk + 2 * dv) + H);
  const hipStream_t s = as_stream(stream);
  const long long L = ld;
  switch (dk) {
    case 64:
      hipLaunchKernelGGL(gdn_prep_kernel<64>, dim3(rows), dim3(256), 0, s, proj, L, beta_bias,
                         decay_logit, q, k, v, beta, g, H, dv);
      break;
    case 128:
      hipLaunchKernelGGL(gdn_prep_kernel<128>, dim3(rows), dim3(256), 0, s, proj, L, beta_bias,
                         decay_logit, q, k, v, beta, g, H, dv);
      break;
    default:
      hipLaunchKernelGGL(gdn_prep_kernel<256>, dim3(rows), dim3(256), 0, s, proj, L, beta_bias,
                         decay_logit, q, k, v, beta, g, H, dv);
      break;
  }
  return launch_status();
}

extern "C" int32_t llmy_gdn_gate_bf16(const llmy_bf16* o, const float* proj, int64_t ld,
                                      int32_t gate_off, llmy_bf16* out, int32_t rows, int32_t HV,
                                      void* stream) {
  LLMY_REQUIRE(rows >= 0 && HV > 0 && HV % 8 == 0 && gate_off >= 0);
  if (rows == 0) return 0;
  LLMY_REQUIRE(o && proj && out);
  LLMY_REQUIRE(ld % 4 == 0 && gate_off % 4 == 0 && ld >= static_cast<int64_t>(gate_off) + HV);
  LLMY_REQUIRE(aligned(o, 16) && aligned(proj, 16) && aligned(out, 16));
  const long long n = static_cast<long long>(rows) * (HV / 8);
  LLMY_REQUIRE((n + 255) / 256 < (1ll << 31));
  hipLaunchKernelGGL(gdn_gate_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                     as_stream(stream), o, proj, static_cast<long long>(ld), gate_off, HV, out,
                     static_cast<long long>(rows));
  return launch_status();
}

extern "C" int32_t llmy_gdn_conv_gate_prefill(const llmy_bf16* h, llmy_bf16* hist, const float* w,
                                              float* out, int32_t B, int32_t T, int32_t D,
                                              int32_t kernel, void* stream) {
  LLMY_REQUIRE(B >= 0 && T >= 0 && D > 0 && kernel == 4);
  if (B == 0 || T == 0) return 0;
  LLMY_REQUIRE(h && hist && w && out);
  const long long n =
      static_cast<long long>(B) * ((T + kConvSpan - 1) / kConvSpan) * static_cast<long long>(D);
  LLMY_REQUIRE((n + 255) / 256 < (1ll << 31));
  hipLaunchKernelGGL(gdn_conv_prefill_kernel<4>, dim3(static_cast<unsigned>((n + 255) / 256)),
                     dim3(256), 0, as_stream(stream), h, hist, w, nullptr, out, B, T, D);
  return launch_status();
}

extern "C" int32_t llmy_gdn_conv_gate_prefill_reset(const llmy_bf16* h, llmy_bf16* hist,
                                                    const float* w, const int32_t* reset,
                                                    float* out, int32_t B, int32_t T, int32_t D,
                                                    int32_t kernel, void* stream) {
  LLMY_REQUIRE(B >= 0 && T >= 0 && D > 0 && kernel == 4);
  if (B == 0 || T == 0) return 0;
  LLMY_REQUIRE(h && hist && w && reset && out);
  const long long n =
      static_cast<long long>(B) * ((T + kConvSpan - 1) / kConvSpan) * static_cast<long long>(D);
  LLMY_REQUIRE((n + 255) / 256 < (1ll << 31));
  hipLaunchKernelGGL(gdn_conv_prefill_kernel<4>, dim3(static_cast<unsigned>((n + 255) / 256)),
                     dim3(256), 0, as_stream(stream), h, hist, w, reset, out, B, T, D);
  return launch_status();
}
