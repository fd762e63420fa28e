// Gated delta-rule decode step: one token per (batch, head), fp32 state
// S [DK, DV] updated in place (model/layers/gated_deltanet.py:140-149):
//
//   pred = k^T S;  S <- g S + beta k (v - pred)^T;  o = (q^T S) * gate
//
// One 256-thread workgroup per (b, h).  Thread t owns columns
// [4*(t % (DV/4)), +4) of rows t / (DV/4) + i * RPP (RPP = 1024/DV rows per
// pass): every state row is read and written as contiguous float4 runs, the
// state lives in registers between the two reductions (k^T S, then q^T S'),
// and the reductions over rows go through LDS in a fixed order, so results
// are deterministic.  The state is read and written exactly once: the kernel
// is HBM-bound on 2 * DK * DV * 4 bytes per (b, h).  Both the state loads
// and the stores carry the non-temporal hint: each state byte is touched once
// per step, and keeping it out of the caches measured 26-27% faster at
// B = 64, H = 16 (dk = dv = 128: 34.6 -> 25.3 us; dk = dv = 64: 11.5 -> 8.8 us).
//
// Two input layouts:
//   op:    q, k [B,H,DK] / v, gate [B,H,DV] bf16, beta, g [B,H] fp32 (q, k
//          already L2-normalised; gate optional);
//   model: the fused fp32 projection row [q | k | v | gate logits | beta
//          logits] of the GDN block (or nparts per-K-block partial products
//          of it, summed here in slice order), from which the kernel applies the
//          per-head L2 norm of q and k (clamp 1e-12, gated_deltanet.py:128-129),
//          beta = sigmoid(logit + bias) (:130), gate = sigmoid(logit) (:131) and
//          g = sigmoid(decay_logit[h]) (:132).
//
// Optional per-row reset (gated_deltanet.py:138-142,165-166; the reference's
// native step takes a per-head mask, llmy_cuda/src/kernels/gdn.cu:28,36-40):
// where reset[b] != 0 the row's state and conv history count as zero before
// the update (the state is still read, so the loads start at once; its values
// are dropped).
#include "common.hpp"
#include "abi_util.hpp"

namespace llmy {

struct GdnStepArgs {
  const uint16_t *q, *k, *v, *gate;
  const float *beta, *g;
  const float* proj;
  long long proj_ld;
  int nparts;             // model variant: slices of proj, [nparts, B, proj_ld]
  long long part_stride;  // floats between slices
  const float* beta_bias;
  const float* decay_logit;
  float* state;
  uint16_t* out;
  int H;
  // optional causal conv gate fused into the model variant
  const uint16_t* conv_h;  // [B, D] mixer input (bf16)
  uint16_t* conv_hist;     // [B, K-1, D]
  const float* conv_w;     // [D, K]
  float* conv_out;         // [B, D] sigmoid(conv)
  int D;
  const int32_t* reset;    // [B] or null: nonzero = the row starts from zero
};

// NP: compile-time bound on the projection slices (1, 4 or 8), so that every
// slice load of a value is issued before the first add.
template <int DK, int DV, bool MODEL, int NP = 1>
__global__ __launch_bounds__(256) void gdn_step_kernel(GdnStepArgs a) {
  constexpr int CPT = DV / 4;        // threads per state row
  constexpr int RPP = 256 / CPT;     // rows per pass
  constexpr int NR = DK / RPP;       // rows per thread
  __shared__ float qs[DK], ks[DK], vs[DV], gs[DV];
  __shared__ float red[RPP][DV];
  __shared__ float bg[2];

  const int bh = blockIdx.x;
  const int b = bh / a.H;
  const int h = bh - b * a.H;
  const int t = threadIdx.x;
  const int c4 = (t % CPT) * 4;
  const int rg = t / CPT;

  float* S = a.state + static_cast<long long>(bh) * DK * DV;
  const bool fresh = a.reset != nullptr && a.reset[b] != 0;
  float4 st[NR];
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const f32x4 v = __builtin_nontemporal_load(
        reinterpret_cast<const f32x4*>(S + (rg + i * RPP) * DV + c4));
    st[i] = make_float4(v[0], v[1], v[2], v[3]);
  }
  if (fresh) {
#pragma unroll
    for (int i = 0; i < NR; ++i) st[i] = make_float4(0.f, 0.f, 0.f, 0.f);
  }

  const int lane = t & 63;
  const int wave = t >> 6;
  if (MODEL) {
    const float* row = a.proj + static_cast<long long>(b) * a.proj_ld;
    const int np = a.nparts;
    const long long ps = a.part_stride;
    // projection value at offset i of the row: the slices summed in order
    // (slices past np repeat the last one and are not added)
    auto pv = [&](int i) {
      float t[NP];
#pragma unroll
      for (int sl = 0; sl < NP; ++sl) t[sl] = row[min(sl, np - 1) * ps + i];
      float v = t[0];
#pragma unroll
      for (int sl = 1; sl < NP; ++sl) v = sl < np ? v + t[sl] : v;
      return v;
    };
    const int HK = a.H * DK, HV = a.H * DV;
    if (wave < 2) {  // wave 0: q, wave 1: k -> L2 normalised
      const float* src = row + (wave == 0 ? 0 : HK) + h * DK;
      float vals[(DK + 63) / 64];
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < (DK + 63) / 64; ++i) {
        const int d = lane + 64 * i;
        vals[i] = d < DK ? pv(static_cast<int>(src - row) + d) : 0.f;
        ss += vals[i] * vals[i];
      }
      const float r = rsqrtf(fmaxf(wave_sum(ss), 1e-12f));
      float* dst = wave == 0 ? qs : ks;
#pragma unroll
      for (int i = 0; i < (DK + 63) / 64; ++i) {
        const int d = lane + 64 * i;
        if (d < DK) dst[d] = vals[i] * r;
      }
    } else if (wave == 2) {
      for (int d = lane; d < DV; d += 64) {
        vs[d] = pv(2 * HK + h * DV + d);
        gs[d] = sigmoidf_(pv(2 * HK + HV + h * DV + d));
      }
    } else if (lane == 0) {
      bg[0] = sigmoidf_(pv(2 * HK + 2 * HV + h) + a.beta_bias[h]);
      bg[1] = sigmoidf_(a.decay_logit[h]);
    }
  } else {
    const long long qk = static_cast<long long>(bh) * DK;
    const long long vv = static_cast<long long>(bh) * DV;
    for (int d = t; d < DK; d += 256) {
      qs[d] = bf2f(a.q[qk + d]);
      ks[d] = bf2f(a.k[qk + d]);
    }
    for (int d = t; d < DV; d += 256) {
      vs[d] = bf2f(a.v[vv + d]);
      gs[d] = a.gate ? bf2f(a.gate[vv + d]) : 1.f;
    }
    if (t == 0) {
      bg[0] = a.beta[bh];
      bg[1] = a.g[bh];
    }
  }
  // After the projection reads: its global stores would otherwise hold them
  // back (the compiler cannot tell the buffers apart).
  if (MODEL && a.conv_h != nullptr) {
    // Causal depthwise conv gate (gated_deltanet.py:257-268) for this head's
    // D/H channels of row b: window = [hist[0..2], h]; out = sigmoid(w . window);
    // the history shifts by one.  Each thread owns one channel.
    const int per = a.D / a.H;
    for (int c = t; c < per; c += 256) {
      const int d = h * per + c;
      uint16_t* hb = a.conv_hist + static_cast<long long>(b) * 3 * a.D + d;
      uint16_t w0 = hb[0], w1 = hb[a.D], w2 = hb[2 * a.D];
      if (fresh) w0 = w1 = w2 = 0;
      const uint16_t w3 = a.conv_h[static_cast<long long>(b) * a.D + d];
      const float4 cw = *reinterpret_cast<const float4*>(a.conv_w + 4 * d);
      float acc = cw.x * bf2f(w0);
      acc = fmaf(cw.y, bf2f(w1), acc);
      acc = fmaf(cw.z, bf2f(w2), acc);
      acc = fmaf(cw.w, bf2f(w3), acc);
      a.conv_out[static_cast<long long>(b) * a.D + d] = sigmoidf_(acc);
      hb[0] = w1;
      hb[a.D] = w2;
      hb[2 * a.D] = w3;
    }
  }
  __syncthreads();

  // pred = k^T S (partial over this thread's rows, then a fixed-order LDS sum)
  float4 pp = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const float kr = ks[rg + i * RPP];
    pp.x = fmaf(kr, st[i].x, pp.x);
    pp.y = fmaf(kr, st[i].y, pp.y);
    pp.z = fmaf(kr, st[i].z, pp.z);
    pp.w = fmaf(kr, st[i].w, pp.w);
  }
  *reinterpret_cast<float4*>(&red[rg][c4]) = pp;
  __syncthreads();
  __shared__ float delta[DV];
  if (t < DV) {
    float pred = 0.f;
#pragma unroll 8
    for (int r = 0; r < RPP; ++r) pred += red[r][t];
    delta[t] = vs[t] - pred;
  }
  __syncthreads();

  const float beta = bg[0];
  const float g = bg[1];
  const float4 dl = *reinterpret_cast<const float4*>(&delta[c4]);
  float4 op = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const int r = rg + i * RPP;
    const float bk = beta * ks[r];
    float4 sn;
    sn.x = fmaf(g, st[i].x, bk * dl.x);
    sn.y = fmaf(g, st[i].y, bk * dl.y);
    sn.z = fmaf(g, st[i].z, bk * dl.z);
    sn.w = fmaf(g, st[i].w, bk * dl.w);
    const f32x4 sv = {sn.x, sn.y, sn.z, sn.w};
    __builtin_nontemporal_store(sv, reinterpret_cast<f32x4*>(S + r * DV + c4));
    const float qr = qs[r];
    op.x = fmaf(qr, sn.x, op.x);
    op.y = fmaf(qr, sn.y, op.y);
    op.z = fmaf(qr, sn.z, op.z);
    op.w = fmaf(qr, sn.w, op.w);
  }
  *reinterpret_cast<float4*>(&red[rg][c4]) = op;
  __syncthreads();
  if (t < DV) {
    float o = 0.f;
#pragma unroll 8
    for (int r = 0; r < RPP; ++r) o += red[r][t];
    a.out[static_cast<long long>(bh) * DV + t] = f2bf(o * gs[t]);
  }
}

template <bool MODEL, int NP>
static int32_t launch_gdn_step_np(const GdnStepArgs& a, int B, int dk, int dv, hipStream_t s) {
  const dim3 grid(B * a.H), block(256);
  if (dk == 64 && dv == 64) {
    hipLaunchKernelGGL((gdn_step_kernel<64, 64, MODEL, NP>), grid, block, 0, s, a);
  } else if (dk == 128 && dv == 128) {
    hipLaunchKernelGGL((gdn_step_kernel<128, 128, MODEL, NP>), grid, block, 0, s, a);
  } else {
    return static_cast<int32_t>(hipErrorInvalidValue);
  }
  return launch_status();
}

template <bool MODEL>
static int32_t launch_gdn_step(const GdnStepArgs& a, int B, int dk, int dv, hipStream_t s) {
  if constexpr (!MODEL) {
    return launch_gdn_step_np<false, 1>(a, B, dk, dv, s);
  } else {
    if (a.nparts <= 1) return launch_gdn_step_np<true, 1>(a, B, dk, dv, s);
    if (a.nparts <= 4) return launch_gdn_step_np<true, 4>(a, B, dk, dv, s);
    return launch_gdn_step_np<true, 8>(a, B, dk, dv, s);
  }
}

}  // namespace llmy

using namespace llmy;

extern "C" int32_t llmy_gdn_step_bf16(const llmy_bf16* q, const llmy_bf16* k, const llmy_bf16* v,
                                      const float* beta, const float* g, const llmy_bf16* gate,
                                      float* state, llmy_bf16* out, int32_t B, int32_t H,
                                      int32_t dk, int32_t dv, void* stream) {
  LLMY_REQUIRE(B >= 0 && H > 0 && ((dk == 64 && dv == 64) || (dk == 128 && dv == 128)));
  if (B == 0) return 0;
  LLMY_REQUIRE(q && k && v && beta && g && state && out);
  LLMY_REQUIRE(aligned(state, 16));
  GdnStepArgs a{};
  a.q = q; a.k = k; a.v = v; a.gate = gate; a.beta = beta; a.g = g;
  a.state = state; a.out = out; a.H = H;
  return launch_gdn_step<false>(a, B, dk, dv, as_stream(stream));
}

extern "C" int32_t llmy_gdn_step_fused_f32(const float* proj, int64_t proj_ld, int32_t nparts,
                                           const float* beta_bias, const float* decay_logit,
                                           float* state, llmy_bf16* out, const llmy_bf16* conv_h,
                                           llmy_bf16* conv_hist, const float* conv_w,
                                           float* conv_out, int32_t D, int32_t conv_kernel,
                                           int32_t B, int32_t H, int32_t dk, int32_t dv,
                                           void* stream) {
  LLMY_REQUIRE(B >= 0 && H > 0 && ((dk == 64 && dv == 64) || (dk == 128 && dv == 128)));
  LLMY_REQUIRE(proj_ld >= static_cast<int64_t>(H) * (2 * dk + 2 * dv + 1));
  LLMY_REQUIRE(nparts >= 1 && nparts <= 8);
  LLMY_REQUIRE(static_cast<long long>(nparts) * B * proj_ld < (1ll << 31));
  if (B == 0) return 0;
  LLMY_REQUIRE(proj && beta_bias && decay_logit && state && out);
  LLMY_REQUIRE(aligned(state, 16));
  if (conv_h != nullptr) {
    LLMY_REQUIRE(conv_hist && conv_w && conv_out && conv_kernel == 4 && D > 0 && D % H == 0);
    LLMY_REQUIRE(aligned(conv_w, 16));
  }
  GdnStepArgs a{};
  a.proj = proj; a.proj_ld = proj_ld; a.beta_bias = beta_bias; a.decay_logit = decay_logit;
  a.nparts = nparts; a.part_stride = static_cast<long long>(B) * proj_ld;
  a.state = state; a.out = out; a.H = H;
  a.conv_h = conv_h; a.conv_hist = conv_hist; a.conv_w = conv_w; a.conv_out = conv_out; a.D = D;
  return launch_gdn_step<true>(a, B, dk, dv, as_stream(stream));
}

extern "C" int32_t llmy_gdn_step_reset_bf16(const llmy_bf16* q, const llmy_bf16* k,
                                            const llmy_bf16* v, const float* beta, const float* g,
                                            const llmy_bf16* gate, const int32_t* reset,
                                            float* state, llmy_bf16* out, int32_t B, int32_t H,
                                            int32_t dk, int32_t dv, void* stream) {
  LLMY_REQUIRE(B >= 0 && H > 0 && ((dk == 64 && dv == 64) || (dk == 128 && dv == 128)));
  if (B == 0) return 0;
  LLMY_REQUIRE(q && k && v && beta && g && reset && state && out);
  LLMY_REQUIRE(aligned(state, 16));
  GdnStepArgs a{};
  a.q = q; a.k = k; a.v = v; a.gate = gate; a.beta = beta; a.g = g;
  a.state = state; a.out = out; a.H = H; a.reset = reset;
  return launch_gdn_step<false>(a, B, dk, dv, as_stream(stream));
}

extern "C" int32_t llmy_gdn_step_fused_reset_f32(const float* proj, int64_t proj_ld,
                                                 int32_t nparts, const float* beta_bias,
                                                 const float* decay_logit, const int32_t* reset,
                                                 float* state, llmy_bf16* out,
                                                 const llmy_bf16* conv_h, llmy_bf16* conv_hist,
                                                 const float* conv_w, float* conv_out, int32_t D,
                                                 int32_t conv_kernel, int32_t B, int32_t H,
                                                 int32_t dk, int32_t dv, void* stream) {
  LLMY_REQUIRE(B >= 0 && H > 0 && ((dk == 64 && dv == 64) || (dk == 128 && dv == 128)));
  LLMY_REQUIRE(proj_ld >= static_cast<int64_t>(H) * (2 * dk + 2 * dv + 1));
  LLMY_REQUIRE(nparts >= 1 && nparts <= 8);
  LLMY_REQUIRE(static_cast<long long>(nparts) * B * proj_ld < (1ll << 31));
  if (B == 0) return 0;
  LLMY_REQUIRE(proj && beta_bias && decay_logit && reset && state && out);
  LLMY_REQUIRE(aligned(state, 16));
  if (conv_h != nullptr) {
    LLMY_REQUIRE(conv_hist && conv_w && conv_out && conv_kernel == 4 && D > 0 && D % H == 0);
    LLMY_REQUIRE(aligned(conv_w, 16));
  }
  GdnStepArgs a{};
  a.proj = proj; a.proj_ld = proj_ld; a.beta_bias = beta_bias; a.decay_logit = decay_logit;
  a.nparts = nparts; a.part_stride = static_cast<long long>(B) * proj_ld;
  a.state = state; a.out = out; a.H = H; a.reset = reset;
  a.conv_h = conv_h; a.conv_hist = conv_hist; a.conv_w = conv_w; a.conv_out = conv_out; a.D = D;
  return launch_gdn_step<true>(a, B, dk, dv, as_stream(stream));
}
