// Banded causal attention, decode: one new query per (batch, head) against a
// ring-buffer KV cache [B, H, W, HD] bf16 (head-major, so one (b, h) window is
// one contiguous slab).  Semantics follow model/layers/hca.py:119-128: the
// new K/V is written to slot pos % W and the query attends to the last
// min(pos + 1, W) tokens including itself; scores in fp32 with scale 1/sqrt(HD).
//
// One 256-thread workgroup per (b, h).  Each wave sweeps 64-key chunks of the
// window with HD/8 lanes per key (8 bf16 = 16 bytes per lane, so one load
// instruction covers 64/(HD/8) whole keys = 1 KiB contiguous), reduces the
// q.k partial dots across those lanes, and keeps an online softmax (running
// max in the log2 domain, rescaled sum and output).  The new token is taken
// from registers rather than re-read from the cache, and the waves' partial
// (max, sum, output) are merged through LDS.
//
// The new row's q, k and v come either as bf16 rows or, for decode batches
// whose projection ran as per-256-wide-K-block partial products, as P fp32
// slices summed here in slice order and rounded to bf16: the same values,
// bit for bit, as a projection kernel that sums its K blocks in that order
// before its bf16 store.
#include "common.hpp"
#include "abi_util.hpp"

namespace llmy {

// q/k/v partial slices: parts [P][B][row] fp32, q at column 0, k at koff, v at voff.
struct QkvParts {
  const float* p;
  int n;
  long long stride;  // floats between slices
  long long row;     // floats between batch rows
  int koff, voff;
};

// The summed slices of one value (column c of row b), in slice order.
__device__ __forceinline__ float sum_parts1(const QkvParts& a, int b, int c) {
  const float* src = a.p + static_cast<long long>(b) * a.row + c;
  float acc = src[0];
  for (int s = 1; s < a.n; ++s) acc += src[s * a.stride];
  return acc;
}

template <int HD, bool PARTS>
__global__ __launch_bounds__(256) void attn_decode_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_new,
    const uint16_t* __restrict__ v_new, long long q_bstride, long long kv_bstride, QkvParts qp,
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
    const int32_t* __restrict__ pos, uint16_t* __restrict__ out, int H, int W,
    float scale_log2) {
  constexpr int LPK = HD / 8;    // lanes per key
  constexpr int KPG = 64 / LPK;  // keys per load group
  constexpr int NIT = LPK;       // load groups per 64-key chunk
  __shared__ float sm_m[4], sm_l[4];
  __shared__ float sm_o[4][HD];

  const int bh = blockIdx.x;
  const int b = bh / H;
  const int h = bh - b * H;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int kk = lane / LPK;
  const int dc = lane % LPK;

  const int p = max(pos[b], 0);  // negative positions are treated as 0
  const int cur = p % W;
  const int n_sweep = min(p + 1, W);
  const long long slab = static_cast<long long>(bh) * W * HD;

  float qf[8], knf[8], vnf[8];
  uint4 qraw, kraw, vraw;
  if (PARTS) {
    // the workgroup's q, k and v rows (3 HD values) summed once, one value
    // per thread, rounded to bf16 and shared through LDS
    __shared__ __align__(16) uint16_t qkv_s[3 * HD];
    for (int e = threadIdx.x; e < 3 * HD; e += 256) {
      const int part = e / HD, dim = e - part * HD;
      const int col = (part == 0 ? 0 : part == 1 ? qp.koff : qp.voff) + h * HD + dim;
      qkv_s[e] = f2bf(sum_parts1(qp, b, col));
    }
    __syncthreads();
    qraw = *reinterpret_cast<const uint4*>(qkv_s + 8 * dc);
    kraw = *reinterpret_cast<const uint4*>(qkv_s + HD + 8 * dc);
    vraw = *reinterpret_cast<const uint4*>(qkv_s + 2 * HD + 8 * dc);
  } else {
    qraw = *reinterpret_cast<const uint4*>(q + b * q_bstride + h * HD + 8 * dc);
    kraw = *reinterpret_cast<const uint4*>(k_new + b * kv_bstride + h * HD + 8 * dc);
    vraw = *reinterpret_cast<const uint4*>(v_new + b * kv_bstride + h * HD + 8 * dc);
  }
  unpack8(qraw, qf);
  unpack8(kraw, knf);
  unpack8(vraw, vnf);
  if (wave == 0 && kk == 0) {
    *reinterpret_cast<uint4*>(k_cache + slab + static_cast<long long>(cur) * HD + 8 * dc) = kraw;
    *reinterpret_cast<uint4*>(v_cache + slab + static_cast<long long>(cur) * HD + 8 * dc) = vraw;
  }

  // Current token: every lane computes its score; only wave 0 (kk == 0 lanes)
  // seeds the softmax with it.
  float s_cur = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) s_cur = fmaf(qf[j], knf[j], s_cur);
#pragma unroll
  for (int off = 1; off < LPK; off <<= 1) s_cur += __shfl_xor(s_cur, off, kWave);
  s_cur *= scale_log2;

  float m_run = -INFINITY, l_run = 0.f;
  float o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = 0.f;
  if (wave == 0) {
    m_run = s_cur;
    if (kk == 0) {
      l_run = 1.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = vnf[j];
    }
  }

  const int nchunks = (n_sweep + 63) >> 6;
  for (int c = wave; c < nchunks; c += 4) {
    float s[NIT];
    uint4 vr[NIT], kr[NIT];
    // HD = 64: the chunk's K loads are issued together ahead of the dot
    // products (the compiler then batches the V loads too); measured 86 ->
    // 83 us on the C5 window.  HD = 128 keeps one key group per step, which
    // holds half the registers (occupancy 4 instead of 3).
    constexpr bool kBatch = NIT <= 8;
    if (kBatch) {
#pragma unroll
      for (int i = 0; i < NIT; ++i) {
        const int key = c * 64 + i * KPG + kk;
        const int kl = min(key, W - 1);
        const long long off = slab + static_cast<long long>(kl) * HD + 8 * dc;
        kr[i] = ld_stream(k_cache + off);
        vr[i] = ld_stream(v_cache + off);
      }
    }
#pragma unroll
    for (int i = 0; i < NIT; ++i) {
      if (!kBatch) {
        const int key = c * 64 + i * KPG + kk;
        const int kl = min(key, W - 1);
        const long long off = slab + static_cast<long long>(kl) * HD + 8 * dc;
        kr[i] = ld_stream(k_cache + off);
        vr[i] = ld_stream(v_cache + off);
      }
      float kf[8];
      unpack8(kr[i], kf);
      float d = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) d = fmaf(qf[j], kf[j], d);
      s[i] = d;
    }
    float mloc = -INFINITY;
#pragma unroll
    for (int i = 0; i < NIT; ++i) {
#pragma unroll
      for (int off = 1; off < LPK; off <<= 1) s[i] += __shfl_xor(s[i], off, kWave);
      const int key = c * 64 + i * KPG + kk;
      const bool valid = key < n_sweep && key != cur;
      s[i] = valid ? s[i] * scale_log2 : -INFINITY;
      mloc = fmaxf(mloc, s[i]);
    }
#pragma unroll
    for (int off = LPK; off < 64; off <<= 1) mloc = fmaxf(mloc, __shfl_xor(mloc, off, kWave));
    const float m_new = fmaxf(m_run, mloc);
    if (m_new == -INFINITY) continue;  // nothing valid yet in this wave (uniform)
    const float alpha = exp2_fast(m_run - m_new);
    l_run *= alpha;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] *= alpha;
#pragma unroll
    for (int i = 0; i < NIT; ++i) {
      const float pi = exp2_fast(s[i] - m_new);  // 0 for masked keys
      l_run += pi;
      if (s[i] != -INFINITY) {
        float vf[8];
        unpack8(vr[i], vf);
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = fmaf(pi, vf[j], o[j]);
      }
    }
    m_run = m_new;
  }

  // Reduce across the keys (kk) that share a dim chunk.
#pragma unroll
  for (int off = LPK; off < 64; off <<= 1) {
    l_run += __shfl_xor(l_run, off, kWave);
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] += __shfl_xor(o[j], off, kWave);
  }
  if (lane < LPK) {
#pragma unroll
    for (int j = 0; j < 8; ++j) sm_o[wave][8 * dc + j] = o[j];
  }
  if (lane == 0) {
    sm_m[wave] = m_run;
    sm_l[wave] = l_run;
  }
  __syncthreads();
  if (threadIdx.x < HD) {
    const int d = threadIdx.x;
    float mstar = sm_m[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) mstar = fmaxf(mstar, sm_m[w]);
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float sc = exp2_fast(sm_m[w] - mstar);
      num = fmaf(sm_o[w][d], sc, num);
      den = fmaf(sm_l[w], sc, den);
    }
    out[static_cast<long long>(bh) * HD + d] = f2bf(num / den);
  }
}

}  // namespace llmy

using namespace llmy;

extern "C" int32_t llmy_banded_attn_decode_bf16(
    const llmy_bf16* q, const llmy_bf16* k_new, const llmy_bf16* v_new, int64_t q_bstride,
    int64_t kv_bstride, llmy_bf16* k_cache, llmy_bf16* v_cache, const int32_t* pos,
    llmy_bf16* out, int32_t B, int32_t H, int32_t head_dim, int32_t W, float scale,
    void* stream) {
  LLMY_REQUIRE(B >= 0 && H > 0 && W > 0 && (head_dim == 64 || head_dim == 128));
  if (B == 0) return 0;
  LLMY_REQUIRE(q && k_new && v_new && k_cache && v_cache && pos && out);
  LLMY_REQUIRE(q_bstride >= static_cast<int64_t>(H) * head_dim && q_bstride % 8 == 0);
  LLMY_REQUIRE(kv_bstride >= static_cast<int64_t>(H) * head_dim && kv_bstride % 8 == 0);
  LLMY_REQUIRE(aligned(q, 16) && aligned(k_new, 16) && aligned(v_new, 16) &&
               aligned(k_cache, 16) && aligned(v_cache, 16) && aligned(out, 2));
  if (B == 0) return 0;
  const float scale_log2 = scale * 1.4426950408889634f;
  const hipStream_t s = as_stream(stream);
  const QkvParts none{};
  if (head_dim == 64) {
    hipLaunchKernelGGL((attn_decode_kernel<64, false>), dim3(B * H), dim3(256), 0, s, q, k_new,
                       v_new, q_bstride, kv_bstride, none, k_cache, v_cache, pos, out, H, W,
                       scale_log2);
  } else {
    hipLaunchKernelGGL((attn_decode_kernel<128, false>), dim3(B * H), dim3(256), 0, s, q, k_new,
                       v_new, q_bstride, kv_bstride, none, k_cache, v_cache, pos, out, H, W,
                       scale_log2);
  }
  return launch_status();
}

extern "C" int32_t llmy_banded_attn_decode_parts_bf16(
    const float* parts, int32_t nparts, int64_t part_stride, int64_t row_stride, int32_t k_off,
    int32_t v_off, llmy_bf16* k_cache, llmy_bf16* v_cache, const int32_t* pos, llmy_bf16* out,
    int32_t B, int32_t H, int32_t head_dim, int32_t W, float scale, void* stream) {
  LLMY_REQUIRE(B >= 0 && H > 0 && W > 0 && (head_dim == 64 || head_dim == 128) && nparts >= 1);
  if (B == 0) return 0;
  LLMY_REQUIRE(parts && k_cache && v_cache && pos && out);
  const int64_t Hhd = static_cast<int64_t>(H) * head_dim;
  LLMY_REQUIRE(k_off >= Hhd && v_off >= k_off + Hhd && row_stride >= v_off + Hhd);
  LLMY_REQUIRE(k_off % 8 == 0 && v_off % 8 == 0 && row_stride % 4 == 0 &&
               (nparts == 1 || (part_stride >= static_cast<int64_t>(B) * row_stride &&
                                part_stride % 4 == 0)));
  LLMY_REQUIRE(aligned(parts, 16) && aligned(k_cache, 16) && aligned(v_cache, 16) &&
               aligned(out, 2));
  const float scale_log2 = scale * 1.4426950408889634f;
  const hipStream_t s = as_stream(stream);
  const QkvParts qp{parts, nparts, part_stride, row_stride, k_off, v_off};
  if (head_dim == 64) {
    hipLaunchKernelGGL((attn_decode_kernel<64, true>), dim3(B * H), dim3(256), 0, s, nullptr,
                       nullptr, nullptr, 0ll, 0ll, qp, k_cache, v_cache, pos, out, H, W,
                       scale_log2);
  } else {
    hipLaunchKernelGGL((attn_decode_kernel<128, true>), dim3(B * H), dim3(256), 0, s, nullptr,
                       nullptr, nullptr, 0ll, 0ll, qp, k_cache, v_cache, pos, out, H, W,
                       scale_log2);
  }
  return launch_status();
}
