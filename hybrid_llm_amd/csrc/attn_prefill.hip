// Banded causal attention, prefill: for every (b, h) and query i,
//   o_i = sum_{j : 0 <= i - j < W} softmax_j(scale * q_i . k_j) v_j
// with fp32 scores and accumulation; q, k, v, o are [B, T, H, HD] bf16 (the
// layout of runpod/kernels/fused_attention.py:14; mask rule :27, scale
// 1/sqrt(HD) of runpod/kernels/triton_banded_attention.py:97-98).
//
// MI355X mapping (v_mfma_f32_32x32x16_bf16, wave64):
//   * a workgroup owns 128 queries of one (b, h); wave w owns 32 of them;
//   * scores are computed transposed, S^T = K Q^T (keys are MFMA rows,
//     queries columns), so each lane holds 16 keys of ONE query: the running
//     max is 15 in-register maxes plus one exchange with the other lane half,
//     and the online-softmax rescale of the accumulator is per lane;
//   * the output is accumulated transposed, O^T = V^T P^T.  Under the key
//     order kappa(h, j) = (j & 3) + 8 (j >> 2) + 4 h (h = lane / 32) the
//     score registers 8s..8s+7 of a 32-key tile are exactly the B operand of
//     key slice s, so P never leaves registers; V is staged transposed in LDS
//     (V^T[dim][key]) so the matching A operand is two 8-byte LDS reads;
//   * K/V tiles of 64 keys are staged once per workgroup in LDS and shared by
//     the 4 waves; the band is walked tile by tile and a wave skips 32-key
//     sub-tiles that lie wholly outside its queries' windows;
//   * blockIdx.x enumerates (query block, b*H + h) with (b, h) fastest, so the
//     consecutive query blocks of one head (which share 3/4 of their K/V
//     window) are B*H apart in launch order and, with B*H a multiple of 8,
//     land on the same XCD and share its L2.
// D layout of a 32x32 MFMA result: lane l, register r holds row
// (r & 3) + 8 (r >> 2) + 4 (l >> 5), column l & 31.
#include "common.hpp"
#include "abi_util.hpp"

namespace llmy {

typedef float f32x16v __attribute__((ext_vector_type(16)));

constexpr int kBM = 128;    // queries per workgroup
constexpr int kBN = 64;     // keys per staged tile
constexpr int kKPad = 8;    // bf16 pad per staged K row (16 bytes)
constexpr int kVPad = 8;    // bf16 pad per staged V^T row

__device__ __forceinline__ uint4 pack8_bf16(const float* v) {
  return uint4{pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]), pack_bf2(v[4], v[5]),
               pack_bf2(v[6], v[7])};
}

template <int HD>
__global__ __launch_bounds__(256) void attn_prefill_kernel(const uint16_t* __restrict__ q,
                                                           const uint16_t* __restrict__ k,
                                                           const uint16_t* __restrict__ v,
                                                           uint16_t* __restrict__ o, int B, int T,
                                                           int H, int W, float scale_log2) {
  static_assert(HD == 64 || HD == 128, "head dim");
  constexpr int ND = HD / 32;   // 32-dim output tiles
  constexpr int NS = HD / 16;   // 16-dim slices of the score MFMA
  __shared__ __align__(16) uint16_t Ks[kBN * (HD + kKPad)];
  __shared__ __align__(16) uint16_t Vt[HD * (kBN + kVPad)];

  const int BH = B * H;
  const int bh = blockIdx.x % BH;
  const int qblk = blockIdx.x / BH;
  const int b = bh / H;
  const int h = bh - b * H;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int half = lane >> 5;
  const int col = lane & 31;
  const long long rs = static_cast<long long>(H) * HD;  // row stride (elements)
  const long long base = static_cast<long long>(b) * T * rs + static_cast<long long>(h) * HD;
  const uint32_t rs32 = static_cast<uint32_t>(rs);      // T * H * HD < 2^31 (host check)

  const int q0 = qblk * kBM;
  const int qw = q0 + 32 * wave;       // first query of this wave
  const int qi = qw + col;             // this lane's query
  const bool q_ok = qi < T;

  // Q^T operand: lane holds Q[qi][16t + 8 half .. +8] for each 16-dim slice t.
  uint4 qf[NS];
#pragma unroll
  for (int t = 0; t < NS; ++t)
    qf[t] = q_ok ? *reinterpret_cast<const uint4*>(q + base + qi * rs + 16 * t + 8 * half)
                 : uint4{0u, 0u, 0u, 0u};

  f32x16v acc[ND];
#pragma unroll
  for (int d = 0; d < ND; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[d][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  const int k_lo = max(0, q0 - W + 1);
  const int k_hi = min(T - 1, q0 + kBM - 1);
  const int t_lo = k_lo / kBN;
  const int t_hi = k_hi / kBN;
  // Software pipeline: the next tile's K/V chunks are fetched into registers
  // while the current tile is being consumed from LDS.
  constexpr int CH = HD / 8;                     // 16-byte chunks per row
  constexpr int NCHK = (kBN * CH + 255) / 256;   // chunks per thread per tile
  uint4 kreg[NCHK], vreg[NCHK];
  // K is fetched row-major (8 lanes per 128-byte row, 16-byte LDS stores).
  // V is fetched as key pairs: entry f = (pair f % 32, chunk f / 32) holds
  // keys 2p and 2p+1 of one 8-dim chunk in vreg[2w], vreg[2w+1], so each of
  // the chunk's 8 dims is stored to V^T as one dword (the two keys' values),
  // lanes of a wave writing consecutive dwords of a row: no bank conflicts
  // (2-byte stores put two lanes on one dword).
  constexpr int NPW = (kBN / 2) * CH / 256;      // key-pair entries per thread
  static_assert(2 * NPW == NCHK, "V pair staging covers the tile");
  static_assert(NCHK * 256 == kBN * CH, "every thread fetches whole chunks");
  // Each thread's chunks sit at fixed (key, column) offsets inside a tile, so
  // a tile's loads are its base plus per-thread offsets plus constants.  K
  // chunk u: row kr0 + u * (256 / CH), column kc0; V pair entry w: rows vr0 and
  // vr0 + 1, column vc0 + 64 w.  Rows past the sequence (the last tile only)
  // are zero: a key there follows every query and is masked.
  const uint32_t kr0 = threadIdx.x / CH, kc0 = 8 * (threadIdx.x % CH);
  const uint32_t vr0 = 2 * (threadIdx.x % (kBN / 2)), vc0 = 8 * (threadIdx.x / (kBN / 2));
  const uint32_t koff0 = kr0 * rs32 + kc0, voff0 = vr0 * rs32 + vc0;
  const uint16_t* kbase = k + base;
  const uint16_t* vbase = v + base;
  auto fetch = [&](int tile) {
    const int kt = tile * kBN;
    const uint16_t* kb = kbase + static_cast<long long>(kt) * rs;
    const uint16_t* vb = vbase + static_cast<long long>(kt) * rs;
    const uint32_t last = static_cast<uint32_t>(T - 1 - kt);
#pragma unroll
    for (int u = 0; u < NCHK; ++u) {
      const uint32_t kr = kr0 + u * (256 / CH);
      kreg[u] = kr <= last ? *reinterpret_cast<const uint4*>(kb + koff0 + u * (256 / CH) * rs32)
                           : uint4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int w = 0; w < NPW; ++w)
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        vreg[2 * w + i] = vr0 + i <= last
                              ? *reinterpret_cast<const uint4*>(vb + voff0 + i * rs32 + 64 * w)
                              : uint4{0u, 0u, 0u, 0u};
      }
  };
  fetch(t_lo);
  for (int tile = t_lo; tile <= t_hi; ++tile) {
    const int kt = tile * kBN;
    // ---- stage K (row-major, padded) and V^T (transposed) for 64 keys
    __syncthreads();
#pragma unroll
    for (int u = 0; u < NCHK; ++u)  // every thread's chunks lie in the tile (NCHK * 256 = kBN * CH)
      *reinterpret_cast<uint4*>(Ks + (kr0 + u * (256 / CH)) * (HD + kKPad) + kc0) = kreg[u];
#pragma unroll
    for (int w = 0; w < NPW; ++w) {
      const int f = threadIdx.x + 256 * w;
      const int p2 = 2 * (f % (kBN / 2)), vc = f / (kBN / 2);
      const uint32_t a4[4] = {vreg[2 * w].x, vreg[2 * w].y, vreg[2 * w].z, vreg[2 * w].w};
      const uint32_t b4[4] = {vreg[2 * w + 1].x, vreg[2 * w + 1].y, vreg[2 * w + 1].z,
                              vreg[2 * w + 1].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // dim 8vc + e: key 2p in the low half, key 2p+1 in the high half (one
        // byte permute: bytes of a4 are selectors 0-3, of b4 4-7)
        const uint32_t word = __builtin_amdgcn_perm(b4[e >> 1], a4[e >> 1],
                                                    (e & 1) ? 0x07060302u : 0x05040100u);
        *reinterpret_cast<uint32_t*>(Vt + (8 * vc + e) * (kBN + kVPad) + p2) = word;
      }
    }
    __syncthreads();
    if (tile < t_hi) fetch(tile + 1);

#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int ks = kt + 32 * sub;  // first key of the 32-key sub-tile
      // skip sub-tiles wholly outside every window of this wave's queries
      if (ks > qw + 31 || ks + 31 < qw - W + 1 || ks >= T) continue;
      // ---- S^T = K Q^T over HD (NS MFMAs)
      f32x16v s;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = 0.f;
#pragma unroll
      for (int t = 0; t < NS; ++t) {
        const uint4 kf = *reinterpret_cast<const uint4*>(Ks + (32 * sub + col) * (HD + kKPad) +
                                                          16 * t + 8 * half);
        s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(kf), as_bf16x8(qf[t]), s, 0, 0, 0);
      }
      // ---- mask + online softmax (log2 domain); register r holds key
      //      kk = ks + (r & 3) + 8 (r >> 2) + 4 half for query qi, kept when
      //      0 <= qi - kk < W: one unsigned compare of dq - c_r against W
      //      (dq < 0 marks a query past T, which fails every compare).
      const int dq = q_ok ? qi - ks - 4 * half : -(1 << 30);
      // a sub-tile inside every window of the wave's 32 queries (all keys at
      // or before the first query, within W of the last) needs no mask
      const bool interior = ks + 31 <= qw && qw + 31 - ks < W && qw + 31 < T;
      if (!interior) {  // wave-uniform: most sub-tiles of the band need no mask
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int cr = (r & 3) + 8 * (r >> 2);
          const bool ok = static_cast<unsigned>(dq - cr) < static_cast<unsigned>(W);
          s[r] = ok ? s[r] : -INFINITY;
        }
      }
      float mloc = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) mloc = fmaxf(mloc, s[r]);
      // Scores stay unscaled; scale_log2 > 0 is applied inside the exponent.
      // Lazy rescale: the exponent offset m_run moves only when some lane's
      // maximum exceeds it by more than kRescaleSlack (log2 units; the wave
      // decides together), so most sub-tiles skip rescaling the accumulator.
      // Weights are then at most 2^kRescaleSlack; the final 1/l uses the
      // same offset, so the result is unchanged up to rounding.
      constexpr float kRescaleSlack = 8.f;
      {  // the other lane half's maximum (lanes l and l ^ 32 hold one query)
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mloc),
                                                         __float_as_uint(mloc), false, false);
        mloc = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
      }
      const bool grow = !(mloc * scale_log2 <= m_run * scale_log2 + kRescaleSlack);
      if (__ballot(grow)) {
        const float m_new = fmaxf(m_run, mloc);
        const float alpha = m_new == -INFINITY
                                ? 1.f
                                : exp2_fast((m_run - m_new) * scale_log2);  // 0 while m_run = -inf
        m_run = m_new;
        l_run *= alpha;
#pragma unroll
        for (int d = 0; d < ND; ++d)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[d][r] *= alpha;
      }
      const float m_sc = m_run == -INFINITY ? 0.f : m_run * scale_log2;
      float p[16];
      float psum = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        p[r] = exp2_fast(fmaf(s[r], scale_log2, -m_sc));
        psum += p[r];
      }
      l_run += psum;
      // ---- O^T += V^T P^T over the two 16-key slices
#pragma unroll
      for (int sl = 0; sl < 2; ++sl) {
        const uint4 pb = pack8_bf16(p + 8 * sl);
        // keys of slice sl for this lane: ks + 16 sl + kappa(half, j)
        const int kb0 = 32 * sub + 16 * sl + 4 * half;  // j = 0..3 -> +0..3, j = 4..7 -> +8..11
#pragma unroll
        for (int d = 0; d < ND; ++d) {
          const uint16_t* vrow = Vt + (32 * d + col) * (kBN + kVPad);
          const uint2 lo = *reinterpret_cast<const uint2*>(vrow + kb0);
          const uint2 hi = *reinterpret_cast<const uint2*>(vrow + kb0 + 8);
          const uint4 va = uint4{lo.x, lo.y, hi.x, hi.y};
          acc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(va), as_bf16x8(pb), acc[d],
                                                           0, 0, 0);
        }
      }
    }
  }

  // ---- normalise and store: acc[d] register r = O[qi][32 d + (r & 3) + 8 (r >> 2) + 4 half]
  const float l_tot = l_run + __shfl_xor(l_run, 32, kWave);
  if (!q_ok) return;
  const float inv = 1.0f / l_tot;
  uint16_t* orow = o + base + qi * rs;
#pragma unroll
  for (int d = 0; d < ND; ++d) {
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int dim = 32 * d + 8 * g4 + 4 * half;
      *reinterpret_cast<uint2*>(orow + dim) =
          make_uint2(pack_bf2(acc[d][4 * g4] * inv, acc[d][4 * g4 + 1] * inv),
                     pack_bf2(acc[d][4 * g4 + 2] * inv, acc[d][4 * g4 + 3] * inv));
    }
  }
}

}  // namespace llmy

using namespace llmy;

extern "C" int32_t llmy_banded_attn_prefill_bf16(const llmy_bf16* q, const llmy_bf16* k,
                                                 const llmy_bf16* v, llmy_bf16* o, int32_t B,
                                                 int32_t T, int32_t H, int32_t head_dim,
                                                 int32_t W, float scale, void* stream) {
  LLMY_REQUIRE(B >= 0 && T >= 0 && H > 0 && W > 0 && (head_dim == 64 || head_dim == 128));
  if (B == 0 || T == 0) return 0;
  LLMY_REQUIRE(q && k && v && o);
  LLMY_REQUIRE(aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && aligned(o, 8));
  LLMY_REQUIRE(static_cast<long long>(T) * H * head_dim < (1ll << 31));  // 32-bit row offsets
  const long long nblk = static_cast<long long>((T + kBM - 1) / kBM) * B * H;
  LLMY_REQUIRE(nblk < (1ll << 31));
  const float scale_log2 = scale * 1.4426950408889634f;
  const hipStream_t s = as_stream(stream);
  if (head_dim == 64)
    hipLaunchKernelGGL(attn_prefill_kernel<64>, dim3(static_cast<unsigned>(nblk)), dim3(256), 0, s,
                       q, k, v, o, B, T, H, W, scale_log2);
  else
    hipLaunchKernelGGL(attn_prefill_kernel<128>, dim3(static_cast<unsigned>(nblk)), dim3(256), 0,
                       s, q, k, v, o, B, T, H, W, scale_log2);
  return launch_status();
}
