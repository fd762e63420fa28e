// Gated delta rule, prefill: the recurrence of model/layers/gated_deltanet.py:140-149
//
//   S_t = g_t S_{t-1} + beta_t k_t (v_t - S_{t-1}^T k_t)^T,   o_t = S_t^T q_t
//
// over T tokens per (batch, head) with an fp32 state S [DK, DV], computed in
// chunks of C = 64 tokens (the reference is sequential over T everywhere:
// gated_deltanet.py:42-53, runpod/kernels/triton_gdn.py:91-114).  Within a
// chunk starting from S0, with Gamma_t = prod_{j<=t} g_j (log-space cumulative
// sums, so every ratio below is <= 1):
//   U  = (I + L)^{-1} [beta (V - Gamma_{t-1} K S0)],
//        L[t,i] = beta_t (Gamma_{t-1} / Gamma_i) k_t . k_i   (i < t)
//      = U0 - W S0,  U0 = (I+L)^{-1} diag(beta) V,  W = (I+L)^{-1} diag(beta Gamma_{t-1}) K
//   O  = Gamma Q S0 + A U,  A[t,i] = (Gamma_t / Gamma_i) q_t . k_i  (i <= t)
//   S' = Gamma_C S0 + K^T diag(Gamma_C / Gamma_t) U
//
// Kernel 1 (gdn_chunk_prep) runs once per (b, h, chunk), all chunks in
// parallel: K K^T and Q K^T on bf16 MFMA (exact: the inputs are bf16 and the
// accumulation fp32), the unit lower-triangular inverse blocked by 16 (four
// diagonal forward substitutions, then three levels of 16 x 16 block
// products), then W, U0, A and the cumulative log-decays.  W and A are
// written as (hi, lo) bf16 planes, U0 and the log-decays as fp32.  Kernel 2
// (gdn_chunk_scan) runs once per (b, h, 32-column slice of the state),
// sequentially over the chunks.  Every product with an fp32 operand uses
// split-bf16 MFMA: x = hi + lo with hi = bf16(x), lo = bf16(x - hi), keeping
// hi*hi + hi*lo + lo*hi (relative error about 2^-16); products of two bf16
// tensors are exact.  Each fp32 operand is split once, where it is made.
//
// Resets (gated_deltanet.py:138-142: the state is zeroed before token t's
// update where reset[b, t]): a reset starts a new segment of the chunk.
// Log-decays are cumulated per segment, the couplings L and A vanish between
// tokens of different segments, S0 reaches only the segment before the first
// reset (Gamma masked to 0 after it), and S' takes only the last segment's
// tokens (Gamma_C / Gamma_t masked to 0 before it, Gamma_C to 0 when the
// chunk resets).  Kernel 1 therefore stores, per token, the two decay factors
// the scan applies (e_t = Gamma_t, d_t = Gamma_C / Gamma_t, masked) instead
// of the log-decays; without resets they are the same expf values the scan
// formed from the log-decays.
//
// MFMA v_mfma_f32_16x16x32_bf16 fragments: A lane l holds A[l%16][8(l/16)+j],
// B lane l holds B[8(l/16)+j][l%16], D lane l holds D[4(l/16)+i][l%16].
#include <mutex>

#include "common.hpp"
#include "abi_util.hpp"

namespace llmy {

constexpr int kC = 64;  // chunk length

__device__ __forceinline__ void split8(const float* x, uint4& hi, uint4& lo) {
  uint16_t h[8], l[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    h[j] = f2bf(x[j]);
    l[j] = f2bf(x[j] - bf2f(h[j]));
  }
  hi = uint4{static_cast<uint32_t>(h[0]) | (static_cast<uint32_t>(h[1]) << 16),
             static_cast<uint32_t>(h[2]) | (static_cast<uint32_t>(h[3]) << 16),
             static_cast<uint32_t>(h[4]) | (static_cast<uint32_t>(h[5]) << 16),
             static_cast<uint32_t>(h[6]) | (static_cast<uint32_t>(h[7]) << 16)};
  lo = uint4{static_cast<uint32_t>(l[0]) | (static_cast<uint32_t>(l[1]) << 16),
             static_cast<uint32_t>(l[2]) | (static_cast<uint32_t>(l[3]) << 16),
             static_cast<uint32_t>(l[4]) | (static_cast<uint32_t>(l[5]) << 16),
             static_cast<uint32_t>(l[6]) | (static_cast<uint32_t>(l[7]) << 16)};
}

__device__ __forceinline__ uint4 gather8_bf16(const uint16_t* p, int stride) {
  return uint4{static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[stride]) << 16),
               static_cast<uint32_t>(p[2 * stride]) | (static_cast<uint32_t>(p[3 * stride]) << 16),
               static_cast<uint32_t>(p[4 * stride]) | (static_cast<uint32_t>(p[5 * stride]) << 16),
               static_cast<uint32_t>(p[6 * stride]) | (static_cast<uint32_t>(p[7 * stride]) << 16)};
}

__device__ __forceinline__ uint32_t pack_bf2u(uint16_t a, uint16_t b) {
  return static_cast<uint32_t>(a) | (static_cast<uint32_t>(b) << 16);
}

__device__ __forceinline__ f32x4 mfma16(const uint4& a, const uint4& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Kernel 1: per-chunk preparation.  Scratch layout per chunk id
// cid = (b*H + h) * NC + c:  W [64][DK], U0 [64][DV] (dk = 128: in the scan's
// fragment order, [64-column slice][16 x 16 tile][lane][4 rows]), A [64][64],
// decay factors [2][64] (e_t then d_t, fp32).  reset [B, T] or null.
template <int DK, int DV>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void gdn_chunk_prep_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const float* __restrict__ beta,
    const float* __restrict__ g, const int32_t* __restrict__ reset, uint16_t* __restrict__ Wg,
    float* __restrict__ U0g, uint16_t* __restrict__ Ag, float* __restrict__ edg, int T, int H,
    int NC, int n_chunks) {
  constexpr int PK = DK + 8, PG = kC + 1, PT = kC + 8;
  constexpr bool kTOut = DK == 128;  // T and factors for gdn_chunk_scan_t_kernel
  // LDS by lifetime, so that two workgroups fit on a CU: region R0 holds K
  // and Q rows (products), then the per-wave block products of the inverse,
  // then K^T and V^T (the B operands of W and U0, staged after the inverse).
  constexpr int R0_KQ = 2 * kC * PK * 2, R0_T = (DK + DV) * PT * 2, R0_P = kC * 17 * 4;
  constexpr int R0 = (R0_KQ > R0_T ? (R0_KQ > R0_P ? R0_KQ : R0_P) : (R0_T > R0_P ? R0_T : R0_P));
  __shared__ __align__(16) unsigned char r0buf[R0];
  uint16_t* const Ks = reinterpret_cast<uint16_t*>(r0buf);
  uint16_t* const Qs = Ks + kC * PK;
  float* const Pm = reinterpret_cast<float*>(r0buf);  // per-wave 16 x 16 block products
  uint16_t* const KsT = reinterpret_cast<uint16_t*>(r0buf);  // K^T [DK][64]: B operand over t
  uint16_t* const VsT = KsT + DK * PT;                      // V^T [DV][64]
  __shared__ float Gm[kC * PG];   // K K^T, then L
  __shared__ float Ti[kC * PG];   // (I + L)^{-1}
  __shared__ float cum[kC], prv[kC], bet[kC], wsc[kC];  // wsc = beta * Gamma_prev
  __shared__ int seg[kC];  // segment of each token (resets seen up to it in the chunk)

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r16 = lane & 15, g4 = lane >> 4;
  const long long rk = static_cast<long long>(H) * DK, rv = static_cast<long long>(H) * DV;

  // Persistent: workgroup w takes chunks w, w + gridDim.x, ...  The next
  // chunk's K and Q rows and per-token g, beta and reset flags are loaded into
  // registers while the current one is worked out (dk = 128: from the block
  // levels of the inverse on; dk = 64: during the W and U0 products).  Every wave issues the same
  // loads (rows past a chunk and the last chunk's "next" re-read valid rows;
  // without resets the flags are read from g and ignored), so each wait counts
  // a fixed number of memory operations after the load it waits for.
  constexpr int SN = kC * (DK / 8) / 256;
  static_assert(SN * 256 == kC * (DK / 8), "staging split");
  uint4 skv[SN], sqv[SN];
  float pg, pb;
  int32_t prs;
  auto prefetch = [&](int cid_) {
    const int bh_ = cid_ / NC, c_ = cid_ - (cid_ / NC) * NC;
    const int b_ = bh_ / H, h_ = bh_ - (bh_ / H) * H;
    const int t0_ = c_ * kC, Tc_ = min(kC, T - t0_);
    const long long kb_ = (static_cast<long long>(b_) * T + t0_) * rk + static_cast<long long>(h_) * DK;
#pragma unroll
    for (int i = 0; i < SN; ++i) {
      const int f = threadIdx.x + 256 * i;
      const int t = f / (DK / 8), cc = f - t * (DK / 8);
      skv[i] = *reinterpret_cast<const uint4*>(k + kb_ + min(t, Tc_ - 1) * rk + 8 * cc);
      // Q only for A, which the dk = 128 scan forms itself
      if constexpr (!kTOut)
        sqv[i] = *reinterpret_cast<const uint4*>(q + kb_ + min(t, Tc_ - 1) * rk + 8 * cc);
    }
    const long long tok = static_cast<long long>(b_) * T + t0_ + min(lane, Tc_ - 1);
    pg = g[tok * H + h_];
    pb = beta[tok * H + h_];
    prs = (reset != nullptr ? reset : reinterpret_cast<const int32_t*>(g))[tok];
  };
  if (static_cast<int>(blockIdx.x) < n_chunks) prefetch(blockIdx.x);
  // the upper 16 x 16 blocks of T = (I + L)^{-1} are zero; no later write
  // touches them (the inverse writes the diagonal and lower blocks)
  for (int e = threadIdx.x; e < kC * kC; e += 256) {
    const int t = e >> 6, i = e & 63;
    if ((i >> 4) > (t >> 4)) Ti[t * PG + i] = 0.f;
  }
  for (int cid = blockIdx.x; cid < n_chunks; cid += gridDim.x) {
  const int bh = cid / NC;
  const int c = cid - bh * NC;
  const int b = bh / H, h = bh - (bh / H) * H;
  const int t0 = c * kC;
  const int Tc = min(kC, T - t0);
  const long long kbase = (static_cast<long long>(b) * T + t0) * rk + static_cast<long long>(h) * DK;
  const long long vbase = (static_cast<long long>(b) * T + t0) * rv + static_cast<long long>(h) * DV;

  // ---- stage K and Q rows from the prefetch registers; padded rows are zero
#pragma unroll
  for (int i = 0; i < SN; ++i) {
    const int f = threadIdx.x + 256 * i;
    const int t = f / (DK / 8), cc = f - t * (DK / 8);
    uint4 kv = skv[i];
    if (t >= Tc) kv = uint4{0u, 0u, 0u, 0u};
    *reinterpret_cast<uint4*>(Ks + t * PK + 8 * cc) = kv;
    if constexpr (!kTOut) {
      uint4 qv = sqv[i];
      if (t >= Tc) qv = uint4{0u, 0u, 0u, 0u};
      *reinterpret_cast<uint4*>(Qs + t * PK + 8 * cc) = qv;
    }
  }
  if (wave == 0) {
    // inclusive prefix sum of log g over the chunk (padded tokens: g = 1, beta = 0)
    float lg = lane < Tc ? logf(pg) : 0.f;
    const float bt = lane < Tc ? pb : 0.f;
    float sc = lg;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float o = __shfl_up(sc, off, kWave);
      if (lane >= off) sc += o;
    }
    // segments: a reset at token r starts a new one; cumulative log-decays
    // restart there (minus the prefix before r)
    const bool rs = reset != nullptr && lane < Tc && prs != 0;
    const unsigned long long rm = __ballot(rs);
    const unsigned long long upto = lane == 63 ? ~0ull : ((2ull << lane) - 1);
    const int sg = __popcll(rm & upto);
    float base = 0.f;
    if (rm != 0) {
      const unsigned long long before = rm & upto;
      const int r0 = before ? 63 - __clzll(static_cast<long long>(before)) : lane;
      const float pre = __shfl(sc - lg, r0, kWave);  // cumulative log-decay before token r0
      if (before) base = pre;
    }
    sc -= base;
    cum[lane] = sc;
    prv[lane] = sc - lg;
    bet[lane] = bt;
    seg[lane] = sg;
    wsc[lane] = sg == 0 ? bt * __expf(sc - lg) : 0.f;
  }
  __syncthreads();

  // ---- K K^T and Q K^T (exact): wave w owns output row block w, 4 column
  // blocks.  K K^T becomes L in LDS; A = (Gamma_t / Gamma_i) q_t . k_i
  // (i <= t) is formed in registers and written as (hi, lo) bf16 planes.
  const long long wo = static_cast<long long>(cid) * kC;
  // per-token factors of this lane's rows, read once: L rows 16 w + 4 g4 + i,
  // the A row 16 w + r16
  float lbet[4], lprv[4];
  int lseg[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = 16 * wave + 4 * g4 + i;
    lbet[i] = bet[t];
    lprv[i] = prv[t];
    lseg[i] = seg[t];
  }
  const float acum = cum[16 * wave + r16];
  const int aseg = seg[16 * wave + r16];
  // this wave's row block of K and Q, read once for the four column blocks
  uint4 kra[DK / 32], qra[DK / 32];
#pragma unroll
  for (int s = 0; s < DK / 32; ++s) {
    kra[s] = *reinterpret_cast<const uint4*>(Ks + (16 * wave + r16) * PK + 32 * s + 8 * g4);
    if constexpr (!kTOut)
      qra[s] = *reinterpret_cast<const uint4*>(Qs + (16 * wave + r16) * PK + 32 * s + 8 * g4);
  }
#pragma unroll
  for (int tj = 0; tj < 4; ++tj) {
    // this column block's factors, requested before its MFMAs
    const float lcum = cum[16 * tj + r16];
    const int lsj = seg[16 * tj + r16];
    float acj[4];
    int asj[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acj[i] = cum[16 * tj + 4 * g4 + i];
      asj[i] = seg[16 * tj + 4 * g4 + i];
    }
    f32x4 a1 = f32x4{0.f, 0.f, 0.f, 0.f}, a2 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < DK / 32; ++s) {
      const uint4 kb = *reinterpret_cast<const uint4*>(Ks + (16 * tj + r16) * PK + 32 * s + 8 * g4);
      a1 = mfma16(kra[s], kb, a1);
      // (K Q^T) block: lane holds 4 consecutive j of row t (dk = 128: the
      // scan forms A itself from the same operands)
      if constexpr (!kTOut) a2 = mfma16(kb, qra[s], a2);
    }
    // L[t, j] = beta_t (Gamma_{t-1} / Gamma_j) k_t . k_j for j < t in the same
    // segment (strictly lower), formed from the K K^T block in registers
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * wave + 4 * g4 + i, j = 16 * tj + r16;
      Gm[t * PG + j] = j < t && lsj == lseg[i] ? lbet[i] * __expf(lprv[i] - lcum) * a1[i] : 0.f;
    }
    if constexpr (!kTOut) {
      const int t = 16 * wave + r16, j0 = 16 * tj + 4 * g4;
      uint16_t hv[4], lv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = j0 + i;
        const float am = j <= t && asj[i] == aseg ? __expf(acum - acj[i]) * a2[i] : 0.f;
        hv[i] = f2bf(am);
        lv[i] = f2bf(am - bf2f(hv[i]));
      }
      uint16_t* arow = Ag + wo * kC * 2 + t * kC + j0;
      *reinterpret_cast<uint2*>(arow) = make_uint2(pack_bf2u(hv[0], hv[1]), pack_bf2u(hv[2], hv[3]));
      *reinterpret_cast<uint2*>(arow + kC * kC) =
          make_uint2(pack_bf2u(lv[0], lv[1]), pack_bf2u(lv[2], lv[3]));
    }
  }
  // K and V rows for the transposed staging after the inverse: item i =
  // (token pair, 8-dim chunk) f = threadIdx.x + 256 i, fetched after the
  // diagonal blocks so their latency hides behind the block levels.  Rows past
  // the chunk are clamped (valid addresses) here and zeroed at the store.
  constexpr int KPI = (kC / 2) * (DK / 8) / 256, VPI = (kC / 2) * (DV / 8) / 256;
  static_assert(KPI * 256 == (kC / 2) * (DK / 8) && VPI * 256 == (kC / 2) * (DV / 8), "pairs");
  uint4 kp[KPI][2], vp[VPI][2];
  __syncthreads();
  // ---- (I + L)^{-1}, blocked by 16: N = I + L is unit lower triangular with
  // 16 x 16 blocks N_ij; T = N^{-1} has T_ii = N_ii^{-1} and, for i > j,
  // T_ij = -T_ii * sum_{m=j}^{i-1} N_im T_mj.  Wave w inverts diagonal block w
  // by forward substitution (lanes 0..15 own its columns; the block's 120
  // entries are read from LDS into registers first, so the substitution waits
  // on no read), then the three off-diagonal levels i - j = 1, 2, 3 are 16 x 16
  // products on fp32 MFMA (v_mfma_f32_16x16x4_f32: A lane l holds
  // A[l % 16][l / 16], B lane l holds B[l / 16][l % 16], D lane l holds
  // D[4 (l / 16) + r][l % 16]), one block per wave and level.
  {
    const int d0 = 16 * wave;
    if (lane < 16) {
      const int j = lane;
      float nv[120];  // N[d0 + t][d0 + i], i < t, at t (t - 1) / 2 + i
#pragma unroll
      for (int t = 1; t < 16; ++t)
#pragma unroll
        for (int i = 0; i < t; ++i) nv[t * (t - 1) / 2 + i] = Gm[(d0 + t) * PG + d0 + i];
      float x[16];
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        // the dot product in four interleaved partial sums (shorter chains)
        float a[4] = {(t == j) ? 1.f : 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < t; ++i) a[i & 3] -= nv[t * (t - 1) / 2 + i] * x[i];
        x[t] = t < j ? 0.f : (a[0] + a[1]) + (a[2] + a[3]);
        Ti[(d0 + t) * PG + d0 + j] = x[t];
      }
    }
    // (the upper blocks of T are zero: set once, never written again)
#pragma unroll
    for (int i = 0; i < (kTOut ? 0 : KPI); ++i) {
      const int f = threadIdx.x + 256 * i;
      const int t2 = 2 * (f % (kC / 2)), cc = f / (kC / 2);
#pragma unroll
      for (int e = 0; e < 2; ++e)
        kp[i][e] = *reinterpret_cast<const uint4*>(k + kbase + min(t2 + e, Tc - 1) * rk + 8 * cc);
    }
#pragma unroll
    for (int i = 0; i < (kTOut ? 0 : VPI); ++i) {
      const int f = threadIdx.x + 256 * i;
      const int t2 = 2 * (f % (kC / 2)), cc = f / (kC / 2);
#pragma unroll
      for (int e = 0; e < 2; ++e)
        vp[i][e] = *reinterpret_cast<const uint4*>(v + vbase + min(t2 + e, Tc - 1) * rv + 8 * cc);
    }
    // dk = 128: the next chunk's rows now, behind the block levels and the T
    // write (this workgroup's last chunk fetches itself again)
    if constexpr (kTOut) prefetch(min(cid + static_cast<int>(gridDim.x), n_chunks - 1));
    __syncthreads();
    const int c16 = lane & 15, k4 = lane >> 4;
#pragma unroll
    for (int lvl = 1; lvl < 4; ++lvl) {
      const int bi = wave, bj = wave - lvl;  // block (bi, bj), bi - bj = lvl
      if (bj >= 0) {
        // P = sum_m N_{bi,m} T_{m,bj}, kept in this wave's rows of Pm (only
        // this wave reads them, and its LDS operations complete in order)
        f32x4 p = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int mm = 0; mm < lvl; ++mm) {
          const int m = bj + mm;
#pragma unroll
          for (int c4 = 0; c4 < 4; ++c4) {
            const float av = Gm[(16 * bi + c16) * PG + 16 * m + 4 * c4 + k4];
            const float bv = Ti[(16 * m + 4 * c4 + k4) * PG + 16 * bj + c16];
            p = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, p, 0, 0, 0);
          }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) Pm[(16 * wave + 4 * k4 + r) * 17 + c16] = p[r];
        // T_{bi,bj} = -T_{bi,bi} P
        f32x4 o = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c4 = 0; c4 < 4; ++c4) {
          const float av = Ti[(16 * bi + c16) * PG + 16 * bi + 4 * c4 + k4];
          const float bv = Pm[(16 * wave + 4 * c4 + k4) * 17 + c16];
          o = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, o, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) Ti[(16 * bi + 4 * k4 + r) * PG + 16 * bj + c16] = -o[r];
      }
      __syncthreads();
    }
  }

  if constexpr (kTOut) {
    // ---- dk = 128: T = (I + L)^{-1} as (hi, lo) bf16 planes [2][64][64] in
    // the chunk's W slot, and per token [Gamma_t | Gamma_C / Gamma_t | beta_t |
    // beta_t Gamma_{t-1}] (masked as below) in its U0 slot: the scan forms
    // U = T (beta V - beta Gamma_prev K S) itself
    uint16_t* Tw = Wg + static_cast<long long>(cid) * kC * DK * 2;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int f = threadIdx.x + 256 * i;
      const int t = f >> 3, c8 = f & 7;
      float x[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = Ti[t * PG + 8 * c8 + j];
      uint4 hi, lo;
      split8(x, hi, lo);
      *reinterpret_cast<uint4*>(Tw + t * kC + 8 * c8) = hi;
      *reinterpret_cast<uint4*>(Tw + kC * kC + t * kC + 8 * c8) = lo;
    }
    for (int f = threadIdx.x; f < 6 * kC; f += 256) {
      // parts 4, 5: the cumulative log-decay and the segment of each token,
      // from which the scan forms A = (Gamma_t / Gamma_i) q_t . k_i
      const int part = f >> 6, t = f & (kC - 1);
      const float ct = cum[t], cl = cum[kC - 1];
      const float fv = part == 0   ? (seg[t] == 0 ? __expf(ct) : 0.f)
                       : part == 1 ? (seg[t] == seg[kC - 1] ? __expf(cl - ct) : 0.f)
                       : part == 2 ? bet[t]
                       : part == 3 ? wsc[t]
                       : part == 4 ? ct
                                   : static_cast<float>(seg[t]);
      U0g[static_cast<long long>(cid) * kC * DV + f] = fv;
    }
    __syncthreads();  // LDS of this chunk is free for the next
  } else {
  // ---- K^T and V^T into R0 (the block products above are done), from the
  // rows fetched before the inverse: each of a pair's 8 dims is stored as one
  // dword holding both tokens (zero past the chunk), the lanes of a wave
  // writing consecutive dwords of a row.
#pragma unroll
  for (int i = 0; i < KPI; ++i) {
    const int f = threadIdx.x + 256 * i;
    const int t2 = 2 * (f % (kC / 2)), cc = f / (kC / 2);
    const uint4 z = uint4{0u, 0u, 0u, 0u};
    const uint4 a0 = t2 < Tc ? kp[i][0] : z, a1 = t2 + 1 < Tc ? kp[i][1] : z;
    const uint32_t w0[4] = {a0.x, a0.y, a0.z, a0.w}, w1[4] = {a1.x, a1.y, a1.z, a1.w};
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const uint32_t lo = (w0[jj >> 1] >> (16 * (jj & 1))) & 0xffffu;
      const uint32_t hi = (w1[jj >> 1] >> (16 * (jj & 1))) & 0xffffu;
      *reinterpret_cast<uint32_t*>(KsT + (8 * cc + jj) * PT + t2) = lo | (hi << 16);
    }
  }
#pragma unroll
  for (int i = 0; i < VPI; ++i) {
    const int f = threadIdx.x + 256 * i;
    const int t2 = 2 * (f % (kC / 2)), cc = f / (kC / 2);
    const uint4 z = uint4{0u, 0u, 0u, 0u};
    const uint4 a0 = t2 < Tc ? vp[i][0] : z, a1 = t2 + 1 < Tc ? vp[i][1] : z;
    const uint32_t w0[4] = {a0.x, a0.y, a0.z, a0.w}, w1[4] = {a1.x, a1.y, a1.z, a1.w};
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const uint32_t lo = (w0[jj >> 1] >> (16 * (jj & 1))) & 0xffffu;
      const uint32_t hi = (w1[jj >> 1] >> (16 * (jj & 1))) & 0xffffu;
      *reinterpret_cast<uint32_t*>(VsT + (8 * cc + jj) * PT + t2) = lo | (hi << 16);
    }
  }
  // the next chunk's rows (this workgroup's last chunk fetches itself again)
  prefetch(min(cid + static_cast<int>(gridDim.x), n_chunks - 1));
  __syncthreads();
  // ---- W = TW K  [64 x DK] (stored as (hi, lo) bf16 planes),  U0 = TU V  [64 x DV] (fp32)
  {
    // wave w takes row blocks (product, tm) = w and w + 4 of the 8 (W: tm 0..3,
    // U0: tm 0..3); their A fragments are scaled and split once, then reused
    // across the column tiles
    for (int pr = wave; pr < 8; pr += 4) {
      const bool isW = pr < 4;
      const int tm = pr & 3;
      const int nd = isW ? DK / 16 : DV / 16;
      const float* sc = isW ? wsc : bet;
      uint4 ahi[kC / 32], alo[kC / 32];
#pragma unroll
      for (int s = 0; s < kC / 32; ++s) {
        // A operand: Ti diag(beta Gamma_prev) (W) or Ti diag(beta) (U0)
        const int col = 32 * s + 8 * g4;
        float av[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) av[j] = Ti[(16 * tm + r16) * PG + col + j] * sc[col + j];
        split8(av, ahi[s], alo[s]);
      }
      const int row = 16 * tm + r16;
      for (int tn = 0; tn < nd; ++tn) {
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < kC / 32; ++s) {
          const uint4 bb = *reinterpret_cast<const uint4*>(
              (isW ? KsT : VsT) + (16 * tn + r16) * PT + 32 * s + 8 * g4);
          if (isW || DK != 128) {
            // transposed product (B^T A^T): lane l ends with row 16 tm + l % 16
            // and the 4 consecutive columns 16 tn + 4 (l / 16) .. +3
            acc = mfma16(bb, ahi[s], acc);
            acc = mfma16(bb, alo[s], acc);
          } else {
            // U0 for the dk = 128 scan: lane l ends with rows 16 tm + 4 (l / 16)
            // .. +3 of column 16 tn + l % 16 (the scan's fragment order)
            acc = mfma16(ahi[s], bb, acc);
            acc = mfma16(alo[s], bb, acc);
          }
        }
        const int col0 = 16 * tn + 4 * g4;
        if (isW) {
          // W as a (hi, lo) pair of bf16 planes [2][64][DK]: W = hi + lo to ~2^-16
          uint16_t* whi = Wg + wo * DK * 2 + row * DK + col0;
          uint16_t hv[4], lv[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            hv[i] = f2bf(acc[i]);
            lv[i] = f2bf(acc[i] - bf2f(hv[i]));
          }
          *reinterpret_cast<uint2*>(whi) =
              make_uint2(pack_bf2u(hv[0], hv[1]), pack_bf2u(hv[2], hv[3]));
          *reinterpret_cast<uint2*>(whi + kC * DK) =
              make_uint2(pack_bf2u(lv[0], lv[1]), pack_bf2u(lv[2], lv[3]));
        } else if (DK != 128) {
          *reinterpret_cast<float4*>(U0g + wo * DV + row * DV + col0) =
              make_float4(acc[0], acc[1], acc[2], acc[3]);
        } else {
          // [64-column slice][16 x 16 tile (row, column) of the slice][lane][4 rows]
          const int sl = tn >> 2, tl = tn & 3;
          *reinterpret_cast<float4*>(U0g + ((wo / kC * 2 + sl) * 16 + tm * 4 + tl) * 256 + lane * 4) =
              make_float4(acc[0], acc[1], acc[2], acc[3]);
        }
      }
    }
  }
  {
    // e_t = Gamma_t (the S0 term of O), d_t = Gamma_C / Gamma_t (the S' update),
    // masked to the segments that see S0 and reach the chunk's end; threads
    // 128..255 store the same values as 0..127 (every wave stores)
    const int e = threadIdx.x & (2 * kC - 1), t = e & (kC - 1);
    const float ct = cum[t], cl = cum[kC - 1];
    edg[2 * wo + e] = e < kC ? (seg[t] == 0 ? __expf(ct) : 0.f)
                             : (seg[t] == seg[kC - 1] ? __expf(cl - ct) : 0.f);
  }
  __syncthreads();  // LDS of this chunk is free for the next
  }
  }
}

// ---------------------------------------------------------------------------
// Kernel 2: sequential scan over chunks for one (b, h, DVS-column state
// slice), 8 wavefronts.  Every slice reads the chunk's K, Q, W and A, so wider
// slices cut that stream: dk = dv = 128 runs 64-column slices (one round of
// workgroups), dk = dv = 64 runs 32-column ones (two workgroups per CU).
// Every fp32 operand enters the MFMA as a (hi, lo) bf16 pair made once: W and
// A arrive split from kernel 1; the state slice lives in the registers of the
// wave that owns each 16 x 16 tile and is split into a transposed LDS copy
// after every update; U is split once into a transposed LDS tile, and so is
// (Gamma_C/Gamma) o U from the fp32 U where LDS holds the extra tile (dk =
// 128; with dk = 64 it is formed from the U split where the state update
// reads it).  Per chunk (tiles spread evenly over the waves):
//   U = U0 - W S
//   O = Gamma Q S + A U                (bf16 out)
//   S = Gamma_C S + K^T diag(Gamma_C / Gamma) U   (owner waves, registers)
// The next chunk's operands (K, Q, W, A, U0, cumulative log-decays) are
// fetched into registers at the start of a chunk and stored to LDS after it.
// Workgroups are placed so the slices of one (b, h) share an XCD (block id
// mod 8) and read the chunk operands through one L2.
constexpr int kScanThreads = 512;


template <int DK, int DV, int DVS>
__global__ __launch_bounds__(kScanThreads) void gdn_chunk_scan_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ Wg, const float* __restrict__ U0g, const uint16_t* __restrict__ Ag,
    const float* __restrict__ edg, float* __restrict__ state, uint16_t* __restrict__ out, int T,
    int H, int NC, int n_units) {
  constexpr int NSL = DV / DVS;
  constexpr int NTN = DVS / 16;                  // column tiles of U, O and S
  constexpr int OT = (kC / 16) * NTN / 8;        // U / O tiles per wave
  constexpr int SU = (DK / 16) * NTN / 8;        // state tiles per wave
  constexpr int PB = DK + 8;                     // bf16 pitch of [*][DK] tiles
  constexpr int PT = kC + 8;                     // bf16 pitch of [*][64] tiles
  constexpr int NT = kScanThreads;
  constexpr int KQ_N = kC * DK / 8 / NT;         // uint4 of K (and of Q) per thread
  constexpr int W_N = 2 * kC * DK / 8 / NT;      // uint4 of W (hi and lo planes) per thread
  constexpr int A_N = 2 * kC * kC / 8 / NT;      // uint4 of A (hi and lo planes) per thread
  static_assert(OT >= 1 && SU >= 1 && KQ_N >= 1 && W_N >= 1 && A_N >= 1, "tile split");
  __shared__ __align__(16) uint16_t Whi[kC * PB], Wlo[kC * PB], Qs[kC * PB];
  __shared__ __align__(16) uint16_t Ahi[kC * PT], Alo[kC * PT];
  __shared__ __align__(16) uint16_t KsT[DK * PT];                  // K^T [DK][64]
  __shared__ __align__(16) uint16_t SThi[DVS * PB], STlo[DVS * PB];  // S^T [DVS][DK]
  __shared__ __align__(16) uint16_t UThi[DVS * PT], UTlo[DVS * PT];  // U^T [DVS][64]
  // (dec o U)^T [DVS][64], split once from the fp32 U where it fits: with
  // dk = 64 two workgroups share a CU's LDS and the state update forms it from
  // the U split instead
  constexpr bool kDU = DK == 128;
  __shared__ __align__(16) uint16_t DThi[kDU ? DVS * PT : 8], DTlo[kDU ? DVS * PT : 8];
  // per token: Gamma_t, Gamma_C / Gamma_t (kernel 1), then one slot per thread
  // past them: every thread stores its prefetched value, so no load of the
  // loop is conditional and every wait on one counts a fixed number of
  // memory operations after it
  __shared__ float ecd[NT];
  float* const ecum = ecd;
  float* const dec = ecd + kC;

  const int per_xcd = (gridDim.x + 7) / 8;
  const int unit = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (unit >= n_units) return;
  const int bh = unit / NSL;
  const int sl = unit - bh * NSL;
  const int b = bh / H, h = bh - (bh / H) * H;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g4 = lane >> 4;
  const long long rk = static_cast<long long>(H) * DK, rv = static_cast<long long>(H) * DV;
  float* Sg = state + (static_cast<long long>(bh) * DK) * DV + DVS * sl;

  // ---- the wave's state tiles in registers (D layout: row d = 16 tm + 4 g4 + i, col 16 tn + r16)
  float sreg[SU][4];
#pragma unroll
  for (int u = 0; u < SU; ++u) {
    const int st = SU * wave + u, tm = st / NTN, tn = st % NTN;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      sreg[u][i] = Sg[static_cast<long long>(16 * tm + 4 * g4 + i) * DV + 16 * tn + r16];
  }
  // transposed (hi, lo) copy of the wave's state tiles: S^T[v][d], 4 consecutive d per lane
#define GDN_SPLIT_STATE()                                                                      \
  do {                                                                                         \
    _Pragma("unroll") for (int u = 0; u < SU; ++u) {                                           \
      const int st = SU * wave + u, tm = st / NTN, tn = st % NTN;                              \
      uint16_t hh[4], ll[4];                                                                   \
      _Pragma("unroll") for (int i = 0; i < 4; ++i) {                                          \
        hh[i] = f2bf(sreg[u][i]);                                                              \
        ll[i] = f2bf(sreg[u][i] - bf2f(hh[i]));                                                \
      }                                                                                        \
      const int off = (16 * tn + r16) * PB + 16 * tm + 4 * g4;                                 \
      *reinterpret_cast<uint2*>(SThi + off) = uint2{pack_bf2u(hh[0], hh[1]), pack_bf2u(hh[2], hh[3])}; \
      *reinterpret_cast<uint2*>(STlo + off) = uint2{pack_bf2u(ll[0], ll[1]), pack_bf2u(ll[2], ll[3])}; \
    }                                                                                          \
  } while (0)
  GDN_SPLIT_STATE();

  // ---- prefetch registers (native vectors, so they stay in VGPRs)
  u32x4 pk[KQ_N], pq[KQ_N], pw[W_N], pa[A_N];
  float pu_nxt[OT][4], pu[OT][4], pc;
#define GDN_FETCH(c_)                                                                          \
  do {                                                                                         \
    const int ft0 = (c_) * kC;                                                                 \
    const int fTc = min(kC, T - ft0);                                                          \
    const long long fcid = static_cast<long long>(bh) * NC + (c_);                             \
    const long long fkb = (static_cast<long long>(b) * T + ft0) * rk + static_cast<long long>(h) * DK; \
    _Pragma("unroll") for (int i = 0; i < KQ_N; ++i) {                                         \
      const int f = tid + NT * i;                                                              \
      /* K: token fastest (conflict-free transposed stores); Q: row-major.  Rows past */      \
      /* the chunk re-read its last row (zeroed at the stash) */                               \
      const int tk = f % kC, ck = f / kC;                                                      \
      const int tq = f / (DK / 8), cq = f % (DK / 8);                                          \
      pk[i] = *reinterpret_cast<const u32x4*>(k + fkb + min(tk, fTc - 1) * rk + 8 * ck);       \
      pq[i] = *reinterpret_cast<const u32x4*>(q + fkb + min(tq, fTc - 1) * rk + 8 * cq);       \
    }                                                                                          \
    _Pragma("unroll") for (int i = 0; i < W_N; ++i)                                            \
      pw[i] = *reinterpret_cast<const u32x4*>(Wg + fcid * kC * DK * 2 + 8 * (tid + NT * i));   \
    _Pragma("unroll") for (int i = 0; i < A_N; ++i)                                            \
      pa[i] = *reinterpret_cast<const u32x4*>(Ag + fcid * kC * kC * 2 + 8 * (tid + NT * i));   \
    _Pragma("unroll") for (int ot = 0; ot < OT; ++ot) {                                        \
      const int tt = OT * wave + ot, tm = tt / NTN, tn = tt % NTN;                             \
      _Pragma("unroll") for (int i = 0; i < 4; ++i)                                            \
        pu_nxt[ot][i] = U0g[(fcid * kC + 16 * tm + 4 * g4 + i) * DV + DVS * sl + 16 * tn + r16]; \
    }                                                                                          \
    pc = edg[fcid * 2 * kC + (tid & (2 * kC - 1))];                                            \
  } while (0)
#define GDN_STASH(c_)                                                                          \
  do {                                                                                         \
    const int sTc = min(kC, T - (c_) * kC);                                                    \
    _Pragma("unroll") for (int i = 0; i < KQ_N; ++i) {                                         \
      const int f = tid + NT * i;                                                              \
      const int tk = f % kC, ck = f / kC;                                                      \
      const int tq = f / (DK / 8), cq = f % (DK / 8);                                          \
      if (tk >= sTc) pk[i] = u32x4{0u, 0u, 0u, 0u};                                            \
      *reinterpret_cast<u32x4*>(Qs + tq * PB + 8 * cq) =                                       \
          tq < sTc ? pq[i] : u32x4{0u, 0u, 0u, 0u};                                            \
      _Pragma("unroll") for (int jj = 0; jj < 8; ++jj)                                         \
        KsT[(8 * ck + jj) * PT + tk] = static_cast<uint16_t>(pk[i][jj >> 1] >> (16 * (jj & 1))); \
    }                                                                                          \
    _Pragma("unroll") for (int i = 0; i < W_N; ++i) {                                          \
      const int f = 8 * (tid + NT * i);                                                        \
      const int pl = f / (kC * DK), rem = f % (kC * DK);                                       \
      const int t = rem / DK, cc = rem % DK;                                                   \
      *reinterpret_cast<u32x4*>((pl ? Wlo : Whi) + t * PB + cc) = pw[i];                       \
    }                                                                                          \
    _Pragma("unroll") for (int i = 0; i < A_N; ++i) {                                          \
      const int f = 8 * (tid + NT * i);                                                        \
      const int pl = f / (kC * kC), rem = f % (kC * kC);                                       \
      const int t = rem / kC, cc = rem % kC;                                                   \
      *reinterpret_cast<u32x4*>((pl ? Alo : Ahi) + t * PT + cc) = pa[i];                       \
    }                                                                                          \
    ecd[tid] = pc;                                                                             \
  } while (0)

  GDN_FETCH(0);
  GDN_STASH(0);
#pragma unroll
  for (int ot = 0; ot < OT; ++ot)
#pragma unroll
    for (int i = 0; i < 4; ++i) pu[ot][i] = pu_nxt[ot][i];
  __syncthreads();
  for (int c = 0; c < NC; ++c) {
    const int t0 = c * kC;
    const int Tc = min(kC, T - t0);
    const float gc = ecum[kC - 1];  // Gamma_C (0 when the chunk resets)
    if (c + 1 < NC) GDN_FETCH(c + 1);
    __syncthreads();

    // ---- U = U0 - W S, split once into U^T and (dec o U)^T
#pragma unroll
    for (int ot = 0; ot < OT; ++ot) {
      const int tt = OT * wave + ot, tm = tt / NTN, tn = tt % NTN;
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < DK / 32; ++s) {
        const int ao = (16 * tm + r16) * PB + 32 * s + 8 * g4;
        const int bo = (16 * tn + r16) * PB + 32 * s + 8 * g4;
        const uint4 ah = *reinterpret_cast<const uint4*>(Whi + ao);
        const uint4 al = *reinterpret_cast<const uint4*>(Wlo + ao);
        const uint4 bhv = *reinterpret_cast<const uint4*>(SThi + bo);
        const uint4 blv = *reinterpret_cast<const uint4*>(STlo + bo);
        acc = mfma16(ah, bhv, acc);
        acc = mfma16(ah, blv, acc);
        acc = mfma16(al, bhv, acc);
      }
      uint16_t uh[4], ul[4], dh[4], dl[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float uval = pu[ot][i] - acc[i];
        uh[i] = f2bf(uval);
        ul[i] = f2bf(uval - bf2f(uh[i]));
        if (kDU) {
          const float dval = dec[16 * tm + 4 * g4 + i] * uval;
          dh[i] = f2bf(dval);
          dl[i] = f2bf(dval - bf2f(dh[i]));
        }
      }
      const int off = (16 * tn + r16) * PT + 16 * tm + 4 * g4;
      *reinterpret_cast<uint2*>(UThi + off) = uint2{pack_bf2u(uh[0], uh[1]), pack_bf2u(uh[2], uh[3])};
      *reinterpret_cast<uint2*>(UTlo + off) = uint2{pack_bf2u(ul[0], ul[1]), pack_bf2u(ul[2], ul[3])};
      if (kDU) {
        *reinterpret_cast<uint2*>(DThi + off) = uint2{pack_bf2u(dh[0], dh[1]), pack_bf2u(dh[2], dh[3])};
        *reinterpret_cast<uint2*>(DTlo + off) = uint2{pack_bf2u(dl[0], dl[1]), pack_bf2u(dl[2], dl[3])};
      }
    }
    __syncthreads();  // U^T, (dec o U)^T complete

    // ---- O = Gamma (Q S) + A U, stored through a buffer resource over the
    // chunk's rows of this slice: a token past the chunk lies beyond its range
    // and the store is dropped, so every lane stores (no branch)
    const __amdgpu_buffer_rsrc_t orsrc = __builtin_amdgcn_make_buffer_rsrc(
        out + (static_cast<long long>(b) * T + t0) * rv + static_cast<long long>(h) * DV + DVS * sl,
        static_cast<short>(0), static_cast<int>(((Tc - 1) * rv + DVS) * 2), 0x00020000);
#pragma unroll
    for (int ot = 0; ot < OT; ++ot) {
      const int tt = OT * wave + ot, tm = tt / NTN, tn = tt % NTN;
      f32x4 qs = f32x4{0.f, 0.f, 0.f, 0.f}, au = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < DK / 32; ++s) {
        const uint4 qa = *reinterpret_cast<const uint4*>(Qs + (16 * tm + r16) * PB + 32 * s + 8 * g4);
        const int bo = (16 * tn + r16) * PB + 32 * s + 8 * g4;
        qs = mfma16(qa, *reinterpret_cast<const uint4*>(SThi + bo), qs);
        qs = mfma16(qa, *reinterpret_cast<const uint4*>(STlo + bo), qs);
      }
#pragma unroll
      for (int s = 0; s < kC / 32; ++s) {
        const int ao = (16 * tm + r16) * PT + 32 * s + 8 * g4;
        const int bo = (16 * tn + r16) * PT + 32 * s + 8 * g4;
        const uint4 ah = *reinterpret_cast<const uint4*>(Ahi + ao);
        const uint4 al = *reinterpret_cast<const uint4*>(Alo + ao);
        const uint4 bhv = *reinterpret_cast<const uint4*>(UThi + bo);
        au = mfma16(ah, bhv, au);
        au = mfma16(ah, *reinterpret_cast<const uint4*>(UTlo + bo), au);
        au = mfma16(al, bhv, au);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 16 * tm + 4 * g4 + i;
        const float o = ecum[t] * qs[i] + au[i];
        __builtin_amdgcn_raw_buffer_store_b16(f2bf(o), orsrc,
                                              static_cast<int>((t * rv + 16 * tn + r16) * 2), 0, 0);
      }
    }
    // ---- S = Gamma_C S + K^T (dec o U): the owner wave updates its tiles in registers
#pragma unroll
    for (int u = 0; u < SU; ++u) {
      const int st = SU * wave + u, tm = st / NTN, tn = st % NTN;
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < kC / 32; ++s) {
        const uint4 ka = *reinterpret_cast<const uint4*>(KsT + (16 * tm + r16) * PT + 32 * s + 8 * g4);
        const int bo = (16 * tn + r16) * PT + 32 * s + 8 * g4;
        if (kDU) {
          acc = mfma16(ka, *reinterpret_cast<const uint4*>(DThi + bo), acc);
          acc = mfma16(ka, *reinterpret_cast<const uint4*>(DTlo + bo), acc);
        } else {
          // dec[t] (U_hi + U_lo) for the fragment's 8 tokens, split again
          const uint4 uhv = *reinterpret_cast<const uint4*>(UThi + bo);
          const uint4 ulv = *reinterpret_cast<const uint4*>(UTlo + bo);
          float hf[8], lf[8], dv[8];
          unpack8(uhv, hf);
          unpack8(ulv, lf);
#pragma unroll
          for (int j = 0; j < 8; ++j) dv[j] = dec[32 * s + 8 * g4 + j] * (hf[j] + lf[j]);
          uint4 dhv, dlv;
          split8(dv, dhv, dlv);
          acc = mfma16(ka, dhv, acc);
          acc = mfma16(ka, dlv, acc);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) sreg[u][i] = gc * sreg[u][i] + acc[i];
    }
    __syncthreads();  // every wave is done with this chunk's LDS operands and S^T
    GDN_SPLIT_STATE();
    if (c + 1 < NC) {
      GDN_STASH(c + 1);
#pragma unroll
      for (int ot = 0; ot < OT; ++ot)
#pragma unroll
        for (int i = 0; i < 4; ++i) pu[ot][i] = pu_nxt[ot][i];
    }
    __syncthreads();
  }
#pragma unroll
  for (int u = 0; u < SU; ++u) {
    const int st = SU * wave + u, tm = st / NTN, tn = st % NTN;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      Sg[static_cast<long long>(16 * tm + 4 * g4 + i) * DV + 16 * tn + r16] = sreg[u][i];
  }
#undef GDN_SPLIT_STATE
#undef GDN_FETCH
#undef GDN_STASH
}


// Kernel 2 for dk = dv = 128 (64-column state slices).  Kernel 1 hands over
// T = (I + L)^{-1} (hi, lo planes) and per token Gamma_t, Gamma_C/Gamma_t,
// beta_t, beta_t Gamma_{t-1}, the cumulative log-decay and the segment; this
// kernel forms U and A itself:
//   U = T Y,  Y = beta o V - (beta Gamma_prev) o (K S)      (= U0 - W S)
//   A[t, i] = (Gamma_t / Gamma_i) q_t . k_i for i <= t in t's segment, with
//             kernel 1's arithmetic (the same bits), by the first token
//             half's waves in phase 1b, where they would wait for the
//             second half's causal products
// Wave w owns the 16 x 16 tiles (token tile 2 tp + a, column tile tn), tp = w
// / 4, tn = w % 4, a = 0, 1 (each fragment read from LDS feeds two MFMAs), and
// the state rows 16 w .. 16 w + 15 of the slice (four tiles, in registers):
//   phase 1   K S and Q S on its tiles, then Y, split into the Y^T planes
//   phase 1b  U = T Y on its tiles (T is unit lower triangular, so the first
//             token half skips the second), then, after every read of Y, U^T
//             and (Gamma_C/Gamma o U)^T as (hi, lo) planes
//   phase 2   O = Gamma (Q S) + A U on its tiles (A is causal likewise), and
//             S = Gamma_C S + K^T (dec o U) on its state rows, the K^T
//             fragment (8 tokens of one dim per lane) gathered from the
//             row-major K tile, then the transposed (hi, lo) copy of S for the
//             next chunk
//   then the next chunk's operands go to LDS.
// Every wave does the same work.  The next chunk's K, Q, T and V rows are
// fetched at the start of a chunk, its per-token factors after phase 1,
// so the loads drain behind the MFMAs; every wave issues the same memory
// operations in the same order in every iteration (the last chunk fetches
// itself again), so each wait for a load counts a fixed number of operations
// after it and the loads of the next chunk stay in flight across it.
template <int DK, int DV, int DVS>
__global__ __launch_bounds__(kScanThreads) void gdn_chunk_scan_t_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const uint16_t* __restrict__ Tg,
    const float* __restrict__ facg, float* __restrict__ state, uint16_t* __restrict__ out, int T,
    int H, int NC, int n_units) {
  static_assert(DK == 128 && DVS == 64, "scan: dk = 128, 64-column slices");
  constexpr int NSL = DV / DVS;
  constexpr int PB = DK + 8, PT = kC + 8, PV = DVS + 8, NT = kScanThreads;
  constexpr int KQ_N = kC * DK / 8 / NT;     // uint4 of K (and of Q) per thread
  constexpr int T_N = 2 * kC * kC / 8 / NT;  // uint4 of T (hi and lo planes) per thread
  static_assert(KQ_N == 2 && T_N == 2 && kC * DVS / 8 == NT, "tile split");
  constexpr int NF = 6;  // per-token factors
  static_assert(NF * kC <= NT, "one factor per thread");
  static_assert(NT / 64 == DK / 16, "one 16-row state stripe per wave");
  __shared__ __align__(16) uint16_t Qs[kC * PB], Ks[kC * PB];        // row-major [t][d]
  __shared__ __align__(16) uint16_t Thi[kC * PT], Tlo[kC * PT];      // T [t][i]
  __shared__ __align__(16) uint16_t Ahi[kC * PT], Alo[kC * PT];      // A [t][i]
  __shared__ __align__(16) uint16_t Vs[kC * PV];                     // V slice [t][v]
  __shared__ __align__(16) uint16_t SThi[DVS * PB], STlo[DVS * PB];  // S^T [DVS][DK]
  __shared__ __align__(16) uint16_t UThi[DVS * PT], UTlo[DVS * PT];  // U^T [DVS][64]
  // (dec o U)^T [DVS][64]; Y^T before phase 1b's barrier
  __shared__ __align__(16) uint16_t DThi[DVS * PT], DTlo[DVS * PT];
  // Gamma_t | Gamma_C / Gamma_t | beta_t | beta_t Gamma_{t-1} | cumulative
  // log-decay | segment
  __shared__ float ecd[NF * kC];
  const float* const ecum = ecd;
  const float* const dec = ecd + kC;
  const float* const bet = ecd + 2 * kC;
  const float* const wsc = ecd + 3 * kC;
  const float* const lcum = ecd + 4 * kC;
  const float* const lseg = ecd + 5 * kC;

  const int per_xcd = (gridDim.x + 7) / 8;
  const int unit = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (unit >= n_units) return;
  const int bh = unit / NSL;
  const int sl = unit - bh * NSL;
  const int b = bh / H, h = bh - (bh / H) * H;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tp = wave >> 2, tn = wave & 3;  // tiles (2 tp + a, tn)
  const int r16 = lane & 15, g4 = lane >> 4;
  const long long rk = static_cast<long long>(H) * DK, rv = static_cast<long long>(H) * DV;
  float* Sg = state + (static_cast<long long>(bh) * DK) * DV + DVS * sl;

  // ---- this wave's state rows 16 wave + 4 g4 + i, column tiles c (D layout)
  f32x4 sreg[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      sreg[c][i] = Sg[static_cast<long long>(16 * wave + 4 * g4 + i) * DV + 16 * c + r16];
  auto split_state = [&]() {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      uint16_t hh[4], ll[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        hh[i] = f2bf(sreg[c][i]);
        ll[i] = f2bf(sreg[c][i] - bf2f(hh[i]));
      }
      const int off = (16 * c + r16) * PB + 16 * wave + 4 * g4;
      *reinterpret_cast<uint2*>(SThi + off) = uint2{pack_bf2u(hh[0], hh[1]), pack_bf2u(hh[2], hh[3])};
      *reinterpret_cast<uint2*>(STlo + off) = uint2{pack_bf2u(ll[0], ll[1]), pack_bf2u(ll[2], ll[3])};
    }
  };
  split_state();

  // ---- prefetch registers
  u32x4 pk[KQ_N], pq[KQ_N], pt[T_N], pv;
  float pc;
  auto fetch1 = [&](int c_) {  // K, Q, V rows (past the chunk: its last row again) and T
    const int ft0 = c_ * kC;
    const int fTc = min(kC, T - ft0);
    const long long fcid = static_cast<long long>(bh) * NC + c_;
    const long long fkb = (static_cast<long long>(b) * T + ft0) * rk + static_cast<long long>(h) * DK;
#pragma unroll
    for (int i = 0; i < KQ_N; ++i) {
      const int f = tid + NT * i;
      const int t = f / (DK / 8), cq = f % (DK / 8);
      pk[i] = *reinterpret_cast<const u32x4*>(k + fkb + min(t, fTc - 1) * rk + 8 * cq);
      pq[i] = *reinterpret_cast<const u32x4*>(q + fkb + min(t, fTc - 1) * rk + 8 * cq);
    }
#pragma unroll
    for (int i = 0; i < T_N; ++i)
      pt[i] = *reinterpret_cast<const u32x4*>(Tg + fcid * kC * DK * 2 + 8 * (tid + NT * i));
    const int tv = tid / (DVS / 8), cv = tid % (DVS / 8);
    pv = *reinterpret_cast<const u32x4*>(
        v + (static_cast<long long>(b) * T + ft0 + min(tv, fTc - 1)) * rv +
        static_cast<long long>(h) * DV + DVS * sl + 8 * cv);
  };
  auto fetch2 = [&](int c_) {  // the per-token factors
    const long long fcid = static_cast<long long>(bh) * NC + c_;
    pc = facg[fcid * kC * DV + (tid < NF * kC ? tid : tid - NF * kC)];
  };
  auto stash = [&](int c_) {
    const int sTc = min(kC, T - c_ * kC);
    const u32x4 z = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < KQ_N; ++i) {
      const int f = tid + NT * i;
      const int t = f / (DK / 8), cq = f % (DK / 8);
      *reinterpret_cast<u32x4*>(Qs + t * PB + 8 * cq) = t < sTc ? pq[i] : z;
      *reinterpret_cast<u32x4*>(Ks + t * PB + 8 * cq) = t < sTc ? pk[i] : z;
    }
#pragma unroll
    for (int i = 0; i < T_N; ++i) {
      const int f = 8 * (tid + NT * i);
      const int pl = f / (kC * kC), rem = f % (kC * kC);
      *reinterpret_cast<u32x4*>((pl ? Tlo : Thi) + (rem / kC) * PT + rem % kC) = pt[i];
    }
    {
      const int tv = tid / (DVS / 8), cv = tid % (DVS / 8);
      *reinterpret_cast<u32x4*>(Vs + tv * PV + 8 * cv) = tv < sTc ? pv : z;
    }
    if (tid < NF * kC) ecd[tid] = pc;
  };
  fetch1(0);
  fetch2(0);
  stash(0);
  __syncthreads();
  for (int c = 0; c < NC; ++c) {
    const int t0 = c * kC;
    const int Tc = min(kC, T - t0);
    const float gc = ecum[kC - 1];  // Gamma_C (0 when the chunk resets)
    // the last chunk fetches itself again (never stored), so every iteration
    // issues the same loads and each wait counts the same operations after it
    const int cn = min(c + 1, NC - 1);
    fetch1(cn);

    // ---- phase 1: K S and Q S on tiles (2 tp + a, tn); K and Q exact in bf16
    // this lane's V, beta, beta Gamma_prev (for Y), Gamma_C / Gamma (for the
    // U split) and Gamma (for O), read once per chunk
    float vv[2][4], bt[2][4], ws[2][4], dv[2][4], ev[2][4];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 16 * (2 * tp + a) + 4 * g4 + i;
        vv[a][i] = bf2f(Vs[t * PV + 16 * tn + r16]);
        bt[a][i] = bet[t];
        ws[a][i] = wsc[t];
        dv[a][i] = dec[t];
        ev[a][i] = ecum[t];
      }
    f32x4 ks[2], qs[2];
#pragma unroll
    for (int a = 0; a < 2; ++a) ks[a] = qs[a] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < DK / 32; ++s) {
      uint4 ka[2], qa[2];
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const int ao = (16 * (2 * tp + a) + r16) * PB + 32 * s + 8 * g4;
        ka[a] = *reinterpret_cast<const uint4*>(Ks + ao);
        qa[a] = *reinterpret_cast<const uint4*>(Qs + ao);
      }
      const int bo = (16 * tn + r16) * PB + 32 * s + 8 * g4;
      const uint4 bhv = *reinterpret_cast<const uint4*>(SThi + bo);
      const uint4 blv = *reinterpret_cast<const uint4*>(STlo + bo);
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        ks[a] = mfma16(ka[a], bhv, ks[a]);
        ks[a] = mfma16(ka[a], blv, ks[a]);
        qs[a] = mfma16(qa[a], bhv, qs[a]);
        qs[a] = mfma16(qa[a], blv, qs[a]);
      }
    }
    // Y = beta o V - (beta Gamma_prev) o (K S), split into the Y^T planes
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const int tm = 2 * tp + a;
      uint16_t yh[4], yl[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float y = bt[a][i] * vv[a][i] - ws[a][i] * ks[a][i];
        yh[i] = f2bf(y);
        yl[i] = f2bf(y - bf2f(yh[i]));
      }
      const int off = (16 * tn + r16) * PT + 16 * tm + 4 * g4;
      *reinterpret_cast<uint2*>(DThi + off) = uint2{pack_bf2u(yh[0], yh[1]), pack_bf2u(yh[2], yh[3])};
      *reinterpret_cast<uint2*>(DTlo + off) = uint2{pack_bf2u(yl[0], yl[1]), pack_bf2u(yl[2], yl[3])};
    }
    __syncthreads();  // Y^T complete; every read of S^T done
    fetch2(cn);

    // ---- phase 1b: U = T Y on tiles (2 tp + a, tn)
    f32x4 u[2];
#pragma unroll
    for (int a = 0; a < 2; ++a) u[a] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < kC / 32; ++s) {
      if (s > tp) break;  // T is lower triangular: tokens 0..31 see no later token
      uint4 th[2], tl[2];
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const int ao = (16 * (2 * tp + a) + r16) * PT + 32 * s + 8 * g4;
        th[a] = *reinterpret_cast<const uint4*>(Thi + ao);
        tl[a] = *reinterpret_cast<const uint4*>(Tlo + ao);
      }
      const int bo = (16 * tn + r16) * PT + 32 * s + 8 * g4;
      const uint4 yhv = *reinterpret_cast<const uint4*>(DThi + bo);
      const uint4 ylv = *reinterpret_cast<const uint4*>(DTlo + bo);
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        u[a] = mfma16(th[a], yhv, u[a]);
        u[a] = mfma16(th[a], ylv, u[a]);
        u[a] = mfma16(tl[a], yhv, u[a]);
      }
    }
    if (tp == 0) {  // uniform
      // A in the first token half's slack (its T Y covers half the tokens):
      // wave tn forms the tiles (tn / 2, tn % 2), (2 + tn / 2, tn % 2) and
      // (2 + tn / 2, 2 + tn % 2) of A's K Q^T, every tile phase 2 reads
      f32x4 a0 = f32x4{0.f, 0.f, 0.f, 0.f}, a1 = a0, a2 = a0;
      const uint16_t* const k0 = Ks + (16 * (tn & 1) + r16) * PB + 8 * g4;
      const uint16_t* const q0 = Qs + (16 * (tn >> 1) + r16) * PB + 8 * g4;
#pragma unroll
      for (int s = 0; s < DK / 32; ++s) {
        const uint4 kv0 = *reinterpret_cast<const uint4*>(k0 + 32 * s);
        const uint4 kv1 = *reinterpret_cast<const uint4*>(k0 + 32 * PB + 32 * s);
        const uint4 qv0 = *reinterpret_cast<const uint4*>(q0 + 32 * s);
        const uint4 qv1 = *reinterpret_cast<const uint4*>(q0 + 32 * PB + 32 * s);
        a0 = mfma16(kv0, qv0, a0);
        a1 = mfma16(kv0, qv1, a1);
        a2 = mfma16(kv1, qv1, a2);
      }
      // A[t, j] = (Gamma_t / Gamma_j) q_t . k_j for j <= t in t's segment, as
      // (hi, lo) planes; the lane holds row t = 16 ti + r16, columns j = 16 tj +
      // 4 g4 + i (kernel 1's arithmetic, so the same bits)
      auto store_a = [&](const f32x4& acc, int ti, int tj) {
        const int t = 16 * ti + r16, j0 = 16 * tj + 4 * g4;
        const float acum = lcum[t], aseg = lseg[t];
        // the column factors read unconditionally, the mask applied by select
        const float4 cj = *reinterpret_cast<const float4*>(lcum + j0);
        const float4 sj = *reinterpret_cast<const float4*>(lseg + j0);
        const float cjv[4] = {cj.x, cj.y, cj.z, cj.w}, sjv[4] = {sj.x, sj.y, sj.z, sj.w};
        uint16_t hv[4], lv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int j = j0 + i;
          const float ex = __expf(acum - cjv[i]) * acc[i];
          const float am = (j <= t) & (sjv[i] == aseg) ? ex : 0.f;
          hv[i] = f2bf(am);
          lv[i] = f2bf(am - bf2f(hv[i]));
        }
        *reinterpret_cast<uint2*>(Ahi + t * PT + j0) =
            make_uint2(pack_bf2u(hv[0], hv[1]), pack_bf2u(hv[2], hv[3]));
        *reinterpret_cast<uint2*>(Alo + t * PT + j0) =
            make_uint2(pack_bf2u(lv[0], lv[1]), pack_bf2u(lv[2], lv[3]));
      };
      store_a(a0, tn >> 1, tn & 1);
      store_a(a1, 2 + (tn >> 1), tn & 1);
      store_a(a2, 2 + (tn >> 1), 2 + (tn & 1));
    }
    __syncthreads();  // every read of Y^T done; A complete
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const int tm = 2 * tp + a;
      uint16_t uh[4], ul[4], dh[4], dl[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float uval = u[a][i];
        uh[i] = f2bf(uval);
        ul[i] = f2bf(uval - bf2f(uh[i]));
        const float dval = dv[a][i] * uval;
        dh[i] = f2bf(dval);
        dl[i] = f2bf(dval - bf2f(dh[i]));
      }
      const int off = (16 * tn + r16) * PT + 16 * tm + 4 * g4;
      *reinterpret_cast<uint2*>(UThi + off) = uint2{pack_bf2u(uh[0], uh[1]), pack_bf2u(uh[2], uh[3])};
      *reinterpret_cast<uint2*>(UTlo + off) = uint2{pack_bf2u(ul[0], ul[1]), pack_bf2u(ul[2], ul[3])};
      *reinterpret_cast<uint2*>(DThi + off) = uint2{pack_bf2u(dh[0], dh[1]), pack_bf2u(dh[2], dh[3])};
      *reinterpret_cast<uint2*>(DTlo + off) = uint2{pack_bf2u(dl[0], dl[1]), pack_bf2u(dl[2], dl[3])};
    }
    __syncthreads();  // U^T and (dec o U)^T complete

    // ---- phase 2: O on tiles (2 tp + a, tn); output rows past the chunk lie
    // beyond the buffer range (the hardware drops those stores)
    {
      const __amdgpu_buffer_rsrc_t orsrc = __builtin_amdgcn_make_buffer_rsrc(
          out + (static_cast<long long>(b) * T + t0) * rv + static_cast<long long>(h) * DV + DVS * sl,
          static_cast<short>(0), static_cast<int>(((Tc - 1) * rv + DVS) * 2), 0x00020000);
      f32x4 au[2];
#pragma unroll
      for (int a = 0; a < 2; ++a) au[a] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < kC / 32; ++s) {
        if (s > tp) break;  // A is causal: tokens 0..31 see no later token
        uint4 ah[2], al[2];
#pragma unroll
        for (int a = 0; a < 2; ++a) {
          const int ao = (16 * (2 * tp + a) + r16) * PT + 32 * s + 8 * g4;
          ah[a] = *reinterpret_cast<const uint4*>(Ahi + ao);
          al[a] = *reinterpret_cast<const uint4*>(Alo + ao);
        }
        const int bo = (16 * tn + r16) * PT + 32 * s + 8 * g4;
        const uint4 uhv = *reinterpret_cast<const uint4*>(UThi + bo);
        const uint4 ulv = *reinterpret_cast<const uint4*>(UTlo + bo);
#pragma unroll
        for (int a = 0; a < 2; ++a) {
          au[a] = mfma16(ah[a], uhv, au[a]);
          au[a] = mfma16(ah[a], ulv, au[a]);
          au[a] = mfma16(al[a], uhv, au[a]);
        }
      }
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = 16 * (2 * tp + a) + 4 * g4 + i;
          const float o = ev[a][i] * qs[a][i] + au[a][i];
          __builtin_amdgcn_raw_buffer_store_b16(
              f2bf(o), orsrc, static_cast<int>((t * rv + 16 * tn + r16) * 2), 0, 0);
        }
    }
    // ---- phase 2: S = Gamma_C S + K^T (dec o U) on state rows 16 wave ..,
    // accumulated onto the decayed state in place
#pragma unroll
    for (int cc = 0; cc < 4; ++cc)
#pragma unroll
      for (int i = 0; i < 4; ++i) sreg[cc][i] *= gc;
#pragma unroll
    for (int s = 0; s < kC / 32; ++s) {
      const uint16_t* kc = Ks + (32 * s + 8 * g4) * PB + 16 * wave + r16;
      uint16_t e[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) e[j] = kc[j * PB];
      const uint4 ka = uint4{pack_bf2u(e[0], e[1]), pack_bf2u(e[2], e[3]), pack_bf2u(e[4], e[5]),
                             pack_bf2u(e[6], e[7])};
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) {
        const int bo = (16 * cc + r16) * PT + 32 * s + 8 * g4;
        sreg[cc] = mfma16(ka, *reinterpret_cast<const uint4*>(DThi + bo), sreg[cc]);
        sreg[cc] = mfma16(ka, *reinterpret_cast<const uint4*>(DTlo + bo), sreg[cc]);
      }
    }
    split_state();
    __syncthreads();  // every wave is done with this chunk's LDS operands; S^T updated
    if (c + 1 < NC) {
      stash(c + 1);
      __syncthreads();
    }
  }
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      Sg[static_cast<long long>(16 * wave + 4 * g4 + i) * DV + 16 * c + r16] = sreg[c][i];
}

}  // namespace llmy

using namespace llmy;

extern "C" int64_t llmy_gdn_prefill_workspace_bytes(int32_t B, int32_t T, int32_t H, int32_t dk,
                                                    int32_t dv) {
  if (B <= 0 || T <= 0 || H <= 0 || dk <= 0 || dv <= 0) return 0;
  const long long nc = (T + kC - 1) / kC;
  const long long chunks = static_cast<long long>(B) * H * nc;
  return chunks * kC * (static_cast<long long>(dk) + dv + kC + 2) * static_cast<long long>(sizeof(float));
}

namespace {

// The prep + scan launches over a caller-sized workspace (validated by the
// entry points below).
// Compute units of the current device (queried once per process).
int device_cus() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cus = n;
  }
  return cus;
}

int32_t gdn_prefill_launch(const llmy_bf16* q, const llmy_bf16* k, const llmy_bf16* v,
                           const float* beta, const float* g, const int32_t* reset, float* state,
                           llmy_bf16* out, void* workspace, int B, int T, int H, int dk,
                           hipStream_t s) {
  const int NC = (T + kC - 1) / kC;
  const long long chunks = static_cast<long long>(B) * H * NC;
  const int dv = dk;
  // workspace, per chunk: W as (hi, lo) bf16 planes, U0 fp32, A as (hi, lo)
  // bf16 planes, decay factors [2][64] fp32.  dk = 128 uses the W slot for T
  // = (I + L)^{-1} ((hi, lo) [2][64][64]) and the U0 slot for the per-token
  // factors [6][64]; its A and decay-factor slots are unused.
  uint16_t* W = static_cast<uint16_t*>(workspace);
  float* U0 = reinterpret_cast<float*>(W + chunks * kC * dk * 2);
  uint16_t* A = reinterpret_cast<uint16_t*>(U0 + chunks * kC * dv);
  float* ed = reinterpret_cast<float*>(A + chunks * kC * kC * 2);
  // persistent prep workgroups: two per CU (the kernel is built for two waves
  // per SIMD), each taking every grid-th chunk
  const int nch = static_cast<int>(chunks);
  if (dk == 64) {
    const int grid = static_cast<int>(std::min<long long>(chunks, 2ll * device_cus()));
    hipLaunchKernelGGL((gdn_chunk_prep_kernel<64, 64>), dim3(static_cast<unsigned>(grid)),
                       dim3(256), 0, s, q, k, v, beta, g, reset, W, U0, A, ed, T, H, NC, nch);
    int32_t st = launch_status();
    if (st != 0) return st;
    const int units = B * H * (64 / 32);
    hipLaunchKernelGGL((gdn_chunk_scan_kernel<64, 64, 32>), dim3((units + 7) / 8 * 8),
                       dim3(kScanThreads), 0, s, q, k, W, U0, A, ed, state, out, T, H, NC, units);
  } else {
    const int grid = static_cast<int>(std::min<long long>(chunks, 2ll * device_cus()));
    hipLaunchKernelGGL((gdn_chunk_prep_kernel<128, 128>), dim3(static_cast<unsigned>(grid)),
                       dim3(256), 0, s, q, k, v, beta, g, reset, W, U0, A, ed, T, H, NC, nch);
    int32_t st = launch_status();
    if (st != 0) return st;
    const int units = B * H * (128 / 64);
    // dk = 128: W's slot holds T, U0's slot the per-token factors
    hipLaunchKernelGGL((gdn_chunk_scan_t_kernel<128, 128, 64>), dim3((units + 7) / 8 * 8),
                       dim3(kScanThreads), 0, s, q, k, v, W, U0, state, out, T, H, NC, units);
  }
  return launch_status();
}

// Workspace of the no-allocation entry point: a fixed device array, one copy
// per GPU (each device holds it from module load until the process ends).
// Host code never passes `scratch` itself (in host code the name is a
// stand-in, not a device address): the per-device address comes from
// hipGetSymbolAddress, once per device, with that device current.
constexpr long long kStaticWorkspaceBytes = 64ll << 20;
__device__ __align__(256) unsigned char scratch[kStaticWorkspaceBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's copy of `scratch` (null on failure).
void* static_workspace() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
      (void)hipGetLastError();
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" int32_t llmy_gdn_prefill_bf16(const llmy_bf16* q, const llmy_bf16* k,
                                         const llmy_bf16* v, const float* beta, const float* g,
                                         float* state, llmy_bf16* out, void* workspace,
                                         int64_t workspace_bytes, int32_t B, int32_t T,
                                         int32_t H, int32_t dk, int32_t dv, void* stream) {
  LLMY_REQUIRE(B >= 0 && T >= 0 && H > 0);
  LLMY_REQUIRE((dk == 64 && dv == 64) || (dk == 128 && dv == 128));
  if (B == 0 || T == 0) return 0;
  LLMY_REQUIRE(q && k && v && beta && g && state && out && workspace);
  LLMY_REQUIRE(workspace_bytes >= llmy_gdn_prefill_workspace_bytes(B, T, H, dk, dv));
  LLMY_REQUIRE(aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && aligned(state, 16) &&
               aligned(workspace, 16));
  const long long chunks = static_cast<long long>(B) * H * ((T + kC - 1) / kC);
  LLMY_REQUIRE(chunks < (1ll << 31));
  return gdn_prefill_launch(q, k, v, beta, g, nullptr, state, out, workspace, B, T, H, dk,
                            as_stream(stream));
}

extern "C" int32_t llmy_gdn_prefill_reset_bf16(const llmy_bf16* q, const llmy_bf16* k,
                                               const llmy_bf16* v, const float* beta,
                                               const float* g, const int32_t* reset, float* state,
                                               llmy_bf16* out, void* workspace,
                                               int64_t workspace_bytes, int32_t B, int32_t T,
                                               int32_t H, int32_t dk, int32_t dv, void* stream) {
  LLMY_REQUIRE(B >= 0 && T >= 0 && H > 0);
  LLMY_REQUIRE((dk == 64 && dv == 64) || (dk == 128 && dv == 128));
  if (B == 0 || T == 0) return 0;
  LLMY_REQUIRE(q && k && v && beta && g && reset && state && out && workspace);
  LLMY_REQUIRE(workspace_bytes >= llmy_gdn_prefill_workspace_bytes(B, T, H, dk, dv));
  LLMY_REQUIRE(aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && aligned(state, 16) &&
               aligned(workspace, 16));
  const long long chunks = static_cast<long long>(B) * H * ((T + kC - 1) / kC);
  LLMY_REQUIRE(chunks < (1ll << 31));
  return gdn_prefill_launch(q, k, v, beta, g, reset, state, out, workspace, B, T, H, dk,
                            as_stream(stream));
}

extern "C" int32_t llmy_gdn_prefill_bf16_noalloc(const llmy_bf16* q, const llmy_bf16* k,
                                                 const llmy_bf16* v, const float* beta,
                                                 const float* g, float* state, llmy_bf16* out,
                                                 int32_t B, int32_t T, int32_t H, int32_t dk,
                                                 int32_t dv, void* stream) {
  LLMY_REQUIRE(B >= 0 && T >= 0 && H > 0);
  LLMY_REQUIRE((dk == 64 && dv == 64) || (dk == 128 && dv == 128));
  if (B == 0 || T == 0) return 0;
  LLMY_REQUIRE(q && k && v && beta && g && state && out);
  LLMY_REQUIRE(aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && aligned(state, 16));
  // beyond the fixed workspace: a distinct status, before anything runs
  if (llmy_gdn_prefill_workspace_bytes(B, T, H, dk, dv) > kStaticWorkspaceBytes)
    return static_cast<int32_t>(hipErrorOutOfMemory);
  void* ws = static_workspace();
  if (!ws) return static_cast<int32_t>(hipErrorInvalidDevicePointer);
  // every workspace byte the scan reads is written by this call's prep kernel
  // first, so what an earlier call left there does not matter
  return gdn_prefill_launch(q, k, v, beta, g, nullptr, state, out, ws, B, T, H, dk,
                            as_stream(stream));
}
