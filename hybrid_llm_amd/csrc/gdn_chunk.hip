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
// accumulation fp32), the unit lower-triangular inverse by per-column forward
// substitution in fp32, then W, U0 (written as fp32), A and the cumulative
// log-decays.  Kernel 2 (gdn_chunk_scan) runs once per (b, h, 32-column slice
// of the state), sequentially over the chunks with the state slice in LDS.
// Every product with an fp32 operand uses split-bf16 MFMA: x = hi + lo with
// hi = bf16(x), lo = bf16(x - hi), keeping hi*hi + hi*lo + lo*hi (relative
// error about 2^-16); products of two bf16 tensors are exact.
//
// MFMA v_mfma_f32_16x16x32_bf16 fragments: A lane l holds A[l%16][8(l/16)+j],
// B lane l holds B[8(l/16)+j][l%16], D lane l holds D[4(l/16)+i][l%16].
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

__device__ __forceinline__ f32x4 mfma16(const uint4& a, const uint4& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Kernel 1: per-chunk preparation.  Scratch layout per chunk id
// cid = (b*H + h) * NC + c:  W [64][DK], U0 [64][DV], A [64][64], cum [64] (fp32).
template <int DK, int DV>
__global__ __launch_bounds__(256) void gdn_chunk_prep_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const float* __restrict__ beta,
    const float* __restrict__ g, float* __restrict__ Wg, float* __restrict__ U0g,
    float* __restrict__ Ag, float* __restrict__ cumg, int T, int H, int NC) {
  constexpr int PK = DK + 8, PV = DV + 8, PG = kC + 1;
  __shared__ __align__(16) uint16_t Ks[kC * PK];
  __shared__ __align__(16) uint16_t Qs[kC * PK];
  __shared__ __align__(16) uint16_t Vs[kC * PV];
  __shared__ float Gm[kC * PG];   // K K^T, then L
  __shared__ float Qk[kC * PG];   // Q K^T
  __shared__ float Ti[kC * PG];   // (I + L)^{-1}
  __shared__ float cum[kC], prv[kC], bet[kC], wsc[kC];  // wsc = beta * Gamma_prev

  const int cid = blockIdx.x;
  const int bh = cid / NC;
  const int c = cid - bh * NC;
  const int b = bh / H, h = bh - (bh / H) * H;
  const int t0 = c * kC;
  const int Tc = min(kC, T - t0);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r16 = lane & 15, g4 = lane >> 4;
  const long long rk = static_cast<long long>(H) * DK, rv = static_cast<long long>(H) * DV;
  const long long kbase = (static_cast<long long>(b) * T + t0) * rk + static_cast<long long>(h) * DK;
  const long long vbase = (static_cast<long long>(b) * T + t0) * rv + static_cast<long long>(h) * DV;

  // ---- stage K, Q (DK) and V (DV) rows; padded rows are zero
  for (int f = threadIdx.x; f < kC * (DK / 8); f += 256) {
    const int t = f / (DK / 8), cc = f - t * (DK / 8);
    uint4 kv = uint4{0u, 0u, 0u, 0u}, qv = uint4{0u, 0u, 0u, 0u};
    if (t < Tc) {
      kv = *reinterpret_cast<const uint4*>(k + kbase + t * rk + 8 * cc);
      qv = *reinterpret_cast<const uint4*>(q + kbase + t * rk + 8 * cc);
    }
    *reinterpret_cast<uint4*>(Ks + t * PK + 8 * cc) = kv;
    *reinterpret_cast<uint4*>(Qs + t * PK + 8 * cc) = qv;
  }
  for (int f = threadIdx.x; f < kC * (DV / 8); f += 256) {
    const int t = f / (DV / 8), cc = f - t * (DV / 8);
    uint4 vv = uint4{0u, 0u, 0u, 0u};
    if (t < Tc) vv = *reinterpret_cast<const uint4*>(v + vbase + t * rv + 8 * cc);
    *reinterpret_cast<uint4*>(Vs + t * PV + 8 * cc) = vv;
  }
  if (wave == 0) {
    // inclusive prefix sum of log g over the chunk (padded tokens: g = 1, beta = 0)
    const long long gi = (static_cast<long long>(b) * T + t0 + min(lane, Tc - 1)) * H + h;
    float lg = lane < Tc ? logf(g[gi]) : 0.f;
    const float bt = lane < Tc ? beta[gi] : 0.f;
    float sc = lg;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float o = __shfl_up(sc, off, kWave);
      if (lane >= off) sc += o;
    }
    cum[lane] = sc;
    prv[lane] = sc - lg;
    bet[lane] = bt;
    wsc[lane] = bt * expf(sc - lg);
  }
  __syncthreads();

  // ---- K K^T and Q K^T (exact): wave w owns output row block w, 4 column blocks
#pragma unroll
  for (int tj = 0; tj < 4; ++tj) {
    f32x4 a1 = f32x4{0.f, 0.f, 0.f, 0.f}, a2 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < DK / 32; ++s) {
      const uint4 ka = *reinterpret_cast<const uint4*>(Ks + (16 * wave + r16) * PK + 32 * s + 8 * g4);
      const uint4 qa = *reinterpret_cast<const uint4*>(Qs + (16 * wave + r16) * PK + 32 * s + 8 * g4);
      const uint4 kb = *reinterpret_cast<const uint4*>(Ks + (16 * tj + r16) * PK + 32 * s + 8 * g4);
      a1 = mfma16(ka, kb, a1);
      a2 = mfma16(qa, kb, a2);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * wave + 4 * g4 + i, j = 16 * tj + r16;
      Gm[t * PG + j] = a1[i];
      Qk[t * PG + j] = a2[i];
    }
  }
  __syncthreads();
  // ---- L (strictly lower) and A = M o Q K^T (lower incl. diagonal)
  for (int e = threadIdx.x; e < kC * kC; e += 256) {
    const int t = e >> 6, i = e & 63;
    const float l = i < t ? bet[t] * expf(prv[t] - cum[i]) * Gm[t * PG + i] : 0.f;
    Gm[t * PG + i] = l;
    const float am = i <= t ? expf(cum[t] - cum[i]) * Qk[t * PG + i] : 0.f;
    Qk[t * PG + i] = am;
  }
  __syncthreads();
  // ---- (I + L)^{-1} by forward substitution; lane j of wave 0 owns column j
  if (wave == 0) {
    const int j = lane;
    for (int t = 0; t < kC; ++t) {
      float a0 = (t == j) ? 1.f : 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
      int i = j;
      for (; i + 3 < t; i += 4) {
        a0 -= Gm[t * PG + i] * Ti[i * PG + j];
        a1 -= Gm[t * PG + i + 1] * Ti[(i + 1) * PG + j];
        a2 -= Gm[t * PG + i + 2] * Ti[(i + 2) * PG + j];
        a3 -= Gm[t * PG + i + 3] * Ti[(i + 3) * PG + j];
      }
      for (; i < t; ++i) a0 -= Gm[t * PG + i] * Ti[i * PG + j];
      Ti[t * PG + j] = t < j ? 0.f : (a0 + a1) + (a2 + a3);
    }
  }
  __syncthreads();

  // ---- W = Ti diag(beta Gamma_prev) K  [64 x DK],  U0 = Ti diag(beta) V  [64 x DV]
  const long long wo = static_cast<long long>(cid) * kC;
  {
    constexpr int NT = 4 * (DK / 16) + 4 * (DV / 16);  // output tiles of both products
    for (int tile = wave; tile < NT; tile += 4) {
      const bool isW = tile < 4 * (DK / 16);
      const int tt = isW ? tile : tile - 4 * (DK / 16);
      const int nd = isW ? DK / 16 : DV / 16;
      const int tm = tt / nd, tn = tt - (tt / nd) * nd;
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < kC / 32; ++s) {
        float av[8];
        const int row = 16 * tm + r16;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
          const int i = 32 * s + 8 * g4 + jj;
          const float sc = isW ? wsc[i] : bet[i];
          av[jj] = Ti[row * PG + i] * sc;
        }
        uint4 ahi, alo;
        split8(av, ahi, alo);
        const uint4 bb = isW ? gather8_bf16(Ks + (32 * s + 8 * g4) * PK + 16 * tn + r16, PK)
                             : gather8_bf16(Vs + (32 * s + 8 * g4) * PV + 16 * tn + r16, PV);
        acc = mfma16(ahi, bb, acc);
        acc = mfma16(alo, bb, acc);
      }
      float* dst = isW ? Wg + wo * DK : U0g + wo * DV;
      const int ld = isW ? DK : DV;
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[(16 * tm + 4 * g4 + i) * ld + 16 * tn + r16] = acc[i];
    }
  }
  for (int e = threadIdx.x; e < kC * kC; e += 256)
    Ag[wo * kC + e] = Qk[(e >> 6) * PG + (e & 63)];
  if (threadIdx.x < kC) cumg[wo + threadIdx.x] = cum[threadIdx.x];
}

// ---------------------------------------------------------------------------
// Kernel 2: sequential scan over chunks for one (b, h, 32-column state slice).
template <int DK, int DV>
__global__ __launch_bounds__(256) void gdn_chunk_scan_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const float* __restrict__ Wg, const float* __restrict__ U0g, const float* __restrict__ Ag,
    const float* __restrict__ cumg, float* __restrict__ state, uint16_t* __restrict__ out, int T,
    int H, int NC) {
  constexpr int DVS = 32;                 // state columns per workgroup
  constexpr int NSL = DV / DVS;
  constexpr int PK = DK + 8, PW = DK + 4, PS = DVS + 4, PG = kC + 1;
  __shared__ __align__(16) float Ss[DK * PS];     // state slice [DK][DVS]
  __shared__ __align__(16) float Us[kC * PS];     // U [64][DVS]
  __shared__ __align__(16) float Ws[kC * PW];     // W [64][DK]
  __shared__ __align__(16) uint16_t Qs[kC * PK];
  __shared__ __align__(16) uint16_t Ks[kC * PK];
  __shared__ float As[kC * PG];
  __shared__ float cum[kC], ecum[kC], dec[kC];  // cum, Gamma_t, Gamma_C / Gamma_t

  const int bh = blockIdx.x / NSL;
  const int sl = blockIdx.x - bh * NSL;
  const int b = bh / H, h = bh - (bh / H) * H;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r16 = lane & 15, g4 = lane >> 4;
  const long long rk = static_cast<long long>(H) * DK, rv = static_cast<long long>(H) * DV;
  float* Sg = state + (static_cast<long long>(bh) * DK) * DV + DVS * sl;

  for (int e = threadIdx.x; e < DK * DVS; e += 256) {
    const int d = e / DVS, cc = e - (e / DVS) * DVS;
    Ss[d * PS + cc] = Sg[static_cast<long long>(d) * DV + cc];
  }

  for (int c = 0; c < NC; ++c) {
    const int t0 = c * kC;
    const int Tc = min(kC, T - t0);
    const long long cid = static_cast<long long>(bh) * NC + c;
    const long long kbase = (static_cast<long long>(b) * T + t0) * rk + static_cast<long long>(h) * DK;
    __syncthreads();  // previous chunk finished with every LDS buffer
    for (int f = threadIdx.x; f < kC * (DK / 8); f += 256) {
      const int t = f / (DK / 8), cc = f - t * (DK / 8);
      uint4 kv = uint4{0u, 0u, 0u, 0u}, qv = uint4{0u, 0u, 0u, 0u};
      if (t < Tc) {
        kv = *reinterpret_cast<const uint4*>(k + kbase + t * rk + 8 * cc);
        qv = *reinterpret_cast<const uint4*>(q + kbase + t * rk + 8 * cc);
      }
      *reinterpret_cast<uint4*>(Ks + t * PK + 8 * cc) = kv;
      *reinterpret_cast<uint4*>(Qs + t * PK + 8 * cc) = qv;
    }
    for (int f = threadIdx.x; f < kC * (DK / 4); f += 256) {
      const int t = f / (DK / 4), cc = f - t * (DK / 4);
      *reinterpret_cast<float4*>(Ws + t * PW + 4 * cc) =
          *reinterpret_cast<const float4*>(Wg + (cid * kC + t) * DK + 4 * cc);
    }
    for (int e = threadIdx.x; e < kC * kC; e += 256)
      As[(e >> 6) * PG + (e & 63)] = Ag[cid * kC * kC + e];
    if (threadIdx.x < kC) {
      const float cv = cumg[cid * kC + threadIdx.x];
      const float cl_ = cumg[cid * kC + kC - 1];
      cum[threadIdx.x] = cv;
      ecum[threadIdx.x] = expf(cv);
      dec[threadIdx.x] = expf(cl_ - cv);
    }
    __syncthreads();

    // ---- U = U0 - W S   [64 x DVS]: 8 tiles of 16x16, 2 per wave
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int tile = 2 * wave + u;
      const int tm = tile >> 1, tn = tile & 1;
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < DK / 32; ++s) {
        uint4 ahi, alo, bhi, blo;
        split8(Ws + (16 * tm + r16) * PW + 32 * s + 8 * g4, ahi, alo);
        float bv[8];
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) bv[jj] = Ss[(32 * s + 8 * g4 + jj) * PS + 16 * tn + r16];
        split8(bv, bhi, blo);
        acc = mfma16(ahi, bhi, acc);
        acc = mfma16(ahi, blo, acc);
        acc = mfma16(alo, bhi, acc);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 16 * tm + 4 * g4 + i, cc = 16 * tn + r16;
        Us[t * PS + cc] = U0g[(cid * kC + t) * DV + DVS * sl + cc] - acc[i];
      }
    }
    __syncthreads();

    // ---- O = Gamma (Q S) + A U  [64 x DVS]; and S' = Gamma_C S + K^T diag(Gamma_C/Gamma) U
    const float cl = cum[kC - 1];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int tile = 2 * wave + u;
      const int tm = tile >> 1, tn = tile & 1;
      f32x4 qs = f32x4{0.f, 0.f, 0.f, 0.f}, au = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < DK / 32; ++s) {
        const uint4 qa = *reinterpret_cast<const uint4*>(Qs + (16 * tm + r16) * PK + 32 * s + 8 * g4);
        float bv[8];
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) bv[jj] = Ss[(32 * s + 8 * g4 + jj) * PS + 16 * tn + r16];
        uint4 bhi, blo;
        split8(bv, bhi, blo);
        qs = mfma16(qa, bhi, qs);
        qs = mfma16(qa, blo, qs);
      }
#pragma unroll
      for (int s = 0; s < kC / 32; ++s) {
        uint4 ahi, alo, bhi, blo;
        float av[8], bv[8];
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
          av[jj] = As[(16 * tm + r16) * PG + 32 * s + 8 * g4 + jj];
          bv[jj] = Us[(32 * s + 8 * g4 + jj) * PS + 16 * tn + r16];
        }
        split8(av, ahi, alo);
        split8(bv, bhi, blo);
        au = mfma16(ahi, bhi, au);
        au = mfma16(ahi, blo, au);
        au = mfma16(alo, bhi, au);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 16 * tm + 4 * g4 + i;
        if (t < Tc) {
          const float o = ecum[t] * qs[i] + au[i];
          out[(static_cast<long long>(b) * T + t0 + t) * rv + static_cast<long long>(h) * DV +
              DVS * sl + 16 * tn + r16] = f2bf(o);
        }
      }
    }
    // state update: [DK x DVS] = 16 tiles, 4 per wave; A = K^T (exact), B = diag(.) U (split)
    f32x4 sacc[4];
    float sold[4][4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int tile = 4 * wave + u;
      const int tm = tile >> 1, tn = tile & 1;
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < kC / 32; ++s) {
        const uint4 ka = gather8_bf16(Ks + (32 * s + 8 * g4) * PK + 16 * tm + r16, PK);
        float bv[8];
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
          const int t = 32 * s + 8 * g4 + jj;
          bv[jj] = dec[t] * Us[t * PS + 16 * tn + r16];
        }
        uint4 bhi, blo;
        split8(bv, bhi, blo);
        acc = mfma16(ka, bhi, acc);
        acc = mfma16(ka, blo, acc);
      }
      sacc[u] = acc;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        sold[u][i] = Ss[(16 * tm + 4 * g4 + i) * PS + 16 * tn + r16];
    }
    __syncthreads();  // every wave has read S for this chunk
    const float gc = expf(cl);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int tile = 4 * wave + u;
      const int tm = tile >> 1, tn = tile & 1;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        Ss[(16 * tm + 4 * g4 + i) * PS + 16 * tn + r16] = gc * sold[u][i] + sacc[u][i];
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < DK * DVS; e += 256) {
    const int d = e / DVS, cc = e - (e / DVS) * DVS;
    Sg[static_cast<long long>(d) * DV + cc] = Ss[d * PS + cc];
  }
}

}  // namespace llmy

using namespace llmy;

extern "C" int64_t llmy_gdn_prefill_workspace_bytes(int32_t B, int32_t T, int32_t H, int32_t dk,
                                                    int32_t dv) {
  if (B <= 0 || T <= 0 || H <= 0 || dk <= 0 || dv <= 0) return 0;
  const long long nc = (T + kC - 1) / kC;
  const long long chunks = static_cast<long long>(B) * H * nc;
  return chunks * kC * (static_cast<long long>(dk) + dv + kC + 1) * static_cast<long long>(sizeof(float));
}

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
  const int NC = (T + kC - 1) / kC;
  const long long chunks = static_cast<long long>(B) * H * NC;
  LLMY_REQUIRE(chunks < (1ll << 31));
  float* W = static_cast<float*>(workspace);
  float* U0 = W + chunks * kC * dk;
  float* A = U0 + chunks * kC * dv;
  float* cum = A + chunks * kC * kC;
  const hipStream_t s = as_stream(stream);
  if (dk == 64) {
    hipLaunchKernelGGL((gdn_chunk_prep_kernel<64, 64>), dim3(static_cast<unsigned>(chunks)),
                       dim3(256), 0, s, q, k, v, beta, g, W, U0, A, cum, T, H, NC);
    int32_t st = launch_status();
    if (st != 0) return st;
    hipLaunchKernelGGL((gdn_chunk_scan_kernel<64, 64>), dim3(B * H * (64 / 32)), dim3(256), 0, s,
                       q, k, W, U0, A, cum, state, out, T, H, NC);
  } else {
    hipLaunchKernelGGL((gdn_chunk_prep_kernel<128, 128>), dim3(static_cast<unsigned>(chunks)),
                       dim3(256), 0, s, q, k, v, beta, g, W, U0, A, cum, T, H, NC);
    int32_t st = launch_status();
    if (st != 0) return st;
    hipLaunchKernelGGL((gdn_chunk_scan_kernel<128, 128>), dim3(B * H * (128 / 32)), dim3(256), 0,
                       s, q, k, W, U0, A, cum, state, out, T, H, NC);
  }
  return launch_status();
}
