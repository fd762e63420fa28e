// Weight-streaming GEMM for the decode path: Y[M, N] = X[M, K] . W[N, K]^T
// with few rows M (the decode batch, or the tokens routed to one expert); the
// weights are read from HBM once per chunk of M and the kernel is HBM-bound.
//
// Mapping onto v_mfma_f32_16x16x32_bf16 (wave64):
//   * tokens are the MFMA rows (A), weight rows the MFMA columns (B); one
//     workgroup owns 16 weight rows and splits K over its S waves (wave w
//     takes the 256-wide K blocks w, w + S, ...), so all of a tile's weight
//     bytes are requested at once; partial sums meet in LDS in wave order
//     (deterministic) and wave 0 runs the fused epilogue;
//   * a 256-wide K block is 8 MFMAs.  Lane l (row r = l%16, group g = l/16)
//     supplies for MFMA j the elements k = kb + 32j + 8g .. +8 of its token
//     row and of its weight row (the instruction's native k order), so the 4
//     lanes of a row read 64 contiguous bytes per load instruction;
//   * weights can be stored in that operand order ("packed": for each 16-row
//     block and 256-wide K block, 8 tiles of 64 lanes x 16 bytes), so one
//     wave's 16-byte-per-lane load of a B operand reads 1 KiB contiguous.
//     The row-major [N, K] layout is also accepted (16-byte pieces of 16
//     different rows per load instruction);
//   * D layout: lane l holds D[4*(l/16) + i][l % 16], i = 0..3.
// Epilogues: bf16/fp32 store, residual add, gated residual add, per-K-block
// partial products, SwiGLU over a (gate, up) row pair, and the gate-weighted
// MoE down store.
//
// Partial products (decode batches): one single-wave workgroup per (16-row
// weight block, 256-wide K block) writes its fp32 product to its own slice;
// the kernel that next reads the rows folds the slices in K order.  A
// workgroup then pulls 32 KiB of activations into its CU instead of the
// whole [M, K] tile, which is what bounds the 4-wave split-K kernel at small
// N, and no residual is read back before the store.
#include "common.hpp"
#include "abi_util.hpp"

#include <algorithm>

namespace llmy {

enum Epilogue : int {
  kStoreBf16 = 0,     // out bf16 [rows, ldo] = acc
  kStoreF32 = 1,      // out f32 [rows, ldo] = acc
  kResidAdd = 2,      // out f32 [rows, ldo] += acc
  kResidGated = 3,    // out f32 [rows, ldo] += acc * aux[row * ldo + n]
  kPartialF32 = 4,    // out f32 [K/256, rows, ldo]: slice s = the product over k in [256s, 256s+256)
  kSwiGLU = 5,        // out bf16 [rows, ldo] = silu(acc_gate) * acc_up  (paired rows)
  kMoeDown = 6,       // out f32 [rows, ldo] = acc * aux[sorted_routes[row]]
};

enum RowMode : int {
  kDense = 0,         // x row m, out row m
  kMoeGather = 1,     // x row sorted_routes[p] / route_k, out row p (p = offsets[e] + m)
  kMoeDirect = 2,     // x row p, out row p
  // Route-indexed (decode): the workgroup of expert e derives its route list
  // {r : ids[r] == e} (ascending) from the router's ids with wavefront ballots;
  // rows are route ids, so no permutation is materialised.
  kRouteGather = 3,   // x row r / route_k, out row r
  kRouteDirect = 4,   // x row r, out row r, gate aux[r]
};

constexpr int kMaxRouteList = 2048;

struct WsArgs {
  const uint16_t* x;
  const uint16_t* w;
  long long w_expert_stride;  // elements between experts' weight blocks
  long long pair_offset;      // elements from a gate row to its up row (kSwiGLU)
  void* out;
  const float* aux;
  const int32_t* offsets;
  const int32_t* sorted_routes;
  const int32_t* ids;  // route-indexed modes: expert id per route [rows_total]
  int M, N, K, ldx, ldo, route_k;
  int rows_total;  // MoE: number of routes (bounds for offsets / sorted_routes)
  int x_rows;      // MoE: rows of x (bounds for the gathered token index)
};

// Packed index of W[n][k] (N % 16 == 0, K % 256 == 0): block (n/16, k/256)
// holds 8 tiles j; tile j lane l element e is W[16*nb + l%16][256*kb + 32*j + 8*(l/16) + e].
__host__ __device__ __forceinline__ long long packed_index(int n, int k, int K) {
  const int nb = n >> 4, r = n & 15;
  const int kb = k >> 8, kk = k & 255;
  const int j = kk >> 5, g = (kk >> 3) & 3, e = kk & 7;
  const int lane = g * 16 + r;
  return ((((static_cast<long long>(nb) * (K >> 8) + kb) * 8 + j) * 64 + lane) << 3) + e;
}

template <int EPI, int MODE, bool PACKED, int MB, int KB, int JT = 8>
__global__ __launch_bounds__(512) void wsgemm_kernel(WsArgs a) {
  constexpr bool kPair = (EPI == kSwiGLU);
  constexpr bool kSplit = (EPI == kPartialF32);  // blockIdx.y = K block, one wave
  constexpr int kSlots = (kPair ? 2 : 1) * MB * 4;
  constexpr int kRows = 16 * MB;  // token rows per chunk
  extern __shared__ float red[];  // [S][kSlots][64]
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int S = blockDim.x >> 6;
  const int n0 = blockIdx.x * 16;
  int row_begin = 0;
  int M = a.M;
  constexpr bool kRouted = (MODE == kRouteGather || MODE == kRouteDirect);
  __shared__ int32_t rlist[kRouted ? kMaxRouteList : 1];
  __shared__ int32_t rcount;
  if (MODE == kDense && !kSplit && gridDim.y > 1) {
    // dense rows split over the grid's y dimension, kRows per workgroup
    row_begin = static_cast<int>(blockIdx.y) * kRows;
    M = min(kRows, a.M - row_begin);
  }
  if (MODE == kMoeGather || MODE == kMoeDirect) {
    // Clamp the (device-resident) offsets so a corrupt permutation cannot
    // move any access out of bounds.
    row_begin = min(max(a.offsets[blockIdx.y], 0), a.rows_total);
    M = min(max(a.offsets[blockIdx.y + 1], row_begin), a.rows_total) - row_begin;
  }
  if (kRouted) {
    if (wave == 0) {
      const int e = blockIdx.y;
      int cnt = 0;
      for (int c0 = 0; c0 < a.rows_total; c0 += 64) {
        const int rr = c0 + lane;
        const int id = rr < a.rows_total ? a.ids[rr] : -1;
        const uint64_t m = __ballot(id == e);
        if (id == e) rlist[cnt + __popcll(m & ((1ull << lane) - 1ull))] = rr;
        cnt += __popcll(m);
      }
      if (lane == 0) rcount = cnt;
    }
    __syncthreads();
    M = rcount;
  }
  if (M <= 0) return;  // uniform over the workgroup: an idle expert reads no weights

  const int r = lane & 15;
  const int g = lane >> 4;
  const int K = a.K;
  const uint16_t* wbase = a.w + (kSplit ? 0ll : static_cast<long long>(blockIdx.y) * a.w_expert_stride);
  // B operand address of (K block kb, MFMA j) for this lane: packed -> tile
  // (kb*8 + j) of the 16-row block; row-major -> row n0 + r, k = kb + 32j + 8g.
  const uint16_t* wlane =
      PACKED ? wbase + (static_cast<long long>(blockIdx.x) * (K >> 8) * 8 * 64 + lane) * 8
             : wbase + static_cast<long long>(n0 + r) * K + 8 * g;

  for (int m0 = 0; m0 < M; m0 += kRows) {
    const int nmb = min(MB, (M - m0 + 15) >> 4);
    const uint16_t* xrow[MB];
    bool valid[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int m = m0 + 16 * mb + r;
      valid[mb] = m < M;
      int src = valid[mb] ? row_begin + m : row_begin;
      if (MODE == kMoeGather) src = min(max(a.sorted_routes[src] / a.route_k, 0), a.x_rows - 1);
      if (MODE == kRouteGather) src = rlist[valid[mb] ? m : 0] / a.route_k;
      if (MODE == kRouteDirect) src = rlist[valid[mb] ? m : 0];
      xrow[mb] = a.x + static_cast<long long>(src) * a.ldx + 8 * g;
    }
    f32x4 acc[MB], accu[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
      accu[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    // Each wave takes KB consecutive pieces of 32*JT k per step (JT = 8: whole
    // 256-wide K blocks; 4: half blocks, twice the waves for a given K);
    // K % (32 * JT * KB) == 0.
    constexpr int KP = 32 * JT;
    const int k_first = kSplit ? static_cast<int>(blockIdx.y) * KP * KB : wave * KP * KB;
    const int k_end = kSplit ? k_first + KP * KB : K;
    for (int kb0 = k_first; kb0 < k_end; kb0 += S * KP * KB) {
      // Issue every load of these K pieces before the first MFMA.
      uint4 bw[KB][JT], bu[KB][JT], av[KB][MB][JT];
#pragma unroll
      for (int q = 0; q < KB; ++q) {
        const int kb = kb0 + KP * q;
#pragma unroll
        for (int j = 0; j < JT; ++j) {
          const long long off =
              PACKED ? (static_cast<long long>(kb >> 8) * 8 + ((kb & 255) >> 5) + j) * 512
                     : kb + 32 * j;
          bw[q][j] = ld_stream(wlane + off);
          if (kPair) bu[q][j] = ld_stream(wlane + a.pair_offset + off);
        }
      }
#pragma unroll
      for (int q = 0; q < KB; ++q) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
          for (int j = 0; j < JT; ++j)
            av[q][mb][j] = (mb < nmb && valid[mb])
                               ? *reinterpret_cast<const uint4*>(xrow[mb] + kb0 + KP * q + 32 * j)
                               : uint4{0u, 0u, 0u, 0u};
        }
      }
#pragma unroll
      for (int q = 0; q < KB; ++q) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
          if (mb < nmb) {
#pragma unroll
            for (int j = 0; j < JT; ++j) {
              acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                  as_bf16x8(av[q][mb][j]), as_bf16x8(bw[q][j]), acc[mb], 0, 0, 0);
              if (kPair)
                accu[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    as_bf16x8(av[q][mb][j]), as_bf16x8(bu[q][j]), accu[mb], 0, 0, 0);
            }
          }
        }
      }
    }

    if (S > 1) {
      __syncthreads();  // the previous chunk's reduction has finished reading
      if (wave > 0) {
        float* dst = red + (static_cast<size_t>(wave) * kSlots) * 64 + lane;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            dst[(mb * 4 + i) * 64] = acc[mb][i];
            if (kPair) dst[(MB * 4 + mb * 4 + i) * 64] = accu[mb][i];
          }
        }
      }
      __syncthreads();
      if (wave == 0) {
        for (int w = 1; w < S; ++w) {
          const float* src = red + (static_cast<size_t>(w) * kSlots) * 64 + lane;
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              acc[mb][i] += src[(mb * 4 + i) * 64];
              if (kPair) accu[mb][i] += src[(MB * 4 + mb * 4 + i) * 64];
            }
          }
        }
      }
    }
    if (wave != 0) continue;

    // Epilogue: lane holds rows m0 + 16mb + 4g + i, column n0 + r.  Every
    // value the epilogue reads (residual, gate) is loaded before the first
    // store: the compiler cannot prove a store and a later load of another
    // row apart, and would otherwise wait out one memory round trip per value.
    const int n = n0 + r;
    float* const outf = static_cast<float*>(a.out) +
                        (kSplit ? static_cast<long long>(blockIdx.y) * a.M * a.ldo : 0ll);
    long long orow[MB][4];
    float in0[MB][4], in1[MB][4];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = m0 + 16 * mb + 4 * g + i;
        const bool ok = mb < nmb && m < M;
        const long long row = ok ? (kRouted ? rlist[m] : row_begin + m) : -1;
        orow[mb][i] = row;
        const long long o = row * a.ldo + n;
        in0[mb][i] = 0.f;
        in1[mb][i] = 1.f;
        if (ok) {
          if (EPI == kResidAdd || EPI == kResidGated) in0[mb][i] = static_cast<const float*>(a.out)[o];
          if (EPI == kResidGated) in1[mb][i] = a.aux[o];
          if (EPI == kMoeDown) {
            const int route = kRouted ? static_cast<int>(row)
                                      : min(max(a.sorted_routes[row], 0), a.rows_total - 1);
            in1[mb][i] = a.aux[route];
          }
        }
      }
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const long long row = orow[mb][i];
        if (row < 0) continue;
        const long long o = row * a.ldo + n;
        const float v = acc[mb][i];
        if (EPI == kStoreBf16) {
          static_cast<uint16_t*>(a.out)[o] = f2bf(v);
        } else if (EPI == kStoreF32 || EPI == kPartialF32) {
          outf[o] = v;
        } else if (EPI == kResidAdd) {
          static_cast<float*>(a.out)[o] = in0[mb][i] + v;
        } else if (EPI == kResidGated) {
          static_cast<float*>(a.out)[o] = in0[mb][i] + v * in1[mb][i];
        } else if (EPI == kSwiGLU) {
          static_cast<uint16_t*>(a.out)[o] = f2bf(siluf_(v) * accu[mb][i]);
        } else if (EPI == kMoeDown) {
          static_cast<float*>(a.out)[o] = v * in1[mb][i];
        }
      }
    }
  }
}

// Dense out[M, N] = x[M, K] . w[N, K]^T for a narrow N (a few 16-row weight
// blocks) and many rows: the weight-streaming kernel with its rows split over
// the grid (16 per workgroup), out row stride ldo.  epi uses the Epilogue
// numbering (store bf16 / fp32, residual add, gated residual add).
int32_t dense_narrow_ws(const uint16_t* x, const uint16_t* w, void* out, const float* aux, int M,
                        int N, int K, int ldo, int epi, bool packed, hipStream_t s);

// Route-indexed MoE gate/up projection for decode (kRouteGather, packed
// weights, a few 16-route chunks per expert): the arithmetic of
// wsgemm_kernel<kSwiGLU, kRouteGather, packed, 1, 1, 8> (S waves, wave w takes
// the 256-wide K blocks w, w + S, ...; partial sums meet in wave order), so the
// two agree bit for bit, but every weight load of the workgroup is requested
// first, before the route scan: the scan's round trip to the router's ids then
// hides behind the weight stream instead of delaying it, and the weights stay
// in registers for every 16-route chunk.  NP K blocks per wave.
template <int NP>
__global__ __launch_bounds__(512) void routed_gate_up_kernel(WsArgs a) {
  extern __shared__ float red[];  // [S][8][64]: gate then up partial sums
  __shared__ int32_t rlist[kMaxRouteList];
  __shared__ int32_t rcount;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int S = blockDim.x >> 6;
  const int e = blockIdx.y;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int K = a.K;
  const uint16_t* wl = a.w + static_cast<long long>(e) * a.w_expert_stride +
                       (static_cast<long long>(blockIdx.x) * (K >> 8) * 8 * 64 + lane) * 8;
  uint4 bw[NP][8], bu[NP][8];
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const long long kb = wave + p * S;  // 256-wide K block
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      bw[p][j] = ld_stream(wl + (kb * 8 + j) * 512);
      bu[p][j] = ld_stream(wl + a.pair_offset + (kb * 8 + j) * 512);
    }
  }
  if (wave == 0) {
    int cnt = 0;
    for (int c0 = 0; c0 < a.rows_total; c0 += 64) {
      const int rr = c0 + lane;
      const int id = rr < a.rows_total ? a.ids[rr] : -1;
      const uint64_t m = __ballot(id == e);
      if (id == e) rlist[cnt + __popcll(m & ((1ull << lane) - 1ull))] = rr;
      cnt += __popcll(m);
    }
    if (lane == 0) rcount = cnt;
  }
  __syncthreads();
  const int M = rcount;

  for (int m0 = 0; m0 < M; m0 += 16) {
    const bool valid = m0 + r < M;
    const int src = rlist[valid ? m0 + r : m0] / a.route_k;
    const uint16_t* xrow = a.x + static_cast<long long>(src) * a.ldx + 8 * g;
    uint4 av[NP][8];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const int kb = (wave + p * S) * 256;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        av[p][j] = valid ? *reinterpret_cast<const uint4*>(xrow + kb + 32 * j)
                         : uint4{0u, 0u, 0u, 0u};
    }
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f}, accu = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int p = 0; p < NP; ++p) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av[p][j]), as_bf16x8(bw[p][j]),
                                                      acc, 0, 0, 0);
        accu = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av[p][j]), as_bf16x8(bu[p][j]),
                                                       accu, 0, 0, 0);
      }
    }
    if (S > 1) {
      __syncthreads();  // the previous chunk's reduction has finished reading
      if (wave > 0) {
        float* dst = red + static_cast<size_t>(wave) * 8 * 64 + lane;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          dst[i * 64] = acc[i];
          dst[(4 + i) * 64] = accu[i];
        }
      }
      __syncthreads();
      if (wave == 0) {
        for (int w = 1; w < S; ++w) {
          const float* sp = red + static_cast<size_t>(w) * 8 * 64 + lane;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            acc[i] += sp[i * 64];
            accu[i] += sp[(4 + i) * 64];
          }
        }
      }
    }
    if (wave != 0) continue;
    // lane holds routes m0 + 4g + i, column 16 * blockIdx.x + r
    const int n = 16 * blockIdx.x + r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int mm = m0 + 4 * g + i;
      if (mm < M)
        static_cast<uint16_t*>(a.out)[static_cast<long long>(rlist[mm]) * a.ldo + n] =
            f2bf(siluf_(acc[i]) * accu[i]);
    }
  }
}

template <int EPI, int MODE, int MB, int KB = 1, int JT = 8>
static int32_t launch_ws(const WsArgs& a, int grid_y, bool packed, hipStream_t s) {
  if (a.K % (32 * JT * KB) != 0) return launch_ws<EPI, MODE, MB, 1, 8>(a, grid_y, packed, s);
  const int waves = std::max(1, std::min(8, a.K / (32 * JT * KB)));
  const size_t lds = waves > 1 ? static_cast<size_t>(waves) * (EPI == kSwiGLU ? 2 : 1) * MB * 4 *
                                     64 * sizeof(float)
                               : 0;
  const dim3 grid(a.N / 16, grid_y), block(64 * waves);
  if (packed)
    hipLaunchKernelGGL((wsgemm_kernel<EPI, MODE, true, MB, KB, JT>), grid, block, lds, s, a);
  else
    hipLaunchKernelGGL((wsgemm_kernel<EPI, MODE, false, MB, KB, JT>), grid, block, lds, s, a);
  return launch_status();
}

int32_t dense_narrow_ws(const uint16_t* x, const uint16_t* w, void* out, const float* aux, int M,
                        int N, int K, int ldo, int epi, bool packed, hipStream_t s) {
  WsArgs a{};
  a.x = x; a.w = w; a.out = out; a.aux = aux;
  a.M = M; a.N = N; a.K = K; a.ldx = K; a.ldo = ldo;
  if ((M + 15) / 16 > 65535) {  // more rows than the grid's y dimension takes: 64 per workgroup
    const int gy = (M + 63) / 64;
    if (gy > 65535) return static_cast<int32_t>(hipErrorInvalidValue);
    switch (epi) {
      case kStoreBf16: return launch_ws<kStoreBf16, kDense, 4>(a, gy, packed, s);
      case kStoreF32: return launch_ws<kStoreF32, kDense, 4>(a, gy, packed, s);
      case kResidAdd: return launch_ws<kResidAdd, kDense, 4>(a, gy, packed, s);
      default: return launch_ws<kResidGated, kDense, 4>(a, gy, packed, s);
    }
  }
  const int grid_y = (M + 15) / 16;
  switch (epi) {
    case kStoreBf16: return launch_ws<kStoreBf16, kDense, 1>(a, grid_y, packed, s);
    case kStoreF32: return launch_ws<kStoreF32, kDense, 1>(a, grid_y, packed, s);
    case kResidAdd: return launch_ws<kResidAdd, kDense, 1>(a, grid_y, packed, s);
    default: return launch_ws<kResidGated, kDense, 1>(a, grid_y, packed, s);
  }
}

// Dense GEMM for large N (the tied LM head): one workgroup owns 64 weight rows
// (4 waves x 16) for up to 64 tokens over the whole K.  Per 256-wide K block
// the token tile [64 x 256] is staged once into LDS with coalesced 16-byte
// loads (rows padded by 16 bytes so the MFMA fragment reads are conflict
// free) and shared by the 4 waves; each wave streams its own packed weight
// tiles from HBM.  Activation traffic is 1/4 of the 16-row split-K kernel's.
constexpr int kLdsRow = 256 + 8;  // bf16 elements per staged token row (16-byte pad)

//
// With EPI = kPartialF32 the grid's y dimension splits K into 256-wide blocks
// (block blockIdx.y only, product written to its own slice, as in
// wsgemm_kernel): four waves then share one staged 32 KiB activation slice
// for 64 weight rows, 2.5x less traffic into each CU than four single-wave
// workgroups of 16 rows.
//
// WV waves per workgroup (16 weight rows each) share the staged tile; with PF
// each wave requests the next K block's weights before the current block's
// MFMAs.
template <int EPI, int WV = 4, bool PF = false>
__global__ __launch_bounds__(64 * WV) void dense_lds_kernel(WsArgs a) {
  constexpr bool kSplit = (EPI == kPartialF32);
  constexpr int kThreads = 64 * WV;
  constexpr int kStage = 2048 / kThreads;  // 16-byte pieces per thread of a [64 x 256] tile
  __shared__ __align__(16) uint16_t As[64 * kLdsRow];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int K = a.K;
  const int M = a.M;
  const int nblk = blockIdx.x * WV + wave;  // this wave's 16-row block
  const bool wave_active = nblk * 16 < a.N;
  const uint16_t* wlane = a.w + (static_cast<long long>(nblk) * (K >> 8) * 8 * 64 + lane) * 8;
  f32x4 acc[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int k_first = kSplit ? static_cast<int>(blockIdx.y) * 256 : 0;
  const int k_end = kSplit ? k_first + 256 : K;
  auto load_w = [&](uint4* dst, int kb) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      dst[j] = ld_stream(wlane + (static_cast<long long>(kb >> 8) * 8 + j) * 512);
  };
  uint4 bw[8];
  if (PF && wave_active) load_w(bw, k_first);
  for (int kb = k_first; kb < k_end; kb += 256) {
    if (!PF && wave_active) load_w(bw, kb);
    // stage the [64 x 256] token tile: flat 16-byte index f = i*kThreads + tid
    uint4 av[kStage];
#pragma unroll
    for (int i = 0; i < kStage; ++i) {
      const int f = i * kThreads + threadIdx.x;
      const int row = f >> 5, c16 = f & 31;
      av[i] = row < M ? *reinterpret_cast<const uint4*>(a.x + static_cast<long long>(row) * a.ldx +
                                                         kb + 8 * c16)
                      : uint4{0u, 0u, 0u, 0u};
    }
    __syncthreads();  // previous block's fragment reads are done
#pragma unroll
    for (int i = 0; i < kStage; ++i) {
      const int f = i * kThreads + threadIdx.x;
      const int row = f >> 5, c16 = f & 31;
      *reinterpret_cast<uint4*>(As + row * kLdsRow + 8 * c16) = av[i];
    }
    __syncthreads();
    uint4 bn[8];
    const bool more = PF && kb + 256 < k_end;
    if (more && wave_active) load_w(bn, kb + 256);
    if (wave_active) {
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint4 af =
              *reinterpret_cast<const uint4*>(As + (16 * mb + r) * kLdsRow + 32 * j + 8 * g);
          acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(af), as_bf16x8(bw[j]),
                                                            acc[mb], 0, 0, 0);
        }
      }
    }
    if (more) {
#pragma unroll
      for (int j = 0; j < 8; ++j) bw[j] = bn[j];
    }
  }
  if (!wave_active) return;
  const int n = nblk * 16 + r;
  float* const outf = static_cast<float*>(a.out) +
                      (kSplit ? static_cast<long long>(blockIdx.y) * M * a.ldo : 0ll);
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 16 * mb + 4 * g + i;
      if (m < M) {
        const long long o = static_cast<long long>(m) * a.ldo + n;
        const float v = acc[mb][i];
        if (EPI == kStoreBf16) static_cast<uint16_t*>(a.out)[o] = f2bf(v);
        else if (EPI == kStoreF32 || EPI == kPartialF32) outf[o] = v;
        else if (EPI == kResidAdd) static_cast<float*>(a.out)[o] += v;
        else static_cast<float*>(a.out)[o] += v * a.aux[o];
      }
    }
  }
}

template <int EPI>
static int32_t launch_dense_lds(const WsArgs& a, hipStream_t s) {
  if (EPI == kPartialF32) {
    const dim3 grid((a.N + 63) / 64, a.K / 256);
    hipLaunchKernelGGL((dense_lds_kernel<EPI>), grid, dim3(256), 0, s, a);
    return launch_status();
  }
  // full K per workgroup: next-block weight prefetch (LM head 17.9 -> 16.2 us);
  // 8 waves per workgroup measured no faster than 4
  const dim3 grid((a.N + 63) / 64);
  hipLaunchKernelGGL((dense_lds_kernel<EPI, 4, true>), grid, dim3(256), 0, s, a);
  return launch_status();
}

// Row-major [batch][N][K] -> packed tiles (same element count).
__global__ __launch_bounds__(256) void pack_kernel(const uint16_t* __restrict__ w,
                                                   uint16_t* __restrict__ out, int N, int K,
                                                   long long total) {
  for (long long i = blockIdx.x * 256ll + threadIdx.x; i < total; i += 256ll * gridDim.x) {
    const long long per = static_cast<long long>(N) * K;
    const long long b = i / per;
    const long long rem = i - b * per;
    const int n = static_cast<int>(rem / K);
    const int k = static_cast<int>(rem - static_cast<long long>(n) * K);
    out[b * per + packed_index(n, k, K)] = w[i];
  }
}

// out[t] (+)= sum_j y[route_pos[t*k + j]] in j order; y [T*k, D] fp32.
__global__ __launch_bounds__(256) void moe_combine_kernel(const float* __restrict__ y,
                                                          const int32_t* __restrict__ route_pos,
                                                          void* __restrict__ out, int T, int D,
                                                          int k, int mode) {
  const int d4 = D >> 2;
  const long long total = static_cast<long long>(T) * d4;
  for (long long i = blockIdx.x * 256ll + threadIdx.x; i < total; i += 256ll * gridDim.x) {
    const int t = static_cast<int>(i / d4);
    const int c = static_cast<int>(i % d4) * 4;
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int j = 0; j < k; ++j) {
      const int p = min(max(route_pos[t * k + j], 0), T * k - 1);
      const float4 v = *reinterpret_cast<const float4*>(y + static_cast<long long>(p) * D + c);
      s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
    }
    const long long o = static_cast<long long>(t) * D + c;
    if (mode == 0) {  // bf16 store
      uint16_t* ob = static_cast<uint16_t*>(out);
      *reinterpret_cast<uint2*>(ob + o) = make_uint2(pack_bf2(s.x, s.y), pack_bf2(s.z, s.w));
    } else if (mode == 1) {  // fp32 store
      *reinterpret_cast<float4*>(static_cast<float*>(out) + o) = s;
    } else {  // fp32 residual add
      float4* of = reinterpret_cast<float4*>(static_cast<float*>(out) + o);
      float4 x = *of;
      x.x += s.x; x.y += s.y; x.z += s.z; x.w += s.w;
      *of = x;
    }
  }
}

// Grouped MFMA GEMMs for MoE prefill (moe_grouped.hip).
int32_t moe_grouped_prefill(const uint16_t* x, const int32_t* offsets, const int32_t* sorted_routes,
                            const float* gates, const uint16_t* w_gate_up, const uint16_t* w_down,
                            uint16_t* act, float* y, int T, int D, int H, int E, int k, bool packed,
                            hipStream_t s);
// Tiled MFMA dense GEMM with the epilogues above (dense_gemm.hip).
int32_t dense_gemm_mfma(const uint16_t* x, const uint16_t* w, void* out, const float* aux,
                        int M, int N, int K, int epi, bool packed, hipStream_t s);

// Rows from which the dense projections switch from the weight-streaming
// kernel (every weight byte read once per 64 rows, HBM-bound) to the MFMA
// tiles (compute-bound); decode batches stay below it.
constexpr int kDenseMfmaMinRows = 256;

}  // namespace llmy

using namespace llmy;

extern "C" int32_t llmy_pack_weights_bf16(const llmy_bf16* w, llmy_bf16* out, int64_t batch,
                                          int32_t N, int32_t K, void* stream) {
  LLMY_REQUIRE(batch >= 0 && N > 0 && N % 16 == 0 && K > 0 && K % 256 == 0);
  if (batch == 0) return 0;
  LLMY_REQUIRE(w && out && w != out);
  const long long total = batch * N * static_cast<long long>(K);
  const int blocks = static_cast<int>(std::min<long long>((total + 255) / 256, 65536));
  hipLaunchKernelGGL(pack_kernel, dim3(blocks), dim3(256), 0, as_stream(stream), w, out, N, K,
                     total);
  return launch_status();
}

extern "C" int32_t llmy_linear_bf16(const llmy_bf16* x, const llmy_bf16* w, void* out,
                                    const float* aux, int32_t M, int32_t N, int32_t K,
                                    int32_t epilogue, int32_t weight_layout, void* stream) {
  LLMY_REQUIRE(M >= 0 && N > 0 && N % 16 == 0 && K > 0 && K % 256 == 0);
  LLMY_REQUIRE(epilogue >= kStoreBf16 && epilogue <= kPartialF32);
  // partial products: decode batches only (one row chunk per workgroup)
  LLMY_REQUIRE(epilogue != kPartialF32 || M <= 64);
  LLMY_REQUIRE(weight_layout == 0 || weight_layout == 1);
  if (M == 0) return 0;
  LLMY_REQUIRE(x && w && out);
  LLMY_REQUIRE(epilogue != kResidGated || aux != nullptr);
  LLMY_REQUIRE(aligned(x, 16) && aligned(w, 16) && aligned(out, 4));
  WsArgs a{};
  a.x = x; a.w = w; a.out = out; a.aux = aux;
  a.M = M; a.N = N; a.K = K; a.ldx = K; a.ldo = N; a.route_k = 1;
  const hipStream_t s = as_stream(stream);
  const bool packed = weight_layout == 1;
  if (epilogue == kPartialF32) {
    LLMY_REQUIRE(static_cast<long long>(K / 256) * M * N < (1ll << 31));
    // packed weights: four waves share a staged activation slice (faster than
    // the single-wave kernel below at every decode shape measured, N = 1024..4112)
    if (packed) return launch_dense_lds<kPartialF32>(a, s);
    // row-major weights: one single-wave workgroup per (16 rows, K block)
    hipLaunchKernelGGL((wsgemm_kernel<kPartialF32, kDense, false, 4, 1, 8>),
                       dim3(N / 16, K / 256), dim3(64), 0, s, a);
    return launch_status();
  }
  if (M >= kDenseMfmaMinRows && aligned(out, 16) && (aux == nullptr || aligned(aux, 16)) &&
      2ll * M * K < (1ll << 31) && 2ll * N * K < (1ll << 31))
    return dense_gemm_mfma(x, w, out, aux, M, N, K, epilogue, packed, s);
  // Large N with packed weights: the LDS-tiled kernel (enough workgroups
  // without splitting K, and 4x less activation traffic).
  if (packed && M <= 64 && N >= 8192) {
    switch (epilogue) {
      case kStoreBf16: return launch_dense_lds<kStoreBf16>(a, s);
      case kStoreF32: return launch_dense_lds<kStoreF32>(a, s);
      case kResidAdd: return launch_dense_lds<kResidAdd>(a, s);
      default: return launch_dense_lds<kResidGated>(a, s);
    }
  }
  switch (epilogue) {
    case kStoreBf16: return launch_ws<kStoreBf16, kDense, 4>(a, 1, packed, s);
    case kStoreF32: return launch_ws<kStoreF32, kDense, 4>(a, 1, packed, s);
    case kResidAdd: return launch_ws<kResidAdd, kDense, 4>(a, 1, packed, s);
    default: return launch_ws<kResidGated, kDense, 4>(a, 1, packed, s);
  }
}

extern "C" int32_t llmy_moe_experts_bf16(const llmy_bf16* x, const int32_t* offsets,
                                         const int32_t* sorted_routes, const float* gates,
                                         const llmy_bf16* w_gate_up, const llmy_bf16* w_down,
                                         llmy_bf16* act, float* y, int32_t T, int32_t D,
                                         int32_t H, int32_t E, int32_t k, int32_t weight_layout,
                                         void* stream) {
  LLMY_REQUIRE(T >= 0 && D > 0 && D % 256 == 0 && H > 0 && H % 256 == 0);
  LLMY_REQUIRE(E > 0 && k > 0 && k <= E && (weight_layout == 0 || weight_layout == 1));
  if (T == 0) return 0;
  LLMY_REQUIRE(x && offsets && sorted_routes && gates && w_gate_up && w_down && act && y);
  LLMY_REQUIRE(aligned(x, 16) && aligned(w_gate_up, 16) && aligned(w_down, 16) &&
               aligned(act, 16) && aligned(y, 16));
  const hipStream_t s = as_stream(stream);
  const bool packed = weight_layout == 1;
  WsArgs a{};
  a.x = x; a.w = w_gate_up; a.out = act; a.offsets = offsets; a.sorted_routes = sorted_routes;
  a.w_expert_stride = 2ll * H * D; a.pair_offset = static_cast<long long>(H) * D;
  a.N = H; a.K = D; a.ldx = D; a.ldo = H; a.route_k = k;
  a.rows_total = T * k; a.x_rows = T;
  WsArgs b{};
  b.x = act; b.w = w_down; b.out = y; b.aux = gates; b.offsets = offsets;
  b.sorted_routes = sorted_routes; b.w_expert_stride = static_cast<long long>(D) * H;
  b.N = D; b.K = H; b.ldx = H; b.ldo = D; b.route_k = k;
  b.rows_total = T * k; b.x_rows = T * k;
  // Few routes per expert (decode): 16-row chunks, half K blocks per wave
  // (8 waves) for the down projection; otherwise 64-row chunks.  (The route-indexed entry
  // point uses the same configurations, so at these sizes the two agree bit
  // for bit.)
  int32_t st;
  // The tiled path addresses each operand block with 32-bit byte offsets.
  const bool tiled_fits = 2ll * T * D < (1ll << 31) && 2ll * T * k * H < (1ll << 31) &&
                          4ll * H * D < (1ll << 31);
  if (T * k <= 16 * E || !tiled_fits) {
    st = launch_ws<kSwiGLU, kMoeGather, 1>(a, E, packed, s);
    if (st != 0) return st;
    return launch_ws<kMoeDown, kMoeDirect, 1, 1, 4>(b, E, packed, s);
  }
  // Prefill: grouped MFMA GEMMs (moe_grouped.hip).
  return moe_grouped_prefill(x, offsets, sorted_routes, gates, w_gate_up, w_down, act, y, T, D,
                             H, E, k, packed, s);
}

extern "C" int32_t llmy_moe_combine(const float* y, const int32_t* route_pos, void* out,
                                    int32_t T, int32_t D, int32_t k, int32_t mode,
                                    void* stream) {
  LLMY_REQUIRE(T >= 0 && D > 0 && D % 4 == 0 && k > 0 && mode >= 0 && mode <= 2);
  if (T == 0) return 0;
  LLMY_REQUIRE(y && route_pos && out);
  LLMY_REQUIRE(aligned(y, 16) && aligned(out, mode == 0 ? 8 : 16));
  const long long work = static_cast<long long>(T) * (D / 4);
  const int blocks = static_cast<int>(std::min<long long>((work + 255) / 256, 4096));
  hipLaunchKernelGGL(moe_combine_kernel, dim3(blocks), dim3(256), 0, as_stream(stream), y,
                     route_pos, out, T, D, k, mode);
  return launch_status();
}

extern "C" int32_t llmy_moe_experts_routed_bf16(const llmy_bf16* x, const int32_t* ids,
                                                const float* gates, const llmy_bf16* w_gate_up,
                                                const llmy_bf16* w_down, llmy_bf16* act, float* y,
                                                int32_t T, int32_t D, int32_t H, int32_t E,
                                                int32_t k, int32_t weight_layout, void* stream) {
  LLMY_REQUIRE(T >= 0 && D > 0 && D % 256 == 0 && H > 0 && H % 256 == 0);
  LLMY_REQUIRE(E > 0 && k > 0 && k <= E && (weight_layout == 0 || weight_layout == 1));
  LLMY_REQUIRE(static_cast<long long>(T) * k <= kMaxRouteList);
  if (T == 0) return 0;
  LLMY_REQUIRE(x && ids && gates && w_gate_up && w_down && act && y);
  LLMY_REQUIRE(aligned(x, 16) && aligned(w_gate_up, 16) && aligned(w_down, 16) &&
               aligned(act, 16) && aligned(y, 16));
  const hipStream_t s = as_stream(stream);
  const bool packed = weight_layout == 1;
  WsArgs a{};
  a.x = x; a.w = w_gate_up; a.out = act; a.ids = ids;
  a.w_expert_stride = 2ll * H * D; a.pair_offset = static_cast<long long>(H) * D;
  a.N = H; a.K = D; a.ldx = D; a.ldo = H; a.route_k = k;
  a.rows_total = T * k; a.x_rows = T;
  WsArgs b{};
  b.x = act; b.w = w_down; b.out = y; b.aux = gates; b.ids = ids;
  b.w_expert_stride = static_cast<long long>(D) * H;
  b.N = D; b.K = H; b.ldx = H; b.ldo = D; b.route_k = k;
  b.rows_total = T * k; b.x_rows = T * k;
  int32_t st;
  // Gate/up through routed_gate_up_kernel where its shape fits (packed
  // weights, D in at most 8 waves of whole 256-wide blocks, 1, 2 or 4 per
  // wave); the same arithmetic as the wsgemm configuration below.  It reads
  // every expert's weights, idle or not, so it is taken only where the routes
  // number at least twice the experts (then about 86% or more of the experts
  // are hit by uniform routing); the generic kernel skips idle experts.
  const int kblk = D / 256, gu_waves = std::min(8, kblk), gu_np = kblk / gu_waves;
  if (T * k <= 16 * E && T * k >= 2 * E && packed && kblk % gu_waves == 0 &&
      (gu_np == 1 || gu_np == 2 || gu_np == 4)) {
    const size_t lds = static_cast<size_t>(gu_waves) * 8 * 64 * sizeof(float);
    const dim3 grid(H / 16, E), block(64 * gu_waves);
    if (gu_np == 1)
      hipLaunchKernelGGL(routed_gate_up_kernel<1>, grid, block, lds, s, a);
    else if (gu_np == 2)
      hipLaunchKernelGGL(routed_gate_up_kernel<2>, grid, block, lds, s, a);
    else
      hipLaunchKernelGGL(routed_gate_up_kernel<4>, grid, block, lds, s, a);
    st = launch_status();
    if (st != 0) return st;
    return launch_ws<kMoeDown, kRouteDirect, 1, 1, 4>(b, E, packed, s);
  }
  if (T * k <= 16 * E) {
    st = launch_ws<kSwiGLU, kRouteGather, 1>(a, E, packed, s);
    if (st != 0) return st;
    return launch_ws<kMoeDown, kRouteDirect, 1, 1, 4>(b, E, packed, s);
  }
  st = launch_ws<kSwiGLU, kRouteGather, 4>(a, E, packed, s);
  if (st != 0) return st;
  return launch_ws<kMoeDown, kRouteDirect, 4>(b, E, packed, s);
}
