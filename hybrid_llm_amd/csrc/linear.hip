// Weight-streaming GEMM for the decode path: Y[M, N] = X[M, K] . W[N, K]^T
// with few rows M (decode batch, or the tokens routed to one expert) and the
// weights read from HBM exactly once per 64-row chunk of M.
//
// Mapping onto v_mfma_f32_16x16x32_bf16 (wave64):
//   * tokens are the MFMA rows (A), weight rows the MFMA columns (B), so one
//     wave owns 16 weight rows and up to 64 tokens (4 row blocks);
//   * a K block of 256 is 8 MFMAs.  Lane l (row/col r = l%16, group g = l/16)
//     loads 128 contiguous bytes, elements [kb + 64g, kb + 64g + 64), of its
//     weight row and of its token row.  MFMA j consumes the j-th 16 bytes, so
//     A and B agree on which k each (lane, slot) holds; over the 8 MFMAs every
//     k of the block is used once.  Per weight row a wave reads 512
//     contiguous bytes per K block, no LDS staging is needed, and the next K
//     block's weights are prefetched into registers during the MFMAs;
//   * D layout: lane l holds D[4*(l/16) + i][l % 16], i = 0..3.
// Epilogues are fused: bf16/fp32 store, residual add, gated residual add,
// SwiGLU over a (gate, up) row pair, and the gate-weighted MoE down store.
#include "common.hpp"
#include "abi_util.hpp"

#include <algorithm>

namespace llmy {

enum Epilogue : int {
  kStoreBf16 = 0,     // out bf16 [rows, ldo] = acc
  kStoreF32 = 1,      // out f32 [rows, ldo] = acc
  kResidAdd = 2,      // out f32 [rows, ldo] += acc
  kResidGated = 3,    // out f32 [rows, ldo] += acc * aux[row * ldo + n]
  kSwiGLU = 4,        // out bf16 [rows, ldo] = silu(acc_gate) * acc_up  (paired rows)
  kMoeDown = 5,       // out f32 [rows, ldo] = acc * aux[sorted_routes[row]]
};

enum RowMode : int {
  kDense = 0,         // x row m, out row m
  kMoeGather = 1,     // x row sorted_routes[p] / route_k, out row p (p = offsets[e] + m)
  kMoeDirect = 2,     // x row p, out row p
};

struct WsArgs {
  const uint16_t* x;
  const uint16_t* w;
  long long w_expert_stride;  // elements between experts' weight blocks
  long long pair_offset;      // elements from a gate row to its up row (kSwiGLU)
  void* out;
  const float* aux;
  const int32_t* offsets;
  const int32_t* sorted_routes;
  int M, N, K, ldx, ldo, route_k;
  int rows_total;  // MoE: number of routes (bounds for offsets / sorted_routes)
  int x_rows;      // MoE: rows of x (bounds for the gathered token index)
};

__device__ __forceinline__ void load128(const uint16_t* p, uint4* v) {
  const uint4* q = reinterpret_cast<const uint4*>(p);
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = q[j];
}

template <int EPI, int MODE>
__global__ __launch_bounds__(256) void wsgemm_kernel(WsArgs a) {
  constexpr bool kPair = (EPI == kSwiGLU);
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n0 = (blockIdx.x * 4 + wave) * 16;
  if (n0 >= a.N) return;  // no block-level synchronisation below
  int row_begin = 0;
  int M = a.M;
  if (MODE != kDense) {
    // Clamp the (device-resident) offsets so a corrupt permutation cannot
    // move any access out of bounds.
    row_begin = min(max(a.offsets[blockIdx.y], 0), a.rows_total);
    M = min(max(a.offsets[blockIdx.y + 1], row_begin), a.rows_total) - row_begin;
  }
  if (M <= 0) return;  // an expert with no routes reads no weights

  const int r = lane & 15;
  const int g = lane >> 4;
  const uint16_t* wrow = a.w + static_cast<long long>(blockIdx.y) * a.w_expert_stride +
                         static_cast<long long>(n0 + r) * a.K + 64 * g;
  const int K = a.K;

  for (int m0 = 0; m0 < M; m0 += 64) {
    const int nmb = min(4, (M - m0 + 15) >> 4);
    const uint16_t* xrow[4];
    bool valid[4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      const int m = m0 + 16 * mb + r;
      valid[mb] = m < M;
      int src = valid[mb] ? row_begin + m : row_begin;
      if (MODE == kMoeGather) src = min(max(a.sorted_routes[src] / a.route_k, 0), a.x_rows - 1);
      xrow[mb] = a.x + static_cast<long long>(src) * a.ldx + 64 * g;
    }
    f32x4 acc[4], accu[4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      acc[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
      accu[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    uint4 bw[8], bu[8], nw[8], nu[8];
    load128(wrow, bw);
    if (kPair) load128(wrow + a.pair_offset, bu);
    for (int kb = 0; kb < K; kb += 256) {
      const bool more = kb + 256 < K;
      if (more) {
        load128(wrow + kb + 256, nw);
        if (kPair) load128(wrow + a.pair_offset + kb + 256, nu);
      }
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        if (mb < nmb) {
          uint4 av[8];
          if (valid[mb]) {
            load128(xrow[mb] + kb, av);
          } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) av[j] = uint4{0u, 0u, 0u, 0u};
          }
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(av[j]), as_bf16x8(bw[j]),
                                                              acc[mb], 0, 0, 0);
            if (kPair)
              accu[mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                  as_bf16x8(av[j]), as_bf16x8(bu[j]), accu[mb], 0, 0, 0);
          }
        }
      }
      if (more) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          bw[j] = nw[j];
          if (kPair) bu[j] = nu[j];
        }
      }
    }

    // Epilogue: lane holds rows m0 + 16mb + 4g + i, column n0 + r.
    const int n = n0 + r;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      if (mb < nmb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = m0 + 16 * mb + 4 * g + i;
          if (m < M) {
            const long long row = row_begin + m;
            const long long o = row * a.ldo + n;
            const float v = acc[mb][i];
            if (EPI == kStoreBf16) {
              static_cast<uint16_t*>(a.out)[o] = f2bf(v);
            } else if (EPI == kStoreF32) {
              static_cast<float*>(a.out)[o] = v;
            } else if (EPI == kResidAdd) {
              static_cast<float*>(a.out)[o] += v;
            } else if (EPI == kResidGated) {
              static_cast<float*>(a.out)[o] += v * a.aux[o];
            } else if (EPI == kSwiGLU) {
              static_cast<uint16_t*>(a.out)[o] = f2bf(siluf_(v) * accu[mb][i]);
            } else if (EPI == kMoeDown) {
              const int route = min(max(a.sorted_routes[row], 0), a.rows_total - 1);
              static_cast<float*>(a.out)[o] = v * a.aux[route];
            }
          }
        }
      }
    }
  }
}

template <int EPI, int MODE>
static int32_t launch_ws(const WsArgs& a, int grid_y, hipStream_t s) {
  const int tiles = (a.N + 63) / 64;
  hipLaunchKernelGGL((wsgemm_kernel<EPI, MODE>), dim3(tiles, grid_y), dim3(256), 0, s, a);
  return launch_status();
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

}  // namespace llmy

using namespace llmy;

extern "C" int32_t llmy_linear_bf16(const llmy_bf16* x, const llmy_bf16* w, void* out,
                                    const float* aux, int32_t M, int32_t N, int32_t K,
                                    int32_t epilogue, void* stream) {
  LLMY_REQUIRE(M >= 0 && N > 0 && N % 16 == 0 && K > 0 && K % 256 == 0);
  LLMY_REQUIRE(epilogue >= kStoreBf16 && epilogue <= kResidGated);
  if (M == 0) return 0;
  LLMY_REQUIRE(x && w && out);
  LLMY_REQUIRE(epilogue != kResidGated || aux != nullptr);
  LLMY_REQUIRE(aligned(x, 16) && aligned(w, 16) && aligned(out, 4));
  WsArgs a{};
  a.x = x; a.w = w; a.out = out; a.aux = aux;
  a.M = M; a.N = N; a.K = K; a.ldx = K; a.ldo = N; a.route_k = 1;
  const hipStream_t s = as_stream(stream);
  switch (epilogue) {
    case kStoreBf16: return launch_ws<kStoreBf16, kDense>(a, 1, s);
    case kStoreF32: return launch_ws<kStoreF32, kDense>(a, 1, s);
    case kResidAdd: return launch_ws<kResidAdd, kDense>(a, 1, s);
    default: return launch_ws<kResidGated, kDense>(a, 1, s);
  }
}

extern "C" int32_t llmy_moe_experts_bf16(const llmy_bf16* x, const int32_t* offsets,
                                         const int32_t* sorted_routes, const float* gates,
                                         const llmy_bf16* w_gate_up, const llmy_bf16* w_down,
                                         llmy_bf16* act, float* y, int32_t T, int32_t D,
                                         int32_t H, int32_t E, int32_t k, void* stream) {
  LLMY_REQUIRE(T >= 0 && D > 0 && D % 256 == 0 && H > 0 && H % 256 == 0);
  LLMY_REQUIRE(E > 0 && k > 0 && k <= E);
  if (T == 0) return 0;
  LLMY_REQUIRE(x && offsets && sorted_routes && gates && w_gate_up && w_down && act && y);
  LLMY_REQUIRE(aligned(x, 16) && aligned(w_gate_up, 16) && aligned(w_down, 16) &&
               aligned(act, 16) && aligned(y, 16));
  const hipStream_t s = as_stream(stream);
  WsArgs a{};
  a.x = x; a.w = w_gate_up; a.out = act; a.offsets = offsets; a.sorted_routes = sorted_routes;
  a.w_expert_stride = 2ll * H * D; a.pair_offset = static_cast<long long>(H) * D;
  a.N = H; a.K = D; a.ldx = D; a.ldo = H; a.route_k = k;
  a.rows_total = T * k; a.x_rows = T;
  int32_t st = launch_ws<kSwiGLU, kMoeGather>(a, E, s);
  if (st != 0) return st;
  WsArgs b{};
  b.x = act; b.w = w_down; b.out = y; b.aux = gates; b.offsets = offsets;
  b.sorted_routes = sorted_routes; b.w_expert_stride = static_cast<long long>(D) * H;
  b.N = D; b.K = H; b.ldx = H; b.ldo = D; b.route_k = k;
  b.rows_total = T * k; b.x_rows = T * k;
  return launch_ws<kMoeDown, kMoeDirect>(b, E, s);
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
