// MoE router (fp32 logits -> top-k -> softmax over the k values) and the
// expert-major token permutation (stable counting sort of the routes).
//
// Router semantics follow model/layers/context_router.py:62,71-74 with the
// context-aware branch off: logits = RMSNorm(x) . W_r^T in fp32, top-k by
// value, gates = softmax of the k selected values.  Ties resolve to the lower
// expert index (the reference's torch.topk leaves this unspecified).
//
// Permutation semantics follow model/layers/moe.py:39-66 (flat route id
// r = t*k + j, grouped by expert, counts = bincount, offsets = exclusive
// cumsum) with the order inside an expert pinned to ascending r, i.e. the
// order of a stable sort of the expert ids.
#include <algorithm>

#include "common.hpp"
#include "abi_util.hpp"

namespace llmy {

// Top-k over the logits held as mine[s] = logit(lane + 64 s) (E <= 256) and
// softmax over the k picks, written to idx_row[0..k) / gates_row[0..k).  Rank
// j is kept by lane j, so no per-lane arrays are indexed dynamically.
__device__ __forceinline__ void topk_softmax_store(const float (&mine)[4], int E, int k,
                                                   int lane, int32_t* __restrict__ idx_row,
                                                   float* __restrict__ gates_row) {
  uint64_t keys[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int e = lane + 64 * s;
    keys[s] = (e < E) ? value_index_key(mine[s], static_cast<uint32_t>(e)) : 0ull;
  }
  int my_idx = 0;
  float my_val = 0.f;
  for (int j = 0; j < k; ++j) {
    uint64_t best = keys[0];
#pragma unroll
    for (int s = 1; s < 4; ++s) best = keys[s] > best ? keys[s] : best;
    best = wave_max_u64(best);
    const int e = static_cast<int>(key_index(best));
    float val = mine[0];
#pragma unroll
    for (int s = 1; s < 4; ++s) val = (e >> 6) == s ? mine[s] : val;
    val = __shfl(val, e & 63, kWave);
    if (lane == j) {
      my_idx = e;
      my_val = val;
    }
    if ((e & 63) == lane) {
#pragma unroll
      for (int s = 0; s < 4; ++s)
        if ((e >> 6) == s) keys[s] = 0ull;
    }
  }
  const float m = __shfl(my_val, 0, kWave);
  const float ex = lane < k ? expf(my_val - m) : 0.f;
  const float inv = 1.0f / wave_sum(ex);
  if (lane < k) {
    idx_row[lane] = my_idx;
    gates_row[lane] = ex * inv;
  }
}


// One wavefront per token, four tokens per 256-thread block.  The normalised
// row is staged in LDS (D floats per wave) so every expert's dot product reads
// it from LDS while the fp32 router matrix streams through L2.
__global__ __launch_bounds__(256) void router_topk_bf16_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ norm_w,
    const float* __restrict__ w, float* __restrict__ logits_out,
    int32_t* __restrict__ idx_out, float* __restrict__ gates_out,
    int T, int D, int E, int k, float eps) {
  extern __shared__ float lds[];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;
  float* h = lds + static_cast<size_t>(wave) * D;
  const uint16_t* xr = x + static_cast<size_t>(t) * D;

  // Stage the row and accumulate sum of squares (fp32, as norms.py:14).
  float ss = 0.0f;
  for (int d = lane * 4; d < D; d += 256) {
    const uint2 raw = *reinterpret_cast<const uint2*>(xr + d);
    const float v0 = __uint_as_float(raw.x << 16);
    const float v1 = __uint_as_float(raw.x & 0xffff0000u);
    const float v2 = __uint_as_float(raw.y << 16);
    const float v3 = __uint_as_float(raw.y & 0xffff0000u);
    h[d] = v0; h[d + 1] = v1; h[d + 2] = v2; h[d + 3] = v3;
    ss += v0 * v0 + v1 * v1 + v2 * v2 + v3 * v3;
  }
  if (norm_w != nullptr) {
    const float r = rsqrtf(wave_sum(ss) / static_cast<float>(D) + eps);
    for (int d = lane * 4; d < D; d += 256) {
#pragma unroll
      for (int j = 0; j < 4; ++j) h[d + j] = (h[d + j] * r) * norm_w[d + j];
    }
  }
  __builtin_amdgcn_wave_barrier();

  // Logits: lane (e mod 64) ends up holding logit e for its slot e / 64.
  float mine[4] = {0.f, 0.f, 0.f, 0.f};
  for (int e = 0; e < E; ++e) {
    const float* wr = w + static_cast<size_t>(e) * D;
    float acc = 0.0f;
    for (int d = lane * 4; d < D; d += 256) {
      const float4 wv = *reinterpret_cast<const float4*>(wr + d);
      acc = fmaf(h[d], wv.x, acc);
      acc = fmaf(h[d + 1], wv.y, acc);
      acc = fmaf(h[d + 2], wv.z, acc);
      acc = fmaf(h[d + 3], wv.w, acc);
    }
    acc = wave_sum(acc);
    if ((e & 63) == lane) mine[e >> 6] = acc;
  }
  if (logits_out != nullptr) {
    for (int s = 0; s < 4; ++s) {
      const int e = lane + 64 * s;
      if (e < E) logits_out[static_cast<size_t>(t) * E + e] = mine[s];
    }
  }

  topk_softmax_store(mine, E, k, lane, idx_out + static_cast<size_t>(t) * k, gates_out + static_cast<size_t>(t) * k);

}

// The same arithmetic for D = 256 NCH (NCH = 1, 2, 4): the normalised row stays
// in registers and the W_r rows of four experts are requested before their
// dot products, so a token waits on one memory round trip per four experts
// instead of one per expert.  Every product, sum and reduction is taken in the
// order of router_topk_bf16_kernel, so logits, ids and gates are identical.
template <int NCH, int TPW>
__global__ __launch_bounds__(256) void router_topk_bf16_nch_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ norm_w,
    const float* __restrict__ w, float* __restrict__ logits_out,
    int32_t* __restrict__ idx_out, float* __restrict__ gates_out,
    int T, int E, int k, float eps) {
  constexpr int D = 256 * NCH;
  constexpr int G = 4;  // experts per batch of W_r loads
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  // TPW tokens per wavefront: each batch of W_r rows is loaded once and used
  // for all of them (a token's products and sums in the same order as with
  // one token per wavefront)
  const int t0 = (blockIdx.x * 4 + wave) * TPW;
  if (t0 >= T) return;
  float h[TPW][NCH][4];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int t = min(t0 + j, T - 1);  // rows past T: the last row again, not stored
    const uint16_t* xr = x + static_cast<size_t>(t) * D;
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const uint2 raw = *reinterpret_cast<const uint2*>(xr + 4 * lane + 256 * c);
      h[j][c][0] = __uint_as_float(raw.x << 16);
      h[j][c][1] = __uint_as_float(raw.x & 0xffff0000u);
      h[j][c][2] = __uint_as_float(raw.y << 16);
      h[j][c][3] = __uint_as_float(raw.y & 0xffff0000u);
      ss += h[j][c][0] * h[j][c][0] + h[j][c][1] * h[j][c][1] + h[j][c][2] * h[j][c][2] +
            h[j][c][3] * h[j][c][3];
    }
    if (norm_w != nullptr) {
      const float r = rsqrtf(wave_sum(ss) / static_cast<float>(D) + eps);
#pragma unroll
      for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) h[j][c][q] = (h[j][c][q] * r) * norm_w[4 * lane + 256 * c + q];
    }
  }
  float mine[TPW][4];
#pragma unroll
  for (int j = 0; j < TPW; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q) mine[j][q] = 0.f;
  for (int e0 = 0; e0 < E; e0 += G) {
    float4 wv[G][NCH];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int e = min(e0 + g, E - 1);  // rows past E are loaded but unused
#pragma unroll
      for (int c = 0; c < NCH; ++c)
        wv[g][c] = *reinterpret_cast<const float4*>(w + static_cast<size_t>(e) * D + 4 * lane +
                                                    256 * c);
    }
#pragma unroll
    for (int j = 0; j < TPW; ++j)
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
          acc = fmaf(h[j][c][0], wv[g][c].x, acc);
          acc = fmaf(h[j][c][1], wv[g][c].y, acc);
          acc = fmaf(h[j][c][2], wv[g][c].z, acc);
          acc = fmaf(h[j][c][3], wv[g][c].w, acc);
        }
        acc = wave_sum(acc);
        const int e = e0 + g;
        if (e < E && (e & 63) == lane) mine[j][e >> 6] = acc;
      }
  }
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int t = t0 + j;
    if (t >= T) break;  // uniform
    if (logits_out != nullptr) {
      for (int s2 = 0; s2 < 4; ++s2) {
        const int e = lane + 64 * s2;
        if (e < E) logits_out[static_cast<size_t>(t) * E + e] = mine[j][s2];
      }
    }
    topk_softmax_store(mine[j], E, k, lane, idx_out + static_cast<size_t>(t) * k,
                       gates_out + static_cast<size_t>(t) * k);
  }
}

// Top-k + softmax from precomputed fp32 logits [T, E]; one wavefront per token.
__global__ __launch_bounds__(256) void router_topk_from_logits_kernel(
    const float* __restrict__ logits, int32_t* __restrict__ idx_out,
    float* __restrict__ gates_out, int T, int E, int k) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;
  float mine[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int e = lane + 64 * s;
    mine[s] = (e < E) ? logits[static_cast<size_t>(t) * E + e] : 0.0f;
  }
  topk_softmax_store(mine, E, k, lane, idx_out + static_cast<size_t>(t) * k, gates_out + static_cast<size_t>(t) * k);

}

constexpr int kPermuteWaves = 16;

// Stable counting sort of n expert ids (read through `get(r)`) by one
// 1024-thread workgroup.  Wave w owns a contiguous run of 64-route chunks, so
// walking the waves in order and the chunks in order visits routes in
// ascending r.
//   pass 1: per-wave expert histograms (LDS integer atomics: order-free);
//   scan:   expert offsets and per-wave bases;
//   pass 2: each chunk ranks its lanes per expert with one ballot per bit of
//           the expert id (a lane's same-expert mask is the AND of the
//           matching ballots or their complements: ceil(log2 E) ballots in
//           place of one per expert) and places route r at offsets[e] +
//           (routes of e before r).
// `cnt` is LDS scratch of kPermuteWaves * E + E + 1 ints.  Ids outside
// [0, E) are not placed.
template <typename Get>
__device__ void permute_block(Get get, int n, int E, int32_t* __restrict__ counts,
                              int32_t* __restrict__ offsets, int32_t* __restrict__ sorted_routes,
                              int32_t* __restrict__ route_pos, int32_t* cnt) {
  const int nw = blockDim.x >> 6;  // waves in the workgroup (<= kPermuteWaves)
  int32_t* offs = cnt + nw * E;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  for (int i = threadIdx.x; i < nw * E; i += blockDim.x) cnt[i] = 0;
  __syncthreads();

  const int nchunks = (n + 63) / 64;
  const int per_wave = (nchunks + nw - 1) / nw;
  const int c0 = wave * per_wave;
  const int c1 = min(nchunks, c0 + per_wave);
  // The wave's ids are read once, all at once, and kept for pass 2 (up to
  // kHeld chunks per wave; beyond that pass 2 reads them again).
  constexpr int kHeld = 16;
  int held[kHeld];
#pragma unroll
  for (int i = 0; i < kHeld; ++i) {
    const int r = (c0 + i) * 64 + lane;
    held[i] = (c0 + i < c1 && r < n) ? get(r) : -1;
  }
#pragma unroll
  for (int i = 0; i < kHeld; ++i) {
    const int e = held[i];
    if (e >= 0 && e < E) atomicAdd(&cnt[wave * E + e], 1);
  }
  for (int c = c0 + kHeld; c < c1; ++c) {
    const int r = c * 64 + lane;
    if (r < n) {
      const int e = get(r);
      if (e >= 0 && e < E) atomicAdd(&cnt[wave * E + e], 1);
    }
  }
  __syncthreads();

  // Per-expert totals and per-wave exclusive bases (serial over 16 waves).
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    int run = 0;
    for (int w = 0; w < nw; ++w) {
      const int c = cnt[w * E + e];
      cnt[w * E + e] = run;
      run += c;
    }
    offs[e] = run;  // total for now
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int e = 0; e < E; ++e) {
      const int c = offs[e];
      counts[e] = c;
      offs[e] = run;
      offsets[e] = run;
      run += c;
    }
    offs[E] = run;
    offsets[E] = run;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < nw * E; i += blockDim.x) cnt[i] += offs[i % E];
  __syncthreads();

  int32_t* running = cnt + wave * E;
  if (E <= kWave) {
    // Lane e keeps expert e's next position for this wave.  Per chunk, one
    // ballot per bit of the expert id (nb = ceil(log2 E) of them) gives every
    // lane the mask of the lanes holding its expert (the AND over the bits of
    // the matching ballot or its complement), which ranks the route among its
    // expert's routes (ascending r); lane e forms its own expert's mask from
    // the same ballots for the count.  One shuffle hands each route its
    // expert's base.  Same placement as below.
    int nb = 0;
    while ((1 << nb) < E) ++nb;
    int next = lane < E ? running[lane] : 0;
    auto place = [&](int c, int e) {
      const int r = c * 64 + lane;
      if (r >= n || e < 0 || e >= E) e = -1;
      const uint64_t valid = __ballot(e >= 0);
      uint64_t mine = valid, lane_set = valid;
      for (int k = 0; k < nb; ++k) {
        const uint64_t bk = __ballot(e >= 0 && ((e >> k) & 1));
        mine &= ((e >> k) & 1) ? bk : ~bk;
        lane_set &= ((lane >> k) & 1) ? bk : ~bk;
      }
      const int add = lane < E ? __popcll(lane_set) : 0;
      const int base = __shfl(next, e < 0 ? 0 : e, kWave);
      if (e >= 0) {
        const int pos = base + __popcll(mine & ((1ull << lane) - 1ull));
        sorted_routes[pos] = r;
        route_pos[r] = pos;
      }
      next += add;
    };
    // The held chunks first, from registers: no load sits in this loop, so
    // the scattered stores of successive chunks stay in flight together (a
    // load here would make each chunk wait for the previous chunk's stores,
    // which share the vector memory counter).
#pragma unroll
    for (int i = 0; i < kHeld; ++i) {
      if (c0 + i >= c1) break;
      place(c0 + i, held[i]);
    }
    for (int c = c0 + kHeld; c < c1; ++c) place(c, c * 64 + lane < n ? get(c * 64 + lane) : -1);
    return;
  }
  // More experts than lanes: the same per-bit masks, with the wave's next
  // positions in LDS (running[e]); the first route of each expert in the
  // chunk advances it.
  int nb = 0;
  while ((1 << nb) < E) ++nb;
  const uint64_t below = (1ull << lane) - 1ull;
  for (int c = c0; c < c1; ++c) {
    const int r = c * 64 + lane;
    int e = -1;
    if (r < n) {
      if (c - c0 < kHeld) {
#pragma unroll
        for (int i = 0; i < kHeld; ++i)
          if (c - c0 == i) e = held[i];
      } else {
        e = get(r);
      }
      if (e < 0 || e >= E) e = -1;
    }
    uint64_t mine = __ballot(e >= 0);
    for (int k = 0; k < nb; ++k) {
      const uint64_t bk = __ballot(e >= 0 && ((e >> k) & 1));
      mine &= ((e >> k) & 1) ? bk : ~bk;
    }
    const int rank = __popcll(mine & below);
    const int base = e >= 0 ? running[e] : 0;
    if (e >= 0) {
      const int pos = base + rank;
      sorted_routes[pos] = r;
      route_pos[r] = pos;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (e >= 0 && rank == 0) running[e] = base + __popcll(mine);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

// Few routes: one wavefront does the whole sort (no cross-wave barriers).
static inline int permute_threads(int n) { return n <= 2048 ? 64 : 1024; }

__global__ __launch_bounds__(1024) void moe_permute_kernel(
    const int32_t* __restrict__ expert_ids, int n, int E, int32_t* __restrict__ counts,
    int32_t* __restrict__ offsets, int32_t* __restrict__ sorted_routes,
    int32_t* __restrict__ route_pos) {
  extern __shared__ int32_t cnt[];
  permute_block([&](int r) { return expert_ids[r]; }, n, E, counts, offsets, sorted_routes,
                route_pos, cnt);
}

// Fused pre-MoE RMSNorm + router for decode (context_router.py:62,71-74;
// moe.py:42-66): one workgroup per token, 4 wavefronts.  Every wave
// normalises the token row itself with the arithmetic of rmsnorm_kernel (so
// h2 equals llmy_rmsnorm_f32_bf16's output bit for bit; wave 0 stores it),
// then wave w computes the logits of experts w, w+4, ... straight from W_r in
// global memory: the W_r loads are issued before the norm, so their latency
// overlaps it, and the lanes split D and meet in one wave reduction per
// expert.  Wave 0 takes the top-k and the softmax from the logits in LDS.
// E * D <= 24576 (at most 24 float4 of W_r per lane).
//
// With nparts > 0 the residual row is first completed from the preceding
// projection's per-K-block partial products: x[t] += sum_p parts[p][t]
// (p ascending), or x[t] += gate[t] * sum_p parts[p][t] for a gated residual
// (one fma per element), and the completed row is written back to x.  Every
// wave reads x[t] before the workgroup barrier; wave 0 writes it after it.
constexpr int kMaxParts = 8;
// Rows from which a partial-free call (a prefill) takes the 32-token block kernel.
constexpr int kRouteBlockRows = 256;
// NPM: compile-time bound on nparts (0, 4 or 8) that sizes the slice registers.
template <int NCH, int NPM>
__global__ __launch_bounds__(256) void moe_route_norm_kernel(
    float* __restrict__ x, const float* __restrict__ parts, int nparts,
    const float* __restrict__ gate, const float* __restrict__ ffn_w,
    const float* __restrict__ router_w, const float* __restrict__ w_router,
    uint16_t* __restrict__ h2, int32_t* __restrict__ idx_out, float* __restrict__ gates_out,
    int T, int E, int k, float eps) {
  constexpr int D = NCH * 256;
  constexpr int MAXE = 24 / NCH;  // experts per wave: E <= 4 * MAXE
  __shared__ float lg[4 * MAXE];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x;
  float4 v[NCH], fw[NCH], rw[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int d = 4 * lane + 256 * c;
    v[c] = *reinterpret_cast<const float4*>(x + static_cast<long long>(t) * D + d);
    fw[c] = *reinterpret_cast<const float4*>(ffn_w + d);
    rw[c] = *reinterpret_cast<const float4*>(router_w + d);
  }
  // W_r rows are requested with the row and the partial slices (one round trip)
  float4 wq[MAXE][NCH];
#pragma unroll
  for (int j = 0; j < MAXE; ++j) {
    const int e = min(wave + 4 * j, E - 1);  // clamped: rows past E are loaded but unused
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      wq[j][c] = *reinterpret_cast<const float4*>(w_router + static_cast<long long>(e) * D +
                                                  4 * lane + 256 * c);
  }
  if (NPM > 0 && nparts > 0) {
    constexpr int NPA = NPM > 0 ? NPM : 1;
    float4 pv[NPA][NCH], gv[NCH];
#pragma unroll
    for (int p = 0; p < NPA; ++p) {
      if (p < nparts) {
#pragma unroll
        for (int c = 0; c < NCH; ++c)
          pv[p][c] = *reinterpret_cast<const float4*>(
              parts + (static_cast<long long>(p) * T + t) * D + 4 * lane + 256 * c);
      }
    }
    if (gate) {
#pragma unroll
      for (int c = 0; c < NCH; ++c)
        gv[c] = *reinterpret_cast<const float4*>(gate + static_cast<long long>(t) * D +
                                                 4 * lane + 256 * c);
    }
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      float4 acc = pv[0][c];
#pragma unroll
      for (int p = 1; p < NPA; ++p) {
        if (p < nparts) {
          acc.x += pv[p][c].x;
          acc.y += pv[p][c].y;
          acc.z += pv[p][c].z;
          acc.w += pv[p][c].w;
        }
      }
      if (gate) {
        v[c].x = fmaf(acc.x, gv[c].x, v[c].x);
        v[c].y = fmaf(acc.y, gv[c].y, v[c].y);
        v[c].z = fmaf(acc.z, gv[c].z, v[c].z);
        v[c].w = fmaf(acc.w, gv[c].w, v[c].w);
      } else {
        v[c].x += acc.x;
        v[c].y += acc.y;
        v[c].z += acc.z;
        v[c].w += acc.w;
      }
    }
  }
  float4 xnew[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) xnew[c] = v[c];

  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < NCH; ++c)
    ss += v[c].x * v[c].x + v[c].y * v[c].y + v[c].z * v[c].z + v[c].w * v[c].w;
  const float r1 = rsqrtf(wave_sum(ss) / static_cast<float>(D) + eps);
  float ss2 = 0.f;
  uint16_t* hrow = h2 + static_cast<long long>(t) * D;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int d = 4 * lane + 256 * c;
    const uint32_t lo = pack_bf2(v[c].x * r1 * fw[c].x, v[c].y * r1 * fw[c].y);
    const uint32_t hi = pack_bf2(v[c].z * r1 * fw[c].z, v[c].w * r1 * fw[c].w);
    if (wave == 0) *reinterpret_cast<uint2*>(hrow + d) = make_uint2(lo, hi);
    v[c].x = __uint_as_float(lo << 16);
    v[c].y = __uint_as_float(lo & 0xffff0000u);
    v[c].z = __uint_as_float(hi << 16);
    v[c].w = __uint_as_float(hi & 0xffff0000u);
    ss2 += v[c].x * v[c].x + v[c].y * v[c].y + v[c].z * v[c].z + v[c].w * v[c].w;
  }
  const float r2 = rsqrtf(wave_sum(ss2) / static_cast<float>(D) + eps);
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    v[c].x = (v[c].x * r2) * rw[c].x;
    v[c].y = (v[c].y * r2) * rw[c].y;
    v[c].z = (v[c].z * r2) * rw[c].z;
    v[c].w = (v[c].w * r2) * rw[c].w;
  }
#pragma unroll
  for (int j = 0; j < MAXE; ++j) {
    const int e = wave + 4 * j;
    if (e < E) {
      float a = 0.f;
#pragma unroll
      for (int c = 0; c < NCH; ++c)
        a += (v[c].x * wq[j][c].x + v[c].y * wq[j][c].y) + (v[c].z * wq[j][c].z + v[c].w * wq[j][c].w);
      a = wave_sum(a);
      if (lane == 0) lg[e] = a;
    }
  }
  __syncthreads();
  if (wave != 0) return;
  if (nparts > 0) {
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      *reinterpret_cast<float4*>(x + static_cast<long long>(t) * D + 4 * lane + 256 * c) = xnew[c];
  }
  float mine[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2) {
    const int e = lane + 64 * s2;
    if (e < E) mine[s2] = lg[e];
  }
  topk_softmax_store(mine, E, k, lane, idx_out + t * k, gates_out + t * k);
}

// The same pre-MoE norms and router for a sequence (nparts == 0), 8 TPW
// tokens per workgroup, 8 wavefronts: wave w normalises tokens TPW w ..
// TPW w + TPW - 1 with moe_route_norm_kernel's arithmetic (so h2 is the same
// bits) and keeps the router input rows in LDS (fp32, rows padded to D + 4);
// the logits [32 rows x E <= 32 experts] then run as fp32 MFMAs
// (v_mfma_f32_32x32x2_f32: exact fp32 products, fp32 sums; with 16 tokens
// rows 16..31 repeat rows 0..15 and are not used), wave w over the D/8-wide
// slice w of the row, and the eight partial tiles are added in wave order.
// W_r is read as 16-byte pieces along d straight from global memory
// (L2-resident, 96 KiB at C5), one piece feeding two MFMAs.  Then wave w
// takes the top-k of its tokens.  A token's results do not depend on TPW;
// TPW = 2 gives a 4096-token prefill 256 workgroups, one per CU.
template <int NCH, int TPW>
__global__ __launch_bounds__(512) void moe_route_norm_blk_kernel(
    const float* __restrict__ x, const float* __restrict__ ffn_w,
    const float* __restrict__ router_w, const float* __restrict__ w_router,
    uint16_t* __restrict__ h2, int32_t* __restrict__ idx_out, float* __restrict__ gates_out,
    int T, int E, int k, float eps) {
  constexpr int D = NCH * 256;
  constexpr int RS = D + 4;          // fp32 per LDS row
  constexpr int KW = D / 8;          // d per wave in the logits
  constexpr int TB = 8 * TPW;        // tokens per workgroup
  static_assert(TPW == 2 || TPW == 4, "tokens per wave");
  extern __shared__ float rs[];      // [TB][RS] router input; then [8][32][32] partials
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t0 = blockIdx.x * TB;
  float4 fw[NCH], rw[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int d = 4 * lane + 256 * c;
    fw[c] = *reinterpret_cast<const float4*>(ffn_w + d);
    rw[c] = *reinterpret_cast<const float4*>(router_w + d);
  }
  // ---- norms of tokens TPW wave .. (rows past T: zero router input)
  float4 v[TPW][NCH];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int t = min(t0 + TPW * wave + j, T - 1);
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      v[j][c] = *reinterpret_cast<const float4*>(x + static_cast<long long>(t) * D + 4 * lane +
                                                 256 * c);
  }
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int tl = TPW * wave + j;
    const bool ok = t0 + tl < T;
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      ss += v[j][c].x * v[j][c].x + v[j][c].y * v[j][c].y + v[j][c].z * v[j][c].z +
            v[j][c].w * v[j][c].w;
    const float r1 = rsqrtf(wave_sum(ss) / static_cast<float>(D) + eps);
    float ss2 = 0.f;
    uint16_t* hrow = h2 + static_cast<long long>(t0 + tl) * D;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int d = 4 * lane + 256 * c;
      const uint32_t lo = pack_bf2(v[j][c].x * r1 * fw[c].x, v[j][c].y * r1 * fw[c].y);
      const uint32_t hi = pack_bf2(v[j][c].z * r1 * fw[c].z, v[j][c].w * r1 * fw[c].w);
      if (ok) *reinterpret_cast<uint2*>(hrow + d) = make_uint2(lo, hi);
      v[j][c].x = __uint_as_float(lo << 16);
      v[j][c].y = __uint_as_float(lo & 0xffff0000u);
      v[j][c].z = __uint_as_float(hi << 16);
      v[j][c].w = __uint_as_float(hi & 0xffff0000u);
      ss2 += v[j][c].x * v[j][c].x + v[j][c].y * v[j][c].y + v[j][c].z * v[j][c].z +
             v[j][c].w * v[j][c].w;
    }
    const float r2 = rsqrtf(wave_sum(ss2) / static_cast<float>(D) + eps);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const float4 r = ok ? make_float4((v[j][c].x * r2) * rw[c].x, (v[j][c].y * r2) * rw[c].y,
                                        (v[j][c].z * r2) * rw[c].z, (v[j][c].w * r2) * rw[c].w)
                          : make_float4(0.f, 0.f, 0.f, 0.f);
      *reinterpret_cast<float4*>(rs + tl * RS + 4 * lane + 256 * c) = r;
    }
  }
  __syncthreads();
  // ---- logits: D[token][expert] over d in [KW wave, KW wave + KW); lane l
  // feeds token / expert l % 32 at d offset l / 32 of each 2-wide step
  const int col = lane & 31, hf = lane >> 5;
  const bool e_ok = col < E;
  const float* wrow = w_router + static_cast<long long>(e_ok ? col : 0) * D + KW * wave;
  const float* arow = rs + (col % TB) * RS + KW * wave;
  typedef float f32x16r __attribute__((ext_vector_type(16)));
  f32x16r acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll 4
  for (int u = 0; u < KW / 4; ++u) {
    const float4 a4 = *reinterpret_cast<const float4*>(arow + 4 * u);
    float4 b4 = *reinterpret_cast<const float4*>(wrow + 4 * u);
    if (!e_ok) b4 = make_float4(0.f, 0.f, 0.f, 0.f);
    // step 2u: d = 4u + hf; step 2u + 1: d = 4u + 2 + hf
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(hf ? a4.y : a4.x, hf ? b4.y : b4.x, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(hf ? a4.w : a4.z, hf ? b4.w : b4.z, acc, 0, 0, 0);
  }
  __syncthreads();   // every read of the router rows is done
  float* part = rs + wave * 1024;   // [token][expert] partial of this wave
#pragma unroll
  for (int r = 0; r < 16; ++r) part[((r & 3) + 8 * (r >> 2) + 4 * hf) * 32 + col] = acc[r];
  __syncthreads();
  // ---- wave order sum, then the top-k of tokens TPW wave ..
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int tl = TPW * wave + j;
    if (t0 + tl >= T) break;   // uniform
    float mine[4] = {0.f, 0.f, 0.f, 0.f};
    if (lane < 32) {
      float a = rs[tl * 32 + lane];
#pragma unroll
      for (int w = 1; w < 8; ++w) a += rs[w * 1024 + tl * 32 + lane];
      mine[0] = a;
    }
    topk_softmax_store(mine, E, k, lane, idx_out + static_cast<size_t>(t0 + tl) * k,
                       gates_out + static_cast<size_t>(t0 + tl) * k);
  }
}

}  // namespace llmy

using namespace llmy;

extern "C" int32_t llmy_router_topk_bf16(const uint16_t* x, const float* norm_w,
                                         const float* w_router, float* logits_out, int32_t* idx,
                                         float* gates, int32_t T, int32_t D, int32_t E, int32_t k,
                                         float eps, void* stream) {
  LLMY_REQUIRE(T >= 0 && D > 0 && D % 4 == 0 && D <= 8192);
  LLMY_REQUIRE(E > 0 && E <= 256 && k > 0 && k <= 32 && k <= E);
  if (T == 0) return 0;
  LLMY_REQUIRE(x && w_router && idx && gates);
  LLMY_REQUIRE(aligned(x, 8) && aligned(w_router, 16) && (norm_w == nullptr || aligned(norm_w, 4)));
  const hipStream_t s = as_stream(stream);
  // long sequences: two tokens per wavefront, so each W_r load serves both
  // (four per wavefront were no faster: the per-token reductions remain)
  constexpr int TPW_ = 2;
  const bool many = T >= 1024;
  const dim3 grid(many ? (T + 4 * TPW_ - 1) / (4 * TPW_) : (T + 3) / 4);
#define LLMY_RT(NCH_)                                                                            \
  if (many)                                                                                      \
    hipLaunchKernelGGL((router_topk_bf16_nch_kernel<NCH_, TPW_>), grid, dim3(256), 0, s, x,      \
                       norm_w, w_router, logits_out, idx, gates, T, E, k, eps);                  \
  else                                                                                           \
    hipLaunchKernelGGL((router_topk_bf16_nch_kernel<NCH_, 1>), grid, dim3(256), 0, s, x, norm_w, \
                       w_router, logits_out, idx, gates, T, E, k, eps);                          \
  return launch_status();
  switch (D) {
    case 256: LLMY_RT(1)
    case 512: LLMY_RT(2)
    case 1024: LLMY_RT(4)
    default: break;
  }
#undef LLMY_RT
  const size_t lds = 4 * static_cast<size_t>(D) * sizeof(float);
  hipLaunchKernelGGL(router_topk_bf16_kernel, dim3((T + 3) / 4), dim3(256), lds,
                     as_stream(stream), x, norm_w, w_router, logits_out, idx, gates, T, D, E, k,
                     eps);
  return launch_status();
}

extern "C" int32_t llmy_router_topk_logits_f32(const float* logits, int32_t* idx, float* gates,
                                               int32_t T, int32_t E, int32_t k, void* stream) {
  LLMY_REQUIRE(T >= 0 && E > 0 && E <= 256 && k > 0 && k <= 32 && k <= E);
  if (T == 0) return 0;
  LLMY_REQUIRE(logits && idx && gates);
  hipLaunchKernelGGL(router_topk_from_logits_kernel, dim3((T + 3) / 4), dim3(256), 0,
                     as_stream(stream), logits, idx, gates, T, E, k);
  return launch_status();
}

extern "C" int32_t llmy_moe_permute(const int32_t* expert_ids, int32_t n_routes, int32_t E,
                                    int32_t* counts, int32_t* offsets, int32_t* sorted_routes,
                                    int32_t* route_pos, void* stream) {
  LLMY_REQUIRE(counts && offsets && n_routes >= 0 && E > 0 && E <= 1024);
  LLMY_REQUIRE(n_routes == 0 || (expert_ids && sorted_routes && route_pos));
  const size_t lds = (static_cast<size_t>(kPermuteWaves) * E + E + 1) * sizeof(int32_t);
  hipLaunchKernelGGL(moe_permute_kernel, dim3(1), dim3(permute_threads(n_routes)), lds,
                     as_stream(stream), expert_ids, n_routes, E, counts, offsets, sorted_routes,
                     route_pos);
  return launch_status();
}

extern "C" int32_t llmy_moe_route_decode(float* x, const float* parts, int32_t nparts,
                                         const float* gate, const float* ffn_w,
                                         const float* router_w,
                                         const float* w_router, llmy_bf16* h2, int32_t* idx,
                                         float* gates, int32_t* counts, int32_t* offsets,
                                         int32_t* sorted_routes, int32_t* route_pos, int32_t T,
                                         int32_t D, int32_t E, int32_t k, float eps,
                                         void* stream) {
  LLMY_REQUIRE(T >= 0 && (D == 256 || D == 512 || D == 1024));
  LLMY_REQUIRE(E > 0 && E <= 256 && k > 0 && k <= 8 && k <= E);
  LLMY_REQUIRE(static_cast<long long>(E) * D <= 24576);
  LLMY_REQUIRE(nparts >= 0 && nparts <= kMaxParts && (nparts > 0 || gate == nullptr));
  const bool permute = counts != nullptr;
  LLMY_REQUIRE(!permute || offsets);
  const hipStream_t s = as_stream(stream);
  const size_t perm_lds = (static_cast<size_t>(kPermuteWaves) * E + E + 1) * sizeof(int32_t);
  if (T > 0) {
    LLMY_REQUIRE(x && ffn_w && router_w && w_router && h2 && idx && gates);
    LLMY_REQUIRE(!permute || (sorted_routes && route_pos));
    LLMY_REQUIRE(aligned(x, 16) && aligned(ffn_w, 16) && aligned(router_w, 16) &&
                 aligned(w_router, 16) && aligned(h2, 8));
    LLMY_REQUIRE(nparts == 0 || (parts && aligned(parts, 16) && (!gate || aligned(gate, 16))));
#define LLMY_ROUTE_NP(NCH, NPM)                                                               \
  hipLaunchKernelGGL((moe_route_norm_kernel<NCH, NPM>), dim3(T), dim3(256), 0, s, x, parts,        \
                     nparts, gate, ffn_w, router_w, w_router, h2, idx, gates, T, E, k, eps)
#define LLMY_ROUTE(NCH)                \
  if (nparts == 0) {                   \
    LLMY_ROUTE_NP(NCH, 0);             \
  } else if (nparts <= 4) {            \
    LLMY_ROUTE_NP(NCH, 4);             \
  } else {                             \
    LLMY_ROUTE_NP(NCH, 8);             \
  }
    if (nparts == 0 && T >= kRouteBlockRows && E <= 32) {
      // a sequence: 16 tokens per workgroup, logits on fp32 MFMA
      const dim3 grid((T + 15) / 16);
      const size_t lds = std::max<size_t>(static_cast<size_t>(16) * (D + 4), 8 * 1024) * sizeof(float);
      switch (D) {
        case 256: hipLaunchKernelGGL((moe_route_norm_blk_kernel<1, 2>), grid, dim3(512), lds, s, x, ffn_w, router_w, w_router, h2, idx, gates, T, E, k, eps); break;
        case 512: hipLaunchKernelGGL((moe_route_norm_blk_kernel<2, 2>), grid, dim3(512), lds, s, x, ffn_w, router_w, w_router, h2, idx, gates, T, E, k, eps); break;
        default: hipLaunchKernelGGL((moe_route_norm_blk_kernel<4, 2>), grid, dim3(512), lds, s, x, ffn_w, router_w, w_router, h2, idx, gates, T, E, k, eps); break;
      }
    } else {
      switch (D) {
        case 256: LLMY_ROUTE(1); break;
        case 512: LLMY_ROUTE(2); break;
        default: LLMY_ROUTE(4); break;
      }
    }
#undef LLMY_ROUTE
#undef LLMY_ROUTE_NP
    const int32_t st = launch_status();
    if (st != 0) return st;
  }
  if (!permute) return 0;
  hipLaunchKernelGGL(moe_permute_kernel, dim3(1), dim3(permute_threads(T * k)), perm_lds, s, idx,
                     T * k, E, counts, offsets, sorted_routes, route_pos);
  return launch_status();
}
