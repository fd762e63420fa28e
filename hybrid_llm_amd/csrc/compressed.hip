// Compressed-memory mixers (CSA, HCA): the attention branches and the
// temporal compressor's state.
//
// Both mixers score H heads of width Dh (CSA: index_heads x index_head_dim,
// model/layers/csa.py:21-24; HCA: one head of width d_model, hca.py:24-25)
// against a candidate set and apply the heads' mean probabilities to one
// value stream of width Dv shared by the heads (csa.py:74-75,131,203-206,257):
//   * local branch: the last W tokens, the current one included
//     (csa.py:55-75,185-206; hca.py:46-63,119-138), dense softmax;
//   * memory branch: the compressor's summaries of complete ratio-token
//     blocks (compressed_attention.py:109-123), visible from the block's last
//     token on (csa.py:94,242; hca.py:79,171), dense softmax (hca.py:84-87) or
//     softmax over each head's top_k (csa.py:99-105; hca.py:88-93; ties keep
//     the lower index; invisible entries weigh 0, none visible gives 0).
//
// MI355X mapping:
//   * selection kernels write, per (query, head), a list of probabilities over
//     the candidate slots (dense: the slot is the index) or of (index,
//     probability) pairs (top-k) into a caller workspace; one apply kernel per
//     query then sums the heads (dense lists) in LDS and streams the value rows
//     once per nonzero weight, 4 channels per thread, fp32 accumulation;
//   * prefill scores are MFMA tiles S^T = K Q^T (v_mfma_f32_32x32x16_bf16, 32
//     candidates x 32 queries, operands straight from global memory so any
//     multiple-of-16 head width works), stored scaled and masked to LDS in
//     row passes sized to the candidate count, then each wave reduces its
//     rows;
//   * decode scores use G = min(64, Dh/8) lanes per candidate (16-byte loads,
//     xor-shuffle sums), one workgroup per (row, head);
//   * memory entries carry a tag = position + 1 (0 = empty slot), so zeroed
//     state is an empty memory and row resets are plain row clears.
// D layout of a 32x32 MFMA result: lane l, register r holds row
// (r & 3) + 8 (r >> 2) + 4 (l >> 5), column l & 31.
#include "common.hpp"
#include "abi_util.hpp"

namespace llmy {

typedef float f32x16c __attribute__((ext_vector_type(16)));

constexpr float kLog2eC = 1.4426950408889634f;
enum CmpMode { kBand = 0, kMemDense = 1, kMemTopK = 2 };
constexpr int kCmpLdsBytes = 135168;  // score budget of one prefill selection workgroup

// One wave turns a row of log2-domain scores into a dense list over n slots:
// slot j reads score srow[j + off] and is a candidate when jlo <= j < jhi
// (non-candidates and -inf scores weigh 0; a row with no finite score is 0).
__device__ __forceinline__ void dense_row(const float* srow, int n, int off, int jlo, int jhi,
                                          int lane, float* out) {
  float m = -INFINITY;
  for (int j = lane; j < n; j += kWave)
    if (j >= jlo && j < jhi) m = fmaxf(m, srow[j + off]);
  m = wave_max(m);
  float s = 0.f;
  if (m != -INFINITY)
    for (int j = lane; j < n; j += kWave)
      if (j >= jlo && j < jhi) s += exp2_fast(srow[j + off] - m);
  s = wave_sum(s);
  const float inv = s > 0.f ? 1.0f / s : 0.f;
  for (int j = lane; j < n; j += kWave)
    out[j] = (j >= jlo && j < jhi && inv > 0.f) ? exp2_fast(srow[j + off] - m) * inv : 0.f;
}

// One wave: the k largest of srow[0, n) (ties to the lower index), softmax
// over them; pairs (index, probability) to iout / wout.  Selections that are
// -inf (fewer than k candidates) weigh 0 with index -1.  sel_s / sel_i: the
// wave's 64-entry LDS staging.
//
// n <= 2048: the scores' order keys (order_key: a larger value has a larger
// key) stay in registers, NPL per lane.  With NPL >= 4 a prefilter first
// finds L, the k-th largest of the 64 lanes' maximum keys (k lanes hold a key
// >= L, so every key of the top k is >= L); the keys >= L (about 45 of 1024
// for unordered scores) are compacted, in index order, one per lane, and the
// selection below runs on them alone.  Past 64 survivors, and for NPL < 4, it
// runs on all keys: the k-th largest key is built bit by bit from the top
// (keep a bit when at least k keys are >= the prefix with it set: up to 32
// counting rounds), then every key above it and the lowest-index ones equal
// to it are selected and compacted with ballots.  Larger rows take k rounds
// of a wave argmax over the LDS row (which it consumes).
//
// Threshold search over the keys a lane holds (NK per lane; counts are
// popcounts of compare masks, so it runs in the scalar unit).  It stops as
// soon as exactly k keys are at or above the candidate prefix: those are the
// top k with no tie at the boundary, and the result then marks them as the
// keys above the threshold (the same set and order as a full search).  0:
// fewer than k keys are nonzero.
template <int NK>
__device__ __forceinline__ uint32_t topk_threshold(const uint32_t* key, int k) {
  uint32_t thr = 0;
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t cand = thr | (1u << bit);
    int c = 0;
#pragma unroll
    for (int i = 0; i < NK; ++i) c += __popcll(__ballot(key[i] >= cand));
    if (c >= k) thr = cand;
    if (c == k) {
      thr = cand - 1u;
      break;
    }
  }
  return thr;
}

// Select the top k of the keys (NK per lane, index idx[i]; scores val[i]) by
// threshold thr: every key above it and, of the keys equal to it, the lowest
// indices (keys are visited in index order: i, then lane).  Selected pairs go
// to sel_s / sel_i in index order; returns their count.
template <int NK>
__device__ __forceinline__ int topk_compact(const uint32_t* key, const float* val, const int* idx,
                                            uint32_t thr, int k, int lane, float* sel_s,
                                            int* sel_i) {
  int gt = 0;
#pragma unroll
  for (int i = 0; i < NK; ++i) gt += __popcll(__ballot(key[i] > thr));
  // thr == 0: fewer than k candidates, all of them are taken
  const int need = thr > 0 ? k - gt : 0;
  const uint64_t below = (1ull << lane) - 1ull;
  int taken = 0, eq_seen = 0;
#pragma unroll
  for (int i = 0; i < NK; ++i) {
    const bool eq = thr > 0 && key[i] == thr;
    const uint64_t meq = __ballot(eq);
    const bool sel = key[i] > thr || (eq && eq_seen + __popcll(meq & below) < need);
    eq_seen += __popcll(meq);
    const uint64_t ms = __ballot(sel);
    if (sel) {
      const int at = taken + __popcll(ms & below);
      sel_s[at] = val[i];
      sel_i[at] = idx[i];
    }
    taken += __popcll(ms);
  }
  return taken;
}

// Softmax over the taken selections in sel_s (index order, sel_i their
// indices) to wout / iout; entries past `taken` or at -inf weigh 0 with index -1.
__device__ __forceinline__ void topk_emit(int taken, int k, int lane, const float* sel_s,
                                          const int* sel_i, float* wout, int32_t* iout) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const float v = lane < taken ? sel_s[lane] : -INFINITY;
  const float m = wave_max(lane < k ? v : -INFINITY);
  const float e = (lane < k && v != -INFINITY) ? exp2_fast(v - m) : 0.f;
  const float sum = wave_sum(e);
  if (lane < k) {
    wout[lane] = sum > 0.f ? e / sum : 0.f;
    iout[lane] = v != -INFINITY ? sel_i[lane] : -1;
  }
}

template <int NPL>
__device__ __forceinline__ void topk_regs(const float* srow, int n, int k, int lane, float* wout,
                                          int32_t* iout, float* sel_s, int* sel_i) {
  uint32_t key[NPL];
#pragma unroll
  for (int i = 0; i < NPL; ++i) {
    const int j = i * kWave + lane;
    key[i] = j < n ? order_key(srow[j]) : 0u;   // 0: below every real key
  }
  const uint64_t below = (1ull << lane) - 1ull;
  int taken = -1;
  if (NPL >= 4) {
    uint32_t lm = key[0];
#pragma unroll
    for (int i = 1; i < NPL; ++i) lm = max(lm, key[i]);
    // at least k lane maxima are >= lbound (0: fewer than k lanes hold a key)
    const uint32_t lbound = topk_threshold<1>(&lm, k);
    int nsv = 0;
#pragma unroll
    for (int i = 0; i < NPL; ++i) nsv += __popcll(__ballot(key[i] >= lbound));
    if (lbound > 0u && nsv <= kWave) {
      // survivors, in index order, to sel_i; then one per lane
      int at0 = 0;
#pragma unroll
      for (int i = 0; i < NPL; ++i) {
        const bool sv = key[i] >= lbound;
        const uint64_t m = __ballot(sv);
        if (sv) sel_i[at0 + __popcll(m & below)] = i * kWave + lane;
        at0 += __popcll(m);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const int idx = lane < nsv ? sel_i[lane] : 0;
      const float val = lane < nsv ? srow[idx] : -INFINITY;
      const uint32_t ky = lane < nsv ? order_key(val) : 0u;
      const uint32_t thr = topk_threshold<1>(&ky, k);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      taken = topk_compact<1>(&ky, &val, &idx, thr, k, lane, sel_s, sel_i);
    }
  }
  if (taken < 0) {
    float val[NPL];
    int idx[NPL];
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      idx[i] = i * kWave + lane;
      val[i] = idx[i] < n ? srow[idx[i]] : -INFINITY;
    }
    taken = topk_compact<NPL>(key, val, idx, topk_threshold<NPL>(key, k), k, lane, sel_s, sel_i);
  }
  topk_emit(taken, k, lane, sel_s, sel_i, wout, iout);
}

__device__ __forceinline__ void topk_row(float* srow, int n, int k, int lane, float* wout,
                                         int32_t* iout, float* sel_s, int* sel_i) {
  if (n <= 128) return topk_regs<2>(srow, n, k, lane, wout, iout, sel_s, sel_i);
  if (n <= 256) return topk_regs<4>(srow, n, k, lane, wout, iout, sel_s, sel_i);
  if (n <= 512) return topk_regs<8>(srow, n, k, lane, wout, iout, sel_s, sel_i);
  if (n <= 1024) return topk_regs<16>(srow, n, k, lane, wout, iout, sel_s, sel_i);
  if (n <= 2048) return topk_regs<32>(srow, n, k, lane, wout, iout, sel_s, sel_i);
  float mine = -INFINITY;
  int32_t mine_idx = -1;
  for (int it = 0; it < k; ++it) {
    uint64_t best = 0;
    for (int j = lane; j < n; j += kWave) best = umax64(best, value_index_key(srow[j], j));
    best = wave_max_u64(best);
    const int idx = static_cast<int>(key_index(best));
    const bool ok = best != 0 && idx >= 0 && idx < n;
    const float v = ok ? srow[idx] : -INFINITY;
    if (lane == it) {
      mine = v;
      mine_idx = (ok && v != -INFINITY) ? idx : -1;
    }
    __builtin_amdgcn_wave_barrier();
    if (ok && lane == 0) srow[idx] = -INFINITY;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  const float m = wave_max(lane < k ? mine : -INFINITY);
  const float e = (lane < k && mine != -INFINITY) ? exp2_fast(mine - m) : 0.f;
  const float s = wave_sum(e);
  if (lane < k) {
    wout[lane] = s > 0.f ? e / s : 0.f;
    iout[lane] = mine_idx;
  }
}

// ---------------------------------------------------------------- prefill
// Workgroup = (head h, 32-query block, row b), h fastest; NW waves (top-k: 16,
// four per SIMD, so the scores' load latency and the selections' scalar
// chains of one wave hide behind the others' -- the block's score rows fill
// up to 132 KiB of LDS and a CU holds one workgroup).  Candidates:
//   band: keys [max(0, t0 - W + 1), min(T - 1, t0 + 31)] of row b (q/k rows
//         b*T + t); the list of query t has W slots, slot j = key t - W + 1 + j;
//   memory: entries [0, nv), nv = min(n, min(T, t0 + 32) / ratio) (rows b*n + i,
//         entry i visible from position (i + 1) ratio - 1 on and, with W > 0 (the
//         decode memory's slots), while it is among the last W entries emitted,
//         i >= (t + 1) / ratio - W, as a token-by-token decode sees them);
//         dense lists have n slots, top-k lists top_k pairs.
// NS = head_dim / 16 when it is at most 8: the 32 queries' fragments stay in
// registers through a pass's scores (128 VGPRs hold a wave at four per SIMD,
// so a tile's fragments are not prefetched); NS = 0: any multiple-of-16 head
// width, operands loaded per 16-wide slice.
// NW waves per workgroup: 16 for top-k lists and for wide heads (NS = 0);
// dense lists of 64- / 128-wide heads (a softmax per row, no selection) run
// 4-wave workgroups, several per CU.
template <int MODE, int NS>
constexpr int sel_waves() {
  return MODE == kMemTopK || NS == 0 ? 16 : 4;
}

template <int MODE, int NS, int NW>
__global__ __launch_bounds__(64 * NW) void cmp_select_prefill_kernel(
    const uint16_t* __restrict__ q, int64_t q_ld, const uint16_t* __restrict__ k, int64_t k_ld,
    int T, int n, int H, int Dh, int W, int ratio, int top_k, int Kmax, int rows_pass,
    float scale_log2, float* __restrict__ wl, int32_t* __restrict__ il) {
  extern __shared__ float sc[];
  __shared__ float sel_s[MODE == kMemTopK ? NW : 1][kWave];
  __shared__ int sel_i[MODE == kMemTopK ? NW : 1][kWave];
  const int h = blockIdx.x % H;
  const int rest = blockIdx.x / H;
  const int nqb = (T + 31) / 32;
  // memory: later query blocks see more entries; they are dispatched first so
  // the short blocks fill in behind them
  const int qb = MODE == kBand ? rest % nqb : nqb - 1 - rest % nqb;
  const int b = rest / nqb;
  const int t0 = qb * 32;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 31, half = lane >> 5;
  int c_lo, nc;
  if (MODE == kBand) {
    c_lo = max(0, t0 - W + 1);
    nc = min(T - 1, t0 + 31) - c_lo + 1;
  } else {
    c_lo = 0;
    nc = min(n, min(T, t0 + 32) / ratio);
  }
  const int ntile = (nc + 31) / 32;
  const int ncp = max(ntile, 1) * 32;
  // score rows one float longer than the candidates: the 32 queries of a tile
  // store each candidate's score to 32 different banks
  const int rsd = ncp + 1;
  const bool q_ok = t0 + col < T;
  const uint16_t* qrow =
      q + static_cast<int64_t>(b * T + (q_ok ? t0 + col : 0)) * q_ld + h * Dh + 8 * half;
  const int64_t krow0 = MODE == kBand ? static_cast<int64_t>(b) * T : static_cast<int64_t>(b) * n;
  constexpr int NQ = NS > 0 ? NS : 1;
  // candidate row of this lane in a tile (past the candidates: the first one,
  // whose score the visibility test below replaces)
  auto krow_of = [&](int tile) {
    const int c0 = c_lo + 32 * tile;
    const bool ok = c0 + col < c_lo + nc;
    return k + (krow0 + (ok ? c0 + col : c_lo)) * k_ld + h * Dh + 8 * half;
  };
  // The candidates query t = t0 + col sees form one interval [vlo, vlo + vspan]:
  // band: max(t - W + 1, c_lo) .. min(t, last candidate); memory: entry i with
  // (i + 1) ratio - 1 <= t, i.e. i < (t + 1) / ratio, and with W > 0 i >=
  // (t + 1) / ratio - W.  An empty interval (or t >= T) puts vlo out of reach.
  int vlo, vspan;
  {
    const int t = t0 + col;
    int lo, hi;
    if (MODE == kBand) {
      lo = max(t - W + 1, c_lo);
      hi = min(t, c_lo + nc - 1);
    } else {
      const int e = (t + 1) / ratio;
      lo = W > 0 ? max(e - W, 0) : 0;
      hi = min(e, nc) - 1;
    }
    const bool any = q_ok && lo <= hi;
    vlo = any ? lo : (1 << 30);
    vspan = any ? hi - lo : 0;
  }
  for (int p0 = 0; p0 < 32; p0 += rows_pass) {
    // the queries' fragments, per pass (dead during the selection)
    uint4 qf[NQ];
    if (NS > 0) {
#pragma unroll
      for (int s = 0; s < NQ; ++s)
        qf[s] = q_ok ? *reinterpret_cast<const uint4*>(qrow + 16 * s) : uint4{0, 0, 0, 0};
    }
    if (ntile == 0) {   // no candidate yet (memory before the first block end)
      for (int i = threadIdx.x; i < rows_pass * rsd; i += 64 * NW) sc[i] = -INFINITY;
    }
    auto store_scores = [&](int tile, const f32x16c& acc) {
      const int row = col - p0;
      if (row >= 0 && row < rows_pass) {
        const int c0 = c_lo + 32 * tile;
        float* dst = sc + row * rsd - c_lo;   // indexed by candidate
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int cj = c0 + (r & 3) + 8 * (r >> 2) + 4 * half;
          const bool vis = static_cast<unsigned>(cj - vlo) <= static_cast<unsigned>(vspan);
          dst[cj] = vis ? acc[r] * scale_log2 : -INFINITY;
        }
      }
    };
    if (NS > 0) {
      // two tiles per round: both tiles' candidate rows are requested together
      for (int tile = wave; tile < ntile; tile += 2 * NW) {
        const int tile2 = tile + NW;
        const bool two = tile2 < ntile;
        uint4 a[NQ], a2[NQ];
        const uint16_t* kr = krow_of(tile);
        const uint16_t* kr2 = krow_of(two ? tile2 : tile);
#pragma unroll
        for (int s = 0; s < NQ; ++s) {
          a[s] = *reinterpret_cast<const uint4*>(kr + 16 * s);
          a2[s] = *reinterpret_cast<const uint4*>(kr2 + 16 * s);
        }
        f32x16c acc, acc2;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = acc2[r] = 0.f;
#pragma unroll
        for (int s = 0; s < NQ; ++s)
          acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a[s]), as_bf16x8(qf[s]), acc,
                                                        0, 0, 0);
        if (two) {
#pragma unroll
          for (int s = 0; s < NQ; ++s)
            acc2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a2[s]), as_bf16x8(qf[s]),
                                                           acc2, 0, 0, 0);
        }
        store_scores(tile, acc);
        if (two) store_scores(tile2, acc2);
      }
    } else {
      for (int tile = wave; tile < ntile; tile += NW) {
        f32x16c acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.f;
        const uint16_t* kr = krow_of(tile);
#pragma unroll 4
        for (int s = 0; s < Dh / 16; ++s) {
          const uint4 a = *reinterpret_cast<const uint4*>(kr + 16 * s);
          const uint4 bq =
              q_ok ? *reinterpret_cast<const uint4*>(qrow + 16 * s) : uint4{0, 0, 0, 0};
          acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), as_bf16x8(bq), acc, 0, 0,
                                                        0);
        }
        store_scores(tile, acc);
      }
    }
    __syncthreads();
    for (int row = wave; row < rows_pass; row += NW) {
      const int t = t0 + p0 + row;
      if (t >= T) continue;
      float* srow = sc + row * rsd;
      const int64_t lb = (static_cast<int64_t>(b * T + t) * H + h) * Kmax;
      if (MODE == kBand) {
        // slot j <-> key t - W + 1 + j (a candidate when >= 0) <-> score
        // index key - c_lo, inside the row for every candidate key
        dense_row(srow, W, t - W + 1 - c_lo, max(0, W - 1 - t), W, lane, wl + lb);
      } else if (MODE == kMemDense) {
        dense_row(srow, Kmax, 0, 0, nc, lane, wl + lb);
      } else {
        topk_row(srow, nc, top_k, lane, wl + lb, il + lb, sel_s[wave], sel_i[wave]);
      }
    }
    __syncthreads();
  }
}

// Launch of the prefill selection: NS specialised for head widths 64 / 128.
template <int MODE>
void select_prefill_launch(dim3 grid, size_t lds, hipStream_t s, const uint16_t* q, int64_t q_ld,
                           const uint16_t* k, int64_t k_ld, int T, int n, int H, int Dh, int W,
                           int ratio, int top_k, int Kmax, int rows, float scale_log2, float* wl,
                           int32_t* il) {
  if (Dh == 128)
    hipLaunchKernelGGL((cmp_select_prefill_kernel<MODE, 8, sel_waves<MODE, 8>()>), grid,
                       dim3(64 * sel_waves<MODE, 8>()), lds, s, q, q_ld, k, k_ld, T, n, H, Dh, W,
                       ratio, top_k, Kmax, rows, scale_log2, wl, il);
  else if (Dh == 64)
    hipLaunchKernelGGL((cmp_select_prefill_kernel<MODE, 4, sel_waves<MODE, 4>()>), grid,
                       dim3(64 * sel_waves<MODE, 4>()), lds, s, q, q_ld, k, k_ld, T, n, H, Dh, W,
                       ratio, top_k, Kmax, rows, scale_log2, wl, il);
  else
    hipLaunchKernelGGL((cmp_select_prefill_kernel<MODE, 0, sel_waves<MODE, 0>()>), grid,
                       dim3(64 * sel_waves<MODE, 0>()), lds, s, q, q_ld, k, k_ld, T, n, H, Dh, W,
                       ratio, top_k, Kmax, rows, scale_log2, wl, il);
}

// ---------------------------------------------------------------- decode
// Scores: workgroup = (chunk of 16 * 64 / G candidates, head h, row b), chunk
// fastest; each wave scores 4 passes of 64 / G candidates with G lanes per
// candidate (16-byte loads, xor-shuffle sums) and writes them, log2-scaled,
// -inf for non-candidates, to sc [B, H, ncand].  band: candidate j in [0, W) <-> key p - W + 1 + j
// (p = pos[b]; keys < 0 are not candidates), the current key from k_new,
// older ones from the ring (slot key % W); chunk 0 also stores its head's slice
// of k_new (and head 0 the v_new row) into slot p % W, which held key p - W,
// outside this step's window.  memory: candidates are the C slots, visible
// when 1 <= tag <= p + 1.
template <int MODE, int G>
__global__ __launch_bounds__(256) void cmp_score_decode_kernel(
    const uint16_t* __restrict__ q, int64_t q_ld, const uint16_t* __restrict__ k_new,
    const uint16_t* __restrict__ v_new, int64_t kv_ld, uint16_t* __restrict__ ring_k,
    uint16_t* __restrict__ ring_v, const uint16_t* __restrict__ mk,
    const int32_t* __restrict__ mtag, const int32_t* __restrict__ pos, int H, int Dh, int Dv,
    int W, int C, float scale_log2, float* __restrict__ sc) {
  constexpr int kCpw = kWave / G;        // candidates per wave pass
  constexpr int kPasses = 4;
  constexpr int kChunk = 4 * kPasses * kCpw;   // candidates per workgroup
  const int ncand = MODE == kBand ? W : C;
  const int nchunk = (ncand + kChunk - 1) / kChunk;
  const int chunk = blockIdx.x % nchunk;
  const int bh = blockIdx.x / nchunk;
  const int h = bh % H;
  const int b = bh / H;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int p = max(pos[b], 0);   // positions are >= 0; the clamp keeps slots in range
  const int Kw = H * Dh;
  if (MODE == kBand && chunk == 0) {
    uint16_t* kslot = ring_k + (static_cast<int64_t>(b) * W + p % W) * Kw + h * Dh;
    const uint16_t* ksrc = k_new + static_cast<int64_t>(b) * kv_ld + h * Dh;
    for (int c = threadIdx.x; c < Dh / 8; c += 256)
      reinterpret_cast<uint4*>(kslot)[c] = reinterpret_cast<const uint4*>(ksrc)[c];
    if (h == 0) {
      uint16_t* vslot = ring_v + (static_cast<int64_t>(b) * W + p % W) * Dv;
      const uint16_t* vsrc = v_new + static_cast<int64_t>(b) * kv_ld;
      for (int c = threadIdx.x; c < Dv / 8; c += 256)
        reinterpret_cast<uint4*>(vslot)[c] = reinterpret_cast<const uint4*>(vsrc)[c];
    }
  }
  const int nch = Dh / 8 / G;                 // 16-byte chunks per lane
  const int gl = lane % G;
  const uint16_t* qh = q + static_cast<int64_t>(b) * q_ld + h * Dh;
  float* srow = sc + static_cast<int64_t>(bh) * ncand;
  // every pass's key row first (rows of invisible candidates are clamped in
  // range and read anyway), so the passes' key loads are in flight together
  int cs[kPasses];
  bool vis[kPasses];
  const uint16_t* kr[kPasses];
#pragma unroll
  for (int ps = 0; ps < kPasses; ++ps) {
    const int c = chunk * kChunk + wave * (kPasses * kCpw) + ps * kCpw + lane / G;
    cs[ps] = c;
    vis[ps] = c < ncand;
    if (MODE == kBand) {
      const int key = p - W + 1 + c;
      vis[ps] = vis[ps] && key >= 0;
      kr[ps] = key == p ? k_new + static_cast<int64_t>(b) * kv_ld + h * Dh
                        : ring_k + (static_cast<int64_t>(b) * W + (key >= 0 ? key % W : 0)) * Kw +
                              h * Dh;
    } else {
      const int cc = c < ncand ? c : 0;
      const int tag = mtag[static_cast<int64_t>(b) * C + cc];
      vis[ps] = vis[ps] && tag >= 1 && tag <= p + 1;
      kr[ps] = mk + (static_cast<int64_t>(b) * C + cc) * Kw + h * Dh;
    }
  }
  float dot[kPasses];
#pragma unroll
  for (int ps = 0; ps < kPasses; ++ps) dot[ps] = 0.f;
  for (int ch = 0; ch < nch; ++ch) {
    const int e = 8 * (gl + G * ch);
    uint4 kk[kPasses];
#pragma unroll
    for (int ps = 0; ps < kPasses; ++ps) kk[ps] = ld_stream(kr[ps] + e);
    float a[8];
    unpack8(*reinterpret_cast<const uint4*>(qh + e), a);
#pragma unroll
    for (int ps = 0; ps < kPasses; ++ps) {
      float bb[8];
      unpack8(kk[ps], bb);
#pragma unroll
      for (int i = 0; i < 8; ++i) dot[ps] = fmaf(a[i], bb[i], dot[ps]);
    }
  }
#pragma unroll
  for (int ps = 0; ps < kPasses; ++ps) {
    float d = dot[ps];
#pragma unroll
    for (int o = G / 2; o >= 1; o >>= 1) d += __shfl_xor(d, o, kWave);
    if (gl == 0 && cs[ps] < ncand) srow[cs[ps]] = vis[ps] ? d * scale_log2 : -INFINITY;
  }
}

// Lists: one wave per (head h, row b) turns its score row into the dense list
// (W or C slots) or the top_k (index, probability) pairs.
template <int MODE>
__global__ __launch_bounds__(64) void cmp_list_decode_kernel(const float* __restrict__ sc,
                                                             int ncand, int top_k, int Kmax,
                                                             float* __restrict__ wl,
                                                             int32_t* __restrict__ il) {
  extern __shared__ float srow[];
  __shared__ float sel_s[kWave];
  __shared__ int sel_i[kWave];
  const int bh = blockIdx.x;
  const int lane = threadIdx.x;
  for (int j = lane; j < ncand; j += kWave) srow[j] = sc[static_cast<int64_t>(bh) * ncand + j];
  __syncthreads();
  const int64_t lb = static_cast<int64_t>(bh) * Kmax;
  if (MODE == kMemTopK) topk_row(srow, ncand, top_k, lane, wl + lb, il + lb, sel_s, sel_i);
  else dense_row(srow, ncand, 0, 0, ncand, lane, wl + lb);
}

// Scores and list of one (head h, row b) in one workgroup, for rows of at
// most kFusedMaxCand candidates when B * H is large enough to fill the GPU:
// the same per-candidate dot products as cmp_score_decode_kernel (G lanes,
// 16-byte chunks in order, xor-shuffle sums), so the scores are bitwise the
// same, written to LDS instead of sc; then wave 0 forms the list as
// cmp_list_decode_kernel does.  Candidate c of pass ps: ps * 4 * (64 / G) +
// wave * (64 / G) + lane / G; the key rows of PB passes are loaded together.
constexpr int kFusedMaxCand = 1024;

template <int MODE, int G>
__global__ __launch_bounds__(256) void cmp_score_list_decode_kernel(
    const uint16_t* __restrict__ q, int64_t q_ld, const uint16_t* __restrict__ k_new,
    const uint16_t* __restrict__ v_new, int64_t kv_ld, uint16_t* __restrict__ ring_k,
    uint16_t* __restrict__ ring_v, const uint16_t* __restrict__ mk,
    const int32_t* __restrict__ mtag, const int32_t* __restrict__ pos, int H, int Dh, int Dv,
    int W, int C, float scale_log2, int top_k, int Kmax, float* __restrict__ wl,
    int32_t* __restrict__ il) {
  extern __shared__ float srow[];
  __shared__ float sel_s[kWave];
  __shared__ int sel_i[kWave];
  constexpr int kCpw = kWave / G;   // candidates per wave pass
  constexpr int PB = 8;             // passes whose key rows are in flight together
  const int ncand = MODE == kBand ? W : C;
  const int bh = blockIdx.x;
  const int h = bh % H;
  const int b = bh / H;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int p = max(pos[b], 0);
  const int Kw = H * Dh;
  if (MODE == kBand) {   // this head's slice of k_new (head 0: the v_new row) to slot p % W
    uint16_t* kslot = ring_k + (static_cast<int64_t>(b) * W + p % W) * Kw + h * Dh;
    const uint16_t* ksrc = k_new + static_cast<int64_t>(b) * kv_ld + h * Dh;
    for (int c = threadIdx.x; c < Dh / 8; c += 256)
      reinterpret_cast<uint4*>(kslot)[c] = reinterpret_cast<const uint4*>(ksrc)[c];
    if (h == 0) {
      uint16_t* vslot = ring_v + (static_cast<int64_t>(b) * W + p % W) * Dv;
      const uint16_t* vsrc = v_new + static_cast<int64_t>(b) * kv_ld;
      for (int c = threadIdx.x; c < Dv / 8; c += 256)
        reinterpret_cast<uint4*>(vslot)[c] = reinterpret_cast<const uint4*>(vsrc)[c];
    }
  }
  const int nch = Dh / 8 / G;
  const int gl = lane % G;
  const uint16_t* qh = q + static_cast<int64_t>(b) * q_ld + h * Dh;
  const int per_pass = 4 * kCpw;
  const int npass = (ncand + per_pass - 1) / per_pass;
  for (int p0 = 0; p0 < npass; p0 += PB) {
    int cs[PB];
    bool vis[PB];
    const uint16_t* kr[PB];
#pragma unroll
    for (int ps = 0; ps < PB; ++ps) {
      const int c = (p0 + ps) * per_pass + wave * kCpw + lane / G;
      cs[ps] = c;
      vis[ps] = c < ncand;
      if (MODE == kBand) {
        const int key = p - W + 1 + c;
        vis[ps] = vis[ps] && key >= 0;
        kr[ps] = key == p ? k_new + static_cast<int64_t>(b) * kv_ld + h * Dh
                          : ring_k + (static_cast<int64_t>(b) * W + (key >= 0 ? key % W : 0)) *
                                         Kw + h * Dh;
      } else {
        const int cc = c < ncand ? c : 0;
        const int tag = mtag[static_cast<int64_t>(b) * C + cc];
        vis[ps] = vis[ps] && tag >= 1 && tag <= p + 1;
        kr[ps] = mk + (static_cast<int64_t>(b) * C + cc) * Kw + h * Dh;
      }
    }
    float dot[PB];
#pragma unroll
    for (int ps = 0; ps < PB; ++ps) dot[ps] = 0.f;
    for (int ch = 0; ch < nch; ++ch) {
      const int e = 8 * (gl + G * ch);
      uint4 kk[PB];
#pragma unroll
      for (int ps = 0; ps < PB; ++ps) kk[ps] = ld_stream(kr[ps] + e);
      float a[8];
      unpack8(*reinterpret_cast<const uint4*>(qh + e), a);
#pragma unroll
      for (int ps = 0; ps < PB; ++ps) {
        float bb[8];
        unpack8(kk[ps], bb);
#pragma unroll
        for (int i = 0; i < 8; ++i) dot[ps] = fmaf(a[i], bb[i], dot[ps]);
      }
    }
#pragma unroll
    for (int ps = 0; ps < PB; ++ps) {
      float d = dot[ps];
#pragma unroll
      for (int o = G / 2; o >= 1; o >>= 1) d += __shfl_xor(d, o, kWave);
      if (gl == 0 && cs[ps] < ncand) srow[cs[ps]] = vis[ps] ? d * scale_log2 : -INFINITY;
    }
  }
  __syncthreads();
  if (wave != 0) return;
  const int64_t lb = static_cast<int64_t>(bh) * Kmax;
  if (MODE == kMemTopK) topk_row(srow, ncand, top_k, lane, wl + lb, il + lb, sel_s, sel_i);
  else dense_row(srow, ncand, 0, 0, ncand, lane, wl + lb);
}

// ---------------------------------------------------------------- apply
// Workgroup = (256-channel block, block of QB consecutive queries of one row),
// channel block fastest; query b*T + t sits at position qpos[b] (qpos NULL:
// t; decode runs QB = 1).  Block slots: memory slot j, or for the band key
// t0 - W + 1 + js with t0 the block's first position, so query t's band slot j
// is block slot j + (t - t0).  First the heads' lists become one weight per
// (query, slot) in LDS: dense lists (il NULL; nslots == Kmax) are summed over
// the heads slot by slot; (index, probability) pairs are added head by head
// (one head's indices are distinct, so each sum runs in head order and the
// result does not depend on scheduling).  Wave 0 compacts the slots any query
// uses; the NW waves split them, each lane 4 channels of every query, so a
// value row is read once for the block; partial sums are added in wave order.
// out = sum / H.  Value key -> row b * rows_per_b + (wrap ? key % wrap : key)
// at v_ld.
constexpr int kApplyMaxH = 16;  // heads whose selections are read in one round trip
#ifndef LLMY_APPLY_DECODE_WAVES
#define LLMY_APPLY_DECODE_WAVES 8
#endif
// single queries: few workgroups per row, so more waves share a row's slots
constexpr int kApplyDecodeWaves = LLMY_APPLY_DECODE_WAVES;

// 8-byte load of a value row piece.  Single-query (decode) applies read each
// row once per step, so their loads carry the non-temporal hint (with
// LLMY_NT); multi-query blocks re-read rows across query blocks and keep the
// plain load.
template <bool kStream>
__device__ __forceinline__ uint2 ld_row8(const uint16_t* p) {
#if defined(LLMY_NT) && LLMY_NT
  if constexpr (kStream) {
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
    return uint2{v.x, v.y};
  }
#endif
  return *reinterpret_cast<const uint2*>(p);
}

template <int QB, int NW>
__global__ __launch_bounds__(64 * NW) void cmp_apply_kernel(
    const float* __restrict__ wl, const int32_t* __restrict__ il, int Kmax, int H, int T,
    const int32_t* __restrict__ qpos, int band_W, int nslots, const uint16_t* __restrict__ v,
    int64_t v_ld, int rows_per_b, int wrap, uint16_t* __restrict__ out, int64_t out_ld,
    int Dv) {
  extern __shared__ float pm[];
  const int nsb = band_W > 0 ? nslots + QB - 1 : nslots;   // block slots
  const int nsp = (nsb + 3) & ~3;
  constexpr int NT = 64 * NW;
  float* red = pm + QB * nsp;                          // [NW][256] partial sums
  int* nz = reinterpret_cast<int*>(red + NW * 256);    // [nsb] compacted slots
  __shared__ int nz_count;
  const int ndb = (Dv + 255) / 256;
  const int nqb = (T + QB - 1) / QB;
  const int blk = blockIdx.x / ndb;
  const int db = blockIdx.x - blk * ndb;
  const int b = blk / nqb;
  const int t0 = (blk - b * nqb) * QB;
  const int nq = min(QB, T - t0);
  const int p0 = qpos ? max(qpos[b], 0) : t0;
  for (int i = threadIdx.x; i < QB * nsp; i += NT) pm[i] = 0.f;
  __syncthreads();
  const int64_t lb0 = (static_cast<int64_t>(b) * T + t0) * H * Kmax;
  if (il && H <= kApplyMaxH && nq * Kmax <= 512) {
    // every head's (slot, weight) entries requested at once (at most RE per
    // thread per head), then added head by head: a head's slots are
    // distinct, so each pass is race-free and every slot sums its heads in
    // head order
    constexpr int RE = (512 + NT - 1) / NT;
    float wr[kApplyMaxH][RE];
    int ir[kApplyMaxH][RE], pr[RE];
#pragma unroll
    for (int r = 0; r < RE; ++r) {
      const int e = threadIdx.x + NT * r;
      pr[r] = e < nq * Kmax ? (e / Kmax) * nsp : -1;
    }
#pragma unroll
    for (int hh = 0; hh < kApplyMaxH; ++hh)
#pragma unroll
      for (int r = 0; r < RE; ++r) {
        const int e = threadIdx.x + NT * r;
        const bool ok = hh < H && pr[r] >= 0;
        const int qq = e / Kmax, j = e - qq * Kmax;
        const int64_t o = lb0 + (static_cast<int64_t>(qq) * H + hh) * Kmax + j;
        wr[hh][r] = ok ? wl[o] : 0.f;
        ir[hh][r] = ok ? il[o] : -1;
      }
#pragma unroll
    for (int hh = 0; hh < kApplyMaxH; ++hh) {
      if (hh >= H) break;  // uniform
#pragma unroll
      for (int r = 0; r < RE; ++r)
        if (ir[hh][r] >= 0 && ir[hh][r] < nslots) pm[pr[r] + ir[hh][r]] += wr[hh][r];
      __syncthreads();
    }
  } else if (il) {
    for (int hh = 0; hh < H; ++hh) {
      for (int e = threadIdx.x; e < nq * Kmax; e += NT) {
        const int qq = e / Kmax, j = e - qq * Kmax;
        const int64_t o = lb0 + (static_cast<int64_t>(qq) * H + hh) * Kmax + j;
        const int idx = il[o];
        if (idx >= 0 && idx < nslots) pm[qq * nsp + idx] += wl[o];
      }
      __syncthreads();
    }
  } else {
    for (int e = threadIdx.x; e < nq * nslots; e += NT) {
      const int qq = e / nslots, j = e - qq * nslots;
      const int64_t o = lb0 + static_cast<int64_t>(qq) * H * Kmax + j;
      float acc = 0.f;
      for (int hh = 0; hh < H; ++hh) acc += wl[o + static_cast<int64_t>(hh) * Kmax];
      pm[qq * nsp + j + (band_W > 0 ? qq : 0)] = acc;
    }
    __syncthreads();
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (wave == 0) {
    int cnt = 0;
    for (int j0 = 0; j0 < nsb; j0 += kWave) {
      const int j = j0 + lane;
      bool live = false;
      if (j < nsb)
#pragma unroll
        for (int qq = 0; qq < QB; ++qq) live = live || pm[qq * nsp + j] != 0.f;
      const uint64_t m = __ballot(live);
      if (live) nz[cnt + __popcll(m & ((1ull << lane) - 1ull))] = j;
      cnt += __popcll(m);
    }
    if (lane == 0) nz_count = cnt;
  }
  __syncthreads();
  const int n = nz_count;
  const int c0 = db * 256 + 4 * lane;
  const int cc = c0 < Dv ? c0 : 0;   // lanes past Dv read a valid column, store nothing
  const int base = band_W > 0 ? p0 - band_W + 1 : 0;
  const uint16_t* vb = v + static_cast<int64_t>(b) * rows_per_b * v_ld + cc;
  auto row_of = [&](int j) {
    const int key = base + j;
    return static_cast<int64_t>(wrap ? key % wrap : key) * v_ld;
  };
  float acc[QB][4];
#pragma unroll
  for (int qq = 0; qq < QB; ++qq)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[qq][c] = 0.f;
  auto add = [&](int j, const uint2& r) {
    const float x0 = __uint_as_float(r.x << 16), x1 = __uint_as_float(r.x & 0xffff0000u);
    const float x2 = __uint_as_float(r.y << 16), x3 = __uint_as_float(r.y & 0xffff0000u);
#pragma unroll
    for (int qq = 0; qq < QB; ++qq) {
      const float w = pm[qq * nsp + j];
      acc[qq][0] = fmaf(w, x0, acc[qq][0]);
      acc[qq][1] = fmaf(w, x1, acc[qq][1]);
      acc[qq][2] = fmaf(w, x2, acc[qq][2]);
      acc[qq][3] = fmaf(w, x3, acc[qq][3]);
    }
  };
  // RU rows in flight per wave (a single query has few workgroups per row, so
  // the sweep is latency-bound); each wave still adds its rows in slot order
  constexpr int RU = QB == 1 ? 16 : 4;
  int i = wave;
  for (; i + NW * (RU - 1) < n; i += NW * RU) {
    int jj[RU];
    uint2 rr[RU];
#pragma unroll
    for (int u = 0; u < RU; ++u) jj[u] = nz[i + NW * u];
#pragma unroll
    for (int u = 0; u < RU; ++u) rr[u] = ld_row8<QB == 1>(vb + row_of(jj[u]));
#pragma unroll
    for (int u = 0; u < RU; ++u) add(jj[u], rr[u]);
  }
  for (; i + 3 * NW < n; i += 4 * NW) {
    const int j0 = nz[i], j1 = nz[i + NW], j2 = nz[i + 2 * NW], j3 = nz[i + 3 * NW];
    const uint2 r0 = ld_row8<QB == 1>(vb + row_of(j0));
    const uint2 r1 = ld_row8<QB == 1>(vb + row_of(j1));
    const uint2 r2 = ld_row8<QB == 1>(vb + row_of(j2));
    const uint2 r3 = ld_row8<QB == 1>(vb + row_of(j3));
    add(j0, r0);
    add(j1, r1);
    add(j2, r2);
    add(j3, r3);
  }
  for (; i < n; i += NW) {
    const int j = nz[i];
    add(j, ld_row8<QB == 1>(vb + row_of(j)));
  }
  const float invH = 1.0f / static_cast<float>(H);
  const int c = db * 256 + threadIdx.x;
#pragma unroll
  for (int qq = 0; qq < QB; ++qq) {
    if (qq >= nq) break;   // workgroup-uniform
    *reinterpret_cast<float4*>(red + wave * 256 + 4 * lane) =
        make_float4(acc[qq][0], acc[qq][1], acc[qq][2], acc[qq][3]);
    __syncthreads();
    if (threadIdx.x < 256 && c < Dv) {
      float sum = red[threadIdx.x];
#pragma unroll
      for (int w = 1; w < NW; ++w) sum += red[w * 256 + threadIdx.x];
      out[(static_cast<int64_t>(b) * T + t0 + qq) * out_ld + c] = f2bf(sum * invH);
    }
    __syncthreads();
  }
}

// Dense lists summed over the heads, for sequences: P[r][j] = sum over h, in
// head order from 0, of wl[(r H + h) Kmax + j] -- the sum the apply forms
// itself, bit for bit -- so the apply reads one list per query instead of H.
// Thread = (row, slot), the H loads requested together.
constexpr int kHeadSumMaxH = 16;

__global__ __launch_bounds__(256) void cmp_head_sum_kernel(const float* __restrict__ wl, int H,
                                                           int Kmax, int64_t n,
                                                           float* __restrict__ P) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= n) return;
  const int64_t r = e / Kmax, j = e - r * Kmax;
  const float* src = wl + r * H * Kmax + j;
  float w[kHeadSumMaxH];
#pragma unroll
  for (int h = 0; h < kHeadSumMaxH; ++h) w[h] = h < H ? src[static_cast<int64_t>(h) * Kmax] : 0.f;
  float acc = 0.f;
#pragma unroll
  for (int h = 0; h < kHeadSumMaxH; ++h)
    if (h < H) acc += w[h];
  P[e] = acc;
}

// Sequence apply on MFMA (prefill): workgroup = (row b, 32-query block,
// 256-channel block), 8 wavefronts.  The block's head-summed weights P [32
// queries][block slots] are accumulated in LDS (fp32, heads in order, as
// above), then O^T = V^T P^T runs as v_mfma_f32_32x32x16_bf16 over 32-slot
// chunks: each chunk's value rows are staged transposed (V^T [channel][slot],
// slot pairs packed per dword, the attention prefill's staging), wave w takes
// the block's channels 32 w .. 32 w + 31, and each P fragment is split into
// (hi, lo) bf16 in registers (so the weights keep fp32 accuracy; the values
// are exact in bf16).  out = acc / H.  Dv % 32 == 0 and at most
// kApplyMfmaSlots block slots (the fp32 P rows fill the LDS).
constexpr int kApplyMfmaSlots = 1088;
constexpr int kApplyVtPitch = 40;   // bf16 per staged V^T row (32 slots + 8 pad)

__global__ __launch_bounds__(512) void cmp_apply_mfma_kernel(
    const float* __restrict__ wl, const int32_t* __restrict__ il, int Kmax, int H, int T,
    int band_W, int nslots, const uint16_t* __restrict__ v, int64_t v_ld, int rows_per_b,
    uint16_t* __restrict__ out, int64_t out_ld, int Dv, float invH) {
  extern __shared__ float pmf[];
  const int nsb = band_W > 0 ? nslots + 31 : nslots;   // block slots
  const int NP = (nsb + 31) & ~31;
  const int RS = NP + 4;                                // fp32 per P row (16-byte pad)
  uint16_t* vt = reinterpret_cast<uint16_t*>(pmf + 32 * RS);   // [256][kApplyVtPitch]
  // after V^T: s_used (kept in the dynamic area, whose 16-byte alignment a
  // static LDS variable ahead of it would break)
  int& s_used = *reinterpret_cast<int*>(vt + 256 * kApplyVtPitch);
  const int ndb = (Dv + 255) / 256;
  const int nqb = (T + 31) / 32;
  const int blk = blockIdx.x / ndb;
  const int db = blockIdx.x - blk * ndb;
  const int b = blk / nqb;
  // memory: later query blocks weigh more slots; they are dispatched first so
  // the short blocks fill in behind them
  const int qb = band_W > 0 ? blk - b * nqb : nqb - 1 - (blk - b * nqb);
  const int t0 = qb * 32;
  const int nq = min(32, T - t0);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c0 = db * 256;
  const int base = band_W > 0 ? t0 - band_W + 1 : 0;    // key of block slot 0

  // ---- P: the 32 queries' weights summed over the heads (head order).
  // Memory rows: s_used = 1 + the last slot any of them weighs (0: none);
  // chunks past it hold only zero weights and are skipped (a causal row sees
  // a prefix of the slots).
  for (int i = tid; i < 32 * RS; i += 512) pmf[i] = 0.f;
  if (tid == 0) s_used = 0;
  __syncthreads();
  int used = 0;
  const int64_t lb0 = (static_cast<int64_t>(b) * T + t0) * H * Kmax;
  if (il && H <= kApplyMaxH && nq * Kmax <= 1024) {
    // every head's (slot, weight) entries requested at once (two per thread
    // per head), then added head by head: a head's slots are distinct, so
    // each pass is race-free and every slot sums its heads in head order
    float wr[kApplyMaxH][2];
    int ir[kApplyMaxH][2], pr[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int e = tid + 512 * r;
      pr[r] = e < nq * Kmax ? (e / Kmax) * RS : -1;
    }
#pragma unroll
    for (int hh = 0; hh < kApplyMaxH; ++hh)
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int e = tid + 512 * r;
        const bool ok = hh < H && pr[r] >= 0;
        const int qq = e / Kmax, j = e - qq * Kmax;
        const int64_t o = lb0 + (static_cast<int64_t>(qq) * H + hh) * Kmax + j;
        wr[hh][r] = ok ? wl[o] : 0.f;
        ir[hh][r] = ok ? il[o] : -1;
      }
#pragma unroll
    for (int hh = 0; hh < kApplyMaxH; ++hh) {
      if (hh >= H) break;  // uniform
#pragma unroll
      for (int r = 0; r < 2; ++r)
        if (ir[hh][r] >= 0 && ir[hh][r] < nslots) {
          pmf[pr[r] + ir[hh][r]] += wr[hh][r];
          if (wr[hh][r] != 0.f) used = max(used, ir[hh][r] + 1);
        }
      __syncthreads();
    }
  } else if (il) {
    for (int hh = 0; hh < H; ++hh) {
      for (int e = tid; e < nq * Kmax; e += 512) {
        const int qq = e / Kmax, j = e - qq * Kmax;
        const int64_t o = lb0 + (static_cast<int64_t>(qq) * H + hh) * Kmax + j;
        const int idx = il[o];
        if (idx >= 0 && idx < nslots) {
          const float w = wl[o];
          pmf[qq * RS + idx] += w;
          if (w != 0.f) used = max(used, idx + 1);
        }
      }
      __syncthreads();
    }
  } else {
    for (int e = tid; e < nq * nslots; e += 512) {
      const int qq = e / nslots, j = e - qq * nslots;
      const int64_t o = lb0 + static_cast<int64_t>(qq) * H * Kmax + j;
      float acc = 0.f;
      for (int hh = 0; hh < H; ++hh) acc += wl[o + static_cast<int64_t>(hh) * Kmax];
      const int col = j + (band_W > 0 ? qq : 0);
      pmf[qq * RS + col] = acc;
      if (acc != 0.f) used = max(used, col + 1);
    }
  }
  if (band_W == 0) {  // uniform; a band's slots are nearly all weighed
    used = static_cast<int>(wave_max(static_cast<float>(used)));  // exact: used <= NP
    if (lane == 0 && used > 0) atomicMax(&s_used, used);
  }
  __syncthreads();
  const int np_used = band_W == 0 ? min(NP, (s_used + 31) & ~31) : NP;

  // ---- V^T staging: thread (slot pair p, channel group g) fetches the two
  // rows' 8 channels (rows clamped into the sequence; their weights are 0)
  const int sp = tid & 15, cg = tid >> 4;   // slots 2 sp, 2 sp + 1; channels 8 cg ..
  const int cch = c0 + 8 * cg;
  const bool ch_ok = cch < Dv;
  const uint16_t* vrow0 = v + static_cast<int64_t>(b) * rows_per_b * v_ld + (ch_ok ? cch : 0);
  uint4 va, vb;
  auto fetch = [&](int s0) {
    const int k0 = min(max(base + s0 + 2 * sp, 0), rows_per_b - 1);
    const int k1 = min(max(base + s0 + 2 * sp + 1, 0), rows_per_b - 1);
    va = ch_ok ? *reinterpret_cast<const uint4*>(vrow0 + static_cast<int64_t>(k0) * v_ld)
               : uint4{0u, 0u, 0u, 0u};
    vb = ch_ok ? *reinterpret_cast<const uint4*>(vrow0 + static_cast<int64_t>(k1) * v_ld)
               : uint4{0u, 0u, 0u, 0u};
  };
  auto stage = [&]() {
    const uint32_t a4[4] = {va.x, va.y, va.z, va.w};
    const uint32_t b4[4] = {vb.x, vb.y, vb.z, vb.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      // channel 8 cg + e: slot 2 sp in the low half, 2 sp + 1 in the high half
      const uint32_t word = __builtin_amdgcn_perm(b4[e >> 1], a4[e >> 1],
                                                  (e & 1) ? 0x07060302u : 0x05040100u);
      *reinterpret_cast<uint32_t*>(vt + (8 * cg + e) * kApplyVtPitch + 2 * sp) = word;
    }
  };

  // ---- O^T = V^T P^T: wave w owns channels c0 + 32 w .. + 31 (all 32 queries)
  const bool w_ok = c0 + 32 * wave < Dv;
  const int col = lane & 31, hf = lane >> 5;
  f32x16c acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.f;
  fetch(0);
  for (int s0 = 0; s0 < np_used; s0 += 32) {
    __syncthreads();   // the previous chunk's V^T reads are done
    stage();
    __syncthreads();
    if (s0 + 32 < np_used) fetch(s0 + 32);
    if (w_ok) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const uint4 af = *reinterpret_cast<const uint4*>(
            vt + (32 * wave + col) * kApplyVtPitch + 16 * ks + 8 * hf);
        const float* pr = pmf + col * RS + s0 + 16 * ks + 8 * hf;
        const float4 p0 = *reinterpret_cast<const float4*>(pr);
        const float4 p1 = *reinterpret_cast<const float4*>(pr + 4);
        const float pv[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
        uint16_t hi[8], lo[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          hi[i] = f2bf(pv[i]);
          lo[i] = f2bf(pv[i] - bf2f(hi[i]));
        }
        auto pk = [](uint16_t x, uint16_t y) {
          return static_cast<uint32_t>(x) | (static_cast<uint32_t>(y) << 16);
        };
        const uint4 bh = uint4{pk(hi[0], hi[1]), pk(hi[2], hi[3]), pk(hi[4], hi[5]),
                               pk(hi[6], hi[7])};
        const uint4 bl = uint4{pk(lo[0], lo[1]), pk(lo[2], lo[3]), pk(lo[4], lo[5]),
                               pk(lo[6], lo[7])};
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(af), as_bf16x8(bh), acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(af), as_bf16x8(bl), acc, 0, 0, 0);
      }
    }
  }
  // ---- lane holds query col, channels 32 w + 8 g4 + 4 hf .. +3 in registers 4 g4 ..
  if (!w_ok || col >= nq) return;
  uint16_t* orow = out + (static_cast<int64_t>(b) * T + t0 + col) * out_ld + c0 + 32 * wave;
#pragma unroll
  for (int g4 = 0; g4 < 4; ++g4)
    *reinterpret_cast<uint2*>(orow + 8 * g4 + 4 * hf) =
        make_uint2(pack_bf2(acc[4 * g4] * invH, acc[4 * g4 + 1] * invH),
                   pack_bf2(acc[4 * g4 + 2] * invH, acc[4 * g4 + 3] * invH));
}

// ---------------------------------------------------------------- compressor
// Prefill (fresh sequences, compressed_attention.py:105-123): workgroup (b, i),
// i < n: mean of block i (bf16); i == n: the tail's sum (fp32) and count.
__global__ __launch_bounds__(256) void cmp_pool_prefill_kernel(
    const uint16_t* __restrict__ h, int64_t h_ld, uint16_t* __restrict__ means,
    float* __restrict__ psum, int32_t* __restrict__ pcnt, int T, int D, int ratio, int n) {
  const int b = blockIdx.x / (n + 1);
  const int i = blockIdx.x - b * (n + 1);
  const int t_lo = i * ratio;
  const int t_hi = i < n ? t_lo + ratio : T;
  for (int d = threadIdx.x; d < D; d += 256) {
    float s = 0.f;
    for (int t = t_lo; t < t_hi; ++t) s += bf2f(h[static_cast<int64_t>(b * T + t) * h_ld + d]);
    if (i < n) means[static_cast<int64_t>(b * n + i) * D + d] = f2bf(s / static_cast<float>(ratio));
    else psum[static_cast<int64_t>(b) * D + d] = s;
  }
  if (i == n && threadIdx.x == 0) pcnt[b] = T - n * ratio;
}

// Decode (compressed_attention.py:177-207): the running sum and count gain
// this token; the mean (bf16) feeds the summary projection every step; a
// completed block is flagged in emit and the sum and count restart.
__global__ __launch_bounds__(256) void cmp_pool_step_kernel(
    const uint16_t* __restrict__ h, int64_t h_ld, float* __restrict__ psum,
    int32_t* __restrict__ pcnt, uint16_t* __restrict__ mean, int32_t* __restrict__ emit, int D,
    int ratio) {
  const int b = blockIdx.x;
  const int cnt = pcnt[b] + 1;
  const bool done = cnt >= ratio;
  for (int d = threadIdx.x; d < D; d += 256) {
    const int64_t o = static_cast<int64_t>(b) * D + d;
    const float s = psum[o] + bf2f(h[static_cast<int64_t>(b) * h_ld + d]);
    mean[o] = f2bf(s / static_cast<float>(cnt));
    psum[o] = done ? 0.f : s;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    pcnt[b] = done ? 0 : cnt;
    emit[b] = done ? 1 : 0;
  }
}

// Decode: a row with emit set stores its summary (kv row: Kw key channels then
// Dv value channels) at slot count % C with tag pos + 1.
__global__ __launch_bounds__(256) void cmp_commit_kernel(
    const uint16_t* __restrict__ kv, int64_t kv_ld, const int32_t* __restrict__ emit,
    const int32_t* __restrict__ pos, uint16_t* __restrict__ mk, uint16_t* __restrict__ mv,
    int32_t* __restrict__ mtag, int32_t* __restrict__ mcount, int C, int Kw, int Dv) {
  const int b = blockIdx.x;
  if (!emit[b]) return;
  const int cnt = mcount[b];
  const int slot = cnt % C;
  const uint16_t* src = kv + static_cast<int64_t>(b) * kv_ld;
  uint16_t* dk = mk + (static_cast<int64_t>(b) * C + slot) * Kw;
  uint16_t* dv = mv + (static_cast<int64_t>(b) * C + slot) * Dv;
  for (int c = threadIdx.x; c < Kw / 8; c += 256)
    reinterpret_cast<uint4*>(dk)[c] = reinterpret_cast<const uint4*>(src)[c];
  for (int c = threadIdx.x; c < Dv / 8; c += 256)
    reinterpret_cast<uint4*>(dv)[c] = reinterpret_cast<const uint4*>(src + Kw)[c];
  __syncthreads();
  if (threadIdx.x == 0) {
    mtag[static_cast<int64_t>(b) * C + slot] = pos[b] + 1;
    mcount[b] = cnt + 1;
  }
}

// Prefill: the last min(n, C) of a row's n summaries (kv rows b*n + i) into
// slots i % C with tags (i + 1) ratio; count n.  Workgroup (b, j).
__global__ __launch_bounds__(256) void cmp_memory_fill_kernel(
    const uint16_t* __restrict__ kv, int64_t kv_ld, uint16_t* __restrict__ mk,
    uint16_t* __restrict__ mv, int32_t* __restrict__ mtag, int32_t* __restrict__ mcount, int n,
    int keep, int ratio, int C, int Kw, int Dv) {
  const int b = blockIdx.x / keep;
  const int i = n - keep + (blockIdx.x - b * keep);
  const int slot = i % C;
  const uint16_t* src = kv + static_cast<int64_t>(b * n + i) * kv_ld;
  uint16_t* dk = mk + (static_cast<int64_t>(b) * C + slot) * Kw;
  uint16_t* dv = mv + (static_cast<int64_t>(b) * C + slot) * Dv;
  for (int c = threadIdx.x; c < Kw / 8; c += 256)
    reinterpret_cast<uint4*>(dk)[c] = reinterpret_cast<const uint4*>(src)[c];
  for (int c = threadIdx.x; c < Dv / 8; c += 256)
    reinterpret_cast<uint4*>(dv)[c] = reinterpret_cast<const uint4*>(src + Kw)[c];
  if (threadIdx.x == 0) {
    mtag[static_cast<int64_t>(b) * C + slot] = (i + 1) * ratio;
    if (i == n - 1) mcount[b] = n;
  }
}

// Prefill: the last min(T, W) rows of each sequence (src rows b*T + t) into
// ring slots t % W.  Workgroup (b, j).
__global__ __launch_bounds__(256) void cmp_ring_fill_kernel(
    const uint16_t* __restrict__ src, int64_t src_ld, uint16_t* __restrict__ ring, int T, int W,
    int keep, int width) {
  const int b = blockIdx.x / keep;
  const int t = T - keep + (blockIdx.x - b * keep);
  const uint16_t* s = src + static_cast<int64_t>(b * T + t) * src_ld;
  uint16_t* d = ring + (static_cast<int64_t>(b) * W + t % W) * width;
  for (int c = threadIdx.x; c < width / 8; c += 256)
    reinterpret_cast<uint4*>(d)[c] = reinterpret_cast<const uint4*>(s)[c];
}

inline bool dh_ok(int Dh) { return Dh >= 16 && Dh % 16 == 0 && Dh <= 4096; }

// decode scoring splits a head over G = min(64, Dh / 8) lanes with xor-shuffle
// sums, a wave scoring 16 candidates: G in {4, 8, 16, 32, 64}, dividing Dh / 8
inline bool dh_decode_ok(int Dh) {
  return Dh == 32 || Dh == 64 || Dh == 128 || Dh == 256 || (Dh % 512 == 0 && Dh <= 4096);
}

// Decode: scores (into sc), then the lists, for one branch; rows of at most
// kFusedMaxCand candidates over B * H >= 512 workgroups take the one-kernel
// form (the same scores and lists).
template <int MODE>
int32_t decode_select(const uint16_t* q, int64_t q_ld, const uint16_t* k_new,
                      const uint16_t* v_new, int64_t kv_ld, uint16_t* ring_k, uint16_t* ring_v,
                      const uint16_t* mk, const int32_t* mtag, const int32_t* pos, int B, int H,
                      int Dh, int Dv, int W, int C, int top_k, int Kmax, float scale_log2,
                      float* sc, float* wl, int32_t* il, hipStream_t s) {
  const int ncand = MODE == kBand ? W : C;
  const int G = min(kWave, Dh / 8);
  if (ncand <= kFusedMaxCand && static_cast<int64_t>(B) * H >= 512) {
    // one workgroup per (row, head): scores in LDS, list formed in place
#define LLMY_SCORE_LIST(GG)                                                                  \
  hipLaunchKernelGGL((cmp_score_list_decode_kernel<MODE, GG>), dim3(B * H), dim3(256),         \
                     static_cast<size_t>(ncand) * 4, s, q, q_ld, k_new, v_new, kv_ld, ring_k,  \
                     ring_v, mk, mtag, pos, H, Dh, Dv, W, C, scale_log2, top_k, Kmax, wl, il)
    switch (G) {
      case 4: LLMY_SCORE_LIST(4); break;
      case 8: LLMY_SCORE_LIST(8); break;
      case 16: LLMY_SCORE_LIST(16); break;
      case 32: LLMY_SCORE_LIST(32); break;
      default: LLMY_SCORE_LIST(64); break;
    }
#undef LLMY_SCORE_LIST
    return launch_status();
  }
  const int chunk = 16 * (kWave / G);
  const dim3 grid(static_cast<unsigned>(B * H * ((ncand + chunk - 1) / chunk)));
#define LLMY_SCORE(GG)                                                                      \
  hipLaunchKernelGGL((cmp_score_decode_kernel<MODE, GG>), grid, dim3(256), 0, s, q, q_ld,   \
                     k_new, v_new, kv_ld, ring_k, ring_v, mk, mtag, pos, H, Dh, Dv, W, C,  \
                     scale_log2, sc)
  switch (G) {
    case 4: LLMY_SCORE(4); break;
    case 8: LLMY_SCORE(8); break;
    case 16: LLMY_SCORE(16); break;
    case 32: LLMY_SCORE(32); break;
    default: LLMY_SCORE(64); break;
  }
#undef LLMY_SCORE
  const int32_t st = launch_status();
  if (st) return st;
  hipLaunchKernelGGL(cmp_list_decode_kernel<MODE>, dim3(B * H), dim3(64),
                     static_cast<size_t>(ncand) * 4, s, sc, ncand, top_k, Kmax, wl, il);
  return launch_status();
}

inline int64_t list_bytes(int64_t queries, int H, int Kmax, bool pairs) {
  return queries * H * Kmax * static_cast<int64_t>(pairs ? 8 : 4);
}

// sequences with dense lists keep the head-summed lists beside them
inline int64_t dense_seq_bytes(int64_t queries, int H, int slots) {
  return list_bytes(queries, H, slots, false) + (H > 1 ? list_bytes(queries, 1, slots, false) : 0);
}

// decode keeps the raw scores of its slots beside the lists
inline int64_t decode_bytes(int64_t rows, int H, int slots, int top_k) {
  return list_bytes(rows, H, top_k > 0 ? top_k : slots, top_k > 0) + rows * H * slots * 4ll;
}

}  // namespace llmy

using namespace llmy;

extern "C" int64_t llmy_cmp_workspace_bytes(int32_t queries, int32_t H, int32_t slots,
                                            int32_t top_k, int32_t decode) {
  if (queries < 0 || H <= 0 || slots <= 0 || top_k < 0) return -1;
  if (decode) return decode_bytes(queries, H, slots, top_k);
  return top_k > 0 ? list_bytes(queries, H, top_k, true) : dense_seq_bytes(queries, H, slots);
}

namespace {

int32_t apply_launch(const float* wl, const int32_t* il, int Kmax, int H, int B, int T,
                     const int32_t* qpos, int band_W, int nslots, const uint16_t* v, int64_t v_ld,
                     int rows_per_b, int wrap, uint16_t* out, int64_t out_ld, int Dv,
                     hipStream_t s, float* head_sum = nullptr) {
  // sequences on MFMA where the block's weights fit the LDS
  if (!qpos && T >= 8 && Dv % 32 == 0 && wrap == 0 &&
      (band_W > 0 ? nslots + 31 : nslots) <= kApplyMfmaSlots) {
    const float invH = 1.0f / static_cast<float>(H);
    if (head_sum && !il && H > 1 && H <= kHeadSumMaxH) {
      // dense lists: sum the heads once, then apply one list per query
      const int64_t n = static_cast<int64_t>(B) * T * Kmax;
      const int64_t nb = (n + 255) / 256;
      if (nb >= (1ll << 31)) return static_cast<int32_t>(hipErrorInvalidValue);
      hipLaunchKernelGGL(cmp_head_sum_kernel, dim3(static_cast<unsigned>(nb)), dim3(256), 0, s,
                         wl, H, Kmax, n, head_sum);
      const int32_t st = launch_status();
      if (st) return st;
      wl = head_sum;
      H = 1;
    }
    const int nsb = band_W > 0 ? nslots + 31 : nslots;
    const int NP = (nsb + 31) & ~31;
    const size_t lds = static_cast<size_t>(32) * (NP + 4) * 4 + 256 * kApplyVtPitch * 2 + 16;
    const int64_t nblk = static_cast<int64_t>(B) * ((T + 31) / 32) * ((Dv + 255) / 256);
    if (nblk >= (1ll << 31)) return static_cast<int32_t>(hipErrorInvalidValue);
    hipLaunchKernelGGL(cmp_apply_mfma_kernel, dim3(static_cast<unsigned>(nblk)), dim3(512), lds,
                       s, wl, il, Kmax, H, T, band_W, nslots, v, v_ld, rows_per_b, out, out_ld,
                       Dv, invH);
    return launch_status();
  }
  // blocks of 8 queries for sequences (a value row serves the whole block),
  // single queries for decode
  const int QB = T >= 8 ? 8 : 1;
  const int nsb = band_W > 0 ? nslots + QB - 1 : nslots;
  const int NW = QB == 8 ? 4 : kApplyDecodeWaves;
  const size_t lds = (static_cast<size_t>(QB) * ((nsb + 3) & ~3) + NW * 256 +
                      static_cast<size_t>(nsb)) * 4;
  if (lds > 147456) return static_cast<int32_t>(hipErrorInvalidValue);
  const int64_t nblk = static_cast<int64_t>(B) * ((T + QB - 1) / QB) * ((Dv + 255) / 256);
  if (nblk >= (1ll << 31)) return static_cast<int32_t>(hipErrorInvalidValue);
  if (QB == 8)
    hipLaunchKernelGGL((cmp_apply_kernel<8, 4>), dim3(static_cast<unsigned>(nblk)), dim3(256), lds, s,
                       wl, il, Kmax, H, T, qpos, band_W, nslots, v, v_ld, rows_per_b, wrap, out,
                       out_ld, Dv);
  else
    hipLaunchKernelGGL((cmp_apply_kernel<1, kApplyDecodeWaves>), dim3(static_cast<unsigned>(nblk)),
                       dim3(64 * kApplyDecodeWaves), lds, s,
                       wl, il, Kmax, H, T, qpos, band_W, nslots, v, v_ld, rows_per_b, wrap, out,
                       out_ld, Dv);
  return launch_status();
}

bool rows_ok(int64_t ld, int width) { return ld >= width && ld % 8 == 0; }

}  // namespace

extern "C" int32_t llmy_cmp_local_prefill_bf16(
    const llmy_bf16* q, int64_t q_ld, const llmy_bf16* k, int64_t k_ld, const llmy_bf16* v,
    int64_t v_ld, llmy_bf16* out, int64_t out_ld, int32_t B, int32_t T, int32_t H,
    int32_t head_dim, int32_t Dv, int32_t W, float scale, void* workspace,
    int64_t workspace_bytes, void* stream) {
  LLMY_REQUIRE(B >= 0 && T >= 0 && H > 0 && dh_ok(head_dim) && Dv > 0 && Dv % 8 == 0 &&
               W >= 1 && W <= 4096);
  if (B == 0 || T == 0) return 0;
  const int Kw = H * head_dim;
  LLMY_REQUIRE(q && k && v && out && workspace);
  LLMY_REQUIRE(rows_ok(q_ld, Kw) && rows_ok(k_ld, Kw) && rows_ok(v_ld, Dv) && out_ld >= Dv &&
               out_ld % 4 == 0);
  LLMY_REQUIRE(aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && aligned(out, 8) &&
               aligned(workspace, 16));
  const int64_t queries = static_cast<int64_t>(B) * T;
  LLMY_REQUIRE(workspace_bytes >= dense_seq_bytes(queries, H, W));
  const int nqb = (T + 31) / 32;
  LLMY_REQUIRE(static_cast<int64_t>(B) * nqb * H < (1ll << 31) && queries < (1ll << 31));
  const int ncp = ((min(T, W + 31) + 31) / 32 + 1) * 32;   // >= any block's candidate span
  int rows = 32;
  while (rows > 1 && static_cast<int64_t>(rows) * (ncp + 1) * 4 > kCmpLdsBytes) rows /= 2;
  LLMY_REQUIRE(static_cast<int64_t>(rows) * (ncp + 1) * 4 <= kCmpLdsBytes);
  const hipStream_t s = as_stream(stream);
  float* wl = static_cast<float*>(workspace);
  select_prefill_launch<kBand>(dim3(B * nqb * H), static_cast<size_t>(rows) * (ncp + 1) * 4, s, q, q_ld,
                               k, k_ld, T, 0, H, head_dim, W, 1, 0, W, rows, scale * kLog2eC, wl,
                               nullptr);
  const int32_t st = launch_status();
  if (st) return st;
  return apply_launch(wl, nullptr, W, H, B, T, nullptr, W, W, v, v_ld, T, 0, out, out_ld, Dv, s,
                      wl + queries * H * W);
}

extern "C" int32_t llmy_cmp_memory_prefill_bf16(
    const llmy_bf16* q, int64_t q_ld, const llmy_bf16* mk, int64_t mk_ld, const llmy_bf16* mv,
    int64_t mv_ld, llmy_bf16* out, int64_t out_ld, int32_t B, int32_t T, int32_t n_entries,
    int32_t ratio, int32_t H, int32_t head_dim, int32_t Dv, int32_t top_k, int32_t slots_window,
    float scale, void* workspace, int64_t workspace_bytes, void* stream) {
  LLMY_REQUIRE(B >= 0 && T >= 0 && H > 0 && dh_ok(head_dim) && Dv > 0 && Dv % 8 == 0 &&
               ratio >= 1 && n_entries >= 0 && top_k >= 0 && top_k <= 64 && slots_window >= 0);
  if (B == 0 || T == 0) return 0;
  LLMY_REQUIRE(n_entries == T / ratio);
  const int Kw = H * head_dim;
  LLMY_REQUIRE(q && out && workspace && (n_entries == 0 || (mk && mv)));
  LLMY_REQUIRE(rows_ok(q_ld, Kw) && out_ld >= Dv && out_ld % 4 == 0);
  LLMY_REQUIRE(n_entries == 0 || (rows_ok(mk_ld, Kw) && rows_ok(mv_ld, Dv) && aligned(mk, 16) &&
                                  aligned(mv, 16)));
  LLMY_REQUIRE(aligned(q, 16) && aligned(out, 8) && aligned(workspace, 16));
  const int64_t queries = static_cast<int64_t>(B) * T;
  const int slots = max(n_entries, 1);
  const int Kmax = top_k > 0 ? top_k : slots;
  LLMY_REQUIRE(workspace_bytes >= (top_k > 0 ? list_bytes(queries, H, Kmax, true)
                                               : dense_seq_bytes(queries, H, Kmax)));
  LLMY_REQUIRE(slots <= 4000);   // the apply's LDS: 9 words per slot + 4 KiB
  const hipStream_t s = as_stream(stream);
  // n_entries == 0: no summary is visible to any query, every list is 0 and
  // the apply writes zeros without reading mk / mv
  const int nqb = (T + 31) / 32;
  LLMY_REQUIRE(static_cast<int64_t>(B) * nqb * H < (1ll << 31) && queries < (1ll << 31));
  const int ncp = ((slots + 31) / 32) * 32;
  int rows = 32;
  while (rows > 1 && static_cast<int64_t>(rows) * (ncp + 1) * 4 > kCmpLdsBytes) rows /= 2;
  LLMY_REQUIRE(static_cast<int64_t>(rows) * (ncp + 1) * 4 <= kCmpLdsBytes);
  float* wl = static_cast<float*>(workspace);
  int32_t* il = top_k > 0 ? reinterpret_cast<int32_t*>(wl + queries * H * Kmax) : nullptr;
  const size_t lds = static_cast<size_t>(rows) * (ncp + 1) * 4;
  if (top_k > 0)
    select_prefill_launch<kMemTopK>(dim3(B * nqb * H), lds, s, q, q_ld, mk, mk_ld, T, n_entries,
                                    H, head_dim, slots_window, ratio, top_k, Kmax, rows,
                                    scale * kLog2eC, wl, il);
  else
    select_prefill_launch<kMemDense>(dim3(B * nqb * H), lds, s, q, q_ld, mk, mk_ld, T, n_entries,
                                     H, head_dim, slots_window, ratio, 0, Kmax, rows,
                                     scale * kLog2eC, wl, il);
  const int32_t st = launch_status();
  if (st) return st;
  return apply_launch(wl, il, Kmax, H, B, T, nullptr, 0, slots, mv, mv_ld, slots, 0, out,
                      out_ld, Dv, s, top_k > 0 ? nullptr : wl + queries * H * Kmax);
}

extern "C" int32_t llmy_cmp_local_decode_bf16(
    const llmy_bf16* q, int64_t q_ld, const llmy_bf16* k_new, const llmy_bf16* v_new,
    int64_t kv_ld, llmy_bf16* ring_k, llmy_bf16* ring_v, const int32_t* pos, llmy_bf16* out,
    int64_t out_ld, int32_t B, int32_t H, int32_t head_dim, int32_t Dv, int32_t W, float scale,
    void* workspace, int64_t workspace_bytes, void* stream) {
  LLMY_REQUIRE(B >= 0 && H > 0 && dh_decode_ok(head_dim) && Dv > 0 && Dv % 8 == 0 && W >= 1 &&
               W <= 7168);
  if (B == 0) return 0;
  const int Kw = H * head_dim;
  LLMY_REQUIRE(q && k_new && v_new && ring_k && ring_v && pos && out && workspace);
  LLMY_REQUIRE(rows_ok(q_ld, Kw) && rows_ok(kv_ld, Kw) && rows_ok(kv_ld, Dv) && out_ld >= Dv &&
               out_ld % 4 == 0);
  LLMY_REQUIRE(aligned(q, 16) && aligned(k_new, 16) && aligned(v_new, 16) &&
               aligned(ring_k, 16) && aligned(ring_v, 16) && aligned(out, 8) &&
               aligned(workspace, 16));
  LLMY_REQUIRE(workspace_bytes >= decode_bytes(B, H, W, 0));
  LLMY_REQUIRE(static_cast<int64_t>(B) * H * ((W + 15) / 16) < (1ll << 31));
  const hipStream_t s = as_stream(stream);
  float* wl = static_cast<float*>(workspace);
  float* sc = wl + static_cast<int64_t>(B) * H * W;
  const int32_t st = decode_select<kBand>(q, q_ld, k_new, v_new, kv_ld, ring_k, ring_v, nullptr,
                                          nullptr, pos, B, H, head_dim, Dv, W, 0, 0, W,
                                          scale * kLog2eC, sc, wl, nullptr, s);
  if (st) return st;
  return apply_launch(wl, nullptr, W, H, B, 1, pos, W, W, ring_v, Dv, W, W, out, out_ld, Dv, s);
}

extern "C" int32_t llmy_cmp_memory_decode_bf16(
    const llmy_bf16* q, int64_t q_ld, const llmy_bf16* mk, const llmy_bf16* mv,
    const int32_t* mtag, const int32_t* pos, llmy_bf16* out, int64_t out_ld, int32_t B,
    int32_t C, int32_t H, int32_t head_dim, int32_t Dv, int32_t top_k, float scale,
    void* workspace, int64_t workspace_bytes, void* stream) {
  LLMY_REQUIRE(B >= 0 && H > 0 && dh_decode_ok(head_dim) && Dv > 0 && Dv % 8 == 0 && C >= 1 &&
               C <= 7168 && top_k >= 0 && top_k <= 64);
  if (B == 0) return 0;
  const int Kw = H * head_dim;
  LLMY_REQUIRE(q && mk && mv && mtag && pos && out && workspace);
  LLMY_REQUIRE(rows_ok(q_ld, Kw) && out_ld >= Dv && out_ld % 4 == 0);
  LLMY_REQUIRE(aligned(q, 16) && aligned(mk, 16) && aligned(mv, 16) && aligned(out, 8) &&
               aligned(workspace, 16));
  const int Kmax = top_k > 0 ? top_k : C;
  LLMY_REQUIRE(workspace_bytes >= decode_bytes(B, H, C, top_k));
  LLMY_REQUIRE(static_cast<int64_t>(B) * H * ((C + 15) / 16) < (1ll << 31));
  const hipStream_t s = as_stream(stream);
  float* wl = static_cast<float*>(workspace);
  const int64_t nl = static_cast<int64_t>(B) * H * Kmax;
  int32_t* il = top_k > 0 ? reinterpret_cast<int32_t*>(wl + nl) : nullptr;
  float* sc = wl + nl * (top_k > 0 ? 2 : 1);
  const int32_t st =
      top_k > 0
          ? decode_select<kMemTopK>(q, q_ld, nullptr, nullptr, 0, nullptr, nullptr, mk, mtag, pos,
                                    B, H, head_dim, Dv, 1, C, top_k, Kmax, scale * kLog2eC, sc,
                                    wl, il, s)
          : decode_select<kMemDense>(q, q_ld, nullptr, nullptr, 0, nullptr, nullptr, mk, mtag,
                                     pos, B, H, head_dim, Dv, 1, C, 0, Kmax, scale * kLog2eC, sc,
                                     wl, il, s);
  if (st) return st;
  return apply_launch(wl, il, Kmax, H, B, 1, pos, 0, C, mv, Dv, C, 0, out, out_ld, Dv, s);
}

extern "C" int32_t llmy_cmp_pool_prefill_bf16(const llmy_bf16* h, int64_t h_ld, llmy_bf16* means,
                                              float* psum, int32_t* pcnt, int32_t B, int32_t T,
                                              int32_t D, int32_t ratio, void* stream) {
  LLMY_REQUIRE(B >= 0 && T >= 0 && D > 0 && ratio >= 1 && h_ld >= D);
  if (B == 0) return 0;
  const int n = T / ratio;
  LLMY_REQUIRE(psum && pcnt && (T == 0 || h) && (n == 0 || means));
  LLMY_REQUIRE(static_cast<int64_t>(B) * (n + 1) < (1ll << 31));
  hipLaunchKernelGGL(cmp_pool_prefill_kernel, dim3(B * (n + 1)), dim3(256), 0, as_stream(stream),
                     h, h_ld, means, psum, pcnt, T, D, ratio, n);
  return launch_status();
}

extern "C" int32_t llmy_cmp_pool_step_bf16(const llmy_bf16* h, int64_t h_ld, float* psum,
                                           int32_t* pcnt, llmy_bf16* mean, int32_t* emit,
                                           int32_t B, int32_t D, int32_t ratio, void* stream) {
  LLMY_REQUIRE(B >= 0 && D > 0 && ratio >= 1 && h_ld >= D);
  if (B == 0) return 0;
  LLMY_REQUIRE(h && psum && pcnt && mean && emit);
  hipLaunchKernelGGL(cmp_pool_step_kernel, dim3(B), dim3(256), 0, as_stream(stream), h, h_ld, psum,
                     pcnt, mean, emit, D, ratio);
  return launch_status();
}

extern "C" int32_t llmy_cmp_commit_bf16(const llmy_bf16* kv, int64_t kv_ld, const int32_t* emit,
                                        const int32_t* pos, llmy_bf16* mk, llmy_bf16* mv,
                                        int32_t* mtag, int32_t* mcount, int32_t B, int32_t C,
                                        int32_t Kw, int32_t Dv, void* stream) {
  LLMY_REQUIRE(B >= 0 && C >= 1 && Kw > 0 && Kw % 8 == 0 && Dv > 0 && Dv % 8 == 0);
  if (B == 0) return 0;
  LLMY_REQUIRE(kv && emit && pos && mk && mv && mtag && mcount);
  LLMY_REQUIRE(kv_ld >= Kw + Dv && kv_ld % 8 == 0 && aligned(kv, 16) && aligned(mk, 16) &&
               aligned(mv, 16));
  hipLaunchKernelGGL(cmp_commit_kernel, dim3(B), dim3(256), 0, as_stream(stream), kv, kv_ld, emit,
                     pos, mk, mv, mtag, mcount, C, Kw, Dv);
  return launch_status();
}

extern "C" int32_t llmy_cmp_memory_fill_bf16(const llmy_bf16* kv, int64_t kv_ld, llmy_bf16* mk,
                                             llmy_bf16* mv, int32_t* mtag, int32_t* mcount,
                                             int32_t B, int32_t n_entries, int32_t ratio,
                                             int32_t C, int32_t Kw, int32_t Dv, void* stream) {
  LLMY_REQUIRE(B >= 0 && n_entries >= 0 && ratio >= 1 && C >= 1 && Kw > 0 && Kw % 8 == 0 &&
               Dv > 0 && Dv % 8 == 0);
  if (B == 0 || n_entries == 0) return 0;
  LLMY_REQUIRE(kv && mk && mv && mtag && mcount);
  LLMY_REQUIRE(kv_ld >= Kw + Dv && kv_ld % 8 == 0 && aligned(kv, 16) && aligned(mk, 16) &&
               aligned(mv, 16));
  const int keep = min(n_entries, C);
  LLMY_REQUIRE(static_cast<int64_t>(B) * keep < (1ll << 31));
  hipLaunchKernelGGL(cmp_memory_fill_kernel, dim3(B * keep), dim3(256), 0, as_stream(stream), kv,
                     kv_ld, mk, mv, mtag, mcount, n_entries, keep, ratio, C, Kw, Dv);
  return launch_status();
}

extern "C" int32_t llmy_cmp_ring_fill_bf16(const llmy_bf16* src, int64_t src_ld, llmy_bf16* ring,
                                           int32_t B, int32_t T, int32_t W, int32_t width,
                                           void* stream) {
  LLMY_REQUIRE(B >= 0 && T >= 0 && W >= 1 && width > 0 && width % 8 == 0);
  if (B == 0 || T == 0) return 0;
  LLMY_REQUIRE(src && ring && src_ld >= width && src_ld % 8 == 0 && aligned(src, 16) &&
               aligned(ring, 16));
  const int keep = min(T, W);
  LLMY_REQUIRE(static_cast<int64_t>(B) * keep < (1ll << 31));
  hipLaunchKernelGGL(cmp_ring_fill_kernel, dim3(B * keep), dim3(256), 0, as_stream(stream), src,
                     src_ld, ring, T, W, keep, width);
  return launch_status();
}
