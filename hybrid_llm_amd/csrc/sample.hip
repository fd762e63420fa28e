// Token sampling over fp32 logits [rows, V].
//
// Greedy: first index of the maximum per row, i.e. torch.argmax semantics as
// used by sample_standalone.py:5609-5610 (NaN counts as the maximum, the
// lowest index wins among equal values).
//
// Temperature + nucleus: sample_standalone.py:5611-5636 and its C twin
// llmy_cuda/src/llmy.cpp:158-201, with the uniform draw supplied per row.
//
// Repetition penalty: sample_standalone.py:5601-5605.
#include "common.hpp"
#include "abi_util.hpp"

namespace llmy {

// One 1024-thread workgroup per row; each thread keeps the best packed
// (value, index) key of its strided slice (loads unrolled 8 deep so the row
// streams with many loads in flight), then waves and the block reduce.
__global__ __launch_bounds__(1024) void argmax_rows_kernel(const float* __restrict__ logits,
                                                           int V, int32_t* __restrict__ out) {
  __shared__ uint64_t part[16];
  const float* row = logits + static_cast<size_t>(blockIdx.x) * V;
  uint64_t best = 0ull;
  for (int base = 0; base < V; base += 8 * 1024) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = base + u * 1024 + threadIdx.x;
      v[u] = i < V ? row[i] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = base + u * 1024 + threadIdx.x;
      if (i < V) {
        const uint64_t key = value_index_key(v[u], static_cast<uint32_t>(i));
        best = key > best ? key : best;
      }
    }
  }
  best = wave_max_u64(best);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t b = part[0];
    for (int w = 1; w < 16; ++w) b = part[w] > b ? part[w] : b;
    out[blockIdx.x] = static_cast<int32_t>(key_index(b));
  }
}


// ---------------------------------------------------------------------------
// Nucleus sampling without a sort.
//
// Per row, with x the raw logits and T the temperature:
//   order   = descending x, equal values by ascending id (the order a stable
//             descending sort gives; dividing by T > 0 does not change it);
//   mass_i  = trunc(2^47 * exp((x_i - max x) / T)), an exact 64-bit integer,
//             so every sum below is exact and independent of summation order;
//   top-k   = the first k ids of the order (k <= 0 or k >= V: all ids);
//   nucleus = the shortest prefix of the top-k order whose mass reaches
//             top_p * (top-k mass) (top_p outside (0, 1): the whole top-k);
//   pick    = the first id of the order whose running mass exceeds
//             u * (nucleus mass), i.e. the inverse-CDF draw of llmy.cpp:195-200.
// Each of the three is "the first id of the order at which a running weight
// reaches a threshold" (weight 1 per id for top-k, mass otherwise).  That id
// is found by a radix select over the 32-bit order keys: three passes over
// 12-, 10- and 10-bit digits, each building a weight histogram of the digits
// (LDS atomics on integers) restricted to the prefix chosen so far and
// scanning it from the top digit down; equal keys share one weight, so the
// rank inside the final tie group is a division.  The nucleus and the draw
// share the first-pass histogram.
//
// One 1024-thread workgroup per row; thread t holds ids [32t, 32t + 32) in
// registers (key and exp value), so V <= 32768.
typedef unsigned long long u64;

constexpr int kNucThreads = 1024;
constexpr int kNucWaves = kNucThreads / kWave;
constexpr int kNucPer = 32;
constexpr int kNucMaxV = kNucThreads * kNucPer;
constexpr float kMassScale = 140737488355328.0f;  // 2^47: a row's mass sum stays below 2^62
constexpr int kTopBins = 4096;                     // first pass: key bits [31:20]
constexpr int kLowBins = 1024;                     // later passes: [19:10], [9:0]

struct NucLds {
  u64 top[kTopBins];
  u64 low[kLowBins];
  u64 wave_tot[kNucWaves];
  u64 pick_above;
  u64 tie_weight;
  uint32_t pick_digit;
  int32_t pick_id;
  float red[kNucWaves];
  float red_min[kNucWaves];
};

// Per-row weighting: x_max and log2(e) / T.
struct NucRow {
  float m;
  float c;
  float b;  // bucket path: buckets per log2 unit below the maximum
};

// Mass of a logit: trunc(2^47 * exp((x - max) / T)); the maximum itself (also
// in a row of infinities) weighs exactly 2^47, NaN weighs 0.
__device__ __forceinline__ u64 nuc_mass(float x, NucRow r) {
  const float e = x == r.m ? 1.f : exp2_fast((x - r.m) * r.c);
  return e > 0.f ? static_cast<u64>(e * kMassScale) : 0ull;
}

// Logit j through an empty asm that "redefines" its value.  Each use in a
// pass goes through it, so the optimiser neither carries keys and masses from
// one pass to the next nor computes every element's key, mass and address
// ahead of the first atomic (32 u64 masses and 32 keys do not fit beside the
// logits at 1024 threads); recomputing them costs a few ALU operations and
// one v_exp_f32 per element.
__device__ __forceinline__ float nuc_x(const float* x, int j) {
  float v = x[j];
  asm volatile("" : "+v"(v));
  return v;
}

// Weight of element j: 1 per live id when counting, else its mass; 0 for ids
// outside the row or outside the top-k.
template <bool kCount>
__device__ __forceinline__ u64 nuc_weight(float xj, uint32_t live, int j, NucRow r) {
  const u64 w = kCount ? 1ull : nuc_mass(xj, r);
  return ((live >> j) & 1u) ? w : 0ull;
}

// Exclusive prefix sum over the block in thread order; *total = block sum.
__device__ __forceinline__ u64 nuc_excl_scan(u64 v, u64* wave_tot, u64* total) {
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  u64 inc = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const u64 o = __shfl_up(inc, off, kWave);
    if (lane >= off) inc += o;
  }
  if (lane == kWave - 1) wave_tot[wave] = inc;
  __syncthreads();
  u64 before = 0, all = 0;
  for (int w = 0; w < kNucWaves; ++w) {
    if (w < wave) before += wave_tot[w];
    all += wave_tot[w];
  }
  __syncthreads();
  *total = all;
  return before + inc - v;
}

// Scans hist from the top digit down; returns the digit at which the running
// weight reaches rem (1 <= rem <= sum of hist) and the weight of the digits
// above it.  Thread t covers the digits nb-1-t*per .. nb-per-t*per.
__device__ __forceinline__ void nuc_scan(const u64* hist, int nb, u64 rem, NucLds& sh, uint32_t* digit,
                         u64* above) {
  const int per = nb / kNucThreads;
  const int t = threadIdx.x;
  u64 s = 0;
  for (int i = 0; i < per; ++i) s += hist[nb - 1 - (t * per + i)];
  u64 total;
  u64 run = nuc_excl_scan(s, sh.wave_tot, &total);
  if (run < rem && rem <= run + s) {  // true for exactly one thread
    for (int i = 0; i < per; ++i) {
      const int d = nb - 1 - (t * per + i);
      const u64 h = hist[d];
      if (run < rem && rem <= run + h) {
        sh.pick_digit = static_cast<uint32_t>(d);
        sh.pick_above = run;
      }
      run += h;
    }
  }
  __syncthreads();
  *digit = sh.pick_digit;
  *above = sh.pick_above;
  __syncthreads();
}

// First-pass histogram of the live weights; returns the block's total weight.
template <bool kCount>
__device__ __forceinline__ u64 nuc_top_hist(const float* x, uint32_t live, NucRow r, NucLds& sh) {
  for (int i = threadIdx.x; i < kTopBins; i += kNucThreads) sh.top[i] = 0ull;
  __syncthreads();
  u64 mine = 0;
#pragma unroll
  for (int j = 0; j < kNucPer; ++j) {
    const float xj = nuc_x(x, j);
    const u64 w = nuc_weight<kCount>(xj, live, j, r);
    if (w) atomicAdd(&sh.top[order_key(xj) >> 20], w);
    mine += w;
  }
  u64 total;
  nuc_excl_scan(mine, sh.wave_tot, &total);  // also orders the histogram writes before any read
  return total;
}

// The first id of the order at which the running live weight reaches thr
// (1 <= thr <= total live weight); sh.top must hold the first-pass histogram
// of the same weights.  *cum = running weight through that id, *key_out = its
// key.
template <bool kCount>
__device__ __forceinline__ int nuc_select(const float* x, uint32_t live, NucRow r, int base, u64 thr, NucLds& sh,
                          u64* cum, uint32_t* key_out) {
  uint32_t digit;
  u64 above;
  nuc_scan(sh.top, kTopBins, thr, sh, &digit, &above);
  uint32_t prefix = digit << 20;
  u64 rem = thr - above, passed = above;
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const int shift = pass == 0 ? 10 : 0;
    const uint32_t hi_mask = 0xffffffffu << (shift + 10);
    for (int i = threadIdx.x; i < kLowBins; i += kNucThreads) sh.low[i] = 0ull;
    __syncthreads();
  #pragma unroll
    for (int j = 0; j < kNucPer; ++j) {
      const float xj = nuc_x(x, j);
      const uint32_t key = order_key(xj);
      if ((key & hi_mask) == prefix) {
        const u64 w = nuc_weight<kCount>(xj, live, j, r);
        if (w) atomicAdd(&sh.low[(key >> shift) & (kLowBins - 1)], w);
      }
    }
    __syncthreads();
    nuc_scan(sh.low, kLowBins, rem, sh, &digit, &above);
    prefix |= digit << shift;
    rem -= above;
    passed += above;
  }
  // Tie group: the live ids with key == prefix, all of one weight; the wanted
  // one is number (rem - 1) / weight of them in id order.
  int mine = 0;
  u64 wt = 0;
#pragma unroll
  for (int j = 0; j < kNucPer; ++j) {
    const float xj = nuc_x(x, j);
    if (order_key(xj) == prefix) {
      const u64 w = nuc_weight<kCount>(xj, live, j, r);
      if (w) {
        ++mine;
        wt = w;
      }
    }
  }
  u64 ties;
  const u64 before = nuc_excl_scan(static_cast<u64>(mine), sh.wave_tot, &ties);
  if (mine > 0 && before == 0) sh.tie_weight = wt;  // the first holder
  __syncthreads();
  const u64 w_tie = sh.tie_weight;
  const u64 rank = (rem - 1) / w_tie;
  if (mine > 0 && before <= rank && rank < before + static_cast<u64>(mine)) {
    int want = static_cast<int>(rank - before);
  #pragma unroll
    for (int j = 0; j < kNucPer; ++j) {
      const float xj = nuc_x(x, j);
      if (order_key(xj) == prefix && nuc_weight<kCount>(xj, live, j, r) != 0ull) {
        if (want == 0) sh.pick_id = base + j;
        --want;
      }
    }
  }
  __syncthreads();
  const int id = sh.pick_id;
  __syncthreads();
  *cum = passed + (rank + 1) * w_tie;
  *key_out = prefix;
  return id;
}

// ---------------------------------------------------------------------------
// Nucleus + draw without top-k, by buckets (the order, masses and thresholds
// of the radix select above, hence the same ids).
//
// An element's bucket is its log2 distance below the row maximum,
// floor((max - x) * log2(e) / T * kFastBins / range), capped at the last
// bucket; the maximum itself is bucket 0.  range is the row's own spread in
// log2 units, (max - min) * log2(e) / T, capped at kFastRange = 48 octaves: a
// mass below 1 (2^-47 of the maximum's) truncates to 0 and never holds a
// threshold, so the capped range still spans every element that can be
// picked, and a narrow row spreads over all the buckets (few members each:
// little LDS atomic contention, small resolves).  The map is monotone (x1 > x2
// gives bucket(x1) <= bucket(x2): a correctly rounded subtraction and products
// with positive constants keep the order), so every element of a lower bucket
// precedes every element of a higher one, and the running mass at a bucket's
// start is the exact sum over the buckets before it.
//
// One scan of the bucket masses places both thresholds (the nucleus size and
// the draw); inside the bucket holding a threshold its members (at most
// kFastCap, else the caller falls back to the radix select) are gathered to
// LDS and each computes its running mass in the exact order (key, then id).
constexpr int kFastBins = 2 * kNucThreads;  // two per thread
constexpr int kFastCap = kNucThreads;
constexpr float kFastRange = 48.f;

struct FastLds {
  u64 mass[kFastBins];
  u64 cand_mass[kFastCap];
  uint32_t cand_key[kFastCap];
  int32_t cand_id[kFastCap];
  u64 wave_tot[kNucWaves];
  u64 above;
  u64 run;
  int32_t ncand;
  int32_t bin;
  int32_t id;
};

__device__ __forceinline__ int fast_bin(float x, NucRow r) {
  if (x == r.m) return 0;
  const float d = ((r.m - x) * r.c) * r.b;
  return d < static_cast<float>(kFastBins - 1) ? static_cast<int>(d) : kFastBins - 1;
}

// Bucket holding running mass thr (1 <= thr <= total), from the scan state of
// thread t (bins 2t, 2t+1: masses h0, h1, exclusive prefix P): sets fs.bin and
// fs.above (the mass of the buckets before it).
__device__ __forceinline__ void fast_find(u64 thr, u64 P, u64 h0, u64 h1, FastLds& fs) {
  if (P < thr && thr <= P + h0 + h1) {  // exactly one thread
    const int t = threadIdx.x;
    if (thr <= P + h0) {
      fs.bin = 2 * t;
      fs.above = P;
    } else {
      fs.bin = 2 * t + 1;
      fs.above = P + h0;
    }
  }
  if (threadIdx.x == 0) fs.ncand = 0;
  __syncthreads();
}

// The member of bucket fs.bin at which the running mass inside the bucket
// reaches rem; false (uniformly) when the bucket has more than kFastCap
// members.  *id = that member, *run = the bucket-local running mass through it.
__device__ __forceinline__ bool fast_resolve(const float* x, uint32_t live, NucRow r, int base, u64 rem,
                             FastLds& fs, int* id, u64* run) {
  const int bin = fs.bin;
#pragma unroll
  for (int j = 0; j < kNucPer; ++j) {
    const float xj = nuc_x(x, j);
    if (fast_bin(xj, r) != bin) continue;  // the mass only for the bucket's members
    const u64 w = nuc_weight<false>(xj, live, j, r);
    if (w != 0ull) {
      const int slot = atomicAdd(&fs.ncand, 1);
      if (slot < kFastCap) {
        fs.cand_key[slot] = order_key(xj);
        fs.cand_id[slot] = base + j;
        fs.cand_mass[slot] = w;
      }
    }
  }
  __syncthreads();
  const int n = fs.ncand;
  if (n > kFastCap) return false;
  const int t = threadIdx.x;
  if (t < n) {
    const uint32_t k = fs.cand_key[t];
    const int my = fs.cand_id[t];
    const u64 w = fs.cand_mass[t];
    u64 before = 0ull;
    // every member read unconditionally, the order test branch-free
#pragma unroll 4
    for (int i = 0; i < n; ++i) {
      const uint32_t ki = fs.cand_key[i];
      const int ii = fs.cand_id[i];
      const u64 mi = fs.cand_mass[i];
      const bool ahead = (ki > k) | ((ki == k) & (ii < my));
      before += ahead ? mi : 0ull;
    }
    if (before < rem && rem <= before + w) {  // exactly one member
      fs.id = my;
      fs.run = before + w;
    }
  }
  __syncthreads();
  *id = fs.id;
  *run = fs.run;
  __syncthreads();
  return true;
}

// The whole draw without top-k; false (uniformly) when a bucket overflows or
// the row has no mass, for the caller's radix path.
__device__ __forceinline__ bool fast_top_p(const float* x, uint32_t live, NucRow r, int base, float top_p,
                           float u, FastLds& fs, int* out_id) {
  const int t = threadIdx.x;
  for (int i = t; i < kFastBins; i += kNucThreads) fs.mass[i] = 0ull;
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kNucPer; ++j) {
    const float xj = nuc_x(x, j);
    const u64 w = nuc_weight<false>(xj, live, j, r);
    atomicAdd(&fs.mass[fast_bin(xj, r)], w);   // adds 0 for ids outside the row
  }
  __syncthreads();
  const u64 h0 = fs.mass[2 * t], h1 = fs.mass[2 * t + 1];
  u64 total;
  const u64 P = nuc_excl_scan(h0 + h1, fs.wave_tot, &total);
  if (total == 0ull) return false;
  u64 kept = total;
  int id;
  u64 run;
  if (top_p > 0.f && top_p < 1.f) {
    u64 thr = static_cast<u64>(ceil(static_cast<double>(top_p) * static_cast<double>(total)));
    thr = thr < 1ull ? 1ull : (thr > total ? total : thr);
    fast_find(thr, P, h0, h1, fs);
    const u64 above = fs.above;
    if (!fast_resolve(x, live, r, base, thr - above, fs, &id, &run)) return false;
    kept = above + run;
  }
  const double ud = static_cast<double>(u);
  u64 y = 1ull;
  if (ud > 0.0) y = static_cast<u64>(floor(ud * static_cast<double>(kept))) + 1ull;
  if (y > kept) y = kept;
  fast_find(y, P, h0, h1, fs);
  const u64 above = fs.above;
  if (!fast_resolve(x, live, r, base, y - above, fs, &id, &run)) return false;
  *out_id = id;
  return true;
}

template <bool kVec4>
__global__ __launch_bounds__(kNucThreads) void top_p_kernel(const float* __restrict__ logits,
                                                            int V, float temperature, int top_k,
                                                            float top_p,
                                                            const float* __restrict__ u,
                                                            int32_t* __restrict__ out) {
  __shared__ NucLds sh;
  __shared__ FastLds fs;
  const int t = threadIdx.x;
  const int lane = t & (kWave - 1), wave = t / kWave;
  const int base = t * kNucPer;
  const float* row = logits + static_cast<size_t>(blockIdx.x) * V;
  float x[kNucPer];
  uint32_t live = 0;
  if (kVec4) {
#pragma unroll
    for (int q = 0; q < kNucPer / 4; ++q) {
      const int i = base + 4 * q;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (i < V) v = *reinterpret_cast<const float4*>(row + i);  // V % 4 == 0
      x[4 * q] = v.x;
      x[4 * q + 1] = v.y;
      x[4 * q + 2] = v.z;
      x[4 * q + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < kNucPer; ++j) x[j] = base + j < V ? row[base + j] : 0.f;
  }
  float m = -INFINITY, mn = INFINITY;
#pragma unroll
  for (int j = 0; j < kNucPer; ++j) {
    const bool ok = base + j < V;
    live |= static_cast<uint32_t>(ok) << j;
    if (ok) {
      m = fmaxf(m, x[j]);
      mn = fminf(mn, x[j]);
    }
  }
  m = wave_max(m);
  mn = -wave_max(-mn);
  if (lane == 0) {
    sh.red[wave] = m;
    sh.red_min[wave] = mn;
  }
  __syncthreads();
  m = sh.red[0];
  mn = sh.red_min[0];
  for (int w = 1; w < kNucWaves; ++w) {
    m = fmaxf(m, sh.red[w]);
    mn = fminf(mn, sh.red_min[w]);
  }
  const float c = 1.4426950408889634f / temperature;  // log2(e) / T
  float range = (m - mn) * c;                          // NaN for a row of one infinity
  if (!(range > 1e-6f)) range = 1e-6f;
  if (range > kFastRange) range = kFastRange;
  const NucRow r{m, c, static_cast<float>(kFastBins) / range};

  // top_k <= 0: the bucket path (top_k >= V, the same id set, stays on the
  // radix path below)
  if (top_k <= 0) {
    int id;
    if (fast_top_p(x, live, r, base, top_p, u[blockIdx.x], fs, &id)) {
      if (t == 0) out[blockIdx.x] = id;
      return;
    }
  }
  u64 cum;
  uint32_t kkey;
  if (top_k > 0 && top_k < V) {
    nuc_top_hist<true>(x, live, r, sh);
    const int kid = nuc_select<true>(x, live, r, base, static_cast<u64>(top_k), sh, &cum, &kkey);
#pragma unroll
    for (int j = 0; j < kNucPer; ++j) {
      const uint32_t key = order_key(nuc_x(x, j));
      const bool in = key > kkey || (key == kkey && base + j <= kid);
      if (!in) live &= ~(1u << j);
    }
  }
  const u64 total = nuc_top_hist<false>(x, live, r, sh);
  u64 kept = total;
  if (top_p > 0.f && top_p < 1.f) {
    u64 thr = static_cast<u64>(ceil(static_cast<double>(top_p) * static_cast<double>(total)));
    thr = thr < 1ull ? 1ull : (thr > total ? total : thr);
    nuc_select<false>(x, live, r, base, thr, sh, &kept, &kkey);
  }
  const double ud = static_cast<double>(u[blockIdx.x]);
  u64 y = 1ull;
  if (ud > 0.0) y = static_cast<u64>(floor(ud * static_cast<double>(kept))) + 1ull;
  if (y > kept) y = kept;
  const int id = nuc_select<false>(x, live, r, base, y, sh, &cum, &kkey);
  if (t == 0) out[blockIdx.x] = id;
}

// ---------------------------------------------------------------------------
// Repetition penalty, in place: every distinct id of recent[r, :] inside
// [0, V) has its logit divided by `penalty` when positive and multiplied by
// it otherwise; an id listed several times is penalised once (the set of
// sample_standalone.py:5602).  An LDS bitmap of claimed ids makes exactly one
// listing of each id apply it.
constexpr int kRepMaxV = 1 << 18;

__global__ __launch_bounds__(1024) void rep_penalty_kernel(float* __restrict__ logits, int V,
                                                           const int32_t* __restrict__ recent,
                                                           int n_recent, float penalty) {
  __shared__ uint32_t claimed[kRepMaxV / 32];
  const int words = (V + 31) / 32;
  for (int i = threadIdx.x; i < words; i += blockDim.x) claimed[i] = 0u;
  __syncthreads();
  float* row = logits + static_cast<size_t>(blockIdx.x) * V;
  const int32_t* ids = recent + static_cast<size_t>(blockIdx.x) * n_recent;
  for (int i = threadIdx.x; i < n_recent; i += blockDim.x) {
    const int id = ids[i];
    if (id < 0 || id >= V) continue;
    const uint32_t bit = 1u << (id & 31);
    if (atomicOr(&claimed[id >> 5], bit) & bit) continue;
    const float v = row[id];
    row[id] = v > 0.f ? v / penalty : v * penalty;
  }
}

}  // namespace llmy

using namespace llmy;

extern "C" int32_t llmy_sample_argmax_f32(const float* logits, int32_t rows, int32_t V,
                                          int32_t* out, void* stream) {
  LLMY_REQUIRE(rows >= 0 && V > 0);
  if (rows == 0) return 0;
  LLMY_REQUIRE(logits && out);
  hipLaunchKernelGGL(argmax_rows_kernel, dim3(rows), dim3(1024), 0, as_stream(stream), logits, V,
                     out);
  return launch_status();
}

extern "C" int32_t llmy_sample_top_p_f32(const float* logits, int32_t rows, int32_t V,
                                         float temperature, int32_t top_k, float top_p,
                                         const float* u, int32_t* out, void* stream) {
  LLMY_REQUIRE(rows >= 0 && V > 0 && V <= kNucMaxV);
  if (rows == 0) return 0;
  LLMY_REQUIRE(logits && out);
  if (!(temperature > 0.f)) {  // greedy, as llmy.cpp:166
    hipLaunchKernelGGL(argmax_rows_kernel, dim3(rows), dim3(1024), 0, as_stream(stream), logits,
                       V, out);
    return launch_status();
  }
  LLMY_REQUIRE(u != nullptr);
  if (V % 4 == 0 && aligned(logits, 16)) {
    hipLaunchKernelGGL(top_p_kernel<true>, dim3(rows), dim3(kNucThreads), 0, as_stream(stream),
                       logits, V, temperature, top_k, top_p, u, out);
  } else {
    hipLaunchKernelGGL(top_p_kernel<false>, dim3(rows), dim3(kNucThreads), 0, as_stream(stream),
                       logits, V, temperature, top_k, top_p, u, out);
  }
  return launch_status();
}

extern "C" int32_t llmy_repetition_penalty_f32(float* logits, int32_t rows, int32_t V,
                                               const int32_t* recent, int32_t n_recent,
                                               float penalty, void* stream) {
  LLMY_REQUIRE(rows >= 0 && V > 0 && V <= kRepMaxV && n_recent >= 0);
  LLMY_REQUIRE(penalty > 0.f);
  if (rows == 0 || n_recent == 0 || penalty == 1.f) return 0;
  LLMY_REQUIRE(logits && recent);
  hipLaunchKernelGGL(rep_penalty_kernel, dim3(rows), dim3(1024), 0, as_stream(stream), logits, V,
                     recent, n_recent, penalty);
  return launch_status();
}
