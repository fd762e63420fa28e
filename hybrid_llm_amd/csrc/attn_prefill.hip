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
//   * tiles arrive by global_load_lds_dwordx4 (global memory straight into
//     LDS, no register holds them) into two stages: the next tile's DMA runs
//     while the current one is consumed, one barrier per tile.  K and V rows
//     are kept row-major with their 16-byte chunks XOR-swizzled by row (K by
//     row & 7, V by 2 (row & 3)), which keeps the 8-lane K fragment reads and
//     the 16-lane transposing V reads free of bank conflicts; a DMA lane
//     fetches the chunk that its fixed LDS slot holds under the swizzle;
//   * the V^T fragments come from the row-major V by ds_read_b64_tr_b16: in
//     each 16-lane group, lane 4a + e receives element e of the 8 bytes that
//     lanes a, a + 4, a + 8 and a + 12 address, so lanes addressing 4
//     consecutive keys at 4 dims each hand every lane one dim of 4 keys;
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

typedef __attribute__((address_space(3))) void lds_void;
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void dma16(const void* src, void* lds_dst) {
  __builtin_amdgcn_global_load_lds(src, (lds_void*)lds_dst, 16, 0, 0);
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const lds_void*)p));
}

// LDS reads as inline asm: with a DMA into the other stage in flight, the
// compiler would make every LDS read wait for it.  Their results are valid
// after lds_settle.
__device__ __forceinline__ u32x4 lds_b128(uint32_t addr) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr) : "memory");
  return v;
}

__device__ __forceinline__ u32x2 lds_tr16(uint32_t addr) {
  u32x2 v;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(v) : "v"(addr) : "memory");
  return v;
}

// Wait for every LDS read of this wave and tie the registers they filled to
// the wait, so no use is scheduled above it.
__device__ __forceinline__ void lds_settle4(u32x4* f) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3])::"memory");
}

__device__ __forceinline__ void lds_settle_v(u32x2* f) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]),
                 "+v"(f[6]), "+v"(f[7])::"memory");
}

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
  constexpr int TILE = kBN * HD;  // bf16 elements of one staged K or V tile
  constexpr int RB = 2 * HD;      // bytes per staged row
  // two stages, each the K tile then the V tile
  __shared__ __align__(16) uint16_t smem[2 * 2 * TILE];

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
  // DMA: per tile and array, 1 KiB blocks j = wave + 4 i of RPB rows each;
  // lane p of block j fills row RPB j + p / CH, 16-byte slot p % CH, which
  // holds the row's chunk (slot ^ swizzle).  Rows past the sequence (the last
  // tile only) re-read row T - 1: those keys follow every query and are masked.
  constexpr int CH = HD / 8;             // 16-byte chunks per row
  constexpr int RPB = 64 / CH;           // rows per 1 KiB block
  constexpr int BPW = kBN / RPB / 4;     // blocks per wave per array
  static_assert(BPW * 4 * RPB == kBN, "the waves' blocks cover the tile");
  uint32_t kdo[BPW], vdo[BPW];
  int drow[BPW];
#pragma unroll
  for (int i = 0; i < BPW; ++i) {
    const int r = RPB * (wave + 4 * i) + lane / CH, sl = lane % CH;
    drow[i] = r;
    kdo[i] = 8 * (sl ^ (r & 7));
    vdo[i] = 8 * (sl ^ (2 * (r & 3)));
  }
  const uint16_t* kbase = k + base;
  const uint16_t* vbase = v + base;
  auto issue = [&](int tile, int st) {
    const int kt = tile * kBN;
    uint16_t* sk = smem + st * 2 * TILE;
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
      const uint32_t ro = static_cast<uint32_t>(min(kt + drow[i], T - 1)) * rs32;
      dma16(kbase + ro + kdo[i], sk + (wave + 4 * i) * 512);
      dma16(vbase + ro + vdo[i], sk + TILE + (wave + 4 * i) * 512);
    }
  };
  // Fragment offsets (bytes from a stage's K or V tile).  K: key row col of the
  // sub-tile, dims 16 t + 8 half (chunk 2 t + half).  V (transposing reads):
  // lane 16 g + y addresses key 4 half + y / 4 (of the 16-key slice's lo or hi
  // 8) at dims 32 d + 16 (g & 1) + 4 (y & 3) .. +3, and receives dim
  // 32 d + col for keys 4 half .. +3 (lo) or 8 + 4 half .. +3 (hi), the
  // B-operand key order of P.
  const uint32_t sbase = lds_addr(smem);
  uint32_t koff[NS], voff[ND];
#pragma unroll
  for (int t = 0; t < NS; ++t) koff[t] = col * RB + 16 * ((2 * t + half) ^ (col & 7));
  {
    const int y = lane & 15, g = lane >> 4, i = y >> 2;
#pragma unroll
    for (int d = 0; d < ND; ++d) {
      const int dim0 = 32 * d + 16 * (g & 1) + 4 * (y & 3);
      voff[d] = (4 * half + i) * RB + 16 * ((dim0 >> 3) ^ (2 * i)) + 2 * (dim0 & 7);
    }
  }
  issue(t_lo, 0);
  for (int tile = t_lo; tile <= t_hi; ++tile) {
    const int kt = tile * kBN;
    const int st = (tile - t_lo) & 1;
    // this wave's DMA of the tile has landed; after the barrier every wave's
    // has, and every wave is done with the other stage, which the next tile's
    // DMA then fills while this one is consumed
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tile < t_hi) issue(tile + 1, st ^ 1);
    const uint32_t kst = sbase + st * 4 * TILE, vst = kst + 2 * TILE;

#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int ks = kt + 32 * sub;  // first key of the 32-key sub-tile
      // skip sub-tiles wholly outside every window of this wave's queries
      if (ks > qw + 31 || ks + 31 < qw - W + 1 || ks >= T) continue;
      // ---- S^T = K Q^T over HD (NS MFMAs)
      f32x16v s;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = 0.f;
      u32x4 kf[NS];
#pragma unroll
      for (int t = 0; t < NS; ++t) kf[t] = lds_b128(kst + 32 * sub * RB + koff[t]);
      static_assert(NS % 4 == 0, "K fragments settle four at a time");
#pragma unroll
      for (int t = 0; t < NS; t += 4) lds_settle4(kf + t);
#pragma unroll
      for (int t = 0; t < NS; ++t)
        s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, kf[t]),
                                                    as_bf16x8(qf[t]), s, 0, 0, 0);
      // V^T fragments of both 16-key slices, requested ahead of the softmax
      u32x2 vf[2][ND][2];
#pragma unroll
      for (int sl = 0; sl < 2; ++sl)
#pragma unroll
        for (int d = 0; d < ND; ++d) {
          const uint32_t va = vst + (32 * sub + 16 * sl) * RB + voff[d];
          vf[sl][d][0] = lds_tr16(va);
          vf[sl][d][1] = lds_tr16(va + 8 * RB);
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
      // ---- O^T += V^T P^T over the two 16-key slices (keys of slice sl for
      //      this lane: ks + 16 sl + kappa(half, j))
      static_assert(ND % 2 == 0, "V fragments settle eight at a time");
#pragma unroll
      for (int q8 = 0; q8 < ND / 2; ++q8) lds_settle_v(&vf[0][0][0] + 8 * q8);
#pragma unroll
      for (int sl = 0; sl < 2; ++sl) {
        const uint4 pb = pack8_bf16(p + 8 * sl);
#pragma unroll
        for (int d = 0; d < ND; ++d) {
          const uint4 va = uint4{vf[sl][d][0].x, vf[sl][d][0].y, vf[sl][d][1].x, vf[sl][d][1].y};
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
