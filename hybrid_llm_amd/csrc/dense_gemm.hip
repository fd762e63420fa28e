// Tiled bf16 MFMA GEMM on gfx950: the dense projections of a sequence
// prefill (llmy_linear_bf16 with many rows), out[M, N] = x[M, K] . w[N, K]^T
// with the linear epilogues, and an N tail (rows past N re-read row N-1,
// their columns are not stored).  The MoE prefill GEMMs are the grouped
// kernel of moe_grouped.hip.
//
// Tiling: a workgroup of 4 wavefronts computes a BM x BN tile of the A rows
// times the B (weight) rows; wavefront (wm, wn) of the 2 x 2 grid owns a
// (BM/2) x (BN/2) sub-tile as (BM/64) x (BN/64) blocks of
// v_mfma_f32_32x32x16_bf16, so LDS traffic is (BM/64 + BN/64) fragment reads
// per (BM/64)(BN/64) MFMAs.  256 x 256 tiles run one workgroup per CU (the
// accumulators fill the AGPR half of the register file); 128-row tiles run
// two per CU when there are more tiles than CUs, one wavefront of each per
// SIMD, so one workgroup's barrier and load waits are covered by the other's
// MFMAs, and one per CU with a deeper ring otherwise.  The MFMA takes the weight
// fragment as its first operand, so each lane ends with four consecutive
// output columns per register group and stores them as one vector.
//
// K advances BK (32 or 64) at a time through a ring of NS LDS stages filled
// by global_load_lds_dwordx4 (global memory straight into LDS) from scalar
// base addresses plus 32-bit lane offsets: while one K tile is multiplied,
// the next NS-1 are in flight.  Tile rows hold BK k with an XOR swizzle of
// their 16-byte chunks, so each DMA instruction reads whole global row
// segments and each fragment read (inline-asm ds_read_b128, see lds_frag) is
// conflict-free.  The loop is a software pipeline with scheduling fences:
// the fragment reads of k-step s+1 are in flight during the MFMAs of step s,
// and the first reads of tile kt+1 during the last MFMAs of tile kt.
//
// Work order: work items (n-tile, m-tile) are grouped 4 m-tiles x all
// n-tiles, m fastest inside a group, and each XCD (block id mod 8) takes a
// contiguous range of them, so the tiles an XCD runs together share few A
// and B tiles in its L2.
#include "common.hpp"
#include "abi_util.hpp"

namespace llmy {

// Dense epilogues (values of the linear entry's epilogue argument).
enum DenseEpi : int { kDenseBf16 = 0, kDenseF32 = 1, kDenseResid = 2, kDenseGated = 3 };

struct TileArgs {
  const uint16_t* x;  // [M, K]
  const uint16_t* w;  // weights, row-major [N, K] or packed
  void* out;          // [M, ldo] (bf16 or fp32 by epilogue)
  const float* aux;   // gated residual: out += acc * aux[m * ldo + n]
  int K, ldo, M;
  int N;        // output columns (last n-tile may be partial)
  int n_tiles;  // output column tiles
  int m_tiles;  // row tiles
  int group_m;  // m-tiles per work group (0: m fastest over all rows)
  int packed;
};

namespace {

constexpr int kThreads = 256;  // 4 wavefronts: one per SIMD
constexpr int kNumXcd = 8;

// Packed operand order of llmy_pack_weights_bf16 (see linear.hip): the 8
// elements W[n][k .. k+7] (k % 8 == 0) are contiguous at this index.
__device__ __forceinline__ long long packed_at(int n, int k, int K) {
  const int nb = n >> 4, r = n & 15;
  const int kb = k >> 8, kk = k & 255;
  const int j = kk >> 5, g = (kk >> 3) & 3;
  const int lane = g * 16 + r;
  return (((static_cast<long long>(nb) * (K >> 8) + kb) * 8 + j) * 64 + lane) << 3;
}

typedef __attribute__((address_space(3))) void lds_void;
// A __shared__ address in the LDS address space (the destination operand of
// global_load_lds).
__device__ __forceinline__ lds_void* as_lds(void* p) { return (lds_void*)p; }

// One global_load_lds_dwordx4: 16 bytes per lane from src into LDS at dst
// (+16 bytes per lane).  Kept in a device function: the builtin inside a
// kernel template body stops the host pass from emitting the launch stub.
__device__ __forceinline__ void dma16(const void* src, void* dst) {
  __builtin_amdgcn_global_load_lds(src, as_lds(dst), 16, 0, 0);
}

// s_waitcnt immediate (gfx9 encoding) that waits until at most n vector
// memory operations of this wavefront are outstanding and for all of its LDS
// operations (vmcnt bits [3:0] and [15:14]; expcnt [6:4] = 7; lgkmcnt
// [11:8] = 0).
constexpr int waitcnt_vm_lgkm0(int n) { return 0x0070 | (n & 15) | ((n >> 4) << 14); }

// 16-byte LDS read at byte address addr + OFF, as inline asm: the compiler's
// LDS-DMA tracking cannot separate the stage being read from the stage being
// filled and would make every read wait for all loads in flight.  The result
// is valid only after a settle below.
template <int OFF>
__device__ __forceinline__ u32x4 lds_frag(uint32_t addr) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF) : "memory");
  return v;
}

// Wait until at most N of this wavefront's LDS operations are outstanding
// (LDS operations complete in order, so every read issued before the last N
// is done) and tie the registers those reads filled to the wait, so every
// later use of them follows it.
template <int N>
__device__ __forceinline__ void settle4(u32x4& a, u32x4& b, u32x4& c, u32x4& d) {
  asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : "i"(N) : "memory");
}
template <int N>
__device__ __forceinline__ void settle2(u32x4& a, u32x4& b) {
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "i"(N) : "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const lds_void*)p));
}

__device__ __forceinline__ f32x16 mfma32(const u32x4& a, const u32x4& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

}  // namespace

template <int BM, int BN, int BK, int NS, int EPI, int OCC = 1>
__global__ __launch_bounds__(kThreads, OCC) void tile_gemm_kernel(TileArgs a) {
  constexpr int WM = BM / 2, WN = BN / 2;  // wavefront sub-tile
  constexpr int FA = WM / 32, FB = WN / 32;  // 32-row / 32-column MFMA blocks per wavefront
  constexpr int ROWB = BK * 2;      // bytes of one tile row in a stage
  constexpr int CPR = BK / 8;       // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;     // tile rows per DMA instruction
  constexpr int SWZ = 16 / CPR;     // rows sharing one swizzle value
  constexpr int KS = BK / 16;       // MFMA k-steps per stage
  constexpr int A_INS = BM / RPI / 4;  // DMA instructions per wavefront per stage
  constexpr int B_INS = BN / RPI / 4;
  constexpr int DPT = A_INS + B_INS;   // DMA instructions per wavefront per K tile
  constexpr int A_BYTES = BM * ROWB;
  constexpr int STAGE_BYTES = (BM + BN) * ROWB;
  constexpr int NF = FA + FB;  // fragment reads per k-step
  static_assert(FA == 2 || FA == 4, "wavefront rows");
  static_assert(FB == 2 || FB == 4, "wavefront columns");
  static_assert(BK == 32 || BK == 64, "K tile");
  static_assert(NS >= 2 && DPT * (NS - 2) <= 63, "vmcnt range");
  __shared__ int s_work[3];  // work flag (-1: none), m0, n-tile

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;

  // ---- which tile: work item w = (n-tile, m-tile), m fastest.
  const int nblk = gridDim.x;
  const int per_xcd = (nblk + kNumXcd - 1) / kNumXcd;
  const int w_item = (blockIdx.x % kNumXcd) * per_xcd + blockIdx.x / kNumXcd;
  if (tid == 0) {
    const bool ok = w_item < a.m_tiles * a.n_tiles;
    int mt = w_item % a.m_tiles, nt = w_item / a.m_tiles;
    if (a.group_m > 0) {
      // groups of group_m m-tiles x all n-tiles, m fastest inside a group,
      // so the tiles an XCD runs together share few A and B tiles
      const int per_group = a.group_m * a.n_tiles;
      const int grp = w_item / per_group, in = w_item % per_group;
      const int gm = min(a.group_m, a.m_tiles - grp * a.group_m);
      mt = grp * a.group_m + in % gm;
      nt = in / gm;
    }
    s_work[0] = ok ? 0 : -1;
    s_work[1] = ok ? mt * BM : 0;
    s_work[2] = ok ? nt : 0;
  }
  __syncthreads();
  if (s_work[0] < 0) return;
  const int m0 = s_work[1], ntile = s_work[2];
  const int rows_e = a.M;
  const int K = a.K;
  const int nk = K / BK;

  // ---- global sources.  A stage holds the A tile (BM rows) then the B tile
  // (BN rows), each row BK k = CPR chunks of 16 bytes, chunk c of row r
  // stored in slot c ^ ((r / SWZ) % CPR).  A ds_read_b128 is served 16 lanes
  // at a time from 256 bytes of banks; the 16 lanes of a fragment read take
  // 16 consecutive rows at one chunk index, which this swizzle spreads over
  // all 16 bank groups.  Each global_load_lds instruction fills RPI
  // consecutive tile rows, lane l taking row l / CPR and slot l % CPR, i.e.
  // one whole row segment per CPR lanes.
  const int dma_row = lane / CPR;
  // Byte offsets (32-bit; the host bounds each operand block below 2 GiB)
  // of the 16 bytes this lane fetches, relative to the operand base: for
  // tile row r the lane takes global chunk (lane % CPR) ^ ((r / SWZ) % CPR).
#define DMA_CH(r) ((lane % CPR) ^ (((r) / SWZ) % CPR))
  uint32_t a_off[A_INS];
#pragma unroll
  for (int q = 0; q < A_INS; ++q) {
    const int r = RPI * (A_INS * wave + q) + dma_row;  // tile row
    const long long m = min(m0 + r, rows_e - 1);        // past the rows: repeat the last
    a_off[q] = static_cast<uint32_t>((m * K + 8 * DMA_CH(r)) * 2);
  }
  const bool packed = a.packed != 0;
  uint32_t b_off[B_INS];
#pragma unroll
  for (int q = 0; q < B_INS; ++q) {
    const int r = RPI * (B_INS * wave + q) + dma_row;  // tile row
    const int n = min(BN * ntile + r, a.N - 1);  // N tail: repeat the last row
    const int ch = DMA_CH(r);
    b_off[q] = static_cast<uint32_t>(
        (packed ? packed_at(n, 8 * ch, K) : static_cast<long long>(n) * K + 8 * ch) * 2);
  }
#undef DMA_CH
  const char* a_base = reinterpret_cast<const char*>(a.x);
  const char* b_base = reinterpret_cast<const char*>(a.w);
  // The wavefront index as a scalar, so LDS destinations (M0) are scalar arithmetic.
  const int wv = __builtin_amdgcn_readfirstlane(wave);

  // NS LDS stages in a ring: K tiles kt+1 .. kt+NS-1 are in flight while
  // tile kt is multiplied.
  __shared__ __align__(1024) unsigned char smem[NS * STAGE_BYTES];
  const uint32_t smem_base = lds_addr(smem);

  // K tile kt of both operands into stage `stage`.  Byte offset of K tile kt
  // within a B row: row-major 2 BK kt; packed: 256-k blocks are 8 KiB apart,
  // 32-k pieces 1 KiB.
#define TILE_ISSUE(kt, stage)                                                               \
  do {                                                                                      \
    const long long ka_ = static_cast<long long>(kt) * BK;                                  \
    const long long kb_ = packed ? (ka_ >> 8) * 4096 + ((ka_ & 255) >> 5) * 512 : ka_;      \
    const char* ab_ = a_base + 2 * ka_;                                                     \
    const char* bb_ = b_base + 2 * kb_;                                                     \
    unsigned char* st_ = smem + (stage) * STAGE_BYTES;                                      \
    _Pragma("unroll") for (int q = 0; q < A_INS; ++q)                                       \
        dma16(ab_ + a_off[q], st_ + (RPI * (A_INS * wv + q)) * ROWB);                       \
    _Pragma("unroll") for (int q = 0; q < B_INS; ++q)                                       \
        dma16(bb_ + b_off[q], st_ + A_BYTES + (RPI * (B_INS * wv + q)) * ROWB);             \
  } while (0)

  f32x16 acc[FA][FB];
#pragma unroll
  for (int i = 0; i < FA; ++i)
#pragma unroll
    for (int j = 0; j < FB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // Fragment address of k-step s: lane l reads tile row (32-row block base) +
  // l%32, chunk 2s + l/32, stored in slot (2s + l/32) ^ ((l%32 / SWZ) % CPR).
  uint32_t frag_off[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s)
    frag_off[s] = (lane & 31) * ROWB + (((2 * s + (lane >> 5)) ^ (((lane & 31) / SWZ) % CPR)) << 4);
  const uint32_t fa_base = (WM * wm) * ROWB;
  const uint32_t fb_base = A_BYTES + (WN * wn) * ROWB;
  constexpr int BLK = 32 * ROWB;  // bytes between 32-row blocks

  // Fragment reads of k-step S of the tile in stage STG into (FA_, FB_).
#define TILE_READ(FA_, FB_, STG, S)                                                        \
  do {                                                                                     \
    const uint32_t xa_ = smem_base + (STG) * STAGE_BYTES + fa_base + frag_off[S];          \
    const uint32_t xb_ = smem_base + (STG) * STAGE_BYTES + fb_base + frag_off[S];          \
    FA_[0] = lds_frag<0>(xa_);                                                             \
    FA_[1] = lds_frag<BLK>(xa_);                                                           \
    if (FA == 4) {                                                                         \
      FA_[FA - 2] = lds_frag<2 * BLK>(xa_);                                                \
      FA_[FA - 1] = lds_frag<3 * BLK>(xa_);                                                \
    }                                                                                      \
    FB_[0] = lds_frag<0>(xb_);                                                             \
    FB_[1] = lds_frag<BLK>(xb_);                                                           \
    if (FB == 4) {                                                                         \
      FB_[FB - 2] = lds_frag<2 * BLK>(xb_);                                                \
      FB_[FB - 1] = lds_frag<3 * BLK>(xb_);                                                \
    }                                                                                      \
  } while (0)

  // Wait until only the N most recent reads are outstanding, tying (FA_, FB_).
#define TILE_SETTLE(FA_, FB_, N)                                       \
  do {                                                                 \
    if (FA == 4) settle4<N>(FA_[0], FA_[1], FA_[FA - 2], FA_[FA - 1]); \
    else settle2<N>(FA_[0], FA_[1]);                                   \
    if (FB == 4) settle4<N>(FB_[0], FB_[1], FB_[FB - 2], FB_[FB - 1]); \
    else settle2<N>(FB_[0], FB_[1]);                                   \
  } while (0)

#define TILE_MMA(FA_, FB_)                                 \
  do {                                                     \
    _Pragma("unroll") for (int i = 0; i < FA; ++i)         \
        _Pragma("unroll") for (int j = 0; j < FB; ++j)     \
            acc[i][j] = mfma32(FB_[j], FA_[i], acc[i][j]); \
  } while (0)

  // Scheduling fence: the compiler keeps every instruction on its side.
#define FENCE() __builtin_amdgcn_sched_barrier(0)

  // Software pipeline.  Before iteration kt: tile kt is in LDS for every
  // wavefront (barrier passed), its step-0 fragment reads are in flight, and
  // tiles kt+1 .. kt+NS-2 are being fetched.  Iteration kt: fetch tile
  // kt+NS-1 into the stage of tile kt-1 (free since the last barrier); for
  // each k-step s, issue the reads of step s+1, wait for those of step s,
  // multiply step s; before the last step's MFMAs, wait for tile kt+1, meet
  // the workgroup, and issue the step-0 reads of tile kt+1, whose latency
  // the last step's MFMAs cover.
#pragma unroll
  for (int t = 0; t < NS - 1; ++t)
    if (t < nk) TILE_ISSUE(t, t);
  if (NS > 2 && nk > NS - 2) __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(DPT * (NS - 2)));
  else __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  u32x4 pa[FA], pb[FB], qa[FA], qb[FB];
  TILE_READ(pa, pb, 0, 0);
  int stage = 0;
  for (int kt = 0; kt < nk; ++kt) {
    const int nxt = stage == NS - 1 ? 0 : stage + 1;
    FENCE();
    if (kt + NS - 1 < nk) TILE_ISSUE(kt + NS - 1, stage == 0 ? NS - 1 : stage - 1);
    FENCE();
    TILE_READ(qa, qb, stage, 1);
    FENCE();
    TILE_SETTLE(pa, pb, NF);
    TILE_MMA(pa, pb);
    FENCE();
    if (KS == 4) {
      TILE_READ(pa, pb, stage, KS - 2);
      FENCE();
      TILE_SETTLE(qa, qb, NF);
      TILE_MMA(qa, qb);
      FENCE();
      TILE_READ(qa, qb, stage, KS - 1);
      FENCE();
      TILE_SETTLE(pa, pb, NF);
      TILE_MMA(pa, pb);
      FENCE();
    }
    TILE_SETTLE(qa, qb, 0);
    FENCE();
    // tile kt+1 landed: the tiles issued after it (up to kt+NS-1) may stay in flight
    if (kt + NS - 1 < nk) __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(DPT * (NS - 2)));
    else __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (kt + 1 < nk) TILE_READ(pa, pb, nxt, 0);
    FENCE();
    TILE_MMA(qa, qb);
    FENCE();
    // the next tile's first reads land before the loop edge: the compiler
    // knows nothing of asm reads in flight and may move their registers
    TILE_SETTLE(pa, pb, 0);
    stage = nxt;
  }
#undef FENCE
#undef TILE_MMA
#undef TILE_SETTLE
#undef TILE_READ
#undef TILE_ISSUE

  // ---- epilogue.  acc[i][j] = (weight block j) . (row block i)^T, so in the
  // 32x32 D layout lane l holds row m = 32 i + (l & 31) of the tile and, in
  // registers 4g .. 4g+3, the four consecutive columns 32 j + 8g + 4(l >> 5)
  // .. +3: every store is a 4-column vector.
#pragma unroll
  for (int i = 0; i < FA; ++i) {
    const int m = m0 + WM * wm + 32 * i + (lane & 31);
    if (m >= rows_e) continue;
    const long long p = m;
    {
      // Residual epilogues load a column block's residual (and gate) groups
      // before its first store: a store and a later load of another group
      // cannot be proved apart, so interleaving them would serialise one
      // memory round trip per group.
#pragma unroll
      for (int j = 0; j < FB; ++j) {
        float4 res[4], gat[4];
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int n = BN * ntile + WN * wn + 32 * j + 8 * g4 + 4 * (lane >> 5);
          const long long o = p * a.ldo + n;
          res[g4] = make_float4(0.f, 0.f, 0.f, 0.f);
          gat[g4] = make_float4(1.f, 1.f, 1.f, 1.f);
          if (n < a.N && (EPI == kDenseResid || EPI == kDenseGated))
            res[g4] = *reinterpret_cast<const float4*>(static_cast<const float*>(a.out) + o);
          if (n < a.N && EPI == kDenseGated)
            gat[g4] = *reinterpret_cast<const float4*>(a.aux + o);
        }
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int n = BN * ntile + WN * wn + 32 * j + 8 * g4 + 4 * (lane >> 5);
          if (n >= a.N) continue;  // N % 16 == 0: a 4-column group is all in or all out
          const long long o = p * a.ldo + n;
          const float v0 = acc[i][j][4 * g4], v1 = acc[i][j][4 * g4 + 1];
          const float v2 = acc[i][j][4 * g4 + 2], v3 = acc[i][j][4 * g4 + 3];
          if (EPI == kDenseBf16) {
            *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.out) + o) =
                make_uint2(pack_bf2(v0, v1), pack_bf2(v2, v3));
          } else if (EPI == kDenseF32) {
            *reinterpret_cast<float4*>(static_cast<float*>(a.out) + o) = make_float4(v0, v1, v2, v3);
          } else if (EPI == kDenseResid) {
            const float4 r = res[g4];
            *reinterpret_cast<float4*>(static_cast<float*>(a.out) + o) =
                make_float4(r.x + v0, r.y + v1, r.z + v2, r.w + v3);
          } else {
            const float4 r = res[g4], g = gat[g4];
            *reinterpret_cast<float4*>(static_cast<float*>(a.out) + o) =
                make_float4(r.x + v0 * g.x, r.y + v1 * g.y, r.z + v2 * g.z, r.w + v3 * g.w);
          }
        }
      }
    }
  }
}

template <int BM, int BN, int BK, int NS, int EPI, int OCC = 1>
int32_t launch_tiles(const TileArgs& g, long long items, hipStream_t s) {
  const unsigned grid = static_cast<unsigned>((items + kNumXcd - 1) / kNumXcd * kNumXcd);
  hipLaunchKernelGGL((tile_gemm_kernel<BM, BN, BK, NS, EPI, OCC>), dim3(grid), dim3(kThreads),
                     0, s, g);
  return launch_status();
}

int32_t dense_narrow_ws(const uint16_t* x, const uint16_t* w, void* out, const float* aux, int M,
                        int N, int K, int ldo, int epi, bool packed, hipStream_t s);

// Dense out[M, N] (epilogue epi) = x[M, K] . w[N, K]^T.  Validated by the
// caller: M >= 1, N >= 1, K % 256 == 0, 16-byte aligned x and w, aux given
// for the gated epilogue.
int32_t dense_gemm_mfma(const uint16_t* x, const uint16_t* w, void* out, const float* aux,
                        int M, int N, int K, int epi, bool packed, hipStream_t s) {
  // operand blocks addressed with 32-bit byte offsets
  if (2ll * M * K >= (1ll << 31) || 2ll * N * K >= (1ll << 31))
    return static_cast<int32_t>(hipErrorInvalidValue);
  TileArgs g{};
  g.x = x;
  g.w = w;
  g.out = out;
  g.aux = aux;
  g.K = K;
  g.ldo = N;
  g.M = M;
  g.N = N;
  g.packed = packed;
  // 256 x 256 tiles (one workgroup per CU, 4 stages of K 32) when there is
  // one per CU; else 128 x 128 tiles, two workgroups per CU with 4 stages of
  // K 32 when there are more tiles than CUs, one per CU with 3 stages of K 64
  // otherwise (the deeper ring covers the load latency that a lone
  // workgroup's 4 wavefronts cannot); all in groups of 4 m-tiles.  Every
  // choice accumulates each output over k in the same order, so the results
  // do not depend on it.
  const bool wide = static_cast<long long>((M + 255) / 256) * ((N + 255) / 256) >= 256;
  const bool crowded = static_cast<long long>((M + 127) / 128) * ((N + 127) / 128) > 256;
  const int bt = wide ? 256 : 128;
  // A narrow column tail (N = 256 n + 16 .. 64, e.g. a 4096-row projection
  // plus its 16 gate rows) would cost a whole 256-wide tile per m-tile, often
  // a second round of workgroups: the whole 256-column tiles run first, and
  // the tail columns follow as a 128-tile launch of their own (the same
  // output rows, column offset and stride N).
  const int tail = wide && N > 256 ? N % 256 : 0;
  if (tail > 0 && tail <= 64) {
    const int n_main = N - tail;
    TileArgs t = g;
    t.N = n_main;
    t.m_tiles = (M + 255) / 256;
    t.n_tiles = n_main / 256;
    t.group_m = 4;
    const long long main_items = static_cast<long long>(t.m_tiles) * t.n_tiles;
    if (main_items >= (1ll << 31) - kNumXcd) return static_cast<int32_t>(hipErrorInvalidValue);
    int32_t st = 0;
#define LLMY_DENSE_T(T_, BK_, NS_, OCC_, ARGS_, ITEMS_)                                           \
  switch (epi) {                                                                                \
    case kDenseBf16: st = launch_tiles<T_, T_, BK_, NS_, kDenseBf16, OCC_>(ARGS_, ITEMS_, s); break; \
    case kDenseF32: st = launch_tiles<T_, T_, BK_, NS_, kDenseF32, OCC_>(ARGS_, ITEMS_, s); break;   \
    case kDenseResid: st = launch_tiles<T_, T_, BK_, NS_, kDenseResid, OCC_>(ARGS_, ITEMS_, s); break; \
    default: st = launch_tiles<T_, T_, BK_, NS_, kDenseGated, OCC_>(ARGS_, ITEMS_, s); break;        \
  }
    LLMY_DENSE_T(256, 32, 4, 1, t, main_items)
    if (st != 0) return st;
#undef LLMY_DENSE_T
    // the tail: rows n_main .. N-1 of w (for the packed order too: 16-row
    // groups are contiguous), output columns n_main .. N-1, through the
    // weight-streaming kernel with the rows split 16 per workgroup (a tile
    // launch would spend a 128-wide tile per 16 columns)
    return dense_narrow_ws(x, w + static_cast<long long>(n_main) * K,
                           static_cast<char*>(out) +
                               static_cast<long long>(n_main) * (epi == kDenseBf16 ? 2 : 4),
                           aux ? aux + n_main : nullptr, M, tail, K, N, epi, packed, s);
  }
  g.m_tiles = (M + bt - 1) / bt;
  g.n_tiles = (N + bt - 1) / bt;
  g.group_m = 4;
  const long long items = static_cast<long long>(g.m_tiles) * g.n_tiles;
  if (items >= (1ll << 31) - kNumXcd) return static_cast<int32_t>(hipErrorInvalidValue);
#define LLMY_DENSE(T_, BK_, NS_, OCC_)                                                          \
  switch (epi) {                                                                               \
    case kDenseBf16: return launch_tiles<T_, T_, BK_, NS_, kDenseBf16, OCC_>(g, items, s); \
    case kDenseF32: return launch_tiles<T_, T_, BK_, NS_, kDenseF32, OCC_>(g, items, s);   \
    case kDenseResid: return launch_tiles<T_, T_, BK_, NS_, kDenseResid, OCC_>(g, items, s); \
    default: return launch_tiles<T_, T_, BK_, NS_, kDenseGated, OCC_>(g, items, s);        \
  }
  if (wide) LLMY_DENSE(256, 32, 4, 1)
  if (crowded) LLMY_DENSE(128, 32, 4, 2)
  LLMY_DENSE(128, 64, 3, 1)
#undef LLMY_DENSE
}

}  // namespace llmy
