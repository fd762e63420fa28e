// Grouped expert GEMMs for MoE prefill on bf16 MFMA (gfx950).
//
// Math (model/layers/moe.py:72-76, expert.py:14-15), per expert e over its
// routes in permuted order p = offsets[e] .. offsets[e+1]-1:
//   act[p, :] = silu(x[t_p] . W_gate[e]^T) * (x[t_p] . W_up[e]^T)   (bf16 out)
//   y[p, :]   = gate[r_p] * (act[p] . W_down[e]^T)                  (fp32 out)
// with r_p = sorted_routes[p] and t_p = r_p / k: the same contract, layouts
// and rounding points as the weight-streaming path of llmy_moe_experts_bf16.
//
// Tiling: a workgroup of 8 wavefronts (2 per SIMD) computes a BM x BN tile
// (BM = 128 routes of one expert; BN = 256 for gate_up, BN = 128 for down).
// The gate_up tile's weight rows are [32 gate | 32 up] per wavefront column,
// so every gate accumulator sits in the same lanes as its up partner and
// SwiGLU is applied in registers.  Wavefront (wm, wn) of the 2 x 4 grid owns
// rows 64 wm .. 64 wm + 63 and columns (BN/4) wn .. as 2 x (BN/128) blocks of
// v_mfma_f32_32x32x16_bf16.
//
// K advances 64 at a time through two LDS stages filled by
// global_load_lds_dwordx4 (global memory straight into LDS, no staging
// registers): while one K tile is multiplied, the next is in flight.  Tile
// rows are 128 bytes with an XOR swizzle of their 16-byte chunks, so each DMA
// instruction reads 8 whole global rows and each MFMA fragment read (inline
// asm ds_read_b128, see lds_frag) is conflict-free.  Per K tile a wavefront
// waits for its own loads (s_waitcnt vmcnt), the workgroup meets at one
// barrier, the next tile is issued, then the tile is multiplied.
//
// Work order: work items (expert, n-tile, m-tile) are numbered expert-major,
// m fastest, and each XCD (block id mod 8) takes a contiguous range of them,
// so the m-tiles that share a weight tile, and the n-tiles that share an
// expert's token rows, run back to back in the same XCD's L2.
//
// The same tiles serve the dense projections of a sequence prefill
// (llmy_linear_bf16 with many rows): MODE 2 is one "expert" owning all M
// rows, BN = 128, an N tail (rows past N re-read row N-1, their columns are
// not stored) and the linear epilogues (bf16 / fp32 store, fp32 residual
// add, gated residual add).
#include "common.hpp"
#include "abi_util.hpp"

namespace llmy {

namespace {

constexpr int kGemmThreads = 512;  // 8 wavefronts: 2 per SIMD
constexpr int kBM = 128;
constexpr int kBK = 64;   // K per pipeline stage (four 16-k MFMA steps)
constexpr int kSteps = kBK / 16;
constexpr int kRowB = kBK * 2;  // bytes of one tile row in a stage (8 chunks of 16)
constexpr int kBlock = 1024;            // one 32 x 16 bf16 MFMA operand block
constexpr int kNumXcd = 8;

struct MoeGemmArgs {
  const uint16_t* x;       // gate_up: token rows [x_rows, K]; down: act [rows_total, K]
  const uint16_t* w;       // expert weights, row-major [E, N_w, K] or packed
  void* out;               // gate_up: act bf16 [rows_total, ldo]; down: y f32 [rows_total, ldo]
  const float* gates;      // down: gate per route id
  const int32_t* offsets;  // [E + 1]
  const int32_t* sorted_routes;
  long long w_expert_stride;  // elements per expert block of w
  long long up_offset;        // gate_up: elements from gate row n to up row n (H * K)
  int K, ldo, E, route_k, rows_total, x_rows;
  int n_tiles;  // output column tiles per expert
  int packed;
  // dense (MODE 2) only
  const float* aux;  // gated residual: out += acc * aux[m * ldo + n]
  int N;             // output columns (the last n-tile may be partial)
  int m_tiles;
};

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

// s_waitcnt immediate (gfx9 encoding) that waits until at most n vector
// memory operations of this wavefront are outstanding (vmcnt bits [3:0] and
// [15:14]; expcnt [6:4] = 7 and lgkmcnt [11:8] = 15 wait for nothing) ...
constexpr int waitcnt_vm(int n) { return 0x0F70 | (n & 15) | ((n >> 4) << 14); }
// ... and also for all of this wavefront's LDS operations (lgkmcnt = 0).
constexpr int waitcnt_vm_lgkm0(int n) { return 0x0070 | (n & 15) | ((n >> 4) << 14); }

// 16-byte LDS read at byte address addr + OFF, as inline asm: the compiler's
// LDS-DMA tracking cannot separate the stage being read from the stages
// being filled and would make every read wait for all loads in flight.  The
// result is valid only after lds_settle().
template <int OFF>
__device__ __forceinline__ u32x4 lds_frag(uint32_t addr) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF) : "memory");
  return v;
}

// Wait for this wavefront's LDS reads; the "+v" operand makes every later use
// of v follow the wait.
__device__ __forceinline__ void lds_settle(u32x4& v) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v) :: "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const lds_void*)p));
}

__device__ __forceinline__ f32x16 mfma32(const u32x4& a, const u32x4& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

}  // namespace

// Dense epilogues (values of the linear entry's epilogue argument).
enum DenseEpi : int { kDenseBf16 = 0, kDenseF32 = 1, kDenseResid = 2, kDenseGated = 3 };

// MODE 0: gate_up + SwiGLU (BN = 256); MODE 1: down + gate scale (BN = 128);
// MODE 2: dense with epilogue EPI (BN = 128).
template <int MODE, int EPI = 0>
__global__ __launch_bounds__(kGemmThreads) void moe_gemm_kernel(MoeGemmArgs a) {
  constexpr int BN = MODE == 0 ? 256 : 128;
  constexpr int CT = BN / 128;       // 32-column MFMA blocks per wavefront (2 x 4 wave grid)
  __shared__ int s_work[3];          // expert, m0, n-tile (or -1: no work)

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;  // rows 64 wm .., columns (BN/4) wn ..

  // ---- which tile.  Dense: work item w = (n-tile, m-tile), m fastest.
  // Grouped: wave 0 scans the experts' m-tile counts.
  if (MODE == 2) {
    if (tid == 0) {
      const int nblk = gridDim.x;
      const int per_xcd = (nblk + kNumXcd - 1) / kNumXcd;
      const int w = (blockIdx.x % kNumXcd) * per_xcd + blockIdx.x / kNumXcd;
      const bool ok = w < a.m_tiles * a.n_tiles;
      s_work[0] = ok ? 0 : -1;
      s_work[1] = ok ? (w % a.m_tiles) * kBM : 0;
      s_work[2] = ok ? w / a.m_tiles : 0;
    }
  } else if (wave == 0) {
    const int nblk = gridDim.x;
    const int per_xcd = (nblk + kNumXcd - 1) / kNumXcd;
    const int w = (blockIdx.x % kNumXcd) * per_xcd + blockIdx.x / kNumXcd;
    int found = -1, m0 = 0, nt = 0;
    int base = 0;  // m-tiles of the experts before this chunk of 64
    for (int e0 = 0; e0 < a.E; e0 += kWave) {
      const int e = e0 + lane;
      int tiles = 0;
      if (e < a.E) {
        const int lo = min(max(a.offsets[e], 0), a.rows_total);
        const int hi = min(max(a.offsets[e + 1], lo), a.rows_total);
        tiles = (hi - lo + kBM - 1) / kBM;
      }
      int inc = tiles;  // inclusive scan over the wave
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) {
        const int o = __shfl_up(inc, off, kWave);
        if (lane >= off) inc += o;
      }
      const int first = (base + inc - tiles) * a.n_tiles;  // first work item of expert e
      const int last = (base + inc) * a.n_tiles;
      const unsigned long long hit = __ballot(e < a.E && w >= first && w < last);
      if (hit) {
        const int src = __ffsll(static_cast<long long>(hit)) - 1;
        const int f = __shfl(first, src, kWave);
        const int t = __shfl(tiles, src, kWave);
        found = e0 + src;
        const int local = w - f;
        nt = local / t;
        m0 = (local - nt * t) * kBM;
        break;
      }
      base += __shfl(inc, kWave - 1, kWave);
    }
    if (lane == 0) {
      s_work[0] = found;
      s_work[1] = m0;
      s_work[2] = nt;
    }
  }
  __syncthreads();
  const int e = s_work[0];
  if (e < 0) return;
  const int m0 = s_work[1], ntile = s_work[2];
  const int row_lo = MODE == 2 ? 0 : min(max(a.offsets[e], 0), a.rows_total);
  const int rows_e =
      MODE == 2 ? a.rows_total : min(max(a.offsets[e + 1], row_lo), a.rows_total) - row_lo;
  const int K = a.K;
  const int nk = K / kBK;

  // ---- global sources.  A stage holds the A tile (128 rows) then the B tile
  // (BN rows), each row 128 bytes = 8 chunks of 8 k, chunk c of row r stored
  // in slot c ^ ((r >> 1) & 7).  A ds_read_b128 is served 16 lanes at a time
  // from 256 bytes of banks; the 16 lanes of a fragment read take 16
  // consecutive rows at one chunk index, which this swizzle spreads over all
  // 16 bank groups (two rows per 256 bytes, 8 slots each).  Each
  // global_load_lds instruction fills 8 consecutive tile rows, lane l taking
  // row 8q + l/8 and slot l%8, i.e. a whole 128-byte global row per 8 lanes.
  constexpr int A_INS = kBM / 8 / 8;  // per wave per stage
  constexpr int B_INS = BN / 8 / 8;
  constexpr int LOADS = A_INS + B_INS;
  constexpr int A_BYTES = kBM * kRowB;
  constexpr int STAGE_BYTES = (kBM + BN) * kRowB;
  const int dma_row = lane >> 3;  // row within the instruction's 8
  // global chunk fetched by this lane for an instruction starting at tile row 8q
  auto dma_chunk = [&](int q) { return (lane & 7) ^ (((8 * q + dma_row) >> 1) & 7); };
  long long a_src[A_INS];
#pragma unroll
  for (int q = 0; q < A_INS; ++q) {
    const int r = 8 * (A_INS * wave + q) + dma_row;  // tile row
    const int m = min(m0 + r, rows_e - 1);            // past the expert: repeat its last row
    const int p = row_lo + m;
    long long src;
    if (MODE == 0) {
      src = min(max(a.sorted_routes[p], 0), a.rows_total - 1) / a.route_k;
      src = min(src, static_cast<long long>(a.x_rows - 1));
    } else {
      src = p;
    }
    a_src[q] = src * K + 8 * dma_chunk(A_INS * wave + q);
  }
  const uint16_t* wexp = a.w + static_cast<long long>(e) * a.w_expert_stride;
  const bool packed = a.packed != 0;
  long long b_src[B_INS];
#pragma unroll
  for (int q = 0; q < B_INS; ++q) {
    const int r = 8 * (B_INS * wave + q) + dma_row;  // tile row
    long long off = 0;
    int n;
    if (MODE == 0) {
      // [gate n0..+31 | up n0..+31 | gate n0+32..+63 | up ...], n0 = 128 * ntile:
      // wavefront column quarter wn gets 32 gate rows and their 32 up rows
      n = 128 * ntile + 32 * (r >> 6) + (r & 31);
      if ((r >> 5) & 1) off = a.up_offset;
    } else if (MODE == 1) {
      n = BN * ntile + r;
    } else {
      n = min(BN * ntile + r, a.N - 1);  // N tail: repeat the last row
    }
    const int ch = dma_chunk(B_INS * wave + q);
    b_src[q] = off + (packed ? packed_at(n, 8 * ch, K) : static_cast<long long>(n) * K + 8 * ch);
  }

  // Two named LDS stages: K tile kt+1 is in flight while tile kt is
  // multiplied (named objects let the compiler's LDS-DMA tracking keep them
  // apart).
  __shared__ __align__(1024) unsigned char st0[STAGE_BYTES];
  __shared__ __align__(1024) unsigned char st1[STAGE_BYTES];

  // Element offset of K tile kt within a B row: row-major 64 kt; packed:
  // 256-k blocks are 4096 elements apart, 64-k tiles 1024.
  auto issue = [&](int kt, unsigned char* st) {
    const long long ka = static_cast<long long>(kt) * kBK;
    const long long kb = packed ? static_cast<long long>(kt >> 2) * 4096 + (kt & 3) * 1024 : ka;
#pragma unroll
    for (int q = 0; q < A_INS; ++q)
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(a.x + a_src[q] + ka),
                                       as_lds(st + (8 * (A_INS * wave + q)) * kRowB), 16, 0, 0);
#pragma unroll
    for (int q = 0; q < B_INS; ++q)
      __builtin_amdgcn_global_load_lds(static_cast<const void*>(wexp + b_src[q] + kb),
                                       as_lds(st + A_BYTES + (8 * (B_INS * wave + q)) * kRowB), 16,
                                       0, 0);
  };

  f32x16 acc[2][CT];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int c = 0; c < CT; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][c][r] = 0.f;

  // Fragment addresses: lane l reads tile row (32-row block base) + l%32,
  // chunk 2s + l/32 of k step s, stored in slot (2s + l/32) ^ ((l%32 >> 1) & 7).
  uint32_t frag_off[kSteps];
#pragma unroll
  for (int s = 0; s < kSteps; ++s)
    frag_off[s] = (lane & 31) * kRowB + (((2 * s + (lane >> 5)) ^ ((lane >> 1) & 7)) << 4);
  const uint32_t fa_base = (64 * wm) * kRowB;
  const uint32_t fb_base = A_BYTES + ((BN / 4) * wn) * kRowB;

  // One K tile: wait for this wave's loads of tile kt and its fragment reads
  // of the previous tile, meet the workgroup at the barrier (then all of tile
  // kt is in LDS and the other buffer is free), fetch tile kt+1 into it,
  // multiply tile kt.
  auto step = [&](int kt, const unsigned char* cur, unsigned char* refill) {
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (kt + 1 < nk) issue(kt + 1, refill);
    const uint32_t ca = lds_addr(cur) + fa_base, cb = lds_addr(cur) + fb_base;
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      u32x4 fa[2], fb[CT];
      const uint32_t xa = ca + frag_off[s], xb = cb + frag_off[s];
      fa[0] = lds_frag<0>(xa);
      fa[1] = lds_frag<32 * kRowB>(xa);
      fb[0] = lds_frag<0>(xb);
      if (CT == 2) fb[CT - 1] = lds_frag<32 * kRowB>(xb);
#pragma unroll
      for (int i = 0; i < 2; ++i) lds_settle(fa[i]);
#pragma unroll
      for (int c = 0; c < CT; ++c) lds_settle(fb[c]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int c = 0; c < CT; ++c) acc[i][c] = mfma32(fa[i], fb[c], acc[i][c]);
    }
  };

  // nk is even (K % 256 == 0, checked by the host)
  issue(0, st0);
  for (int kt = 0; kt < nk; kt += 2) {
    step(kt, st0, st1);
    step(kt + 1, st1, st0);
  }

  // ---- epilogue: D layout of 32x32 blocks: lane l, reg r -> row (r&3) + 8(r>>2) + 4(l>>5), col l&31
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = 64 * wm + 32 * i + (r & 3) + 8 * (r >> 2) + 4 * (lane >> 5);
      const int m = m0 + row;
      if (m >= rows_e) continue;
      const long long p = row_lo + m;
      if (MODE == 0) {
        uint16_t* act = static_cast<uint16_t*>(a.out) + p * a.ldo;
        const float g = acc[i][0][r], u = acc[i][1][r];
        act[128 * ntile + 32 * wn + (lane & 31)] = f2bf(siluf_(g) * u);
      } else if (MODE == 2) {
        const int n = BN * ntile + 32 * wn + (lane & 31);
        if (n >= a.N) continue;
        const long long o = p * a.ldo + n;
        const float v = acc[i][0][r];
        if (EPI == kDenseBf16) {
          static_cast<uint16_t*>(a.out)[o] = f2bf(v);
        } else if (EPI == kDenseF32) {
          static_cast<float*>(a.out)[o] = v;
        } else if (EPI == kDenseResid) {
          static_cast<float*>(a.out)[o] += v;
        } else {
          static_cast<float*>(a.out)[o] += v * a.aux[o];
        }
      } else {
        const int route = min(max(a.sorted_routes[p], 0), a.rows_total - 1);
        const float gs = a.gates[route];
        float* y = static_cast<float*>(a.out) + p * a.ldo;
#pragma unroll
        for (int c = 0; c < CT; ++c) y[BN * ntile + 32 * wn + 32 * c + (lane & 31)] = acc[i][c][r] * gs;
      }
    }
  }
}

// Launch both GEMMs; returns the launch status.  Shapes were validated by the
// caller: D % 256 == 0, H % 256 == 0, rows_total = T * k >= 1.
int32_t moe_gemm_prefill(const uint16_t* x, const int32_t* offsets, const int32_t* sorted_routes,
                         const float* gates, const uint16_t* w_gate_up, const uint16_t* w_down,
                         uint16_t* act, float* y, int T, int D, int H, int E, int k, bool packed,
                         hipStream_t s) {
  const int rows_total = T * k;
  const int max_mtiles = (rows_total + kBM - 1) / kBM + E;  // sum over experts of ceil(n_e/BM)
  MoeGemmArgs g{};
  g.x = x;
  g.w = w_gate_up;
  g.out = act;
  g.offsets = offsets;
  g.sorted_routes = sorted_routes;
  g.w_expert_stride = 2ll * H * D;
  g.up_offset = static_cast<long long>(H) * D;
  g.K = D;
  g.ldo = H;
  g.E = E;
  g.route_k = k;
  g.rows_total = rows_total;
  g.x_rows = T;
  g.n_tiles = H / 128;
  g.packed = packed;
  long long blocks = static_cast<long long>(max_mtiles) * g.n_tiles;
  blocks = (blocks + kNumXcd - 1) / kNumXcd * kNumXcd;
  hipLaunchKernelGGL(moe_gemm_kernel<0>, dim3(static_cast<unsigned>(blocks)), dim3(kGemmThreads),
                     0, s, g);
  const int32_t st = launch_status();
  if (st != 0) return st;
  MoeGemmArgs d = g;
  d.x = act;
  d.w = w_down;
  d.out = y;
  d.gates = gates;
  d.w_expert_stride = static_cast<long long>(D) * H;
  d.up_offset = 0;
  d.K = H;
  d.ldo = D;
  d.x_rows = rows_total;
  d.n_tiles = D / 128;
  blocks = static_cast<long long>(max_mtiles) * d.n_tiles;
  blocks = (blocks + kNumXcd - 1) / kNumXcd * kNumXcd;
  hipLaunchKernelGGL(moe_gemm_kernel<1>, dim3(static_cast<unsigned>(blocks)), dim3(kGemmThreads),
                     0, s, d);
  return launch_status();
}

// Dense out[M, N] (epilogue epi) = x[M, K] . w[N, K]^T on the same tiles.
// Validated by the caller: M >= 1, N >= 1, K % 256 == 0, 16-byte aligned
// x and w, aux given for the gated epilogue.
int32_t dense_gemm_mfma(const uint16_t* x, const uint16_t* w, void* out, const float* aux,
                        int M, int N, int K, int epi, bool packed, hipStream_t s) {
  MoeGemmArgs g{};
  g.x = x;
  g.w = w;
  g.out = out;
  g.aux = aux;
  g.K = K;
  g.ldo = N;
  g.E = 1;
  g.route_k = 1;
  g.rows_total = M;
  g.x_rows = M;
  g.N = N;
  g.n_tiles = (N + 127) / 128;
  g.m_tiles = (M + kBM - 1) / kBM;
  g.packed = packed;
  long long blocks = static_cast<long long>(g.m_tiles) * g.n_tiles;
  if (blocks >= (1ll << 31) - kNumXcd) return static_cast<int32_t>(hipErrorInvalidValue);
  blocks = (blocks + kNumXcd - 1) / kNumXcd * kNumXcd;
  const dim3 grid(static_cast<unsigned>(blocks)), block(kGemmThreads);
  switch (epi) {
    case kDenseBf16: hipLaunchKernelGGL((moe_gemm_kernel<2, kDenseBf16>), grid, block, 0, s, g); break;
    case kDenseF32: hipLaunchKernelGGL((moe_gemm_kernel<2, kDenseF32>), grid, block, 0, s, g); break;
    case kDenseResid: hipLaunchKernelGGL((moe_gemm_kernel<2, kDenseResid>), grid, block, 0, s, g); break;
    default: hipLaunchKernelGGL((moe_gemm_kernel<2, kDenseGated>), grid, block, 0, s, g); break;
  }
  return launch_status();
}

}  // namespace llmy
