// Grouped expert GEMMs of MoE prefill on gfx950.
//
// Math (model/layers/moe.py:72-76, expert.py:14-15), per expert e over its
// routes in permuted order p = offsets[e] .. offsets[e+1]-1:
//   gate_up: act[p, :] = silu(x[t_p] . W_gate[e]^T) * (x[t_p] . W_up[e]^T)  (bf16 out)
//   down:    y[p, :]   = gate[r_p] * (act[p] . W_down[e]^T)                 (fp32 out)
// with r_p = sorted_routes[p], t_p = r_p / k: the contract of
// llmy_moe_experts_bf16 (the rounding points of the weight-streaming path).
//
// Work item = (expert, m-chunk, n-slab).  An expert's n_e rows are split into
// ceil(n_e / 256) chunks of near-equal size (<= 256 rows), and its weight rows
// into slabs of 256 (gate_up: 128 gate + the 128 matching up rows, i.e. 128
// output columns; down: 256 output columns), so a weight byte is read from
// HBM once per m-chunk and a chunk's token rows once per slab.
//
// Persistent workgroups, one per CU, each of 8 wavefronts (two per SIMD, so
// one wavefront's barrier and waits are covered by the other's MFMAs).  A
// workgroup takes every gridDim/8-th item of its XCD's contiguous range
// (items are numbered expert-major, then slab, then chunk, so the chunks
// sharing a weight slab and the slabs sharing an expert's rows run together
// in one XCD's L2), works out up to four at a time, and runs their K steps as
// one continuous stream: the DMA pipeline runs ahead across item boundaries
// and each item's epilogue overlaps the next item's first loads.
//
// Tile: the chunk's 256 rows x the slab's 256 weight rows.  Wavefront
// (wm, wn) of the 2 x 4 grid owns the 32-row token blocks wm, wm + 2, wm + 4,
// wm + 6 (interleaved, so a short chunk keeps both rows of wavefronts equally
// busy) against 64 weight rows (gate_up: 32 gate + their 32 up rows), as
// 4 x 2 v_mfma_f32_32x32x16_bf16 accumulators.  The weight fragment is the
// MFMA's first operand, so each lane ends with groups of four consecutive
// output columns of one row, and a gate accumulator sits in the same lanes as
// its up partner (SwiGLU in registers).
//
// Per 32-wide K step a stage holds the chunk's 256 token rows x 64 bytes
// (16-byte chunks XOR-swizzled by row, so the DMA writes and the 16-lane
// fragment reads are conflict-free) and the slab's 16 weight fragments of
// 16 rows x 32 k (1 KiB each, in fragment order: lane l holds row l % 16 at
// k 8 (l / 16) .. +7, the packed operand order of llmy_pack_weights_bf16).
// Both arrive by global_load_lds_dwordx4 (global memory straight into LDS:
// no register holds data in flight), P = 4 steps ahead, through a ring of
// P + 1 stages (160 KiB).  Each wavefront issues 4 of a step's 32 DMA
// instructions, unconditionally (past the stream's end they re-read its last
// step into a stage no step reads), so the wait counts hold.  Token blocks
// past a chunk's last row issue no MFMA; DMA instructions whose 16 rows are
// all past it read one 16-byte line.
//
// Step schedule (g = stream step; fragments of the two 16-wide k halves in
// two register sets):
//   reads of half 1; MFMAs of half 0 (read during the previous step); wait
//   for half 1 and for step g+1's DMA; barrier (stage g is free, stage g+1
//   complete); reads of half 0 of step g+1; the first MFMA of half 1, then
//   the DMA of step g+1+P into stage g (its issue overlaps that MFMA), then
//   the other MFMAs of half 1, which cover the reads; wait for them (no
//   fragment read is in flight across a loop edge or an epilogue); at an
//   item's last step, its epilogue.
//
// Set-up: the first 64 experts' route ranges are loaded once per workgroup
// and held one per lane, so finding an item needs no memory access, and the
// route loads of a batch's items are issued together.
#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "abi_util.hpp"

namespace llmy {

struct GroupedArgs {
  const uint16_t* x;        // token rows: gate_up x [x_rows, K]; down act [rows_total, K]
  const uint16_t* w;        // weights [E, Nw, K], row-major or packed per expert
  void* out;                // gate_up: act bf16 [rows_total, ldo]; down: y fp32 [rows_total, ldo]
  const float* gates;       // down: gate per route id
  const int32_t* offsets;   // [E + 1]
  const int32_t* sorted_routes;
  long long w_expert_stride;  // elements per expert block of w
  int up_rows;                // gate_up: first up row (H)
  int K, ldo, E, route_k, rows_total, x_rows;
  int n_slabs;                // weight slabs per expert
};

namespace {

constexpr int kGThreads = 512;           // 8 wavefronts, two per SIMD
constexpr int kGChunk = 256;             // rows per m-chunk at most
constexpr int kGXcd = 8;
constexpr int kGStage = kGChunk * 64;    // token rows of a stage: 256 rows x 32 bf16
constexpr int kGBatch = 4;               // items worked out at a time

typedef __attribute__((address_space(3))) void glds_void;

__device__ __forceinline__ void g_dma16(const void* src, void* dst) {
  __builtin_amdgcn_global_load_lds(src, (glds_void*)dst, 16, 0, 0);
}

__device__ __forceinline__ uint32_t g_lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const glds_void*)p));
}

// 16-byte LDS read at addr + OFF (inline asm: the compiler would otherwise make
// each read wait for every LDS DMA in flight).  Valid after a g_settle.
template <int OFF>
__device__ __forceinline__ u32x4 g_frag(uint32_t addr) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF) : "memory");
  return v;
}

// Wait until at most N LDS operations of this wavefront are outstanding and
// tie the 6 registers those reads filled to the wait.
template <int N>
__device__ __forceinline__ void g_settle(u32x4* f) {
  asm volatile("s_waitcnt lgkmcnt(%6)"
               : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5])
               : "i"(N)
               : "memory");
}

// s_waitcnt immediate (gfx9 encoding): vmcnt <= n (bits [3:0] and [15:14]);
// expcnt (bits [6:4] = 7) and lgkmcnt (bits [11:8] = 15) left open.
constexpr int g_vmcnt(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0F70; }

__device__ __forceinline__ f32x16 mfma32(const u32x4& w, const u32x4& t, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, w),
                                                 __builtin_bit_cast(bf16x8, t), c, 0, 0, 0);
}

// Rows of chunk c when n rows are split into nc near-equal chunks.
__device__ __forceinline__ void chunk_rows(int n, int nc, int c, int& start, int& rows) {
  const int base = n / nc, rem = n % nc;
  start = c * base + min(c, rem);
  rows = base + (c < rem ? 1 : 0);
}

// Expert e's row range [lo, lo + n), clamped to the routes.
__device__ __forceinline__ void expert_rows(const GroupedArgs& a, int e, int& lo, int& n) {
  lo = min(max(a.offsets[e], 0), a.rows_total);
  n = min(max(a.offsets[e + 1], lo), a.rows_total) - lo;
}

// Row range of expert e0 + lane (e0 a multiple of 64); empty past E.  The
// kernel loads the first 64 experts' ranges once (lo0, n0) and reuses them.
__device__ __forceinline__ void lane_rows(const GroupedArgs& a, int e0, int lo0, int n0, int& lo,
                                          int& n) {
  if (e0 == 0) {
    lo = lo0;
    n = n0;
    return;
  }
  const int e = e0 + (threadIdx.x & 63);
  lo = n = 0;
  if (e < a.E) expert_rows(a, e, lo, n);
}

// Number of work items (a wavefront-wide sum; every lane gets it).
__device__ int count_items(const GroupedArgs& a, int lo0, int n0) {
  int total = 0;
  for (int e0 = 0; e0 < a.E; e0 += kWave) {
    int lo, n;
    lane_rows(a, e0, lo0, n0, lo, n);
    int items = (n + kGChunk - 1) / kGChunk * a.n_slabs;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) items += __shfl_xor(items, off, kWave);
    total += items;
  }
  return total;
}

// Work item `it` (< the item count): its expert, first row, row count and slab.
// Wavefront-wide; every lane gets the same values.
__device__ void find_item(const GroupedArgs& a, int it, int lo0, int n0, int& e, int& row0,
                          int& rows, int& slab) {
  const int lane = threadIdx.x & 63;
  e = -1;
  row0 = rows = slab = 0;
  int base = 0;
  for (int e0 = 0; e0 < a.E; e0 += kWave) {
    const int ee = e0 + lane;
    int lo, n;
    lane_rows(a, e0, lo0, n0, lo, n);
    const int nc = (n + kGChunk - 1) / kGChunk;
    const int items = nc * a.n_slabs;
    int inc = items;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const int o = __shfl_up(inc, off, kWave);
      if (lane >= off) inc += o;
    }
    const int first = base + inc - items;
    const unsigned long long hit = __ballot(ee < a.E && it >= first && it < first + items);
    if (hit) {
      const int src = __ffsll(static_cast<long long>(hit)) - 1;
      int r0 = 0, rr = 0, sl = 0;
      if (lane == src) {
        const int local = it - first;
        sl = local / nc;
        int start;
        chunk_rows(n, nc, local % nc, start, rr);
        r0 = lo + start;
      }
      e = e0 + src;
      row0 = __shfl(r0, src, kWave);
      rows = __shfl(rr, src, kWave);
      slab = __shfl(sl, src, kWave);
      return;
    }
    base += __shfl(inc, kWave - 1, kWave);
  }
}

template <typename T>
__device__ __forceinline__ T sel4(int i, T v0, T v1, T v2, T v3) {
  return i == 0 ? v0 : i == 1 ? v1 : i == 2 ? v2 : v3;
}

}  // namespace

template <int MODE, bool PACKED>
__global__ __launch_bounds__(kGThreads, 1) void grouped_gemm_kernel(GroupedArgs a) {
  constexpr int P = 4;                // prefetch distance in K steps
  constexpr int NS = P + 1;           // stages
  constexpr int L = 4;                // DMA instructions per wavefront per step
  constexpr int STAGE = 2 * kGStage;  // token rows, then 16 weight fragments
  constexpr int B_STEP = PACKED ? 1024 : 64;  // bytes between K steps of one fragment
  static_assert(P * L <= 63, "vmcnt range");
  __shared__ __align__(1024) unsigned char smem[NS * STAGE];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  // The waves of a workgroup go to the SIMDs in turn (wave w to SIMD w % 4),
  // so wm = w / 4 pairs a wm = 0 and a wm = 1 wave on every SIMD: each SIMD
  // then runs the same number of active token blocks when a chunk's block
  // count is odd.
  const int wm = wave >> 2, wn = wave & 3;
  const int lr = lane & 31, lh = lane >> 5;
  const int K = a.K;
  const int nk = K >> 5;  // 32-wide K steps
  const uint32_t smem_base = g_lds_addr(smem);

  // this workgroup's items: XCD x = blockIdx % 8 owns items
  // [x * per_xcd, (x + 1) * per_xcd); its workgroups take them in turn
  int lo0 = 0, n0 = 0;  // expert `lane`'s routes (experts 0 .. 63)
  if (lane < a.E) expert_rows(a, lane, lo0, n0);
  const int n_items = __builtin_amdgcn_readfirstlane(count_items(a, lo0, n0));
  const int per_xcd = (n_items + kGXcd - 1) / kGXcd;
  const int grid_xcd = gridDim.x / kGXcd;  // workgroups per XCD (the host launches a multiple of 8)
  const int xcd = blockIdx.x % kGXcd, slot = blockIdx.x / kGXcd;
  const int x_end = min(n_items, (xcd + 1) * per_xcd);

  // Fragment read addresses (v_mfma_f32_32x32x16_bf16 operands: lane l holds
  // row l % 32 at k 8 (l / 32) .. +7 of the 16-wide k half h).  Token block i
  // of the wavefront (stage rows 32 (2 i + wm) + l % 32) at 4 KiB i, chunk
  // 2 h + l / 32 in its swizzled slot; weight block jb (stage fragments
  // 4 wn + 2 jb + (l % 32) / 16) at 2 KiB jb, chunk 2 h + l / 32.
  const uint32_t a_frag0 = smem_base + wm * 2048 + lr * 64 + ((lh ^ ((lr >> 2) & 3)) << 4);
  const uint32_t a_frag1 = smem_base + wm * 2048 + lr * 64 + (((2 + lh) ^ ((lr >> 2) & 3)) << 4);
  const uint32_t b_frag = smem_base + kGStage + (4 * wn + (lr >> 4)) * 1024 + lh * 256 +
                          (lane & 15) * 16;
  const char* a_base = reinterpret_cast<const char*>(a.x);

  for (int first = xcd * per_xcd + slot; first < x_end; first += kGBatch * grid_xcd) {
    // ---- up to four items: descriptors and this wavefront's DMA sources
    int nb = 0;
    int d_row0[kGBatch], d_rows[kGBatch], d_slab[kGBatch], d_e[kGBatch];
    uint32_t d_aoff[kGBatch][2], d_boff[kGBatch][2];
    float d_gate[kGBatch][4];
#pragma unroll
    for (int b = 0; b < kGBatch; ++b) {
      const int it = first + b * grid_xcd;
      int e = -1, row0 = 0, rows = 1, slab = 0;
      if (it < x_end) find_item(a, it, lo0, n0, e, row0, rows, slab);
      if (e >= 0) nb = b + 1;
      else { e = 0; row0 = 0; rows = 1; slab = 0; }  // unused slot: any in-bounds item
      d_e[b] = __builtin_amdgcn_readfirstlane(e);
      d_row0[b] = __builtin_amdgcn_readfirstlane(row0);
      d_rows[b] = __builtin_amdgcn_readfirstlane(rows);
      d_slab[b] = __builtin_amdgcn_readfirstlane(slab);
    }
    // The items' route loads are issued together, without branches (rows
    // clamped into the item), so their latencies overlap.
#pragma unroll
    for (int b = 0; b < kGBatch; ++b) {
      // token rows: instruction q fills stage rows 16 (2 w + q) .. +15; lane l
      // writes bytes 16 l of that 1 KiB (row l / 4, slot l % 4), holding the
      // row's chunk (l % 4) ^ (l / 16); groups past the chunk read row 0
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int g = 2 * wave + q;
        const bool live = 16 * g < d_rows[b];
        const int r = 16 * g + (lane >> 2);
        const int p = d_row0[b] + min(r, d_rows[b] - 1);
        long long src = p;
        if (MODE == 0) {
          src = min(max(a.sorted_routes[p], 0), a.rows_total - 1) / a.route_k;
          src = min(src, static_cast<long long>(a.x_rows - 1));
        }
        const int ch = (lane & 3) ^ (lane >> 4);
        d_aoff[b][q] = live ? static_cast<uint32_t>((src * K + 8 * ch) * 2) : 0u;
      }
      // weight fragments: stage fragment f = 2 w + q holds rows n0 .. n0 + 15
      // of the slab (f = 4 c + j for wavefront column c): gate_up j < 2 gate
      // rows 128 s + 32 c + 16 j, j >= 2 the up rows H + 128 s + 32 c +
      // 16 (j - 2); down rows 256 s + 64 c + 16 j
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int f = 2 * wave + q, c = f >> 2, j = f & 3;
        int nr;
        if (MODE == 0) nr = (j >= 2 ? a.up_rows : 0) + 128 * d_slab[b] + 32 * c + 16 * (j & 1);
        else nr = 256 * d_slab[b] + 64 * c + 16 * j;
        if (PACKED)
          d_boff[b][q] =
              static_cast<uint32_t>((static_cast<long long>(nr >> 4) * nk) * 1024 + lane * 16);
        else
          d_boff[b][q] = static_cast<uint32_t>(
              ((static_cast<long long>(nr + (lane & 15)) * K) + 8 * (lane >> 4)) * 2);
      }
      // down: the gate of each of this lane's four output rows (0 past the chunk)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        d_gate[b][i] = 0.f;
        if (MODE == 1) {
          const int m = 32 * (2 * i + wm) + lr;
          const int route =
              min(max(a.sorted_routes[d_row0[b] + min(m, d_rows[b] - 1)], 0), a.rows_total - 1);
          const float gv = a.gates[route];
          d_gate[b][i] = m < d_rows[b] ? gv : 0.f;
        }
      }
    }
    nb = __builtin_amdgcn_readfirstlane(nb);

    // ---- the DMA stream: next step to issue is K step dk of item di; past
    // the last item's last step it re-issues that step
    int di = 0, dk = 0;
    uint32_t dma_a0 = d_aoff[0][0], dma_a1 = d_aoff[0][1];
    uint32_t dma_b0 = d_boff[0][0], dma_b1 = d_boff[0][1];
    const char* dma_w = reinterpret_cast<const char*>(a.w + static_cast<long long>(d_e[0]) *
                                                               a.w_expert_stride);
    // DMA of the stream's next step into the stage at byte offset OFF, then advance
#define G_ISSUE_NEXT(OFF)                                                                   \
  do {                                                                                      \
    unsigned char* st_ = smem + (OFF) + (2 * wave) * 1024;                                  \
    const char* ab_ = a_base + 64 * dk;                                                     \
    const char* bb_ = dma_w + B_STEP * dk;                                                  \
    g_dma16(ab_ + dma_a0, st_);                                                             \
    g_dma16(ab_ + dma_a1, st_ + 1024);                                                      \
    g_dma16(bb_ + dma_b0, st_ + kGStage);                                                   \
    g_dma16(bb_ + dma_b1, st_ + kGStage + 1024);                                            \
    if (++dk == nk) {                                                                       \
      if (di + 1 < nb) {                                                                    \
        ++di;                                                                               \
        dk = 0;                                                                             \
        dma_a0 = sel4(di, d_aoff[0][0], d_aoff[1][0], d_aoff[2][0], d_aoff[3][0]);          \
        dma_a1 = sel4(di, d_aoff[0][1], d_aoff[1][1], d_aoff[2][1], d_aoff[3][1]);          \
        dma_b0 = sel4(di, d_boff[0][0], d_boff[1][0], d_boff[2][0], d_boff[3][0]);          \
        dma_b1 = sel4(di, d_boff[0][1], d_boff[1][1], d_boff[2][1], d_boff[3][1]);          \
        dma_w = reinterpret_cast<const char*>(                                              \
            a.w + static_cast<long long>(sel4(di, d_e[0], d_e[1], d_e[2], d_e[3])) *        \
                      a.w_expert_stride);                                                   \
      } else {                                                                              \
        dk = nk - 1;                                                                        \
      }                                                                                     \
    }                                                                                       \
  } while (0)
    // fragment reads of k half H of the step in the stage at byte offset OFF:
    // F[i] token block i, F[4 + jb] weight block jb
#define G_READ(F, OFF, H)                                              \
  do {                                                                 \
    const uint32_t o_ = (OFF);                                         \
    const uint32_t xa_ = ((H) ? a_frag1 : a_frag0) + o_;               \
    F[0] = g_frag<0>(xa_);                                             \
    F[1] = g_frag<4096>(xa_);                                          \
    F[2] = g_frag<8192>(xa_);                                          \
    F[3] = g_frag<12288>(xa_);                                         \
    F[4] = g_frag<512 * (H)>(b_frag + o_);                             \
    F[5] = g_frag<2048 + 512 * (H)>(b_frag + o_);                      \
  } while (0)
#define G_FENCE() __builtin_amdgcn_sched_barrier(0)

    f32x16 acc[4][2];

    // prologue: steps 0 .. P in flight (stages 0 .. P), step 0 complete, its
    // half 0 requested
#pragma unroll
    for (int s = 0; s <= P; ++s) G_ISSUE_NEXT(s * STAGE);
    __builtin_amdgcn_s_waitcnt(g_vmcnt(P * L));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    u32x4 h0[6], h1[6];
    uint32_t off = 0;  // stage of the current step (stream step g is in stage g % NS)
    G_READ(h0, off, 0);
    g_settle<0>(h0);

    // K steps of one item with NA active token blocks in this wavefront.
    // Stream step g+1+P lands in the stage of step g (NS = P + 1), which the
    // barrier has just freed.
    auto k_loop = [&](auto na_c) {
      constexpr int NA = decltype(na_c)::value;
      for (int kk = 0; kk < nk; ++kk) {
        G_FENCE();
        G_READ(h1, off, 1);
        G_FENCE();
#pragma unroll
        for (int i = 0; i < NA; ++i) {
          acc[i][0] = mfma32(h0[4], h0[i], acc[i][0]);
          acc[i][1] = mfma32(h0[5], h0[i], acc[i][1]);
        }
        G_FENCE();
        g_settle<0>(h1);
        // the next step's DMA landed (the DMA of the P - 1 after it stays in flight)
        __builtin_amdgcn_s_waitcnt(g_vmcnt((P - 1) * L));
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        // the next step's half-0 reads, then the DMA of step g+1+P into the
        // freed stage, issued behind the first MFMA so its issue overlaps it
        const uint32_t freed = off;
        off = off + STAGE == NS * STAGE ? 0 : off + STAGE;
        G_READ(h0, off, 0);
        G_FENCE();
        if (NA > 0) acc[0][0] = mfma32(h1[4], h1[0], acc[0][0]);
        G_FENCE();
        G_ISSUE_NEXT(freed);
        G_FENCE();
        if (NA > 0) acc[0][1] = mfma32(h1[5], h1[0], acc[0][1]);
#pragma unroll
        for (int i = 1; i < NA; ++i) {
          acc[i][0] = mfma32(h1[4], h1[i], acc[i][0]);
          acc[i][1] = mfma32(h1[5], h1[i], acc[i][1]);
        }
        G_FENCE();
        // The next step's half-0 reads land before the loop edge (and before
        // an epilogue): the compiler knows nothing of the asm reads in flight
        // and may move a register that one of them is still to fill.
        g_settle<0>(h0);
      }
    };

    for (int bi = 0; bi < nb; ++bi) {
      const int rows = sel4(bi, d_rows[0], d_rows[1], d_rows[2], d_rows[3]);
      const int row0 = sel4(bi, d_row0[0], d_row0[1], d_row0[2], d_row0[3]);
      const int slab = sel4(bi, d_slab[0], d_slab[1], d_slab[2], d_slab[3]);
      // active token blocks of this wavefront: i = 0 .. na-1 (block 2 i + wm < nblk)
      const int nblk = (rows + 31) >> 5;
      const int na = min(4, max(0, (nblk - wm + 1) >> 1));
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
      switch (na) {
        case 4: k_loop(std::integral_constant<int, 4>{}); break;
        case 3: k_loop(std::integral_constant<int, 3>{}); break;
        case 2: k_loop(std::integral_constant<int, 2>{}); break;
        case 1: k_loop(std::integral_constant<int, 1>{}); break;
        default: k_loop(std::integral_constant<int, 0>{}); break;
      }
      // ---- epilogue of item bi: acc[i][jb] lane l holds chunk row
      // 32 (2 i + wm) + l % 32 and, in registers 4 g4 .. 4 g4 + 3, weight
      // rows 32 jb + 8 g4 + 4 (l / 32) .. +3 of the wavefront column
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = 32 * (2 * i + wm) + lr;
        if (i >= na || m >= rows) continue;
        const long long p = row0 + m;
        if (MODE == 0) {
          uint16_t* act = static_cast<uint16_t*>(a.out) + p * a.ldo;
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            const int col = 128 * slab + 32 * wn + 8 * g4 + 4 * lh;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = silu_fast(acc[i][0][4 * g4 + r]) * acc[i][1][4 * g4 + r];
            *reinterpret_cast<uint2*>(act + col) =
                make_uint2(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]));
          }
        } else {
          const float gs = sel4(bi, d_gate[0][i], d_gate[1][i], d_gate[2][i], d_gate[3][i]);
          float* yrow = static_cast<float*>(a.out) + p * a.ldo;
#pragma unroll
          for (int jb = 0; jb < 2; ++jb)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
              const int col = 256 * slab + 64 * wn + 32 * jb + 8 * g4 + 4 * lh;
              *reinterpret_cast<float4*>(yrow + col) =
                  make_float4(acc[i][jb][4 * g4] * gs, acc[i][jb][4 * g4 + 1] * gs,
                              acc[i][jb][4 * g4 + 2] * gs, acc[i][jb][4 * g4 + 3] * gs);
            }
        }
      }
    }
#undef G_FENCE
#undef G_READ
#undef G_ISSUE_NEXT
    // drain: the re-read DMA past the stream's end and the last fragment
    // reads land before the next batch (or the workgroup's end) reuses LDS
    __builtin_amdgcn_s_waitcnt(g_vmcnt(0));
    g_settle<0>(h0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }
}

template <int MODE, bool PACKED>
static int32_t launch_grouped(const GroupedArgs& g, int grid, hipStream_t s) {
  hipLaunchKernelGGL((grouped_gemm_kernel<MODE, PACKED>), dim3(grid), dim3(kGThreads), 0, s, g);
  return launch_status();
}

// One persistent workgroup per CU (a multiple of 8: an equal share per XCD).
static int grouped_grid() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cus = n;
  }
  return std::max(kGXcd, cus / kGXcd * kGXcd);
}

// Both grouped GEMMs of one MoE prefill (gate_up + SwiGLU into act, then the
// gate-scaled down projection into y).  Validated by the caller: D % 256 == 0,
// H % 256 == 0, rows_total = T * k >= 1, operand blocks below 2 GiB.
int32_t moe_grouped_prefill(const uint16_t* x, const int32_t* offsets, const int32_t* sorted_routes,
                            const float* gates, const uint16_t* w_gate_up, const uint16_t* w_down,
                            uint16_t* act, float* y, int T, int D, int H, int E, int k, bool packed,
                            hipStream_t s) {
  const int rows_total = T * k;
  const int grid = grouped_grid();
  GroupedArgs g{};
  g.x = x;
  g.w = w_gate_up;
  g.out = act;
  g.offsets = offsets;
  g.sorted_routes = sorted_routes;
  g.w_expert_stride = 2ll * H * D;
  g.up_rows = H;
  g.K = D;
  g.ldo = H;
  g.E = E;
  g.route_k = k;
  g.rows_total = rows_total;
  g.x_rows = T;
  g.n_slabs = H / 128;
  int32_t st = packed ? launch_grouped<0, true>(g, grid, s) : launch_grouped<0, false>(g, grid, s);
  if (st != 0) return st;
  GroupedArgs d = g;
  d.x = act;
  d.w = w_down;
  d.out = y;
  d.gates = gates;
  d.w_expert_stride = static_cast<long long>(D) * H;
  d.up_rows = 0;
  d.K = H;
  d.ldo = D;
  d.x_rows = rows_total;
  d.n_slabs = D / 256;
  return packed ? launch_grouped<1, true>(d, grid, s) : launch_grouped<1, false>(d, grid, s);
}

}  // namespace llmy
