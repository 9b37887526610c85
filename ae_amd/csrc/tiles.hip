// Tiled expert kernels of the MoE layer, for batches in which every active expert sees many
// tokens (prefill-sized batches): the two grouped SwiGLU contractions as MFMA tiles.
//
// Once an expert's token count reaches ~100, its weights are no longer the only large
// operand: each weight byte feeds enough multiply-adds that the contraction is bound by the
// matrix cores and by on-chip bandwidth, not by HBM. The streaming kernels (experts.hip) then
// spend their time re-reading small token tiles per 16 weight rows. Here a workgroup owns a
// 256-row x 128-token output tile:
//
//   - each of its 4 waves owns 64 weight rows (four 16-row MFMA tiles) and streams them on its
//     own: per K step, 8 loads of 8 rows x 128 bytes (consecutive lanes on consecutive bytes, so
//     every 4-lane quad reads 64 contiguous bytes) into a wave-private LDS tile, read back as
//     MFMA A fragments. Loading the fragments directly from memory (16 rows x 64 bytes per
//     instruction, a different row in every lane of a quad) ran the kernel at half the rate. A
//     wave reads back only its own writes and LDS operations of one wave run in order, so the
//     tile needs no barrier;
//   - the 128 token rows of the tile are loaded once per workgroup per K step (128 bytes of
//     each row, 4 16-byte loads per thread) into a double-buffered LDS stage and read by all
//     4 waves as MFMA B fragments;
//   - one K step = 128 bytes of K per row = two v_mfma_f32_16x16x32 k-groups; per wave and
//     step: 8 weight loads, 16 LDS fragment reads, 64 MFMAs (4 weight tiles x 8 token tiles x
//     2 k-groups), accumulators 4 x 8 x 4 fp32 per lane;
//   - the next K step's weights and token rows are in flight while a step is multiplied; two
//     workgroups per CU (LDS 32 KB and <= 256 registers per lane each) cover each other's
//     waits.
//
// LDS layout of a token stage and of a weight tile: row q's 16-byte slot s of the step sits
// at slot 8*q + (s ^ (q % 8)). Measured with SQ_LDS_BANK_CONFLICT on the gate/up kernel: no
// conflict cycles for fragment reads (16 lanes: rows q0..q0+15 at one slot) and row writes
// (8 lanes: one row, 8 slots); without the XOR, conflicts take 60% of the LDS cycles (and
// (q ^ (q >> 3)) % 8, conflict-free under an 8- or 16-lane bank model, 33%). Every address is
// a per-lane base plus a compile-time offset.
//
//   tile_gateup_kernel  workgroup = (token range of up to 128 sorted positions of one expert,
//                       128 intermediate columns): wave w owns gate rows [c0+32w, +32) and the
//                       matching up rows, and writes act = round(silu(round(gate)) * round(up)).
//   tile_down_kernel    workgroup = (token range, 256 rows of W2, K split): wave w owns W2 rows
//                       [r0+64w, +64) over the split's K slice and writes fp32 partials
//                       part[split][f][h], summed by combine_kernel.
//
// The arithmetic and rounding points are those of the streaming kernels (and of
// stack_fused_moe, specmoe/layers/fused_moe_kernel.py:319-349); only the fp32 accumulation
// order over K differs.
#include "expert_items.h"

namespace smx {

constexpr int kTStep = 128;                                   // K bytes per row per step
constexpr int kTSlots = kTStep / 16;                          // 16-byte slots per row per step
constexpr int kTBTiles = kTileTok / kTokTile;                 // 16-token MFMA tiles (8)
constexpr int kTATiles = 4;                                   // 16-row weight tiles per wave
constexpr int kTBLoads = kTileTok * kTSlots / kExpertThreads; // token loads per thread per step
constexpr int kTRowsPerLoad = kExpertThreads / kTSlots;       // token rows one load covers (32)
constexpr int kTStage = kTileTok * kTSlots;                   // 16-byte slots per LDS stage

static_assert(kTBLoads * kTRowsPerLoad == kTileTok, "token loads cover the tile");
static_assert(kTileGateCols == kExpertWaves * 2 * kRowTile, "gate/up: 2 gate + 2 up tiles per wave");
static_assert(kTileDownRows == kExpertWaves * kTATiles * kRowTile, "down: 4 W2 tiles per wave");

__device__ __forceinline__ int tswz(int r) { return r & 7; }

// The wave's four weight tiles: a buffer resource on the expert page, a per-lane offset (row
// l / 8, slot l % 8 of an 8-row group) and a wave-uniform byte offset per tile (first row + K
// start); two loads per tile per step (rows 0-7 and 8-15).
struct WTiles {
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t lane_off;
  uint32_t row8;                // bytes of 8 rows
  uint32_t row0[kTATiles];
};

struct WRegs {
  u32x4 v[kTATiles][2];  // loaded: [tile][rows 0-7 / 8-15]; fragments: [tile][k-group]
};

template <int CP>
__device__ __forceinline__ void load_w(WRegs& r, const WTiles& w, int step) {
  const uint32_t kb = static_cast<uint32_t>(step) * kTStep;
#pragma unroll
  for (int i = 0; i < kTATiles; ++i)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      r.v[i][h] = __builtin_amdgcn_raw_buffer_load_b128(w.rsrc, w.lane_off, w.row0[i] + kb + h * w.row8, CP);
}

// Loaded rows into the wave's LDS tile (64 rows x 8 slots); `wa[h]` = the lane's slot for
// rows 8h + l / 8 of tile 0.
__device__ __forceinline__ void store_w(const WRegs& r, u32x4* tile, const int (&wa)[2]) {
#pragma unroll
  for (int i = 0; i < kTATiles; ++i)
#pragma unroll
    for (int h = 0; h < 2; ++h) tile[wa[h] + i * kRowTile * kTSlots] = r.v[i][h];
}

// MFMA A fragments of the step from the wave's tile: lane (g, m) = (l / 16, l % 16) takes
// row m of each tile at slot 4u + g (k-group u); `rb0`, `rb1` are the lane's slots for u = 0, 1.
__device__ __forceinline__ void read_frags(WRegs& f, const u32x4* tile, int rb0, int rb1) {
#pragma unroll
  for (int i = 0; i < kTATiles; ++i) {
    f.v[i][0] = tile[i * kRowTile * kTSlots + rb0];
    f.v[i][1] = tile[i * kRowTile * kTSlots + rb1];
  }
}

// The workgroup's token rows: thread tid loads rows tid/8 + 32j (j < 4), slot tid%8.
struct TRows {
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t base;              // K start of the walk (wave-uniform)
  uint32_t off[kTBLoads];     // per thread: row byte offset + 16 * slot
};

struct TRegs {
  u32x4 v[kTBLoads];
};

__device__ __forceinline__ void load_t(TRegs& r, const TRows& t, int step) {
  const uint32_t kb = t.base + static_cast<uint32_t>(step) * kTStep;
#pragma unroll
  for (int j = 0; j < kTBLoads; ++j) r.v[j] = __builtin_amdgcn_raw_buffer_load_b128(t.rsrc, t.off[j], kb, 0);
}

__device__ __forceinline__ void store_t(const TRegs& r, u32x4* stage, int wbase) {
#pragma unroll
  for (int j = 0; j < kTBLoads; ++j) stage[wbase + j * kTRowsPerLoad * kTSlots] = r.v[j];
}

// Token rows of a step straight into an LDS stage (buffer_load ... lds, 16 bytes per lane, no
// registers): instruction j of wave w fills stage slots [256 j + 64 w, +64) in lane order. Slot
// 256 j + 64 w + l is row q = 32 j + 8 w + l / 8 at position l % 8, which the swizzled layout
// assigns the row's slot (l % 8) ^ swz(q); the per-lane offsets `off` (set for this path)
// select those bytes.
__device__ __forceinline__ void dma_t(const TRows& t, u32x4* stage, int step) {
  const uint32_t kb = t.base + static_cast<uint32_t>(step) * kTStep;
  const int w = wave_id();
#pragma unroll
  for (int j = 0; j < kTBLoads; ++j)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        t.rsrc, (__attribute__((address_space(3))) void*)(stage + j * kTRowsPerLoad * kTSlots + w * kWave),
        16, t.off[j], kb, 0, 0);
}

// Workgroup barrier without a memory fence: the token stages are filled by LDS DMA, and a
// fence would wait for every DMA in flight (also those for later steps); the callers wait for
// the stage they need with an explicit vmcnt. The memory clobber keeps the compiler from
// moving LDS accesses across it.
__device__ __forceinline__ void bare_barrier() { asm volatile("s_barrier" ::: "memory"); }

// 64 MFMAs of one step: acc[i][bt] += A_i . B_bt over the step's two k-groups. The 16 B
// fragments (k-group u, token tile bt) are read from the stage two ahead of their use, in a
// ring of three, and a scheduling barrier closes each group (one read, then the four MFMAs of
// the fragment read two groups before), so that the compiler keeps that distance: a
// fragment's LDS latency then overlaps eight MFMAs of this wave. With kStore, the next step's
// weights (`wnext`, loaded two steps back) go to the wave's tile one write every second
// group, spread over the step rather than gathered before the barrier; the tile's A fragments
// of this step were read before (a wave's LDS operations run in issue order).
template <int DT, bool kStore = false>
__device__ __forceinline__ void mma_step(const WRegs& a, const u32x4* stage, int rb0, int rb1,
                                         f32x4 (&acc)[kTATiles][kTBTiles],
                                         const WRegs* wnext = nullptr, u32x4* tile = nullptr,
                                         const int* wa = nullptr) {
  constexpr int kFrags = 2 * kTBTiles;
  static_assert(kFrags / 2 == kTATiles * 2, "one weight write every second group");
  auto slot = [&](int n) { return (n % kTBTiles) * kTokTile * kTSlots + (n < kTBTiles ? rb0 : rb1); };
  u32x4 b[3];
  b[0] = stage[slot(0)];
  b[1] = stage[slot(1)];
#pragma unroll
  for (int n = 0; n < kFrags; ++n) {
    if (n + 2 < kFrags) b[(n + 2) % 3] = stage[slot(n + 2)];
    if constexpr (kStore) {
      if (n % 2 == 1) {
        const int q = n / 2, i = q / 2, h = q % 2;
        tile[wa[h] + i * kRowTile * kTSlots] = wnext->v[i][h];
      }
    }
    const int u = n / kTBTiles, bt = n % kTBTiles;
#pragma unroll
    for (int i = 0; i < kTATiles; ++i) acc[i][bt] = Elem<DT>::mfma(a.v[i][u], b[n % 3], acc[i][bt]);
    __builtin_amdgcn_sched_barrier(0);
  }
}

struct TWalk {
  WTiles w;
  TRows t;
  int wbase;     // per thread: LDS slot of its first token load
  int wa[2];     // per lane: LDS slot of its weight loads (rows 0-7 / 8-15 of tile 0)
  int rb0, rb1;  // per lane: LDS slot of its A and B fragments, k-group 0 / 1, tile 0
};

// Vector-memory operations a wave issues after its token DMA of a step, until the wait that
// must see that DMA landed: the same step's weights, then the next step's DMA and weights. The
// waits below count on this issue order (the hardware retires a wave's vector-memory loads in
// order), so every DMA group and weight group is fenced from the compiler's scheduler by a
// sched_barrier: without them the compiler issued the prologue's first weight loads ahead of
// its DMA, and the prologue's wait then left the first DMA in flight at the barrier -- other
// waves read that quarter of the first stage before it landed (stale LDS, NaN on occasion).
constexpr int kVmAfterDma = 2 * kTATiles * 2 + kTBLoads;  // 8 + 4 + 8

// One step of the 16-bit walk, for step c: its token rows are in stage `cur` and its weights in
// the wave's tile. Step c+2's token rows go out by DMA into `dma_dst` (the stage step c-1 read)
// and then its weights into `issue_to`; during the MFMAs, step c+1's weights (`next`, loaded two
// steps back) are written to the tile; then the wave waits until step c+1's DMA has landed -- loads
// issued after it: step c+1's weights (8), step c+2's DMA (4) and weights (8) -- and the
// workgroup meets at the barrier.
template <int CP, int DT>
__device__ __forceinline__ void dma_step(WRegs& issue_to, const WRegs& next, WRegs& frag,
                                         const u32x4* cur, u32x4* dma_dst, u32x4* wtile,
                                         const TWalk& wk, int issue, f32x4 (&acc)[kTATiles][kTBTiles]) {
  dma_t(wk.t, dma_dst, issue);
  __builtin_amdgcn_sched_barrier(0);
  load_w<CP>(issue_to, wk.w, issue);
  __builtin_amdgcn_sched_barrier(0);
  read_frags(frag, wtile, wk.rb0, wk.rb1);
  mma_step<DT, true>(frag, cur, wk.rb0, wk.rb1, acc, &next, wtile, wk.wa);
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(kVmAfterDma));
  bare_barrier();
}

// acc += the wave's 64 weight rows . the workgroup's 128 token rows over n K steps (n even),
// 16-bit types. Token rows go by DMA into three LDS stages, two steps ahead; weights two steps
// ahead into two register sets, written to the wave's tile one step ahead (after the step's
// fragments were read from it). The loop is unrolled by six so that every stage and register
// set is a fixed object (the compiler then sees that a DMA in flight and the stage being read
// do not alias). Step indices past the end are clamped to the last step (reloads in bounds,
// into stages and registers no later step reads), so the body has no branches apart from the
// exits between step pairs. Two workgroups per CU cover each other's waits.
template <int CP, int DT>
__device__ __forceinline__ void tile_walk(const TWalk& wk, int n, u32x4* st0, u32x4* st1,
                                          u32x4* st2, u32x4* wtile,
                                          f32x4 (&acc)[kTATiles][kTBTiles]) {
  WRegs r0, r1, frag;
  // issue order: step 0's DMA, its weights, step 1's DMA, its weights (kVmAfterDma after the
  // first DMA), so that the wait before the barrier sees step 0's token rows in LDS
  dma_t(wk.t, st0, 0);
  __builtin_amdgcn_sched_barrier(0);
  load_w<CP>(r0, wk.w, 0);
  __builtin_amdgcn_sched_barrier(0);
  dma_t(wk.t, st1, min(1, n - 1));
  __builtin_amdgcn_sched_barrier(0);
  load_w<CP>(r1, wk.w, min(1, n - 1));
  __builtin_amdgcn_sched_barrier(0);
  store_w(r0, wtile, wk.wa);
  __builtin_amdgcn_s_waitcnt(vmcnt_imm(kVmAfterDma));  // step 0's DMA
  bare_barrier();
  for (int c = 0;; c += 6) {
    const int l = n - 1;
    dma_step<CP, DT>(r0, r1, frag, st0, st2, wtile, wk, min(c + 2, l), acc);
    dma_step<CP, DT>(r1, r0, frag, st1, st0, wtile, wk, min(c + 3, l), acc);
    if (c + 2 >= n) break;
    dma_step<CP, DT>(r0, r1, frag, st2, st1, wtile, wk, min(c + 4, l), acc);
    dma_step<CP, DT>(r1, r0, frag, st0, st2, wtile, wk, min(c + 5, l), acc);
    if (c + 4 >= n) break;
    dma_step<CP, DT>(r0, r1, frag, st1, st0, wtile, wk, min(c + 6, l), acc);
    dma_step<CP, DT>(r1, r0, frag, st2, st1, wtile, wk, min(c + 7, l), acc);
    if (c + 6 >= n) break;
  }
}

// The same walk with weights loaded one step ahead (one register set), for fp32 (whose four
// MFMAs per fragment need more registers than a second weight set leaves).
template <int CP, int DT>
__device__ __forceinline__ void tile_walk_1(const TWalk& wk, int n, u32x4* s0, u32x4* s1,
                                            u32x4* wtile, f32x4 (&acc)[kTATiles][kTBTiles]) {
  WRegs raw, frag;
  TRegs tnext;
  load_t(tnext, wk.t, 0);
  load_w<CP>(raw, wk.w, 0);
  store_t(tnext, s0, wk.wbase);
  store_w(raw, wtile, wk.wa);
  wg_barrier();
  for (int c = 0; c < n; ++c) {
    u32x4* cur = (c & 1) ? s1 : s0;
    u32x4* nxt = (c & 1) ? s0 : s1;
    const int nx = min(c + 1, n - 1);
    load_t(tnext, wk.t, nx);
    load_w<CP>(raw, wk.w, nx);
    __builtin_amdgcn_sched_barrier(0);
    read_frags(frag, wtile, wk.rb0, wk.rb1);
    mma_step<DT>(frag, cur, wk.rb0, wk.rb1, acc);
    __builtin_amdgcn_sched_barrier(0);
    store_t(tnext, nxt, wk.wbase);
    store_w(raw, wtile, wk.wa);
    wg_barrier();
  }
}

// The 16-bit walk ends with reloads of its last step still in flight, DMAs into its LDS stages
// among them. The wave waits for them before it ends (after its output stores, so the wait
// costs nothing the end of the program would not), so that no DMA of this workgroup can land
// in LDS that a later workgroup on the CU has been given.
template <int DT>
__device__ __forceinline__ void drain_walk() {
  if constexpr (DT != kF32) __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
}

template <int CP, int DT>
__device__ __forceinline__ void walk(const TWalk& wk, int n, u32x4* s0, u32x4* s1, u32x4* s2,
                                     u32x4* wtile, f32x4 (&acc)[kTATiles][kTBTiles]) {
  if constexpr (DT == kF32) tile_walk_1<CP, DT>(wk, n, s0, s1, wtile, acc);
  else tile_walk<CP, DT>(wk, n, s0, s1, s2, wtile, acc);
}

// Per-thread byte offset of token row `row`'s slot for this thread: the DMA path (16-bit
// types) loads the slot its fixed LDS position holds, the register path its own slot.
template <int DT>
__device__ __forceinline__ uint32_t token_off(int row, int64_t row_bytes) {
  const int tid = threadIdx.x;
  int slot = tid % kTSlots;
  if constexpr (DT != kF32) slot ^= tswz(tid / kTSlots);
  return static_cast<uint32_t>(row * row_bytes + slot * 16);
}

// Per-thread LDS addressing of the token stage (see the layout note at the top).
__device__ __forceinline__ void stage_addressing(TWalk& wk) {
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int q = tid / kTSlots;  // first token row this thread loads
  wk.wbase = q * kTSlots + ((tid % kTSlots) ^ tswz(q & 15));
  const int r = lane & 15, g = lane >> 4;
  wk.rb0 = r * kTSlots + (g ^ tswz(r));
  wk.rb1 = r * kTSlots + ((4 + g) ^ tswz(r));
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int row = 8 * h + (lane >> 3);  // rows of this lane's weight loads (tile 0)
    wk.wa[h] = row * kTSlots + ((lane & 7) ^ tswz(row));
  }
}

// Token rows of a workgroup's range: position q of the range (clamped to the last one; rows
// past the range are computed and discarded).
__device__ __forceinline__ int range_row(const ExpertArgs& a, const WorkItem& it, int q, bool gather) {
  const int pos = it.off + min(q, it.m - 1);
  if (!gather) return pos;
  return it.shared ? pos : a.rb.sorted_f[pos] / a.k;
}

__device__ __forceinline__ void zero_acc(f32x4 (&acc)[kTATiles][kTBTiles]) {
#pragma unroll
  for (int i = 0; i < kTATiles; ++i)
#pragma unroll
    for (int bt = 0; bt < kTBTiles; ++bt) acc[i][bt] = f32x4{0.f, 0.f, 0.f, 0.f};
}

template <int DT>
__global__ __launch_bounds__(kExpertThreads, 2) void tile_gateup_kernel(ExpertArgs a) {
  using S = typename Elem<DT>::S;
  const int wave = wave_id();
  const int lane = lane_id();
  const bool in_shared = static_cast<int>(blockIdx.x) < a.sh.gateup_blocks;
  const int Iw = in_shared ? a.sh.I : a.I;
  const int groups = (Iw + kTileGateCols - 1) / kTileGateCols;
  WorkItem it;
  if (!work_item<S>(a, a.sh.gateup_blocks, groups, it, a.rb.hdr, a.rb.ranges)) return;
  __shared__ u32x4 st0[kTStage], st1[kTStage], st2[DT == kF32 ? 1 : kTStage];
  __shared__ u32x4 wtiles[kExpertWaves][kTATiles * kRowTile * kTSlots];
  const int H = a.H, I = it.I;
  const int64_t row_bytes = static_cast<int64_t>(H) * sizeof(S);
  const int last = I / kRowTile - 1;  // last 16-column tile of the intermediate dimension
  int ct[2];                          // the wave's two 16-column tiles (clamped)
  bool own[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int tcol = (it.tg * kTileGateCols) / kRowTile + 2 * wave + i;
    own[i] = tcol <= last;
    ct[i] = min(tcol, last);
  }
  TWalk wk;
  wk.w.rsrc = make_rsrc(it.page, static_cast<uint32_t>(it.page_bytes));
  wk.w.lane_off = static_cast<uint32_t>((lane >> 3) * row_bytes + (lane & 7) * 16);
  wk.w.row8 = static_cast<uint32_t>(8 * row_bytes);
  // tiles 0, 1: gate rows; tiles 2, 3: the matching up rows (W3 starts I rows after W1)
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    wk.w.row0[i] = static_cast<uint32_t>(static_cast<int64_t>(ct[i]) * kRowTile * row_bytes);
    wk.w.row0[i + 2] = static_cast<uint32_t>((static_cast<int64_t>(I) + ct[i] * kRowTile) * row_bytes);
  }
  wk.t.rsrc = make_rsrc(a.x, static_cast<uint32_t>(static_cast<int64_t>(a.T) * row_bytes));
  wk.t.base = 0;
  const int tid = threadIdx.x;
#pragma unroll
  for (int j = 0; j < kTBLoads; ++j) {
    const int tok = range_row(a, it, tid / kTSlots + j * kTRowsPerLoad, true);
    wk.t.off[j] = token_off<DT>(tok, row_bytes);
  }
  stage_addressing(wk);
  f32x4 acc[kTATiles][kTBTiles];
  zero_acc(acc);
  const int n = static_cast<int>(row_bytes / kTStep);
  // Weight rows are re-read by the other token ranges of the expert: normal caching.
  walk<0, DT>(wk, n, st0, st1, st2, wtiles[wave], acc);

  S* act = static_cast<S*>(it.shared ? a.sh.act : a.act);
  const int f16out = it.shared ? 0 : a.f16out;
  const int g = lane >> 4;
#pragma unroll
  for (int bt = 0; bt < kTBTiles; ++bt) {
    const int q = bt * kTokTile + (lane & 15);
    if (q >= it.m) continue;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if (!own[i]) continue;
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float gate = round_out<DT>(acc[i][bt][e], f16out);
        const float up = round_out<DT>(acc[i + 2][bt][e], f16out);
        o[e] = silu_f32(gate) * up;
      }
      store4<DT>(act, static_cast<int64_t>(it.off + q) * I + ct[i] * kRowTile + 4 * g, o[0], o[1], o[2], o[3]);
    }
  }
  drain_walk<DT>();
}

template <int DT>
__global__ __launch_bounds__(kExpertThreads, 2) void tile_down_kernel(ExpertArgs a) {
  using S = typename Elem<DT>::S;
  const int wave = wave_id();
  const int lane = lane_id();
  const int rgroups = (a.H + kTileDownRows - 1) / kTileDownRows;
  const bool in_shared = static_cast<int>(blockIdx.x) < a.sh.down_blocks;
  const int splits = in_shared ? a.sh.splits : a.splits;
  const int split_steps = in_shared ? a.sh.split_steps : a.split_steps;  // 64-byte units
  WorkItem it;
  if (!work_item<S>(a, a.sh.down_blocks, rgroups * splits, it, a.rb.hdr, a.rb.ranges)) return;
  __shared__ u32x4 st0[kTStage], st1[kTStage], st2[DT == kF32 ? 1 : kTStage];
  __shared__ u32x4 wtiles[kExpertWaves][kTATiles * kRowTile * kTSlots];
  const int sp = it.tg / rgroups;
  const int rg = it.tg - sp * rgroups;
  const int H = a.H, I = it.I;
  const int rows = it.shared ? a.T : a.T * a.k;  // rows of act and of one split of part
  const int64_t row_bytes = static_cast<int64_t>(I) * sizeof(S);
  const int64_t k0 = static_cast<int64_t>(sp) * split_steps * kStepBytes;
  const int last = H / kRowTile - 1;
  int ht[kTATiles];
  bool own[kTATiles];
#pragma unroll
  for (int i = 0; i < kTATiles; ++i) {
    const int t = (rg * kTileDownRows) / kRowTile + kTATiles * wave + i;
    own[i] = t <= last;
    ht[i] = min(t, last);
  }
  TWalk wk;
  wk.w.rsrc = make_rsrc(it.page, static_cast<uint32_t>(it.page_bytes));
  wk.w.lane_off = static_cast<uint32_t>((lane >> 3) * row_bytes + (lane & 7) * 16);
  wk.w.row8 = static_cast<uint32_t>(8 * row_bytes);
  // W2 starts after W1 and W3 (2*I rows of H elements = 2*H rows of I elements)
#pragma unroll
  for (int i = 0; i < kTATiles; ++i)
    wk.w.row0[i] = static_cast<uint32_t>((2 * static_cast<int64_t>(H) + ht[i] * kRowTile) * row_bytes + k0);
  const void* actp = it.shared ? a.sh.act : a.act;
  wk.t.rsrc = make_rsrc(actp, static_cast<uint32_t>(static_cast<int64_t>(rows) * row_bytes));
  wk.t.base = static_cast<uint32_t>(k0);
  const int tid = threadIdx.x;
#pragma unroll
  for (int j = 0; j < kTBLoads; ++j) {
    const int row = range_row(a, it, tid / kTSlots + j * kTRowsPerLoad, false);
    wk.t.off[j] = token_off<DT>(row, row_bytes);
  }
  stage_addressing(wk);
  f32x4 acc[kTATiles][kTBTiles];
  zero_acc(acc);
  const int n = split_steps * kStepBytes / kTStep;
  walk<0, DT>(wk, n, st0, st1, st2, wtiles[wave], acc);

  float* part = it.shared ? a.sh.part : a.part;
  const int g = lane >> 4;
#pragma unroll
  for (int bt = 0; bt < kTBTiles; ++bt) {
    const int q = bt * kTokTile + (lane & 15);
    if (q >= it.m) continue;
    const int f = it.shared ? it.off + q : a.rb.sorted_f[it.off + q];
    float* dst = part + (static_cast<int64_t>(sp) * rows + f) * H;
#pragma unroll
    for (int i = 0; i < kTATiles; ++i)
      if (own[i]) *reinterpret_cast<f32x4*>(dst + ht[i] * kRowTile + 4 * g) = acc[i][bt];
  }
  drain_walk<DT>();
}

int64_t tile_grid_blocks(int stage, int64_t H, int64_t I, int shared_blocks, int max_ranges, int splits) {
  const int64_t groups = stage == 0 ? (I + kTileGateCols - 1) / kTileGateCols
                                    : (H + kTileDownRows - 1) / kTileDownRows * splits;
  return shared_blocks + max_ranges * groups;
}

template <int DT>
static hipError_t tile_launch(int stage, const ExpertArgs& a, int max_ranges, hipStream_t s) {
  // The 16-bit walk consumes K steps in pairs: the plan gives every walk an even step count
  // (H and I are whole 256-byte chunks, split counts divide half the steps); refuse otherwise.
  if (DT != kF32) {
    const int64_t eb = dtype_bytes(DT);
    const bool odd = stage == 0 ? (a.H * eb / kTStep) % 2 != 0
                                : (a.split_steps * kStepBytes / kTStep) % 2 != 0 ||
                                      (a.sh.I > 0 && (a.sh.split_steps * kStepBytes / kTStep) % 2 != 0);
    if (odd) return hipErrorInvalidValue;
  }
  if (stage == 0) {
    const int64_t blocks = tile_grid_blocks(0, a.H, a.I, a.sh.gateup_blocks, max_ranges, 1);
    tile_gateup_kernel<DT><<<static_cast<unsigned>(blocks), kExpertThreads, 0, s>>>(a);
  } else {
    const int64_t blocks = tile_grid_blocks(1, a.H, a.I, a.sh.down_blocks, max_ranges, a.splits);
    tile_down_kernel<DT><<<static_cast<unsigned>(blocks), kExpertThreads, 0, s>>>(a);
  }
  return hipGetLastError();
}

static hipError_t tile_stage(int stage, int dtype, const ExpertArgs& a, int max_ranges, hipStream_t s) {
  switch (dtype) {
    case kF32: return tile_launch<kF32>(stage, a, max_ranges, s);
    case kF16: return tile_launch<kF16>(stage, a, max_ranges, s);
    default: return tile_launch<kBF16>(stage, a, max_ranges, s);
  }
}

hipError_t launch_tile_gateup(int dtype, const ExpertArgs& a, int max_ranges, hipStream_t s) {
  return tile_stage(0, dtype, a, max_ranges, s);
}

hipError_t launch_tile_down(int dtype, const ExpertArgs& a, int max_ranges, hipStream_t s) {
  return tile_stage(1, dtype, a, max_ranges, s);
}

}  // namespace smx
