// Device code of the weight-streaming gate/up launch (gateup_kernel and the pieces of the
// expert streams it shares with the down kernel), included by the translation units that
// instantiate it: experts.hip (the gate/up launches) and layer1.hip (the single-launch layer
// form, whose gate/up workgroups publish their activation rows to the down workgroups of the
// same launch).
#pragma once

#include "expert_items.h"
#include "topk_device.h"

namespace smx {

// MFMA output layout (16x16 f32 accumulator): lane l, register i holds row 4*(l/16)+i of the
// A operand's 16 rows and column l%16 of the B operand's 16 columns. Operand fragments:
// lane l holds 16 contiguous bytes of A row l%16 (resp. B column l%16) at K group l/16.
//
// Weight loads do not use the fragment layout directly (16 rows x 64 bytes per instruction
// streams from HBM ~15% slower than wider row segments). Each 16-row tile is loaded in
// chunks of 256 bytes per row by four instructions of 4 rows x 256 bytes (lane l: row
// 4i + l/16, bytes 16*(l%16)), written to a wave-private LDS tile, and read back as
// fragments. The LDS tile stores row r's 16-byte slot c at slot 17*r + c: the row pitch of
// 17 slots puts the 16 slots a 16-lane group touches, row-wise on write and column-wise on
// read, in 16 distinct bank groups (no conflicts), and keeps every address a per-lane base
// plus a compile-time offset. One wave's LDS operations execute in order, so a wave reads
// back its own writes and overwrites a tile only after reading it: no barriers.
//
// Loads are buffer loads: a scalar resource (base, size) plus a 32-bit per-lane offset and a
// wave-uniform scalar offset (tile, instruction and chunk), which keeps the per-lane address
// state to one VGPR per stream.

constexpr int kPitch = 17;                        // LDS row pitch in 16-byte slots
constexpr int kTileSlots = kRowTile * kPitch;     // slots per LDS tile (4352 bytes)
template <int R>
struct Raw {
  u32x4 v[4][R];  // [instruction][tile]
};

struct WeightStream {
  __amdgpu_buffer_rsrc_t rsrc;  // the expert's page
  uint32_t base;                // byte offset of tile 0's first row at chunk 0
  uint32_t tile_stride;         // bytes between consecutive tiles
  uint32_t row4;                // bytes of 4 rows
  uint32_t lane_off;            // per lane: row l/16, byte column 16*(l%16)
};

// CP: cache policy of the weight loads (kNonTemporal when every weight byte is read once).
template <int CP, int R>
__device__ __forceinline__ void load_raw(Raw<R>& c, const WeightStream& w, int chunk) {
  const uint32_t cbase = w.base + static_cast<uint32_t>(chunk) * (kStepBytes * kUnroll);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < R; ++r)
      c.v[i][r] = __builtin_amdgcn_raw_buffer_load_b128(
          w.rsrc, w.lane_off, cbase + r * w.tile_stride + i * w.row4, CP);
}

// Token operand, shared by the workgroup. The W waves of a workgroup (W = 4, 2 or 1) work on
// the same expert and step through K together. Each chunk of the MT token tiles (16 token rows
// x 256 bytes each) is loaded once per workgroup -- wave w loads the 4-row groups w, w + W, ...
// of every tile, one 4-row x 256-byte instruction per group (4 / W per tile) -- into a
// double-buffered LDS tile with the same padded layout as the weight tiles, and every wave reads
// its MFMA B fragments from there. One barrier per chunk; every wave of a workgroup runs the
// same number of chunks.
template <int MT, int W>
struct SharedTokens {
  static constexpr int kGroups = 4 / W;  // 4-row groups per tile loaded by one wave
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t base;                 // byte offset of the K range (wave-uniform)
  uint32_t off[MT][kGroups];     // per lane: offset of row 4*(wave + W*n) + l/16 of tile j, + 16*(l%16)
};

template <int MT, int W>
struct RawTokens {
  u32x4 v[MT][4 / W];
};

template <int MT, int W>
__device__ __forceinline__ void load_tokens(RawTokens<MT, W>& rb, const SharedTokens<MT, W>& t, int chunk) {
  const uint32_t cbase = t.base + static_cast<uint32_t>(chunk) * (kStepBytes * kUnroll);
#pragma unroll
  for (int j = 0; j < MT; ++j)
#pragma unroll
    for (int n = 0; n < 4 / W; ++n)
      rb.v[j][n] = __builtin_amdgcn_raw_buffer_load_b128(t.rsrc, t.off[j][n], cbase, 0);
}

// wv: the wave's index among the W waves that share the token stage.
template <int MT, int W>
__device__ __forceinline__ void store_tokens(const RawTokens<MT, W>& rb, u32x4* bt, int wv) {
  const int lane = lane_id();
#pragma unroll
  for (int n = 0; n < 4 / W; ++n) {
    u32x4* wr = bt + kPitch * (4 * (wv + W * n) + (lane >> 4)) + (lane & 15);
#pragma unroll
    for (int j = 0; j < MT; ++j) wr[j * kTileSlots] = rb.v[j][n];
  }
}

// One step of the workgroup's two-deep pipeline, for chunk c. On entry this chunk's weights
// are in `cur` (issued two steps back), chunk c+1's weights are in flight in the other
// register set, this chunk's token tile is published in `bt` and chunk c+1's token rows are
// in flight in `tnext`. Writing `cur` into the wave's LDS tile frees it at once, so chunk
// c+2's token rows (into `tfree`) and weights (into `cur`; `issue_chunk` is where step c+2
// falls in the workgroup's chunk order) are issued before the MFMAs: two
// chunks of weights stay in flight while this one is multiplied. Then chunk c+1's token rows,
// issued a step ago, are published into `bt_next`; barrier. Token loads are issued before
// weight loads, so waiting for a token chunk never waits for the weights issued with it.
template <int CP, int DT, int R, int MT, int W, bool kIssue, bool kNext>
__device__ __forceinline__ void wg_step(Raw<R>& cur, const RawTokens<MT, W>& tnext,
                                        RawTokens<MT, W>& tfree, u32x4* lds, const u32x4* bt,
                                        u32x4* bt_next, const WeightStream& w,
                                        const SharedTokens<MT, W>& t, int issue_chunk,
                                        f32x4 (&acc)[R][MT], int wv) {
  const int lane = lane_id();
  u32x4* wr = lds + kPitch * (lane >> 4) + (lane & 15);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < R; ++r) wr[r * kTileSlots + 4 * kPitch * i] = cur.v[i][r];
  // Keep the refill after the LDS writes (so it reuses `cur`'s registers) and ahead of the
  // MFMA sequence (so it is in flight while they run).
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (kIssue) {
    load_tokens(tfree, t, issue_chunk);
    load_raw<CP>(cur, w, issue_chunk);
  }
  __builtin_amdgcn_sched_barrier(0);
  const u32x4* rd = lds + kPitch * (lane & 15) + (lane >> 4);
  const u32x4* brd = bt + kPitch * (lane & 15) + (lane >> 4);
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    u32x4 af[R];
#pragma unroll
    for (int r = 0; r < R; ++r) af[r] = rd[r * kTileSlots + 4 * u];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const u32x4 bf = brd[mt * kTileSlots + 4 * u];
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r][mt] = Elem<DT>::mfma(af[r], bf, acc[r][mt]);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (kNext) store_tokens(tnext, bt_next, wv);
  wg_barrier();
}

// Issue the first two weight chunks of a stream (they need only the expert page, so they go
// out before the token rows are looked up).
template <int CP, int R>
__device__ __forceinline__ void issue_weights(Raw<R>& a, Raw<R>& b, const WeightStream& w,
                                              const ChunkOrder& ord) {
  load_raw<CP>(a, w, ord.at(0));
  if (ord.n > 1) load_raw<CP>(b, w, ord.at(1));
}

// acc[r][mt] += A_r (16 rows x nchunks*256 bytes) . B_mt, the workgroup streaming the token
// chunks through `bsh` (two buffers of MT tiles) while each wave streams its own weights;
// chunks 0 and 1 of the weights are already in flight in `a` and `b` (issue_weights).
template <int CP, int DT, int R, int MT, int W>
__device__ __forceinline__ void stream_wg(const WeightStream& w, const SharedTokens<MT, W>& t,
                                          const ChunkOrder& ord, u32x4* lds, u32x4* bsh,
                                          f32x4 (&acc)[R][MT], Raw<R>& a, Raw<R>& b, int wv) {
  RawTokens<MT, W> t0, t1;
  u32x4* b0 = bsh;
  u32x4* b1 = bsh + MT * kTileSlots;
  const int nchunks = ord.n;
  load_tokens(t0, t, ord.at(0));
  if (nchunks > 1) load_tokens(t1, t, ord.at(1));
  store_tokens(t0, b0, wv);
  wg_barrier();
  int c = 0;
  for (; c + 3 < nchunks; c += 2) {
    wg_step<CP, DT, R, MT, W, true, true>(a, t1, t0, lds, b0, b1, w, t, ord.at(c + 2), acc, wv);
    wg_step<CP, DT, R, MT, W, true, true>(b, t0, t1, lds, b1, b0, w, t, ord.at(c + 3), acc, wv);
  }
  const int rem = nchunks - c;  // 1, 2 or 3 chunks left
  if (rem == 3) {
    wg_step<CP, DT, R, MT, W, true, true>(a, t1, t0, lds, b0, b1, w, t, ord.at(c + 2), acc, wv);
    wg_step<CP, DT, R, MT, W, false, true>(b, t0, t1, lds, b1, b0, w, t, 0, acc, wv);
    wg_step<CP, DT, R, MT, W, false, false>(a, t1, t0, lds, b0, b1, w, t, 0, acc, wv);
  } else if (rem == 2) {
    wg_step<CP, DT, R, MT, W, false, true>(a, t1, t0, lds, b0, b1, w, t, 0, acc, wv);
    wg_step<CP, DT, R, MT, W, false, false>(b, t0, t1, lds, b1, b0, w, t, 0, acc, wv);
  } else {
    wg_step<CP, DT, R, MT, W, false, false>(a, t1, t0, lds, b0, b1, w, t, 0, acc, wv);
  }
}

// The token passes of one gate/up workgroup with MT token tiles per pass: wave `wave` owns
// weight-row tile p (gate rows [16p, 16p+16) and the matching up rows); `owner` is false for
// a wave past the expert's last tile (it streams tile p again and stores nothing).
// `sorted`: the routing's sorted flat assignments (global memory, or the workgroup's LDS copy).
// KS (4-wave workgroups): the K walk is split between wave pairs -- waves 0, 1 own tiles 2tg,
// 2tg + 1 over the first half of the chunks, waves 2, 3 the same tiles over the second half,
// each half with its own token stage -- and the second half's sums reach the first through LDS
// before the epilogue: items of half the length, so a launch's last round of workgroups drains
// in half the time. bsh then holds two stages.
// CO: the activation rows are stored at device scope (store4_agent), for the single-launch
// layer whose down workgroups read them in the same launch.
// The weight stream of wave tile p of an item (tile 0: gate rows [16p, 16p+16); tile 1: the
// matching up rows) and the wave's chunk order (KS: its K half). Needs only the item's page,
// I and rotation.
template <int DT, bool KS>
__device__ __forceinline__ void gateup_stream(const ExpertArgs& a, const WorkItem& it, int p,
                                              WeightStream& ws, ChunkOrder& ord) {
  using S = typename Elem<DT>::S;
  const int lane = lane_id();
  const int h = KS ? wave_id() >> 1 : 0;
  const int64_t row_bytes = static_cast<int64_t>(a.H) * sizeof(S);
  ws.rsrc = make_rsrc(it.page, static_cast<uint32_t>(it.page_bytes));
  ws.base = static_cast<uint32_t>(kRowTile * p * row_bytes);
  ws.tile_stride = static_cast<uint32_t>(it.I * row_bytes);
  ws.row4 = static_cast<uint32_t>(4 * row_bytes);
  ws.lane_off = static_cast<uint32_t>((lane >> 4) * row_bytes + (lane & 15) * 16);
  const int nch = static_cast<int>(row_bytes / (kStepBytes * kUnroll));
  ord = rotated_order(KS ? nch / 2 : nch, it.rot);
  ord.base = h * ord.n;
}

// PRE: the item's first two weight chunks are already in flight in *pa, *pb (issued by
// gateup_stream + issue_weights for the same item and tile before the routing); the item then
// has one pass (m <= MT token tiles: the host's condition for such items).
template <int CP, int DT, int MT, int W, bool KS = false, bool CO = false, bool PRE = false>
__device__ __forceinline__ void gateup_passes(const ExpertArgs& a, const WorkItem& it, int p,
                                              bool owner, u32x4* lds, u32x4* bsh,
                                              const int32_t* sorted, Raw<2>* pa = nullptr,
                                              Raw<2>* pb = nullptr) {
  using S = typename Elem<DT>::S;
  static_assert(!KS || W == kExpertWaves, "the K split pairs the waves of a 4-wave workgroup");
  constexpr int WT = KS ? 2 : W;  // waves sharing one token stage
  const int lane = lane_id();
  const int wave = wave_id();
  const int h = KS ? wave >> 1 : 0;     // K half
  const int wv = KS ? wave & 1 : wave;  // index among the waves of the token stage
  const int r = lane & 15, g = lane >> 4;
  const int I = it.I, off = it.off, m = it.m;
  const int64_t row_bytes = static_cast<int64_t>(a.H) * sizeof(S);
  WeightStream ws;
  ChunkOrder ord;
  gateup_stream<DT, KS>(a, it, p, ws, ord);
  u32x4* stage = bsh + h * 2 * MT * kTileSlots;
  S* act = static_cast<S*>(it.shared ? a.sh.act : a.act);
  const int f16out = it.shared ? 0 : a.f16out;
  const float rk = 1.0f / static_cast<float>(a.k);  // flat assignment f -> token f / k
  for (int q0 = 0; q0 < m; q0 += kTokTile * MT) {
    Raw<2> wa, wb;
    if constexpr (PRE) {
      wa = *pa;
      wb = *pb;
    } else {
      issue_weights<CP>(wa, wb, ws, ord);
    }
    SharedTokens<MT, WT> tb;
    tb.rsrc = make_rsrc(a.x, static_cast<uint32_t>(static_cast<int64_t>(a.T) * row_bytes));
    tb.base = 0;
#pragma unroll
    for (int j = 0; j < MT; ++j)
#pragma unroll
      for (int n = 0; n < 4 / WT; ++n) {
        const int q = min(q0 + j * kTokTile + 4 * (wv + WT * n) + (lane >> 4), m - 1);
        const int tok = it.shared ? off + q : div_small(sorted[off + q], a.k, rk);
        tb.off[j][n] = static_cast<uint32_t>(tok * row_bytes + (lane & 15) * 16);
      }
    f32x4 acc[2][MT];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[i][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    stream_wg<CP, DT, 2, MT, WT>(ws, tb, ord, lds, stage, acc, wa, wb, wv);
    if constexpr (KS) {
      // the second half's sums into the first half's waves, through the wave tiles (wave w + 2
      // is wave w's partner; its tile is 2 * kTileSlots slots per wave further on)
      f32x4* red = reinterpret_cast<f32x4*>(lds);
      if (h == 1) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) red[(i * MT + mt) * kWave + lane] = acc[i][mt];
      }
      wg_barrier();
      if (h == 0) {
        const f32x4* pr = reinterpret_cast<const f32x4*>(lds + 4 * kTileSlots);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) acc[i][mt] = acc[i][mt] + pr[(i * MT + mt) * kWave + lane];
      }
      wg_barrier();  // the tiles are free for the next pass
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int q = q0 + mt * kTokTile + r;
      if (owner && h == 0 && q < m) {
        float o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float gate = round_out<DT>(acc[0][mt][i], f16out);
          const float up = round_out<DT>(acc[1][mt][i], f16out);
          o[i] = silu_f32(gate) * up;
        }
        const int64_t idx = static_cast<int64_t>(off + q) * I + kRowTile * p + 4 * g;
        if constexpr (CO) store4_agent<DT>(act, idx, o[0], o[1], o[2], o[3]);
        else store4<DT>(act, idx, o[0], o[1], o[2], o[3]);
      }
    }
  }
}

// Workgroup = (work item, W consecutive weight tiles): wave w owns tile W*tg + w. A wave
// past the expert's last tile streams the last tile again and stores nothing, so every
// wave of a workgroup runs the same chunks and barriers. The token tiles per pass follow
// the item's token count (up to MT): an expert with few tokens streams its weights with
// one tile of 16 tokens.
template <int CP, int DT, int MT, int W, bool KS = false, bool CO = false, bool PRE = false>
__device__ __forceinline__ void gateup_item(const ExpertArgs& a, const WorkItem& it, int p,
                                            bool owner, u32x4* lds, u32x4* bsh,
                                            const int32_t* sorted, Raw<2>* pa = nullptr,
                                            Raw<2>* pb = nullptr) {
  if (MT == 1 || it.m <= kTokTile)
    gateup_passes<CP, DT, 1, W, KS, CO, PRE>(a, it, p, owner, lds, bsh, sorted, pa, pb);
  else if (MT == 2 || it.m <= 2 * kTokTile)
    gateup_passes<CP, DT, (MT >= 2 ? 2 : 1), W, KS, CO, PRE>(a, it, p, owner, lds, bsh, sorted, pa, pb);
  else if (MT == 3 || it.m <= 3 * kTokTile)
    gateup_passes<CP, DT, (MT >= 3 ? 3 : 1), W, KS, CO, PRE>(a, it, p, owner, lds, bsh, sorted, pa, pb);
  else
    gateup_passes<CP, DT, MT, W, KS, CO, PRE>(a, it, p, owner, lds, bsh, sorted, pa, pb);
}

// The down workgroups of the single-launch layer (defined in layer1.hip, the one translation
// unit that instantiates gateup_kernel with FD). `stage`: LDS for the activation rows.
template <int DT, int RG, int W>
__device__ void layer_down_role(const ExpertArgs& a, u32x4* stage);

// kMulti: the launch may hold experts split into several token ranges (T > span). Their
// items load weights with normal caching (the ranges of a weight group read the same rows
// side by side); every other item streams with the non-temporal hint.
// RG > 0: the routing runs inside the launch (a.rt; RG lanes per token in the top-k): wave 0
// of every routed workgroup routes the batch into the workgroup's LDS (route_small_wave), the
// workgroup meets at a barrier and takes its work item and token rows from there; the first
// routed workgroup also writes the records (and the top-k results) the later kernels read.
// The shared-expert workgroups need no routing and start at once.
// RM: the larger in-launch form (up to kGateupSortMax assignments over E <= 64, T <= 64): the
// workgroup's 4 waves run the top-k (RG lanes per token; or load caller ids), then wave 0 sorts
// the assignments (sort_wave) into the workgroup's LDS; the first routed workgroup also
// writes the records and top-k results, and its threads the token mask.
// P: the workgroup walks the items b = blockIdx.x, + gridDim.x, ... < a.gu_items (a grid of at
// most one residency of the chip, for batches with more items than that): the routing (with
// RG > 0) is done once per workgroup, at the start, and every later item starts with its weight
// loads instead of a routing prologue under load. Every such workgroup routes; the first writes
// the records.
// KS: the K walk of every item is split between wave pairs (gateup_passes): a workgroup covers
// TW = 2 weight tiles instead of W.
// FD: the single-launch layer (a.ls, a.lo): workgroups from a.ls.gu_blocks on are the down
// workgroups of the fused down projection + combine (layer_down_role); the gate/up workgroups
// before them store their activation rows at device scope and, when every store of the
// workgroup has completed, publish a.ls.epoch in their flag. Items per workgroup, never per
// wave: every wave of a workgroup has the same role.
template <bool kMulti, int DT, int MT, int RG, bool RM = false, int W = kExpertWaves, bool P = false,
          bool KS = false, bool FD = false, bool ST = false>
__global__ __launch_bounds__(W * kWave, 2) void gateup_kernel(ExpertArgs a) {
  using S = typename Elem<DT>::S;
  constexpr int TW = KS ? 2 : W;  // weight tiles per workgroup
  static_assert(!FD || (RG > 0 && !RM && !P && !KS && MT == 1 && !kMulti),
                "the single-launch layer takes one token, routed inside the launch by one wave");
  static_assert(!ST || (RG > 0 && RM && !FD && !kMulti && W == kExpertWaves),
                "expert-ordered items: the multi-wave in-launch routing, 4-wave workgroups");
  static_assert(!ST || MT <= kExpertItemsMaxTiles, "expert-ordered items: at most two token tiles");
  __shared__ u32x4 lds_all[W][2 * kTileSlots];
  if constexpr (FD) {
    if (static_cast<int>(blockIdx.x) >= a.ls.gu_blocks) {
      layer_down_role<DT, RG, W>(a, &lds_all[0][0]);
      return;
    }
  }
  const int wave = wave_id();
  // routing: whether this workgroup has a routed item, and whether it writes the records
  const bool in_shared = P ? false : static_cast<int>(blockIdx.x) < a.sh.gateup_blocks;
  const bool writer_wg = P ? blockIdx.x == 0 : static_cast<int>(blockIdx.x) == a.sh.gateup_blocks;
  const int32_t* hdr = a.rb.hdr;
  const RangeRec* ranges = a.rb.ranges;
  const int32_t* sorted = a.rb.sorted_f;
  // ST: the workgroup's first item is known before the routing (expert_item): its first two
  // weight chunks are issued now, and the routing below runs while they are in flight. The
  // routing's own loads (caller ids -- one per thread: T*k <= 256 -- and the expert-to-slot
  // map) are issued before them: vector loads complete in issue order, so waiting for these
  // does not wait for the weights.
  [[maybe_unused]] int st_id = 0;
  [[maybe_unused]] int64_t st_slot = -1;
  [[maybe_unused]] Raw<2> pre_a, pre_b;
  [[maybe_unused]] bool pre = false;
  if constexpr (ST) {
    if (!in_shared) {
      const int tid = threadIdx.x;
      if (a.rt.logits == nullptr && tid < a.T * a.k) st_id = a.rt.ids_in[tid];
      if (tid < a.rt.E) st_slot = a.e2s[tid];
    }
    __builtin_amdgcn_sched_barrier(0);
    const int b0 = static_cast<int>(blockIdx.x);
    const int tiles = (b0 < a.sh.gateup_blocks ? a.sh.I : a.I) / kRowTile;
    WorkItem it0;
    pre = (!P || b0 < a.gu_items) &&
          expert_item<S, TW>(a, b0, a.sh.gateup_blocks, (tiles + TW - 1) / TW,
                             (tiles + kExpertWaves - 1) / kExpertWaves, it0, nullptr);
    // The loads are issued on every path (without a first item: from an empty buffer resource,
    // which returns zeros and reads nothing), so that every path has the same loads in flight
    // after the routing's: the waits for those then leave the weights outstanding.
    if (!pre) {
      it0.page = static_cast<const char*>(a.pool);
      it0.page_bytes = 0;
      it0.I = a.I;
      it0.rot = 0;
    }
    const int praw = pre ? it0.tg * TW + (KS ? wave & 1 : wave) : 0;
    WeightStream ws;
    ChunkOrder ord;
    gateup_stream<DT, KS>(a, it0, praw < tiles ? praw : tiles - 1, ws, ord);
    // both chunks on every path (a one-chunk walk loads chunk 0 twice and never uses pre_b)
    load_raw<kNonTemporal>(pre_a, ws, ord.at(0));
    load_raw<kNonTemporal>(pre_b, ws, ord.at(ord.n > 1 ? 1 : 0));
  }
  if constexpr (RG > 0 && RM) {
    __shared__ int16_t ids_l[kGateupSortMax];
    __shared__ int64_t slot_l[kWave];
    __shared__ SortWaveLds sw;
    __shared__ RangeRec rr_l[kSortRangesMax];
    __shared__ int32_t sf_l[kGateupSortMax];
    __shared__ int32_t hdr_l[4];
    __shared__ int32_t cnt_l[kWave];       // own-range form: routable assignments per expert
    __shared__ int32_t wcnt_l[kExpertWaves];
    __shared__ int32_t me_l, j_l;
    if (!in_shared) {
      const int lane = lane_id();
      const int tid = threadIdx.x;
      const int N = a.T * a.k;
      const int E = a.rt.E;
      const bool writer = writer_wg;
      const int64_t my_slot = ST ? st_slot : (tid < E ? a.e2s[tid] : -1);
      if (tid < kWave) cnt_l[tid] = 0;
      if (tid == 0) me_l = -1;
      auto keep = [&](int t, int slot, float wv, int id) {
        const int f = t * a.k + slot;
        if (writer) {
          a.rt.w_out[f] = wv;
          a.rt.ids_out[f] = id;
        }
        ids_l[f] = static_cast<int16_t>(id);
      };
      if (a.rt.logits != nullptr) {
        constexpr int TPW = TopkGroup<RG, 1>::kTokens;
        const int stride = W * TPW;
        for (int t0 = wave * TPW + lane / RG; t0 - lane / RG < a.T; t0 += stride * kTokBatch)
          topk_batch<DT, RG, 1>(a.rt.logits, a.T, E, a.k, a.rt.renorm != 0, t0, stride, keep);
      } else if constexpr (ST) {
        if (tid < N) ids_l[tid] = static_cast<int16_t>((st_id >= 0 && st_id < E) ? st_id : -2);
      } else {
        for (int f = tid; f < N; f += W * kWave) {
          const int x = a.rt.ids_in[f];
          ids_l[f] = static_cast<int16_t>((x >= 0 && x < E) ? x : -2);
        }
      }
      if (tid < kWave) slot_l[tid] = (my_slot >= 0 && my_slot < a.rt.num_slots) ? my_slot : -1;
      __syncthreads();
      if (writer) {
        for (int t = tid; t < a.T; t += W * kWave) {
          uint32_t m = 0;
          for (int j = 0; j < a.k; ++j) {
            const int e = ids_l[t * a.k + j];
            if (e >= 0 && slot_l[e] >= 0) m |= 1u << j;
          }
          a.rb.tmask[t] = static_cast<int32_t>(m);
        }
      }
      if (P || writer) {
        // the whole sort: the writer's records are the later kernels', and a walking workgroup
        // takes several items
        if (wave == 0) {
          AlignOutputs g{}, l{};
          g.span = a.rb.span;
          l.hdr = hdr_l;
          l.ranges = rr_l;
          l.sorted_f = sf_l;
          l.by_expert = ST;
          if (writer) {
            g.hdr = a.rb.hdr;
            g.ranges = a.rb.ranges;
            g.sorted_f = a.rb.sorted_f;
            g.fpos = a.rb.fpos;
            g.fslot = a.rb.fpos ? a.rb.fslot : nullptr;
          }
          sort_wave<true>(ids_l, slot_l, N, E, sw, g, l);
        }
      } else {
        // Own-range form: only the record of this workgroup's range j and its expert's sorted
        // assignments -- the values sort_wave gives them (counts of routable assignments per
        // expert, exclusive scans over the experts, the expert's assignments in ascending f).
        // ST: j is the expert (expert-ordered items), its record kept even when it is empty.
        for (int f = tid; f < N; f += W * kWave) {
          const int e = ids_l[f];
          if (e >= 0 && slot_l[e] >= 0) atomicAdd(&cnt_l[e], 1);
        }
        __syncthreads();
        const int span = a.rb.span;
        const int groups = (a.I / kRowTile + TW - 1) / TW;
        if (wave == 0) {
          const int c = lane < E ? cnt_l[lane] : 0;
          const int nr = div_small(c + span - 1, span, 1.0f / static_cast<float>(span));
          const int act = c > 0 ? 1 : 0;
          const int ic = wave_incl_scan(c), ia = wave_incl_scan(act), ir = wave_incl_scan(nr);
          const int j = (static_cast<int>(blockIdx.x) - a.sh.gateup_blocks) / groups;
          if (ST ? lane == j : (c > 0 && j >= ir - nr && j < ir)) {
            RangeRec rec{};
            rec.slot = slot_l[lane];
            rec.off = ic - c;
            rec.cnt = c;
            rec.key = lane;
            rec.j0 = ir - nr;
            rec.nr = nr;
            rr_l[j] = rec;  // j < the launch's range bound (ST: j < E) <= kSortRangesMax
            if (c > 0) me_l = lane;
          }
          if (lane == kWave - 1) {
            hdr_l[0] = ir;
            hdr_l[kHdrSingleRanges] = ir == ia ? 1 : 0;
            j_l = j;
          }
        }
        __syncthreads();
        const int me = me_l;
        if (me >= 0) {
          const int off = rr_l[j_l].off;
          const uint64_t below = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
          int base = off;
          for (int f0 = 0; f0 < N; f0 += W * kWave) {
            const int f = f0 + tid;
            const bool hit = f < N && ids_l[f] == me;
            const uint64_t m = ballot(hit);
            if (lane == 0) wcnt_l[wave] = __popcll(m);
            __syncthreads();
            int before = base, total = base;
            for (int w = 0; w < W; ++w) {
              const int n = wcnt_l[w];
              if (w < wave) before += n;
              total += n;
            }
            if (hit) sf_l[before + __popcll(m & below)] = f;
            base = total;
            __syncthreads();
          }
        }
      }
      __syncthreads();
      hdr = hdr_l;
      ranges = rr_l;
      sorted = sf_l;
    }
    if constexpr (ST) {
      // the routed items read only these LDS tables (shared items read neither): as LDS
      // pointers on every path their reads wait for LDS alone, not for the weights in flight
      ranges = rr_l;
      sorted = sf_l;
    }
  } else if constexpr (RG > 0) {
    __shared__ SmallRouteLds sc;
    __shared__ RangeRec rr_l[kSmallRangesMax];
    __shared__ int32_t sf_l[kWave];
    __shared__ int32_t hdr_l[4];
    if (!in_shared) {
      if (wave == 0) {
        SmallRouteOut g, l;
        l.hdr = hdr_l;
        l.ranges = rr_l;
        l.sorted_f = sf_l;
        if (writer_wg) {
          g.w = a.rt.w_out;
          g.ids = a.rt.ids_out;
          g.hdr = a.rb.hdr;
          g.ranges = a.rb.ranges;
          g.sorted_f = a.rb.sorted_f;
          g.tmask = a.rb.tmask;
          g.fpos = a.rb.fpos;
          g.fslot = a.rb.fpos ? a.rb.fslot : nullptr;
        }
        route_small_wave<DT, RG>(a.rt.logits, a.T, a.rt.E, a.k, a.rt.renorm, a.rt.ids_in, a.e2s,
                                 a.rt.num_slots, a.rb.span, sc, g, l);
      }
      __syncthreads();
      hdr = hdr_l;
      ranges = rr_l;
      sorted = sf_l;
    }
  }
  __shared__ u32x4 bsh[(KS ? 4 : 2) * MT * kTileSlots];
  u32x4* lds = lds_all[wave];
  const int nitems = P ? a.gu_items : static_cast<int>(blockIdx.x) + 1;
  int b_first = blockIdx.x;
  if constexpr (ST) {
    // The first item, its weights in flight since before the routing (pre is false only for a
    // workgroup whose first item is empty: past the items, or an expert without a valid slot,
    // which the routing gives no tokens). Peeled off the walk so that pre_a and pre_b are dead
    // after it.
    b_first += gridDim.x;
    if (pre) {
      const int b = blockIdx.x;
      const int tiles = (b < a.sh.gateup_blocks ? a.sh.I : a.I) / kRowTile;
      WorkItem it;
      if (expert_item<S, TW>(a, b, a.sh.gateup_blocks, (tiles + TW - 1) / TW,
                             (tiles + kExpertWaves - 1) / kExpertWaves, it, ranges)) {
        const int praw = it.tg * TW + (KS ? wave & 1 : wave);
        const bool owner = praw < tiles;
        gateup_item<kNonTemporal, DT, MT, W, KS, FD, true>(a, it, owner ? praw : tiles - 1, owner, lds,
                                                           bsh, sorted, &pre_a, &pre_b);
      }
    }
  }
  for (int b = b_first; b < nitems; b += gridDim.x) {
    const int Iw = b < a.sh.gateup_blocks ? a.sh.I : a.I;
    const int tiles = Iw / kRowTile;
    const int groups = (tiles + TW - 1) / TW;
    const int groups4 = (tiles + kExpertWaves - 1) / kExpertWaves;
    WorkItem it;
    // XCD order only with the routing kernel's records (inside the launch it measured slower:
    // DeepSeek-V2-Lite 32 tokens 175.8 -> 177.0 us, Qwen1.5-MoE 32 tokens 162.4 -> 163.8)
    if constexpr (ST) {
      if (!expert_item<S, TW>(a, b, a.sh.gateup_blocks, groups, groups4, it, ranges)) continue;
    } else if (!work_item<S, TW, RG == 0>(a, b, a.sh.gateup_blocks, groups, groups4, it, hdr, ranges)) {
      continue;
    }
    const int praw = it.tg * TW + (KS ? wave & 1 : wave);
    const bool owner = praw < tiles;
    const int p = owner ? praw : tiles - 1;
    if (kMulti && it.nr > 1) gateup_item<0, DT, MT, W, KS, FD>(a, it, p, owner, lds, bsh, sorted);
    else gateup_item<kNonTemporal, DT, MT, W, KS, FD>(a, it, p, owner, lds, bsh, sorted);
  }
  if constexpr (FD) {
    // Publication: every wave's stores have completed (at device scope: store4_agent), then
    // the workgroup meets, then one store of the flag. A workgroup without an item publishes
    // too: the down workgroups wait for every flag.
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __syncthreads();
    if (threadIdx.x == 0 && a.ls.publish)
      __hip_atomic_store(a.ls.flags + blockIdx.x, a.ls.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}


}  // namespace smx
