// Expert kernels of the verify-step MoE: weight-streaming grouped SwiGLU on MFMA.
//
// At verify-step token counts every routed expert sees few tokens, so the expert weights
// are the only large operand: each weight byte is read from HBM exactly once, by one wave,
// with 16-byte-per-lane loads of 4 rows x 256 bytes transposed through LDS into MFMA A
// fragments, and the few token rows ride along as the B operand (L2-resident). The MFMA
// makes the flops free, so the kernels run at the rate weights stream in.
//
//   gateup_kernel   wave = (token range of an active expert, 16 intermediate columns):
//                   streams the 16 matching rows of W1 (gate) and W3 (up) over K = H, then
//                   fuses the epilogue act = round(silu(round(gate)) * round(up)) into `act`
//                   (row = sorted position).
//   down_kernel     wave = (token range, 32 rows of W2, K split): streams W2 over its K slice
//                   of I and writes fp32 partials part[split][f][h].
//   combine_kernel  y[t] = round(sum_j round(w[t,j] * sum_split part[split][t*k+j])), one wave
//                   per assignment of a token (and one for the shared expert's partials).
//
// Arithmetic and rounding points follow stack_fused_moe
// (specmoe/layers/fused_moe_kernel.py:319-349): C1 rounded to the activation dtype (:203),
// silu_and_mul (:337), the down GEMM scaled by the routing weight before rounding (:197-203),
// and the fp32 top-k sum rounded once (:344-347).
#include <atomic>
#include <type_traits>

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
template <int CP, int DT, int MT, int W, bool KS = false>
__device__ __forceinline__ void gateup_passes(const ExpertArgs& a, const WorkItem& it, int p,
                                              bool owner, u32x4* lds, u32x4* bsh,
                                              const int32_t* sorted) {
  using S = typename Elem<DT>::S;
  static_assert(!KS || W == kExpertWaves, "the K split pairs the waves of a 4-wave workgroup");
  constexpr int WT = KS ? 2 : W;  // waves sharing one token stage
  const int lane = lane_id();
  const int wave = wave_id();
  const int h = KS ? wave >> 1 : 0;     // K half
  const int wv = KS ? wave & 1 : wave;  // index among the waves of the token stage
  const int r = lane & 15, g = lane >> 4;
  const int H = a.H, I = it.I, off = it.off, m = it.m;
  const int64_t row_bytes = static_cast<int64_t>(H) * sizeof(S);
  WeightStream ws;  // tile 0: gate rows [16p, 16p+16); tile 1: the matching up rows
  ws.rsrc = make_rsrc(it.page, static_cast<uint32_t>(it.page_bytes));
  ws.base = static_cast<uint32_t>(kRowTile * p * row_bytes);
  ws.tile_stride = static_cast<uint32_t>(I * row_bytes);
  ws.row4 = static_cast<uint32_t>(4 * row_bytes);
  ws.lane_off = static_cast<uint32_t>((lane >> 4) * row_bytes + (lane & 15) * 16);
  const int nch = static_cast<int>(row_bytes / (kStepBytes * kUnroll));
  ChunkOrder ord = rotated_order(KS ? nch / 2 : nch, it.rot);
  ord.base = h * ord.n;
  u32x4* stage = bsh + h * 2 * MT * kTileSlots;
  S* act = static_cast<S*>(it.shared ? a.sh.act : a.act);
  const int f16out = it.shared ? 0 : a.f16out;
  const float rk = 1.0f / static_cast<float>(a.k);  // flat assignment f -> token f / k
  for (int q0 = 0; q0 < m; q0 += kTokTile * MT) {
    Raw<2> wa, wb;
    issue_weights<CP>(wa, wb, ws, ord);
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
        store4<DT>(act, static_cast<int64_t>(off + q) * I + kRowTile * p + 4 * g, o[0], o[1], o[2], o[3]);
      }
    }
  }
}

// Workgroup = (work item, W consecutive weight tiles): wave w owns tile W*tg + w. A wave
// past the expert's last tile streams the last tile again and stores nothing, so every
// wave of a workgroup runs the same chunks and barriers. The token tiles per pass follow
// the item's token count (up to MT): an expert with few tokens streams its weights with
// one tile of 16 tokens.
template <int CP, int DT, int MT, int W, bool KS = false>
__device__ __forceinline__ void gateup_item(const ExpertArgs& a, const WorkItem& it, int p,
                                            bool owner, u32x4* lds, u32x4* bsh,
                                            const int32_t* sorted) {
  if (MT == 1 || it.m <= kTokTile) gateup_passes<CP, DT, 1, W, KS>(a, it, p, owner, lds, bsh, sorted);
  else if (MT == 2 || it.m <= 2 * kTokTile) gateup_passes<CP, DT, (MT >= 2 ? 2 : 1), W, KS>(a, it, p, owner, lds, bsh, sorted);
  else if (MT == 3 || it.m <= 3 * kTokTile) gateup_passes<CP, DT, (MT >= 3 ? 3 : 1), W, KS>(a, it, p, owner, lds, bsh, sorted);
  else gateup_passes<CP, DT, MT, W, KS>(a, it, p, owner, lds, bsh, sorted);
}

// kMulti: the launch may hold experts split into several token ranges (T > span). Their
// items load weights with normal caching (the ranges of a weight group read the same rows
// side by side); every other item streams with the non-temporal hint.
// RG > 0: the routing runs inside the launch (a.rt; RG lanes per token in the top-k): wave 0
// of every routed workgroup routes the batch into the workgroup's LDS (route_small_wave), the
// workgroup meets at a barrier and takes its work item and token rows from there; the first
// routed workgroup also writes the records (and the top-k results) the later kernels read.
// The shared-expert workgroups need no routing and start at once.
// RM: the larger in-launch form (up to kSortWaveMax assignments over E <= 64, T <= 64): the
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
template <bool kMulti, int DT, int MT, int RG, bool RM = false, int W = kExpertWaves, bool P = false,
          bool KS = false>
__global__ __launch_bounds__(W * kWave, 2) void gateup_kernel(ExpertArgs a) {
  constexpr int TW = KS ? 2 : W;  // weight tiles per workgroup
  const int wave = wave_id();
  // routing: whether this workgroup has a routed item, and whether it writes the records
  const bool in_shared = P ? false : static_cast<int>(blockIdx.x) < a.sh.gateup_blocks;
  const bool writer_wg = P ? blockIdx.x == 0 : static_cast<int>(blockIdx.x) == a.sh.gateup_blocks;
  const int32_t* hdr = a.rb.hdr;
  const RangeRec* ranges = a.rb.ranges;
  const int32_t* sorted = a.rb.sorted_f;
  if constexpr (RG > 0 && RM) {
    __shared__ int16_t ids_l[kSortWaveMax];
    __shared__ int64_t slot_l[kWave];
    __shared__ SortWaveLds sw;
    __shared__ RangeRec rr_l[kSortRangesMax];
    __shared__ int32_t sf_l[kSortWaveMax];
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
      const int64_t my_slot = tid < E ? a.e2s[tid] : -1;
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
          if (c > 0 && j >= ir - nr && j < ir) {
            RangeRec rec{};
            rec.slot = slot_l[lane];
            rec.off = ic - c;
            rec.cnt = c;
            rec.key = ia - act;
            rec.j0 = ir - nr;
            rec.nr = nr;
            rr_l[j] = rec;  // j < the launch's range bound <= kSortRangesMax
            me_l = lane;
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
  __shared__ u32x4 lds_all[W][2 * kTileSlots];
  __shared__ u32x4 bsh[(KS ? 4 : 2) * MT * kTileSlots];
  u32x4* lds = lds_all[wave];
  const int nitems = P ? a.gu_items : static_cast<int>(blockIdx.x) + 1;
  for (int b = blockIdx.x; b < nitems; b += gridDim.x) {
    const int Iw = b < a.sh.gateup_blocks ? a.sh.I : a.I;
    const int tiles = Iw / kRowTile;
    const int groups = (tiles + TW - 1) / TW;
    const int groups4 = (tiles + kExpertWaves - 1) / kExpertWaves;
    WorkItem it;
    // XCD order only with the routing kernel's records (inside the launch it measured slower:
    // DeepSeek-V2-Lite 32 tokens 175.8 -> 177.0 us, Qwen1.5-MoE 32 tokens 162.4 -> 163.8)
    if (!work_item<typename Elem<DT>::S, TW, RG == 0>(a, b, a.sh.gateup_blocks, groups, groups4, it, hdr,
                                                     ranges))
      continue;
    const int praw = it.tg * TW + (KS ? wave & 1 : wave);
    const bool owner = praw < tiles;
    const int p = owner ? praw : tiles - 1;
    if (kMulti && it.nr > 1) gateup_item<0, DT, MT, W, KS>(a, it, p, owner, lds, bsh, sorted);
    else gateup_item<kNonTemporal, DT, MT, W, KS>(a, it, p, owner, lds, bsh, sorted);
  }
}

// The token passes of one down workgroup with MT token tiles per pass: wave `wave` owns W2
// rows [32*rt, 32*rt + 32) over the K slice of split sp.
template <int CP, int DT, int MT, int R>
__device__ __forceinline__ void down_passes(const ExpertArgs& a, const WorkItem& it, int rt,
                                            bool owner, int sp, int split_steps, u32x4* lds,
                                            u32x4* bsh) {
  using S = typename Elem<DT>::S;
  const int lane = lane_id();
  const int wave = wave_id();
  const int r = lane & 15, g = lane >> 4;
  const int H = a.H, I = it.I, off = it.off, m = it.m;
  const int rows = it.shared ? a.T : a.T * a.k;  // rows of act and of one split of part
  const int64_t row_bytes = static_cast<int64_t>(I) * sizeof(S);
  const int64_t k0_bytes = static_cast<int64_t>(sp) * split_steps * kStepBytes;
  WeightStream ws;  // tiles: rows [(rt*R + i)*16, +16) of W2 (after W1, W3), this split's K slice
  ws.rsrc = make_rsrc(it.page, static_cast<uint32_t>(it.page_bytes));
  ws.base = static_cast<uint32_t>(2 * H * row_bytes + rt * R * kRowTile * row_bytes + k0_bytes);
  ws.tile_stride = static_cast<uint32_t>(kRowTile * row_bytes);
  ws.row4 = static_cast<uint32_t>(4 * row_bytes);
  ws.lane_off = static_cast<uint32_t>((lane >> 4) * row_bytes + (lane & 15) * 16);
  const void* act = it.shared ? a.sh.act : a.act;
  float* part = it.shared ? a.sh.part : a.part;
  const ChunkOrder ord{split_steps / kUnroll, 0};
  for (int q0 = 0; q0 < m; q0 += kTokTile * MT) {
    Raw<R> wa, wb;
    issue_weights<CP>(wa, wb, ws, ord);
    SharedTokens<MT, kExpertWaves> tb;
    tb.rsrc = make_rsrc(act, static_cast<uint32_t>(static_cast<int64_t>(rows) * row_bytes));
    tb.base = static_cast<uint32_t>(k0_bytes);
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      const int q = min(q0 + j * kTokTile + 4 * wave + (lane >> 4), m - 1);
      tb.off[j][0] = static_cast<uint32_t>((off + q) * row_bytes + (lane & 15) * 16);
    }
    f32x4 acc[R][MT];
#pragma unroll
    for (int i = 0; i < R; ++i)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[i][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    stream_wg<CP, DT, R, MT, kExpertWaves>(ws, tb, ord, lds, bsh, acc, wa, wb, wave);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int q = q0 + mt * kTokTile + r;
      if (owner && q < m) {
        const int f = it.shared ? off + q : a.rb.sorted_f[off + q];
        float* dst = part + (static_cast<int64_t>(sp) * rows + f) * H;
#pragma unroll
        for (int i = 0; i < R; ++i)
          *reinterpret_cast<f32x4*>(dst + (rt * R + i) * kRowTile + 4 * g) = acc[i][mt];
      }
    }
  }
}

// Workgroup = (work item, K split, 4 consecutive pairs of W2 row tiles): wave w owns rows
// [32*(4*group + w), +32). Waves past the last pair repeat it and store nothing. Token tiles
// per pass as in gateup_kernel.
template <int CP, int DT, int MT, int R>
__device__ __forceinline__ void down_item(const ExpertArgs& a, const WorkItem& it, int rt,
                                          bool owner, int sp, int split_steps, u32x4* lds,
                                          u32x4* bsh) {
  if (MT == 1 || it.m <= kTokTile) down_passes<CP, DT, 1, R>(a, it, rt, owner, sp, split_steps, lds, bsh);
  else if (MT == 2 || it.m <= 2 * kTokTile) down_passes<CP, DT, (MT >= 2 ? 2 : 1), R>(a, it, rt, owner, sp, split_steps, lds, bsh);
  else if (MT == 3 || it.m <= 3 * kTokTile) down_passes<CP, DT, (MT >= 3 ? 3 : 1), R>(a, it, rt, owner, sp, split_steps, lds, bsh);
  else down_passes<CP, DT, MT, R>(a, it, rt, owner, sp, split_steps, lds, bsh);
}

// R: W2 row tiles per wave (kDownRows; 1 doubles the workgroups of a grid too small to fill
// the chip).
template <bool kMulti, int DT, int MT, int R = kDownRows>
__global__ __launch_bounds__(kExpertThreads, 2) void down_kernel(ExpertArgs a) {
  const int wave = wave_id();
  const int rtiles = a.H / (kRowTile * R);
  const int groups = (rtiles + kExpertWaves - 1) / kExpertWaves;
  const bool in_shared = static_cast<int>(blockIdx.x) < a.sh.down_blocks;
  const int splits = in_shared ? a.sh.splits : a.splits;
  const int split_steps = in_shared ? a.sh.split_steps : a.split_steps;
  WorkItem it;
  if (!work_item<typename Elem<DT>::S, true>(a, a.sh.down_blocks, groups * splits, it, a.rb.hdr, a.rb.ranges))
    return;
  const int sp = div_small(it.tg, groups, 1.0f / static_cast<float>(groups));
  const int tg = it.tg - sp * groups;
  const int rtraw = tg * kExpertWaves + wave;
  const bool owner = rtraw < rtiles;
  const int rt = owner ? rtraw : rtiles - 1;
  __shared__ u32x4 lds_all[kExpertWaves][R * kTileSlots];
  __shared__ u32x4 bsh[2 * MT * kTileSlots];
  u32x4* lds = lds_all[wave];
  if (kMulti && it.nr > 1) down_item<0, DT, MT, R>(a, it, rt, owner, sp, split_steps, lds, bsh);
  else down_item<kNonTemporal, DT, MT, R>(a, it, rt, owner, sp, split_steps, lds, bsh);
}

__device__ __forceinline__ float load_scalar(const void* base, int dtype, int64_t i) {
  switch (dtype) {
    case kF32: return load_as_f32<kF32>(base, i);
    case kF16: return load_as_f32<kF16>(base, i);
    default: return load_as_f32<kBF16>(base, i);
  }
}

constexpr int kCombineBatch = 8;        // split loads in flight per lane
constexpr int kCombineMaxWaves = 16;

// Sum over the splits of one partial row segment (4 outputs per lane), in split order.
__device__ __forceinline__ f32x4 split_sum(const float* src, int64_t split_stride, int splits) {
  f32x4 v = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < splits; s0 += kCombineBatch) {
    f32x4 a[kCombineBatch];
#pragma unroll
    for (int u = 0; u < kCombineBatch; ++u)
      a[u] = s0 + u < splits ? *reinterpret_cast<const f32x4*>(src + (s0 + u) * split_stride)
                             : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < kCombineBatch; ++u)
      if (s0 + u < splits) v += a[u];
  }
  return v;
}

// Workgroup = (token t, 256 consecutive outputs: lane l owns outputs 4l..4l+3 of the chunk).
// Work item i < k is assignment t*k + i: its splits are summed in split order and the term
// round(w * sum) goes to LDS; item k (block form with a shared expert) is the shared
// expert's split sum. Wave w takes items w, w + waves, ... Wave 0 then adds the k terms in
// j order (y = round(sum_j term_j), deterministic) and applies the block form
// y = round(round(round(y) * scale) + s * round(shared)) with s = 1 or
// round(sigmoid(gate logit)) and the product rounded, as the unfused block computes it.
template <int DT>
__global__ __launch_bounds__(kCombineMaxWaves * kWave) void combine_kernel(CombineArgs c) {
  __shared__ f32x4 terms[kMaxTopK + 1][kWave];
  const int lane = lane_id();
  const int wave = wave_id();
  const int waves = blockDim.x / kWave;
  const int chunks = (c.H + 4 * kWave - 1) / (4 * kWave);
  const int t = blockIdx.x / chunks;
  const int h = ((blockIdx.x - t * chunks) * kWave + lane) * 4;
  const bool live = h < c.H;
  const uint32_t vm = static_cast<uint32_t>(c.tmask[t]);
  const int items = c.k + (c.part_s != nullptr ? 1 : 0);
  // the shared-expert gate logit, loaded with everything else (used by wave 0 at the end)
  const bool gated = c.block && c.part_s != nullptr && c.sgate != nullptr;
  const float z = gated && wave == 0 ? load_scalar(c.sgate, c.sgate_dtype, t) : 0.0f;
  for (int i = wave; i < items; i += waves) {
    f32x4 term = {0.f, 0.f, 0.f, 0.f};
    if (i < c.k) {
      // The partials and the weight are loaded together with the token's mask (no dependent
      // round trip); a dropped assignment's rows were not written by this call and are
      // discarded by the select below.
      if (live) {
        const int64_t f = static_cast<int64_t>(t) * c.k + i;
        const f32x4 v = split_sum(c.part + f * c.H + h, static_cast<int64_t>(c.T) * c.k * c.H, c.splits);
        const float wf = c.w[f];
        const bool routed = (vm >> i) & 1u;
#pragma unroll
        for (int e = 0; e < 4; ++e) term[e] = routed ? round_out<DT>(v[e] * wf, c.f16out) : 0.0f;
      }
    } else if (live) {
      term = split_sum(c.part_s + static_cast<int64_t>(t) * c.H + h, static_cast<int64_t>(c.T) * c.H, c.splits_s);
    }
    terms[i][lane] = term;
  }
  __syncthreads();
  if (wave != 0 || !live) return;
  f32x4 y = {0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < c.k; ++j)
    if ((vm >> j) & 1u) y += terms[j][lane];
  if (c.block) {
    const bool scaled = c.scale != 1.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      y[e] = Elem<DT>::round(y[e]);
      if (scaled) y[e] = Elem<DT>::round(y[e] * c.scale);
    }
    if (c.part_s) {
      const f32x4 d = terms[c.k][lane];
      float gs = 1.0f;
      if (gated) gs = Elem<DT>::round(1.0f / (1.0f + __expf(-z)));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float sh = Elem<DT>::round(d[e]);
        if (gated) sh = Elem<DT>::round(gs * sh);
        y[e] += sh;
      }
    }
  }
  store4<DT>(c.y, static_cast<int64_t>(t) * c.H + h, y[0], y[1], y[2], y[3]);
}

// Combine for large batches: one thread per 8 consecutive outputs of a token, every
// assignment of the token (and the shared expert) summed in the same order as combine_kernel
// -- splits in order from 0, then round(w * sum) added over j in order, then the block form --
// so both kernels give identical bits. No LDS or barriers; at thousands of tokens the
// per-(token, 256 outputs) workgroups of combine_kernel are bound by workgroup dispatch.
constexpr int kCombineRowThreads = 256;
constexpr int kCombineRowOuts = 8;
constexpr int kCombineRowBatch = 8;  // assignments whose partials are loaded together

template <int DT>
__global__ __launch_bounds__(kCombineRowThreads) void combine_rows_kernel(CombineArgs c) {
  // thread g owns outputs [8g, 8g + 8): token g / (H/8); T*H/8 < 2^31 (one chunk of the call)
  const int per_t = c.H / kCombineRowOuts;
  const int g = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
  if (g >= c.T * per_t) return;
  const int t = c.T * per_t < (1 << 23) ? div_small(g, per_t, 1.0f / static_cast<float>(per_t)) : g / per_t;
  const int h = (g - t * per_t) * kCombineRowOuts;
  const int64_t idx = static_cast<int64_t>(t) * c.H + h;
  const int64_t split_stride = static_cast<int64_t>(c.T) * c.k * c.H;
  // The token's gate logit and its shared-expert partials of the first two splits are loaded
  // first, with the routed partials of the first split, so that the thread waits for one round
  // of loads per routed split (not one per assignment, nor another for the shared expert's).
  // Without a shared expert the same loads read a routed row (in bounds) and are unused.
  const bool shared = c.block && c.part_s != nullptr;
  const bool gated = shared && c.sgate != nullptr;
  const float zs = gated ? load_scalar(c.sgate, c.sgate_dtype, t) : 0.0f;
  const int64_t sstride = static_cast<int64_t>(c.T) * c.H;
  const float* ssrc = shared ? c.part_s + static_cast<int64_t>(t) * c.H + h
                             : c.part + static_cast<int64_t>(t) * c.k * c.H + h;
  const int64_t s1 = shared && c.splits_s > 1 ? sstride : 0;
  const f32x4 ps0a = *reinterpret_cast<const f32x4*>(ssrc);
  const f32x4 ps0b = *reinterpret_cast<const f32x4*>(ssrc + 4);
  const f32x4 ps1a = *reinterpret_cast<const f32x4*>(ssrc + s1);
  const f32x4 ps1b = *reinterpret_cast<const f32x4*>(ssrc + s1 + 4);
  const uint32_t vm = static_cast<uint32_t>(c.tmask[t]);
  f32x4 y0 = {0.f, 0.f, 0.f, 0.f}, y1 = {0.f, 0.f, 0.f, 0.f};
  // kCombineRowBatch assignments at a time: their weights and partials (from clamped j, in
  // bounds: every row f = t*k + j of part exists) are loaded together, then summed over the
  // splits in split order and added over j in order -- the arithmetic of combine_kernel.
  for (int j0 = 0; j0 < c.k; j0 += kCombineRowBatch) {
    const float* src0 = c.part + (static_cast<int64_t>(t) * c.k) * c.H + h;
    float wf[kCombineRowBatch];
    f32x4 v0[kCombineRowBatch], v1[kCombineRowBatch];
#pragma unroll
    for (int jj = 0; jj < kCombineRowBatch; ++jj) {
      const int j = min(j0 + jj, c.k - 1);
      wf[jj] = c.w[static_cast<int64_t>(t) * c.k + j];
      v0[jj] = f32x4{0.f, 0.f, 0.f, 0.f};
      v1[jj] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    for (int sp = 0; sp < c.splits; ++sp) {
      f32x4 a0[kCombineRowBatch], a1[kCombineRowBatch];
#pragma unroll
      for (int jj = 0; jj < kCombineRowBatch; ++jj) {
        const int j = min(j0 + jj, c.k - 1);
        const float* src = src0 + static_cast<int64_t>(j) * c.H + sp * split_stride;
        a0[jj] = *reinterpret_cast<const f32x4*>(src);
        a1[jj] = *reinterpret_cast<const f32x4*>(src + 4);
      }
      __builtin_amdgcn_sched_barrier(0);  // every load of the split issued before the first add
#pragma unroll
      for (int jj = 0; jj < kCombineRowBatch; ++jj) {
        v0[jj] += a0[jj];
        v1[jj] += a1[jj];
      }
    }
#pragma unroll
    for (int jj = 0; jj < kCombineRowBatch; ++jj) {
      const int j = j0 + jj;
      if (j < c.k && ((vm >> j) & 1u)) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          y0[e] += round_out<DT>(v0[jj][e] * wf[jj], c.f16out);
          y1[e] += round_out<DT>(v1[jj][e] * wf[jj], c.f16out);
        }
      }
    }
  }
  if (c.block) {
    const bool scaled = c.scale != 1.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      y0[e] = Elem<DT>::round(y0[e]);
      y1[e] = Elem<DT>::round(y1[e]);
      if (scaled) {
        y0[e] = Elem<DT>::round(y0[e] * c.scale);
        y1[e] = Elem<DT>::round(y1[e] * c.scale);
      }
    }
    if (shared) {
      f32x4 d0 = {0.f, 0.f, 0.f, 0.f}, d1 = {0.f, 0.f, 0.f, 0.f};
      d0 += ps0a;
      d1 += ps0b;
      if (c.splits_s > 1) {
        d0 += ps1a;
        d1 += ps1b;
      }
      for (int sp = 2; sp < c.splits_s; ++sp) {
        d0 += *reinterpret_cast<const f32x4*>(ssrc + sp * sstride);
        d1 += *reinterpret_cast<const f32x4*>(ssrc + sp * sstride + 4);
      }
      float gs = 1.0f;
      if (gated) gs = Elem<DT>::round(1.0f / (1.0f + __expf(-zs)));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float s0 = Elem<DT>::round(d0[e]), s1 = Elem<DT>::round(d1[e]);
        if (gated) {
          s0 = Elem<DT>::round(gs * s0);
          s1 = Elem<DT>::round(gs * s1);
        }
        y0[e] += s0;
        y1[e] += s1;
      }
    }
  }
  store4<DT>(c.y, idx, y0[0], y0[1], y0[2], y0[3]);
  store4<DT>(c.y, idx + 4, y1[0], y1[1], y1[2], y1[3]);
}

// ---------------------------------------------------------------------------------------
// Down projection fused with the combine, for batches of a few tokens. One wave per output
// row h computes every term of y[:, h] -- the dot of W2 row h of each routed assignment's
// expert with that assignment's activation row (and, in the block form, of the shared
// expert's W2 row h with the token's shared activation row) -- and lanes 0..T-1 then apply
// the combine's arithmetic and store y[t, h]. No fp32 partials are written and no combine
// kernel runs. A wave's terms form one stream of 1 KB units (16 bytes per lane of the weight
// row and of the activation row), kRowsDepth units in flight across term boundaries; each row
// of an active expert's W2 is read by one wave.
// Terms run in sorted-position order (an expert's tokens back to back: a row that several
// tokens need is read from HBM once and then from L2), then the shared expert's T rows.
// Arithmetic: term = round(w * dot) per routed assignment, summed in j order; block form as
// combine_kernel. The dot runs in fp32 over the lane's elements in K order, then a fixed
// reduction across lanes (DPP steps within rows of 16, then the four row sums).
// Units in flight per wave, measured on the DeepSeek-V2-Lite block at one token (us per
// layer): 2: 34.5, 3: 32.9, 4: 32.4, 6: 33.0, 8: 33.3, 12: 34.3, 16: 36.4, 24: 37.3 (the split
// down kernel + combine: 37.1). 2 or 4 waves per row taking interleaved units, and a cursor
// stepping over several units at once, were 4-6 us slower.
// ---------------------------------------------------------------------------------------
constexpr int kRowsWaves = 4;                                   // rows (waves) per workgroup
constexpr int kRowsDepth = 4;                                   // units in flight per wave
constexpr int kRowsUnit = kWave * 16;                           // bytes per unit
constexpr int kRowsMaxAssign = kRowsMaxTokens * kMaxTopK;
constexpr int kRowsMaxTerms = kRowsMaxAssign + kRowsMaxTokens;
static_assert(kRowsUnit == kRowsUnitBytes, "unit size of the host-side rule");

struct RowTerm {
  uint64_t w;   // byte address of row 0 of the term's W2
  uint64_t a;   // byte address of the term's activation row
  int rowb;     // bytes per row
  int units;    // kRowsUnit units per row
};

// Wave-uniform position in the term stream: term, unit within it, and the term's row.
struct RowCursor {
  int tau, u, rowb, units;
  uint64_t w, a;
};

__device__ __forceinline__ void row_cursor_at(RowCursor& c, const RowTerm* terms, int tau, int h) {
  const RowTerm& r = terms[tau];
  c.tau = tau;
  c.u = 0;
  c.rowb = uniform(r.rowb);
  c.units = uniform(r.units);
  c.w = static_cast<uint64_t>(uniform64(static_cast<int64_t>(r.w))) +
        static_cast<uint64_t>(h) * static_cast<uint64_t>(c.rowb);
  c.a = static_cast<uint64_t>(uniform64(static_cast<int64_t>(r.a)));
}

// acc + the 16-byte lane slices' element products, in element order.
template <int DT>
__device__ __forceinline__ float dot16(const u32x4& wv, const u32x4& xv, float acc) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if constexpr (DT == kF32) {
      acc = fmaf(__uint_as_float(wv[e]), __uint_as_float(xv[e]), acc);
    } else {
      using S = typename Elem<DT>::S;
      acc = fmaf(Elem<DT>::to_f32(static_cast<S>(wv[e] & 0xffffu)),
                 Elem<DT>::to_f32(static_cast<S>(xv[e] & 0xffffu)), acc);
      acc = fmaf(Elem<DT>::to_f32(static_cast<S>(wv[e] >> 16)),
                 Elem<DT>::to_f32(static_cast<S>(xv[e] >> 16)), acc);
    }
  }
  return acc;
}

// 16-byte load from a global-memory byte address (global, not flat, instructions: their
// completion is tracked by the vector-memory counter alone).
typedef const __attribute__((address_space(1))) u32x4* GlobalU32x4;

template <int CP>
__device__ __forceinline__ u32x4 load16(uint64_t addr) {
  if constexpr (CP == kNonTemporal)
    return __builtin_nontemporal_load(reinterpret_cast<GlobalU32x4>(addr));
  else
    return *reinterpret_cast<GlobalU32x4>(addr);
}

// PRE: a shared expert whose rows have more than kRowsDepth units (the host's choice).
template <int DT, int CP, bool PRE>
__global__ __launch_bounds__(kRowsWaves * kWave) void down_rows_kernel(RowsArgs a) {
  using S = typename Elem<DT>::S;
  __shared__ RowTerm terms[kRowsMaxTerms];
  __shared__ int fpos_l[kRowsMaxAssign];
  __shared__ float w_l[kRowsMaxAssign];
  __shared__ float vals[kRowsWaves][kRowsMaxTerms];
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = wave_id();
  const int h = blockIdx.x * kRowsWaves + wave;
  const int N = a.T * a.k;
  const int rowb = a.I * static_cast<int>(sizeof(S));
  const int units = (rowb + kRowsUnit - 1) / kRowsUnit;
  const bool shared = a.page_s != nullptr;
  const bool gated = a.block && shared && a.sgate != nullptr;
  const int Ts = shared ? a.T : 0;  // shared-expert terms 0..T-1, then the routed terms
  const int rowb_s = a.Is * static_cast<int>(sizeof(S));
  const int units_s = (rowb_s + kRowsUnit - 1) / kRowsUnit;
  RowCursor ic;  // issue cursor
  u32x4 wr[kRowsDepth], ar[kRowsDepth];
  int nterms = Ts;
  // Issue the cursor's unit into ring slot d and advance; past the last unit the cursor
  // stays on it (reloads in bounds, never consumed).
  auto issue = [&](int d) {
    const int o = ic.u * kRowsUnit + lane * 16;
    const int oc = o < ic.rowb ? o : ic.rowb - 16;
    wr[d] = load16<CP>(ic.w + static_cast<uint64_t>(oc));
    ar[d] = load16<0>(ic.a + static_cast<uint64_t>(oc));
    if (++ic.u == ic.units) {
      if (ic.tau + 1 < nterms) row_cursor_at(ic, terms, ic.tau + 1, h);
      else ic.u = ic.units - 1;
    }
  };
  // Term table: the shared expert's row for token t is term t; routed assignment f becomes
  // term Ts + fpos[f]. Its loads are independent of one another (one latency) and are issued
  // first, by every lane (from clamped, in-bounds indices, N >= 1) so that no branch hides
  // their count: loads complete in issue order, and the table is then waited for without
  // waiting for the weight loads issued after it.
  const int fi = tid < N ? tid : N - 1;
  const int tt = div_small(fi, a.k, 1.0f / static_cast<float>(a.k));
  const int jt = fi - tt * a.k;
  const uint32_t m = static_cast<uint32_t>(a.tmask[tt]);
  const int pos = a.fpos[fi];
  const int64_t slot = a.fslot[fi];
  const float wt = a.w[fi];
  // lane t's shared-expert gate logit (used by lane t at the end). Its load converts under a
  // dtype branch, which waits for it at once: issued here, that wait covers only the table.
  const float zt = gated ? load_scalar(a.sgate, a.sgate_dtype, lane < a.T ? lane : a.T - 1) : 0.0f;
  int routed = 0;
  __builtin_amdgcn_sched_barrier(0);
  // PRE: the shared expert's rows need no routing record, so the first kRowsDepth units of
  // token 0's shared term (which has more units than that: the cursor stays inside it, and no
  // table entry is needed) are issued before the table is used; its latency overlaps them.
  if constexpr (PRE) {
    ic.tau = 0;
    ic.u = 0;
    ic.rowb = rowb_s;
    ic.units = units_s;
    ic.w = reinterpret_cast<uint64_t>(a.page_s) +
           (2ull * static_cast<uint64_t>(a.H) + static_cast<uint64_t>(h)) * static_cast<uint64_t>(rowb_s);
    ic.a = reinterpret_cast<uint64_t>(a.act_s);
#pragma unroll
    for (int d = 0; d < kRowsDepth; ++d) issue(d);
  }
  __builtin_amdgcn_sched_barrier(0);
  if (shared && tid < a.T) {
    RowTerm r;
    r.w = reinterpret_cast<uint64_t>(a.page_s) + 2ull * static_cast<uint64_t>(a.H) * static_cast<uint64_t>(rowb_s);
    r.a = reinterpret_cast<uint64_t>(a.act_s) + static_cast<uint64_t>(tid) * static_cast<uint64_t>(rowb_s);
    r.rowb = rowb_s;
    r.units = units_s;
    terms[tid] = r;
  }
  if (tid < N) {
    w_l[tid] = wt;
    routed = (m >> jt) & 1u;
    fpos_l[tid] = routed ? pos : -1;
    if (routed) {
      RowTerm r;
      r.w = reinterpret_cast<uint64_t>(a.pool) + static_cast<uint64_t>(slot * a.page_bytes) +
            2ull * static_cast<uint64_t>(a.H) * static_cast<uint64_t>(rowb);
      r.a = reinterpret_cast<uint64_t>(a.act) + static_cast<uint64_t>(pos) * static_cast<uint64_t>(rowb);
      r.rowb = rowb;
      r.units = units;
      terms[Ts + pos] = r;
    }
  }
  const int nr = __syncthreads_count(routed);
  nterms = Ts + nr;
  const int total = nr * units + Ts * units_s;
  if (total > 0) {
    RowCursor cc;
    row_cursor_at(cc, terms, 0, h);
    float part = 0.0f;
    if constexpr (!PRE) {
      ic = cc;
#pragma unroll
      for (int d = 0; d < kRowsDepth; ++d) issue(d);
    }
    for (int i = 0; i < total; i += kRowsDepth) {
#pragma unroll
      for (int d = 0; d < kRowsDepth; ++d) {
        if (i + d < total) {
          const int o = cc.u * kRowsUnit + lane * 16;
          if (o < cc.rowb) part = dot16<DT>(wr[d], ar[d], part);
          if (++cc.u == cc.units) {  // the term's last unit: its dot goes to LDS
            const float v = group_reduce<kWave>(part, [](float x, float y) { return x + y; });
            if (lane == 0) vals[wave][cc.tau] = v;
            part = 0.0f;
            if (cc.tau + 1 < nterms) row_cursor_at(cc, terms, cc.tau + 1, h);
          }
        }
        issue(d);
      }
    }
  }
  __builtin_amdgcn_wave_barrier();
  if (lane >= a.T) return;
  // lane t: y[t, h] in the combine's arithmetic
  const int t = lane;
  float y = 0.0f;
  for (int j = 0; j < a.k; ++j) {
    const int f = t * a.k + j;
    const int p = fpos_l[f];
    if (p >= 0) y += round_out<DT>(vals[wave][Ts + p] * w_l[f], a.f16out);
  }
  if (a.block) {
    y = Elem<DT>::round(y);
    if (a.scale != 1.0f) y = Elem<DT>::round(y * a.scale);
    if (shared) {
      float sh = Elem<DT>::round(vals[wave][t]);
      if (gated) sh = Elem<DT>::round(Elem<DT>::round(1.0f / (1.0f + __expf(-zt))) * sh);
      y += sh;
    }
  }
  static_cast<S*>(a.y)[static_cast<int64_t>(t) * a.H + h] = Elem<DT>::from_f32(y);
}

hipError_t launch_down_rows(int dtype, const RowsArgs& a, hipStream_t s) {
  if (a.T < 1 || a.T > kRowsMaxTokens || a.k > kMaxTopK || a.H % kRowsWaves != 0)
    return hipErrorInvalidValue;
  const unsigned blocks = static_cast<unsigned>(a.H / kRowsWaves);
  // a token's expert rows are read once at T = 1 (streaming hint); larger batches may read a
  // row twice in a row (two tokens of one expert) and keep it in L2
  const bool once = a.T == 1;
  const int64_t rowb_s = static_cast<int64_t>(a.Is) * dtype_bytes(dtype);
  const bool pre = a.page_s != nullptr && (rowb_s + kRowsUnit - 1) / kRowsUnit > kRowsDepth;
  auto go = [&](auto dt, auto cp, auto pr) {
    down_rows_kernel<decltype(dt)::value, decltype(cp)::value, decltype(pr)::value>
        <<<blocks, kRowsWaves * kWave, 0, s>>>(a);
  };
  auto by_pre = [&](auto dt, auto cp) {
    if (pre) go(dt, cp, std::true_type{});
    else go(dt, cp, std::false_type{});
  };
  auto by_cp = [&](auto dt) {
    if (once) by_pre(dt, std::integral_constant<int, kNonTemporal>{});
    else by_pre(dt, std::integral_constant<int, 0>{});
  };
  switch (dtype) {
    case kF32: by_cp(std::integral_constant<int, kF32>{}); break;
    case kF16: by_cp(std::integral_constant<int, kF16>{}); break;
    default: by_cp(std::integral_constant<int, kBF16>{}); break;
  }
  return hipGetLastError();
}

// Resident 4-wave expert workgroups of the current device: two per CU (their launch bounds).
// The per-device cache is read and written by concurrent callers: relaxed atomics suffice (every
// writer stores the same value, and a reader that sees 0 queries the device itself).
static int resident_slots() {
  static std::atomic<int> cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 512;
  if (dev < 64) {
    const int c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  const int slots = 2 * cus;
  if (dev < 64) cached[dev].store(slots, std::memory_order_relaxed);
  return slots;
}

// Gate/up launch of W waves per workgroup (fewer waves only for batches of at most two
// token tiles with every expert one token range: the grids that can leave CUs idle). A
// 4-wave grid with more items than one residency of the chip (a.gu_items > 0 asks for it)
// runs as G workgroups that walk ceil(items / G) items each (G a multiple of 8, so that every
// workgroup stays on one XCD's items), when such a G keeps at least 7/8 of the slots busy.
template <bool kMulti, int DT, int MT, int RG, bool RM>
static void launch_gateup_w(const ExpertArgs& a, int max_ranges, hipStream_t s) {
  auto go = [&](auto wc, auto ksc) {
    constexpr int W = decltype(wc)::value;
    constexpr bool KS = decltype(ksc)::value;
    constexpr int TW = KS ? 2 : W;
    const int64_t groups = (a.I / kRowTile + TW - 1) / TW;
    const int64_t items = a.sh.gateup_blocks + max_ranges * groups;
    const int slots = resident_slots();
    if constexpr (W == kExpertWaves) {
      // the fewest workgroups that walk equal item counts, if that keeps 7/8 of the slots busy
      const int64_t per = (items + slots - 1) / slots;
      const int64_t g = ((items + per - 1) / per + 7) / 8 * 8;
      if (a.gu_items > 0 && items > slots && 8 * g >= 7 * static_cast<int64_t>(slots)) {
        ExpertArgs b = a;
        b.gu_items = static_cast<int>(items);
        gateup_kernel<kMulti, DT, MT, RG, RM, W, true, KS><<<static_cast<unsigned>(g), W * kWave, 0, s>>>(b);
        return;
      }
    }
    gateup_kernel<kMulti, DT, MT, RG, RM, W, false, KS><<<static_cast<unsigned>(items), W * kWave, 0, s>>>(a);
  };
  using No = std::false_type;
  if constexpr (!kMulti && MT <= 2) {
    if (a.gu_waves == 1) return go(std::integral_constant<int, 1>{}, No{});
    if (a.gu_waves == 2) return go(std::integral_constant<int, 2>{}, No{});
  }
  if constexpr (MT <= 2) {
    if (a.gu_ks) return go(std::integral_constant<int, kExpertWaves>{}, std::true_type{});
  }
  go(std::integral_constant<int, kExpertWaves>{}, No{});
}

template <bool kMulti, int DT, int MT>
static void launch_stage_m(int stage, const ExpertArgs& a, int max_ranges, hipStream_t s) {
  if (stage == 0) {
    launch_gateup_w<kMulti, DT, MT, 0, false>(a, max_ranges, s);
  } else {
    const int R = a.down_rows == 1 ? 1 : kDownRows;
    const int64_t groups = (a.H / (kRowTile * R) + kExpertWaves - 1) / kExpertWaves;
    const int64_t blocks = a.sh.down_blocks + max_ranges * groups * a.splits;
    if (R == 1) down_kernel<kMulti, DT, MT, 1><<<static_cast<unsigned>(blocks), kExpertThreads, 0, s>>>(a);
    else down_kernel<kMulti, DT, MT><<<static_cast<unsigned>(blocks), kExpertThreads, 0, s>>>(a);
  }
}

template <int DT, int MT>
static hipError_t launch_stage_t(int stage, const ExpertArgs& a, int max_ranges, hipStream_t s) {
  // no expert can have more tokens than one pass holds when T <= span
  if (a.T <= a.rb.span) launch_stage_m<false, DT, MT>(stage, a, max_ranges, s);
  else launch_stage_m<true, DT, MT>(stage, a, max_ranges, s);
  return hipGetLastError();
}

template <int DT>
static hipError_t launch_stage_dt(int stage, const ExpertArgs& a, int max_ranges, int tok_tiles,
                                  hipStream_t s) {
  switch (tok_tiles) {
    case 1: return launch_stage_t<DT, 1>(stage, a, max_ranges, s);
    case 2: return launch_stage_t<DT, 2>(stage, a, max_ranges, s);
    case 3: return launch_stage_t<DT, 3>(stage, a, max_ranges, s);
    default: return launch_stage_t<DT, 4>(stage, a, max_ranges, s);
  }
}

static hipError_t launch_stage(int stage, int dtype, const ExpertArgs& a, int max_ranges,
                               int tok_tiles, hipStream_t s) {
  switch (dtype) {
    case kF32: return launch_stage_dt<kF32>(stage, a, max_ranges, tok_tiles, s);
    case kF16: return launch_stage_dt<kF16>(stage, a, max_ranges, tok_tiles, s);
    default: return launch_stage_dt<kBF16>(stage, a, max_ranges, tok_tiles, s);
  }
}

template <int DT, int MT, bool RM>
static void launch_gateup_routed(const ExpertArgs& a, int max_ranges, int route_g, hipStream_t s) {
  switch (route_g) {
    case 8: launch_gateup_w<false, DT, MT, 8, RM>(a, max_ranges, s); break;
    case 16: launch_gateup_w<false, DT, MT, 16, RM>(a, max_ranges, s); break;
    case 32: launch_gateup_w<false, DT, MT, 32, RM>(a, max_ranges, s); break;
    default: launch_gateup_w<false, DT, MT, 64, RM>(a, max_ranges, s); break;
  }
}

template <int DT>
static void launch_gateup_routed_dt(const ExpertArgs& a, int max_ranges, int tok_tiles, int route_g,
                                    bool multi, hipStream_t s) {
  if (!multi) {
    if (tok_tiles <= 1) launch_gateup_routed<DT, 1, false>(a, max_ranges, route_g, s);
    else launch_gateup_routed<DT, 2, false>(a, max_ranges, route_g, s);
    return;
  }
  switch (tok_tiles) {
    case 1: launch_gateup_routed<DT, 1, true>(a, max_ranges, route_g, s); break;
    case 2: launch_gateup_routed<DT, 2, true>(a, max_ranges, route_g, s); break;
    case 3: launch_gateup_routed<DT, 3, true>(a, max_ranges, route_g, s); break;
    default: launch_gateup_routed<DT, 4, true>(a, max_ranges, route_g, s); break;
  }
}

hipError_t launch_gateup(int dtype, const ExpertArgs& a, int max_ranges, int tok_tiles, hipStream_t s,
                         int route_g, bool route_multi) {
  if (route_g == 0) return launch_stage(0, dtype, a, max_ranges, tok_tiles, s);
  // routing inside the launch, every expert one token range (T <= span): one wave routes
  // T*k <= 64 assignments over E <= 64 experts in at most 4 top-k passes; the multi-wave form
  // takes up to kSortWaveMax assignments and up to four token tiles
  if (route_g != 8 && route_g != 16 && route_g != 32 && route_g != 64) return hipErrorInvalidValue;
  if (a.rt.E > kWave || a.T > a.rb.span || tok_tiles > kMaxTokTiles) return hipErrorInvalidValue;
  if (route_multi) {
    if (a.T * a.k > kSortWaveMax) return hipErrorInvalidValue;
  } else if (a.T * a.k > kWave || tok_tiles > 2 ||
             (a.rt.logits != nullptr && a.T * route_g > kWave * kSmallRoutePasses)) {
    return hipErrorInvalidValue;
  }
  switch (dtype) {
    case kF32: launch_gateup_routed_dt<kF32>(a, max_ranges, tok_tiles, route_g, route_multi, s); break;
    case kF16: launch_gateup_routed_dt<kF16>(a, max_ranges, tok_tiles, route_g, route_multi, s); break;
    default: launch_gateup_routed_dt<kBF16>(a, max_ranges, tok_tiles, route_g, route_multi, s); break;
  }
  return hipGetLastError();
}

hipError_t launch_down(int dtype, const ExpertArgs& a, int max_ranges, int tok_tiles, hipStream_t s) {
  return launch_stage(1, dtype, a, max_ranges, tok_tiles, s);
}

hipError_t launch_combine(int dtype, const CombineArgs& c, hipStream_t s) {
  if (c.rows) {
    // One-wave workgroups until the grid holds a few workgroups per CU: at 128 tokens of
    // hidden 2048 the 256-thread form has 128 workgroups, half the CUs.
    const int64_t outs = static_cast<int64_t>(c.T) * c.H / kCombineRowOuts;
    const int threads = outs >= static_cast<int64_t>(kCombineRowThreads) * 1024 ? kCombineRowThreads : kWave;
    const unsigned blocks = static_cast<unsigned>((outs + threads - 1) / threads);
    switch (dtype) {
      case kF32: combine_rows_kernel<kF32><<<blocks, threads, 0, s>>>(c); break;
      case kF16: combine_rows_kernel<kF16><<<blocks, threads, 0, s>>>(c); break;
      default: combine_rows_kernel<kBF16><<<blocks, threads, 0, s>>>(c); break;
    }
    return hipGetLastError();
  }
  const int chunks = (c.H + 4 * kWave - 1) / (4 * kWave);
  const unsigned blocks = static_cast<unsigned>(static_cast<int64_t>(c.T) * chunks);
  const int items = c.k + (c.part_s != nullptr ? 1 : 0);
  const int threads = (items < kCombineMaxWaves ? items : kCombineMaxWaves) * kWave;
  switch (dtype) {
    case kF32: combine_kernel<kF32><<<blocks, threads, 0, s>>>(c); break;
    case kF16: combine_kernel<kF16><<<blocks, threads, 0, s>>>(c); break;
    default: combine_kernel<kBF16><<<blocks, threads, 0, s>>>(c); break;
  }
  return hipGetLastError();
}

}  // namespace smx
