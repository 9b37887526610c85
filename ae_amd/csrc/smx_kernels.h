// Internal interface between the kernel translation units and the C ABI (capi.hip).
#pragma once

#include "smx_common.h"

namespace smx {

// Routing limits (one workgroup sorts all assignments in LDS).
constexpr int kRouteMaxWaves = 16;                  // waves of the single routing workgroup
constexpr int kRouteMaxThreads = kRouteMaxWaves * kWave;
constexpr int kMaxExperts = 256;
constexpr int kMaxExpertsPerLane = kMaxExperts / kWave;
constexpr int kMaxAssignments = 16384;  // T * top_k
constexpr int kMaxTopK = 16;
constexpr int kBlockExperts = 8;        // experts per lane of the block top-k (topk_device.h)
constexpr int kTokBatch = 1;            // wave-passes of tokens a wave computes together
// Token passes of 64/G tokens (T * G <= 256) of the one-wave routing: each pass is a dependent
// chain of group reductions, so beyond a few passes the multi-wave kernel is faster.
constexpr int kSmallRoutePasses = 4;

// Expert-kernel geometry.
constexpr int kExpertThreads = 256;                 // 4 independent waves per workgroup
constexpr int kExpertWaves = kExpertThreads / kWave;
constexpr int kRowTile = 16;                        // weight rows per MFMA tile
constexpr int kTokTile = 16;                        // token columns per MFMA tile
constexpr int kStepBytes = 64;                      // row bytes one 16-byte/lane load step covers
constexpr int kUnroll = 4;                          // load steps per chunk (256 bytes per row)
constexpr int kDownRows = 2;                        // row tiles per wave in the down projection
                                                    // (1 for grids that would not fill the chip)
constexpr int kMaxTokTiles = 4;                     // token tiles per pass (64 tokens)
// Expert-ordered gate/up items: token tiles per pass at most. The first item's prefetched
// chunks are copied into the stream's registers; with three or four token tiles that copy
// exceeds the registers of two workgroups per CU (the kernels spill).
constexpr int kExpertItemsMaxTiles = 2;

static_assert(kUnroll * kStepBytes == 256 && kRowTile == 16,
              "a weight chunk is four 4-row x 256-byte loads covering one 16-row tile");

// In-launch routing (the gate/up kernel routes a small batch itself and keeps the range records
// in the workgroup's LDS). The one-wave form takes at most 64 assignments; the multi-wave form
// sorts with the one-wave sort (sort_wave) at most kGateupSortMax given ids (the top-k from
// logits inside the launch: at most kSortWaveMax assignments), over at most 64 experts; with
// given ids an expert's assignments may span several token ranges (T > span). The
// routing kernel sorts with sort_wave up to kSortWaveMax assignments. Range records at most:
// one per active expert plus one per further span (>= kTokTile sorted positions) of an
// expert's assignments.
constexpr int kSortWaveMax = 256;
constexpr int kGateupSortMax = 768;
constexpr int kSmallRangesMax = kWave + kWave / kTokTile;
constexpr int kSortRangesMax = kWave + kGateupSortMax / kTokTile;

// Tiled expert kernels (tiles.hip), for experts that see many tokens: output tiles of
// 128 token rows by 128 intermediate columns (gate/up) or 256 W2 rows (down) per workgroup.
constexpr int kTileTok = 128;        // sorted positions per work range
constexpr int kTileGateCols = 128;   // intermediate columns per gate/up workgroup
constexpr int kTileDownRows = 256;   // W2 rows per down workgroup

// Work ranges of the expert kernels: up to `span` consecutive sorted positions of one active
// expert. An expert with more tokens than one pass of the kernels holds is split into nr
// ranges, numbered j0 .. j0 + nr - 1; each of them holds the same record (the expert's), so a
// workgroup finds its expert from any range index in one load. The kernels number the items
// of an expert (range r, weight group g) so that the nr ranges of one weight group run side
// by side on one XCD and read the same rows at about the same time.
struct RangeRec {
  int64_t slot;  // pool slot of the expert
  int32_t off;   // first sorted position of the expert
  int32_t cnt;   // sorted positions of the expert
  int32_t key;   // expert index (the gate/up K-walk rotation)
  int32_t j0;    // first range of the expert
  int32_t nr;    // ranges of the expert: ceil(cnt / span)
  int32_t pad;
};

// hdr[kHdrSingleRanges] (global records only): 1 when every active expert is one work range.
constexpr int kHdrSingleRanges = 2;

struct RouteBuffers {
  int32_t* hdr;         // [0] ranges, [1] dropped-assignment flag, [2] one range per expert
  RangeRec* ranges;     // [max_ranges] in expert order, then range order
  int32_t* sorted_f;    // [T*k] flat assignment index f = t*k + j at each sorted position
  int32_t* tmask;       // [T] bit j set: assignment t*k+j contributes (routable expert and slot)
  int32_t* fpos;        // [T*k] sorted position of each contributing assignment (may be null)
  int64_t* fslot;       // [T*k] pool slot of each contributing assignment (with fpos)
  int span;             // sorted positions per range (the tokens of one kernel pass)
};

// An always-active expert that every token passes through (the shared expert of the
// Qwen-MoE and DeepSeek-V2 MoE blocks). It runs in the leading workgroups of the gate/up and
// down launches: token range v (`span` tokens) of the batch is one work item,
// like one routed expert's token list.
struct SharedArgs {
  const void* page;     // [3 * I * H] page in the routed layout; null when absent
  int I;                // intermediate size of the shared expert (0 when absent)
  void* act;            // [T, I] silu(gate)*up, row = token
  float* part;          // [splits, T, H] fp32 partial down projections, row = token
  int splits;           // K splits of its down projection
  int split_steps;      // load steps per split
  int tok_groups;       // token ranges
  int gateup_blocks;    // leading workgroups of the gate/up launch that run it
  int down_blocks;      // leading workgroups of the down launch that run it
};

// Routing done inside the gate/up launch for small batches (T*k <= 64 assignments over E <= 64
// experts, at most 64/G tokens per pass in 4 passes): no routing launch. Every routed workgroup
// routes the batch itself (one wave, into LDS) and takes its work item from that; the first
// routed workgroup also writes the routing records and top-k results for the later kernels.
struct InRoute {
  const void* logits;      // [T, E] router logits in the activation dtype (null: ids given)
  const int32_t* ids_in;   // [T, k] caller ids when logits is null
  float* w_out;            // [T, k] top-k weights out (logits given)
  int32_t* ids_out;        // [T, k] top-k ids out (logits given)
  int64_t num_slots;
  int E, renorm;
};

// The single-launch layer (layer1.hip): one launch holds the gate/up workgroups [0, gu_blocks)
// and after them the down workgroups of the fused down projection + combine. A gate/up
// workgroup stores its activation rows through to device scope, waits for the stores to
// complete, and then stores `epoch` into its flag; a down workgroup waits (bounded in time)
// until every flag holds `epoch` and then reads the activation rows at device scope.
struct LayerSync {
  uint64_t* flags;      // [gu_blocks] (workspace)
  uint64_t* status;     // (workspace) set to `epoch` by a down workgroup that gave up waiting
  uint64_t epoch;       // this call's value: unique within the process, never 0
  int gu_blocks;        // gate/up workgroups; the down workgroups follow them in the grid
  int publish;          // 0: the gate/up workgroups do not publish (tests of the give-up path)
  int64_t wait_ticks;   // longest wait of a down workgroup, in wall-clock (s_memrealtime) ticks
};

// The combine arguments of the single-launch layer's down workgroups (as RowsArgs).
struct LayerOut {
  void* y;              // [T, H]
  int block;
  float scale;
  const void* sgate;
  int sgate_dtype;
};

struct ExpertArgs {
  const void* x;        // [T, H] hidden states
  const void* pool;     // [num_slots, page_elems] expert pages
  int64_t page_elems;
  const int64_t* e2s;   // [E] expert -> pool slot
  RouteBuffers rb;
  int T, H, I, k;
  void* act;            // [T*k, I] silu(gate)*up, row = sorted position
  float* part;          // [splits, T*k, H] fp32 partial down projections, row = f
  int splits;           // K splits of the down projection
  int split_steps;      // load steps per split
  int f16out;           // fp32 runs: routed gate/up outputs rounded to fp16 (reference stores)
  int down_rows;        // W2 row tiles per down wave: kDownRows, or 1
  int gu_waves;         // waves per gate/up workgroup: kExpertWaves, or 2 or 1 (more, smaller
                        // workgroups for grids that would leave CUs idle); sh.gateup_blocks and
                        // the launch's grid follow it
  int gu_items;         // host: nonzero lets a gate/up grid larger than one residency of the
                        // chip run as workgroups that walk several items; kernel: the item count
  int gu_ks;            // 4-wave gate/up workgroups split each item's K walk between wave pairs
                        // (2 weight tiles per workgroup; sh.gateup_blocks and the grid follow it)
  InRoute rt;           // used by the gate/up launch with routing inside (route_g > 0)
  SharedArgs sh;
  LayerSync ls;         // the single-launch layer only
  LayerOut lo;          // the single-launch layer only
};

struct CombineArgs {
  const float* part;
  const float* w;       // [T*k]
  const int32_t* tmask; // [T] contributing assignments of each token (RouteBuffers::tmask)
  void* y;              // [T, H]
  int T, H, k, splits;
  // Block form y = round(round(routed * scale) + s * shared), used when `block` is set.
  int block;
  float scale;               // routed scaling factor
  const float* part_s;       // [splits_s, T, H] shared-expert partials, null when absent
  int splits_s;
  const void* sgate;         // [T] shared-expert gate logits (s = sigmoid), null: s = 1
  int sgate_dtype;
  int rows;                  // thread-per-outputs kernel (large batches) instead of per-token
  int f16out;                // fp32 runs: each routed term rounded to fp16 (reference stores)
};

// Down projection fused with the combine for batches of a few tokens (experts.hip,
// down_rows_kernel): one wave per output row, every term of y[:, row] in one launch.
constexpr int kRowsMaxTokens = 8;                       // largest batch the kernel takes
constexpr int kRowsUnitBytes = 1024;                    // one 16-byte load per lane of a wave
// By default the fused kernel runs when each wave's terms stream at most this many units
// (weight bytes per output row, in 1 KB units): DeepSeek-V2-Lite and Qwen1.5-MoE blocks at
// one token (23 units) run ~5 us faster per layer than the split down kernel + combine and
// DeepSeek-V2-Lite at two tokens (46) 1.5 us faster; Mixtral at one token (56 units, 114 vs
// 113 us) and DeepSeek-V2-Lite at four (92 units, 82 vs 76 us) run slower.
constexpr int kRowsDefaultMaxUnits = 48;

struct RowsArgs {
  const void* pool;          // [num_slots, page] expert pages
  int64_t page_bytes;
  const void* act;           // [T*k, I] silu(gate)*up, row = sorted position
  const int32_t* tmask;      // [T] contributing assignments (RouteBuffers::tmask)
  const int32_t* fpos;       // [T*k] sorted position of each contributing assignment
  const int64_t* fslot;      // [T*k] pool slot of each contributing assignment
  const float* w;            // [T*k] routing weights
  const void* page_s;        // shared-expert page (null: none)
  const void* act_s;         // [T, Is]
  int Is;
  void* y;                   // [T, H]
  int T, H, I, k;
  // block form, as CombineArgs
  int block;
  float scale;
  const void* sgate;
  int sgate_dtype;
  int f16out;                // as CombineArgs::f16out
};

hipError_t launch_down_rows(int dtype, const RowsArgs& a, hipStream_t s);

// The single-launch layer for one token (layer1.hip): the gate/up launch with routing inside
// (route_g lanes per token, 4 waves per workgroup) followed, in the same grid, by one down
// workgroup per 4 output rows. Its limits: T = 1, E <= 64, the down waves' W2 units
// (kLayerMaxUnits) and the activation rows staged in LDS (kLayerMaxActBytes).
constexpr int kLayerMaxUnits = 24;
constexpr int kLayerMaxActBytes = 32768;
constexpr int kLayerMaxGuBlocks = 512;  // gate/up workgroups one polling wave watches (8 per lane)
hipError_t launch_layer1(int dtype, const ExpertArgs& a, int max_ranges, int route_g, hipStream_t s);

// Post-attention residual add + RMSNorm + router gate (+ shared-expert gate row, + top-k).
constexpr int kNormThreads = 256;
constexpr int kNormWaves = kNormThreads / kWave;
constexpr int kNormMaxH = 16384;  // one token's fp32 row is staged in LDS

struct NormGateArgs {
  const void* x;          // [T, H] hidden states
  void* residual;         // [T, H] in/out (null: no residual add)
  void* xn;               // [T, H] normalized out (may alias x)
  const void* norm_w;     // [H]
  float eps;
  const void* gate_w;     // [E, H] router gate (null: norm only)
  const void* sgate_w;    // [H] shared-expert gate row (null: none)
  void* logits;           // [T, E] router logits out (dtype)
  void* sgate_logits;     // [T] shared-expert gate logits out (dtype)
  float* topk_w;          // [T, k] top-k weights out (null: no top-k)
  int32_t* topk_ids;      // [T, k]
  int T, H, E, k, renorm, dtype;
  // One token and E <= 64: the expert sort of the token's picks written here (the records the
  // routing kernels write), in place of a routing launch. route = 0: not written.
  int route;
  RouteBuffers rb;
  const int64_t* e2s;     // [E] expert -> pool slot
  int64_t num_slots;
};

hipError_t launch_norm_gate(const NormGateArgs& a, hipStream_t s);

hipError_t launch_topk_softmax(const void* logits, int ldt, int T, int E, int k, int renorm,
                               float* w, int32_t* ids, hipStream_t s);
// Grouped top-k (ng groups of E / ng experts, topk_group of them selectable; bias: the
// sigmoid scores with a correction bias, else softmax). Limits checked by the caller.
hipError_t launch_grouped_topk(const void* logits, int ldt, int T, int E, int k, int renorm, int ng,
                               int tg, const float* bias, float* w, int32_t* ids, hipStream_t s);
hipError_t launch_align(const int32_t* ids, int N, int E, int bm, int32_t* sorted_ids,
                        int32_t* expert_ids, int32_t* ntp, hipStream_t s);
hipError_t launch_route(const void* logits, int ldt, int T, int E, int k, int renorm,
                        float* w_out, int32_t* ids_out, const int32_t* ids_in,
                        const int64_t* e2s, int64_t num_slots, const RouteBuffers& rb,
                        hipStream_t s);
// route_g > 0: the routing runs inside the launch (a.rt), with route_g lanes per token in the
// top-k; route_multi: the multi-wave form (up to 256 assignments); expert_items: its routed
// items in expert order (every expert one range of one pass), the first item's weights issued
// before the routing.
hipError_t launch_gateup(int dtype, const ExpertArgs& a, int max_ranges, int tok_tiles,
                         hipStream_t s, int route_g = 0, bool route_multi = false,
                         bool expert_items = false);
hipError_t launch_down(int dtype, const ExpertArgs& a, int max_ranges, int tok_tiles,
                       hipStream_t s);
hipError_t launch_combine(int dtype, const CombineArgs& c, hipStream_t s);
// Workgroups of a tiled launch (stage 0: gate/up, 1: down): the shared expert's leading
// workgroups, then every work range's weight groups (down: times the K splits).
int64_t tile_grid_blocks(int stage, int64_t H, int64_t I, int shared_blocks, int max_ranges, int splits);
hipError_t launch_tile_gateup(int dtype, const ExpertArgs& a, int max_ranges, hipStream_t s);
hipError_t launch_tile_down(int dtype, const ExpertArgs& a, int max_ranges, hipStream_t s);

}  // namespace smx
