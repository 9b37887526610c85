// C ABI of libspecmoe_mi355x.so (declared in include/specmoe_mi355x.h).
//
// Host code only: argument checks, the launch plan (a pure function of the shapes, so the
// grid never depends on routing results and nothing waits on the device), workspace layout,
// and the stream-ordered launch sequence route -> gate/up -> down -> combine.
#include "../../include/specmoe_mi355x.h"
#include "smx_kernels.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <mutex>
#include <random>

// Device-resident scratch of smx_fused_moe_forward_noalloc: the workspace of a call that may
// not allocate. Each GPU the library runs on holds its own copy (allocated with the code object
// when the library is first used on that device) until the process ends. Host code never passes
// `scratch` itself to a kernel or a copy: in host code the name is a stand-in, not a device
// address; the device address comes from hipGetSymbolAddress, once per device.
static __device__ __align__(256) char scratch[SMX_NOALLOC_SCRATCH_BYTES];

namespace {

using namespace smx;

constexpr int kVersion = 1 * 10000 + 1 * 100 + 0;
constexpr size_t kAlign = 256;
// Down-projection waves to aim for: K is split into the fewest parts that give this many
// (two per SIMD). Fewer, longer splits stream better (Mixtral T=32: 4 splits 148 us, 2 splits
// 143 us, 1 split 154 us) as long as the chip is covered (DeepSeek-V2-Lite T=1: 1 split
// 14.1 us, 11 splits 12.2 us).
constexpr int64_t kTargetDownWaves = 2048;
constexpr int64_t kDownFillBlocks = 512;  // one residency: two down workgroups per CU, 256 CUs
// Tiled path (tiles.hip): its down workgroups to aim for (two per CU), and the default
// expected tokens per active expert at which it takes over from the streaming kernels
// (measured crossover: Mixtral 64 tokens per expert 613 vs 637 us, 32: 590 vs 502 us;
// Qwen1.5-MoE 68: 378 vs 466 us, 34: 456 vs 293 us).
constexpr int64_t kTileTargetDownBlocks = 512;
// From this many expected tokens per active expert the down projection aims for 4x the
// workgroups: with ~2 rounds of workgroups the last round ran mostly empty (Mixtral 4096 tokens:
// 1072 workgroups on 512 slots; 2 K splits: down 1164 -> 1035 us, the combine's extra split 33 ->
// 56 us). Below it the extra splits cost more in the combine than they save.
constexpr int64_t kTileLargeTokens = 512;
// Batches from this many tokens combine with one thread per 8 outputs (combine_rows_kernel);
// smaller ones with one workgroup per (token, 256 outputs), one wave per assignment. Measured
// per layer, rows vs per-token: Mixtral 128 tokens 492.4 vs 493.3 us, DeepSeek-V2-Lite 128
// tokens 213.2 vs 213.6; at 64 tokens rows is 1.5-2 us slower (201.4 vs 199.6).
constexpr int64_t kCombineRowsMinTokens = 128;
constexpr int64_t kTileMinTokensDefault = 64;
int64_t g_tile_min_tokens = kTileMinTokensDefault;
// Batches of at most this many tokens run the down projection and the combine as one kernel
// (down_rows_kernel) instead of the split down kernel plus the combine; negative: the default
// rule (batches whose output rows each stream at most kRowsDefaultMaxUnits weight units).
int64_t g_rows_max_tokens = -1;
// fp32 runs round the routed GEMM outputs to fp16 as the reference stores them (opt-in).
bool g_fp32_f16out = false;
// Small batches route inside the gate/up launch (smx_set_routing_in_gateup).
bool g_route_in_gateup = true;
// Waves per gate/up workgroup (smx_set_gateup_waves): 0 = the default rule (gateup_waves).
int g_gateup_waves = 0;
// Gate/up grids larger than one residency of the chip run as workgroups walking several items
// (smx_set_gateup_item_walk).
bool g_gateup_walk = true;
// Routed gate/up items in expert order, the first item's weights issued before the in-launch
// routing (smx_set_gateup_expert_items).
bool g_expert_items = true;
// One-token layers as one launch where the plan allows (smx_set_single_launch_layer). Off by
// default: measured on the DeepSeek-V2-Lite block at one token, 37.0 us per layer against 31.1
// for the two launches (timelines: while the down workgroups stream their W2 rows the last
// gate/up workgroups end at ~27.5 us instead of ~19 us, and ~8 us of wait, staging and dot
// products follow the last publication).
bool g_layer1 = false;
// The single-launch layer's in-launch wait (smx_set_layer_sync_test): whether the gate/up
// workgroups publish (0 only in tests of the give-up path) and the longest wait of a down
// workgroup. Measured layers take ~30 us; the bound only ends a wait that would never end.
int g_sync_publish = 1;
constexpr int64_t kSyncWaitDefaultUs = 100000;
int64_t g_sync_wait_us = kSyncWaitDefaultUs;
// The default rule: 4 waves per workgroup, unless the 4-wave grid holds between one and two
// workgroups per CU and 2 waves (twice the workgroups) balance the work over the CUs better by
// more than kGateupBalanceMargin: a grid of n workgroups keeps n / (kChipCUs * ceil(n /
// kChipCUs)) of the CUs' time busy when the CUs holding the most workgroups finish last (one
// to two workgroups per CU at 4 waves leaves many CUs half idle; larger grids have the K split
// and the item walk).
// Measured, us per layer, 4 / 2 / 1 waves (same box): DeepSeek-V2-Lite 2 tokens (286
// workgroups at 4; balance 0.56 vs 0.75 at 2 waves) 51.8 / 48.1 / 50.0 (later 49.8 / 46.1);
// 1 token (176; 0.69 vs 0.69) 31.1 / 31.9 / 31.8 (later 30.3 / 31.1; rocprof gate/up 18.5 /
// 19.7 us); 4 tokens (506; 0.99 vs 0.99) 73.3 / 73.9 / 82.6; Qwen1.5-MoE 1 token (176) 31.2 /
// 30.3 / 30.5; Mixtral 1 token (448; 0.875 vs 0.875) 113.5 / 118.7 / 114.1; the fp32 layer of
// hidden 1024, ffn 2816, 8 experts at 32 tokens (352; 0.69 vs 0.92) 68.4 / 62.3 / 75.0 (gate/up
// 43.7 / 38.9 / 52.9).
constexpr int64_t kChipCUs = 256;
constexpr double kGateupBalanceMargin = 0.05;

// Share of the CUs' time a grid of n equal workgroups keeps busy (the CUs that hold the most of
// them finish last).
double cu_balance(int64_t n) {
  if (n <= 0) return 0.0;
  return static_cast<double>(n) / static_cast<double>(kChipCUs * ((n + kChipCUs - 1) / kChipCUs));
}
// 4-wave gate/up launches of at most two token tiles over rows of at most kGateupKSplitChunks
// 256-byte chunks split each item's K walk between wave pairs (items of half the length: the
// launch's last round drains in half the time), unless smx_set_gateup_waves fixes the workgroup
// shape. Measured, us per layer, split / not (same box): DeepSeek-V2-Lite 16 tokens 149.4-149.8 /
// 152.2-152.6 (gate/up 94.5-95.0 / 98.2-98.4), 32 tokens 175.8-176.4 / 176.5-176.6, 8 tokens
// 121.9-122.2 / 122.6-123.5; Qwen1.5-MoE 16 and 32 tokens even. Mixtral rows (32 chunks): 8
// tokens 321.2-322.0 / 326.7-327.1, but 16 tokens 375.7-376.5 / 364.7-365.7 and 32 tokens
// 436.8-436.9 / 420.9-421.0 (its walking workgroups take twice the items), hence the chunk limit.
// A grid of about one residency has no last round to shorten, and only the split's costs (two
// token stages, the LDS sum) remain: DeepSeek-V2-Lite 1 token (176 4-wave workgroups) 31.2 /
// 29.8, 4 tokens (~506) 73.4-74.2 / 72.7-73.2; hence the grid minimum (1.25 residencies).
constexpr bool kGateupKSplit = true;
constexpr int64_t kGateupKSplitChunks = 16;
constexpr int64_t kGateupKSplitMinBlocks = 640;

// tiles: 16-row weight tiles of one routed expert; s_tiles: of the shared expert (0: none);
// items: routed work items expected; s_groups: the shared expert's token ranges.
int gateup_waves(int64_t tiles, int64_t s_tiles, int64_t items, int64_t s_groups, int tok_tiles) {
  if (tok_tiles > 2) return kExpertWaves;
  if (g_gateup_waves > 0) return g_gateup_waves;
  const int64_t blocks4 = items * ((tiles + kExpertWaves - 1) / kExpertWaves) +
                          s_groups * ((s_tiles + kExpertWaves - 1) / kExpertWaves);
  const int64_t blocks2 = items * ((tiles + 1) / 2) + s_groups * ((s_tiles + 1) / 2);
  return blocks4 > kChipCUs && blocks4 < 2 * kChipCUs &&
                 cu_balance(blocks2) > cu_balance(blocks4) + kGateupBalanceMargin
             ? 2 : kExpertWaves;
}

bool fused_down(int64_t T, int64_t H, int64_t I, int64_t k, int64_t Is, int dtype) {
  if (T < 1 || T > kRowsMaxTokens || H % 4 != 0) return false;
  if (g_rows_max_tokens >= 0) return T <= g_rows_max_tokens;
  const int64_t eb = dtype_bytes(dtype);
  const int64_t units = T * (k * ((I * eb + kRowsUnitBytes - 1) / kRowsUnitBytes) +
                             (Is * eb + kRowsUnitBytes - 1) / kRowsUnitBytes);
  return units <= kRowsDefaultMaxUnits;
}

// Optional measurement events (smx_set_profile_events): recorded on the launch stream
// before routing and after each of the four kernels.
constexpr int kProfileEvents = 5;
hipEvent_t g_profile[kProfileEvents] = {};
bool g_profiling = false;

void mark(int i, hipStream_t s) {
  if (g_profiling) (void)hipEventRecord(g_profile[i], s);
}

size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

bool valid_dtype(int dt) { return dt == kF32 || dt == kF16 || dt == kBF16; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

struct Plan {
  bool tiled = false;  // tiled expert kernels (many tokens per expert) instead of streaming
  bool rows = false;   // down projection fused with the combine (a few tokens)
  int N = 0;
  int max_active = 0;  // experts that can be active: min(E, T*k)
  int span = 0;        // sorted positions per work range: the tokens of one kernel pass
  int max_ranges = 0;  // work ranges at most: every active expert, plus one per further span
  int tok_tiles = 1;
  int splits = 1;
  int split_steps = 0;
  int down_rows = kDownRows;  // W2 row tiles per down wave
  int gu_waves = kExpertWaves;  // waves per gate/up workgroup
  bool gu_ks = false;           // gate/up K walk split between wave pairs (kGateupKSplit)
  size_t hdr = 0, ranges = 0, sorted_f = 0, w = 0, ids = 0;
  size_t tmask = 0, fpos = 0, fslot = 0;
  size_t act = 0, part = 0, total = 0;
  // shared expert (Is > 0)
  int Is = 0, s_splits = 1, s_split_steps = 0, s_tok_groups = 0, s_gateup_blocks = 0, s_down_blocks = 0;
  size_t act_s = 0, part_s = 0;
  // whole-layer form: router logits and shared-expert gate logits
  size_t logits = 0, sgl = 0;
  // single-launch layer (one token, fused down): eligible, its gate/up workgroups and the
  // workspace offset of their flags (the status word follows them)
  bool layer1 = false;
  int sync_blocks = 0;
  size_t sync = 0;
};

// Shape limits shared by the workspace query and the entry points.
int check_shape(int64_t T, int64_t H, int64_t I, int64_t E, int64_t k, int dtype) {
  if (T < 0 || H <= 0 || I <= 0 || E <= 0 || k <= 0 || !valid_dtype(dtype)) return SMX_ERR_INVALID_ARG;
  if (k > E) return SMX_ERR_INVALID_ARG;
  if (E > kMaxExperts || k > kMaxTopK) return SMX_ERR_UNSUPPORTED;
  const int64_t eb = dtype_bytes(dtype);
  const int64_t chunk = static_cast<int64_t>(kStepBytes) * kUnroll;  // bytes per pipelined chunk
  if ((H * eb) % chunk != 0 || (I * eb) % chunk != 0) return SMX_ERR_UNSUPPORTED;
  if (H % (kRowTile * kDownRows) != 0 || I % kRowTile != 0) return SMX_ERR_UNSUPPORTED;
  if (H > (1 << 20) || I > (1 << 20)) return SMX_ERR_UNSUPPORTED;
  return SMX_OK;
}

// Tokens per pass of the kernels: the expert sort holds at most kMaxAssignments assignments in
// one workgroup's LDS, and per-lane offsets into the hidden states and activations are 32-bit.
// Calls with more tokens run as consecutive passes over token chunks on the same stream (each
// token's output depends on its own row only), sharing the workspace.
int64_t chunk_tokens(int64_t T, int64_t H, int64_t I, int64_t k, int64_t Is, int dtype) {
  const int64_t eb = dtype_bytes(dtype);
  const int64_t lim = (int64_t{1} << 31) - 1;
  int64_t c = kMaxAssignments / k;
  c = std::min(c, lim / (H * eb));
  c = std::min(c, lim / (k * I * eb));
  if (Is > 0) c = std::min(c, lim / (Is * eb));
  return std::max<int64_t>(1, std::min(T, c));
}

// Smallest divisor of n that is >= want (n when want > n).
int64_t divisor_at_least(int64_t n, int64_t want) {
  for (int64_t d = want < 1 ? 1 : want; d < n; ++d)
    if (n % d == 0) return d;
  return n;
}

// Largest divisor of n that is <= want (at least 1).
int64_t divisor_at_most(int64_t n, int64_t want) {
  int64_t s = 1;
  for (int64_t d = 1; d <= n && d <= want; ++d)
    if (n % d == 0) s = d;
  return s;
}

// Limits of the shared expert's intermediate size (the routed limits on I, plus 32-bit
// offsets into its page and activations).
int check_shared(int64_t T, int64_t H, int64_t Is, int dtype) {
  if (Is < 0) return SMX_ERR_INVALID_ARG;
  if (Is == 0) return SMX_OK;
  const int64_t eb = dtype_bytes(dtype);
  const int64_t chunk = static_cast<int64_t>(kStepBytes) * kUnroll;
  if ((Is * eb) % chunk != 0 || Is % kRowTile != 0 || Is > (1 << 20)) return SMX_ERR_UNSUPPORTED;
  if (3 * H * Is * eb >= (int64_t{1} << 32)) return SMX_ERR_UNSUPPORTED;
  (void)T;
  return SMX_OK;
}

// Limits of the residual-add + RMSNorm + gate kernel: whole 16-byte vectors per row and one
// row staged in LDS.
int check_norm(int64_t H, int dtype) {
  if (H <= 0 || !valid_dtype(dtype)) return SMX_ERR_INVALID_ARG;
  if ((H * dtype_bytes(dtype)) % 16 != 0 || H > kNormMaxH) return SMX_ERR_UNSUPPORTED;
  return SMX_OK;
}

// Is = intermediate size of the always-active shared expert, 0 when there is none; `layer`
// adds the buffers of the whole-layer form (router logits, shared-expert gate logits).
Plan make_plan(int64_t T, int64_t H, int64_t I, int64_t E, int64_t k, int dtype, int64_t Is = 0,
               bool layer = false) {
  Plan p;
  p.N = static_cast<int>(T * k);
  p.max_active = static_cast<int>(E < p.N ? E : p.N);
  const int64_t eb = dtype_bytes(dtype);
  // Experts expected to be active under uniform routing, E * (1 - (1 - k/E)^T): small batches
  // activate fewer than min(E, T*k) experts (T=4, top-2 of 8: 5.5), and the split count is
  // sized for the workgroups that will run.
  double active = static_cast<double>(E) * (1.0 - std::pow(1.0 - static_cast<double>(k) / E, static_cast<double>(T)));
  if (active > p.max_active) active = p.max_active;
  if (active < 1.0) active = 1.0;
  p.tiled = p.N > 0 && static_cast<double>(p.N) / active >= static_cast<double>(g_tile_min_tokens);
  int64_t s = 1;
  if (p.tiled) {
    p.span = kTileTok;
    p.max_ranges = p.max_active + p.N / p.span;
    // K steps of 128 bytes; the down projection's K is split into the fewest parts that give
    // kTileTargetDownBlocks workgroups over the ranges expected
    const int64_t nsteps = I * eb / 128;
    // ranges expected under uniform routing: each active expert holds ceil(N / active / 128)
    const int64_t ex = static_cast<int64_t>(active + 0.5);
    const int64_t per_expert = (static_cast<int64_t>(p.N / active + 0.5) + kTileTok - 1) / kTileTok;
    const int64_t ranges = ex * (per_expert < 1 ? 1 : per_expert);
    const int64_t units = ranges * ((H + kTileDownRows - 1) / kTileDownRows);
    const int64_t target = static_cast<double>(p.N) / active >= kTileLargeTokens ? 4 * kTileTargetDownBlocks
                                                                               : kTileTargetDownBlocks;
    const int64_t want = (target + units - 1) / units;
    // each split walks an even number of steps (the kernels' loop is unrolled by two), so the
    // split count divides nsteps / 2 (whole: I * eb is a multiple of 256 bytes)
    s = divisor_at_least(nsteps / 2, want);
    if (s > 4 * want) s = divisor_at_most(nsteps / 2, want);
    p.splits = static_cast<int>(s);
    p.split_steps = static_cast<int>(nsteps / s * 2);  // in 64-byte units
    if (Is > 0) {
      const int64_t ssteps = Is * eb / 128;
      const int64_t per = nsteps / s;
      const int64_t ss = divisor_at_most(ssteps / 2, (ssteps + per - 1) / per);
      p.Is = static_cast<int>(Is);
      p.s_splits = static_cast<int>(ss);
      p.s_split_steps = static_cast<int>(ssteps / ss * 2);
      p.s_tok_groups = static_cast<int>((T + p.span - 1) / p.span);
      p.s_gateup_blocks = static_cast<int>(p.s_tok_groups * ((Is + kTileGateCols - 1) / kTileGateCols));
      p.s_down_blocks = static_cast<int>(p.s_tok_groups * ((H + kTileDownRows - 1) / kTileDownRows) * ss);
    }
  } else {
    p.rows = fused_down(T, H, I, k, Is, dtype);
    const int64_t tiles = (T + kTokTile - 1) / kTokTile;
    p.tok_tiles = static_cast<int>(tiles < 1 ? 1 : (tiles > kMaxTokTiles ? kMaxTokTiles : tiles));
    p.span = kTokTile * p.tok_tiles;
    p.max_ranges = p.max_active + p.N / p.span;
    const int64_t nchunks = I * eb / (static_cast<int64_t>(kStepBytes) * kUnroll);
    const int64_t ex = static_cast<int64_t>(active + 0.5);
    // Down-projection split for R row tiles per wave: the fewest splits that reach the wave
    // target, unless the chunk count's divisors overshoot it by more than 4x (a prime count
    // leaves only 1 and itself); the shared expert's waves stream about as many chunks as a
    // routed wave. Returns the workgroups expected.
    int64_t ss = 1;
    // workgroups of the down grid for R row tiles per wave and sv routed splits (the shared
    // expert's splits follow: its waves stream about as many chunks as a routed wave)
    auto down_grid = [&](int R, int64_t sv, int64_t* ssv) {
      const int64_t rgroups = (H / (kRowTile * R) + kExpertWaves - 1) / kExpertWaves;
      int64_t blocks = ex * rgroups * sv;
      int64_t sso = 1;
      if (Is > 0) {
        const int64_t schunks = Is * eb / (static_cast<int64_t>(kStepBytes) * kUnroll);
        const int64_t per = nchunks / sv;
        sso = divisor_at_most(schunks, (schunks + per - 1) / per);
        blocks += ((T + p.span - 1) / p.span) * rgroups * sso;
      }
      if (ssv) *ssv = sso;
      return blocks;
    };
    auto down_split = [&](int R) {
      const int64_t units = ex * (H / (kRowTile * R));
      int64_t want = (kTargetDownWaves + units - 1) / units;
      if (want < 1) want = 1;
      s = divisor_at_least(nchunks, want);
      if (s > 4 * want) s = divisor_at_most(nchunks, want);
      return down_grid(R, s, &ss);
    };
    // Two row tiles per wave, unless that grid would not fill one residency of the chip (two
    // workgroups per CU): then one, which doubles the workgroups. Measured, us per down launch,
    // two vs one row tiles, same box: DeepSeek-V2-Lite 3 tokens (304 workgroups) 25.7 vs 22.2,
    // 4 tokens (368) 26.7 vs 24.4, 6 tokens (496) 38.2 vs 34.8; Qwen1.5-MoE 4 tokens (304)
    // 24.1 vs 24.1, 8 tokens (464) 27.6 vs 28.9. Full grids lose with one: Qwen1.5-MoE 16
    // tokens (704) 41.0 vs 42.2, Mixtral 32 tokens 142.9 vs 147.7.
    // Past two residencies, also one where the last round of two-tile workgroups would be at
    // most half full: the launch then drains on half-length workgroups. Measured, two vs one:
    // DeepSeek-V2-Lite 48 tokens (1040 workgroups) 67.4 vs 63.3, 64 (1056) 68.9 vs 65.7, 128
    // (1088) 72.6 vs 70.7; Qwen1.5-MoE 96 (1088) 70.7 vs 69.0, 128 (1088) 70.9 vs 70.4. Below
    // two residencies the results were mixed (Qwen1.5-MoE 32 tokens, 912: 55.3 vs 56.4;
    // DeepSeek-V2-Lite 16, 848: 52.2 vs 49.5), and there the rule keeps two.
    // Between one and two residencies with the last round at most half full, the grid of at
    // most two residencies (both row-tile counts, every split of the K chunks) of the fewest
    // rounds per workgroup byte -- rounds x (bytes / workgroups), the time of equal workgroups
    // dealt in rounds -- keeping the wave-target grid on ties. Measured on the fp32 layer of hidden 1024, ffn 2816, 8
    // experts at 32 tokens (704 workgroups: 2 row tiles, 11 splits), us per down launch: 1
    // row tile and 4 splits (512) 21.3, 2 and 4 (256) 21.7, 1 and 11 (1408) 22.2, 2 and 11 22.9,
    // 2 and 22 (1408) 25.5, 2 and 2 (128) 28.0; per layer 68.4 -> 65.7 (fewer partials too).
    const int64_t b2 = down_split(kDownRows);
    const int64_t last = b2 % kDownFillBlocks;
    auto rounds_per_byte = [](int64_t b) {
      return static_cast<double>((b + kDownFillBlocks - 1) / kDownFillBlocks) / static_cast<double>(b);
    };
    if (b2 < kDownFillBlocks || (b2 > 2 * kDownFillBlocks && last > 0 && 2 * last <= kDownFillBlocks)) {
      p.down_rows = 1;
      down_split(1);
    } else if (b2 > kDownFillBlocks && last > 0 && 2 * last <= kDownFillBlocks) {
      // Up to four residencies where every active expert is expected to hold at most two
      // assignments (its down items are then plain weight streams, whose time follows their
      // bytes) and a W2 row is not a power-of-two number of bytes. Measured, us per layer, two ->
      // four residencies: Mixtral-8x7B 4 tokens 269.1 -> 265.4 (4 -> 8 splits), DBRX 1 token
      // 249.1 -> 243.6, 4 tokens 584.8 -> 582.5, Qwen1.5-MoE 12 tokens 110.4 -> 108.6,
      // DeepSeek-V2-Lite 12 tokens 150.0 -> 147.0; Mixtral-8x22B (ffn 16384: 32 KB rows) 2 tokens
      // 367.5 -> 381.6 with 8 splits of 4 KB, hence the pitch condition.
      const int64_t w2_row = I * eb;
      const bool wide = static_cast<double>(p.N) <= 2.0 * active && (w2_row & (w2_row - 1)) != 0;
      const int64_t cap = (wide ? 4 : 2) * kDownFillBlocks;
      double best = rounds_per_byte(b2) * (1.0 - 1e-9);
      int best_r = kDownRows;
      int64_t best_s = s;
      for (int R : {kDownRows, 1}) {
        for (int64_t d = 1; d <= nchunks; ++d) {
          if (nchunks % d != 0) continue;
          const int64_t b = down_grid(R, d, nullptr);
          const double c = rounds_per_byte(b);
          if (b <= cap && c < best) {
            best = c;
            best_r = R;
            best_s = d;
          }
        }
      }
      p.down_rows = best_r;
      s = best_s;
      down_grid(best_r, best_s, &ss);
    }
    p.splits = static_cast<int>(s);
    p.split_steps = static_cast<int>(nchunks / s * kUnroll);
    // every expert is one token range (T <= span) wherever fewer waves per workgroup apply
    if (T <= p.span)
      p.gu_waves = gateup_waves(I / kRowTile, Is / kRowTile, ex, (T + p.span - 1) / p.span, p.tok_tiles);
    const int64_t hchunks = H * eb / (static_cast<int64_t>(kStepBytes) * kUnroll);
    const int64_t blocks4 = ex * ((I / kRowTile + kExpertWaves - 1) / kExpertWaves) +
                            (Is > 0 ? (T + p.span - 1) / p.span * ((Is / kRowTile + kExpertWaves - 1) / kExpertWaves) : 0);
    p.gu_ks = kGateupKSplit && g_gateup_waves == 0 && p.gu_waves == kExpertWaves && p.tok_tiles <= 2 &&
              hchunks % 2 == 0 && hchunks >= 4 && hchunks <= kGateupKSplitChunks &&
              blocks4 >= kGateupKSplitMinBlocks;
    const int gu_tiles = p.gu_ks ? 2 : p.gu_waves;  // weight tiles per gate/up workgroup
    if (Is > 0) {
      // its token ranges match the kernel's token-tile span
      const int64_t schunks = Is * eb / (static_cast<int64_t>(kStepBytes) * kUnroll);
      p.Is = static_cast<int>(Is);
      p.s_splits = static_cast<int>(ss);
      p.s_split_steps = static_cast<int>(schunks / ss * kUnroll);
      p.s_tok_groups = static_cast<int>((T + p.span - 1) / p.span);
      p.s_gateup_blocks = static_cast<int>(p.s_tok_groups * ((Is / kRowTile + gu_tiles - 1) / gu_tiles));
      p.s_down_blocks = static_cast<int>(p.s_tok_groups * ((H / (kRowTile * p.down_rows) + kExpertWaves - 1) / kExpertWaves) * ss);
    }
  }
  if (p.rows && T == 1) {
    // The single-launch form (layer1.hip): 4-wave gate/up workgroups without the K split (their
    // grid: the shared expert's, then every range's weight groups), the down waves' W2 units
    // and the activation rows within the kernel's registers and LDS, 4 output rows per
    // workgroup, and the in-launch routing of one token (E <= 64).
    const int64_t gu_tiles = p.gu_ks ? 2 : p.gu_waves;
    const int64_t groups = (I / kRowTile + gu_tiles - 1) / gu_tiles;
    const int64_t units = (I * eb + kRowsUnitBytes - 1) / kRowsUnitBytes;
    const int64_t units_s = (Is * eb + kRowsUnitBytes - 1) / kRowsUnitBytes;
    const int64_t act_bytes = (Is * eb + 15) / 16 * 16 + k * I * eb;
    p.sync_blocks = static_cast<int>(p.s_gateup_blocks + p.max_ranges * groups);
    p.layer1 = p.gu_waves == kExpertWaves && !p.gu_ks && E <= kWave && H % kExpertWaves == 0 &&
               units_s + k * units <= kLayerMaxUnits && act_bytes <= kLayerMaxActBytes &&
               p.sync_blocks <= kLayerMaxGuBlocks;
  }
  size_t o = 0;
  p.hdr = o;        o = align_up(o + 64);
  p.ranges = o;     o = align_up(o + sizeof(RangeRec) * static_cast<size_t>(p.max_ranges > 0 ? p.max_ranges : 1));
  p.sorted_f = o;   o = align_up(o + sizeof(int32_t) * p.N);
  p.tmask = o;      o = align_up(o + sizeof(int32_t) * T);
  if (p.rows) {
    p.fpos = o;     o = align_up(o + sizeof(int32_t) * p.N);
    p.fslot = o;    o = align_up(o + sizeof(int64_t) * p.N);
  }
  p.w = o;          o = align_up(o + sizeof(float) * p.N);
  p.ids = o;        o = align_up(o + sizeof(int32_t) * p.N);
  p.act = o;        o = align_up(o + static_cast<size_t>(eb) * p.N * I);
  // the fused down kernel writes y directly: no fp32 partials
  p.part = o;       if (!p.rows) o = align_up(o + sizeof(float) * static_cast<size_t>(s) * p.N * H);
  if (Is > 0) {
    p.act_s = o;    o = align_up(o + static_cast<size_t>(eb) * T * Is);
    p.part_s = o;   if (!p.rows) o = align_up(o + sizeof(float) * static_cast<size_t>(p.s_splits) * T * H);
  }
  if (layer) {
    p.logits = o;   o = align_up(o + static_cast<size_t>(eb) * T * E);
    p.sgl = o;      o = align_up(o + static_cast<size_t>(eb) * T);
  }
  if (p.layer1) {
    p.sync = o;     o = align_up(o + sizeof(uint64_t) * (static_cast<size_t>(p.sync_blocks) + 1));
  }
  p.total = o;
  return p;
}

// Workspace of a call of T tokens: the larger of the plans of its full token chunks and of its
// last, partial one.
size_t workspace_for(int64_t T, int64_t H, int64_t I, int64_t E, int64_t k, int dtype, int64_t Is,
                     bool layer) {
  const int64_t tc = chunk_tokens(T, H, I, k, Is, dtype);
  size_t total = make_plan(tc, H, I, E, k, dtype, Is, layer).total;
  const int64_t rest = T % tc;
  if (T > tc && rest > 0) total = std::max(total, make_plan(rest, H, I, E, k, dtype, Is, layer).total);
  return total;
}

RouteBuffers carve(const Plan& p, void* ws) {
  char* b = static_cast<char*>(ws);
  RouteBuffers rb;
  rb.hdr = reinterpret_cast<int32_t*>(b + p.hdr);
  rb.ranges = reinterpret_cast<RangeRec*>(b + p.ranges);
  rb.sorted_f = reinterpret_cast<int32_t*>(b + p.sorted_f);
  rb.tmask = reinterpret_cast<int32_t*>(b + p.tmask);
  rb.fpos = p.rows ? reinterpret_cast<int32_t*>(b + p.fpos) : nullptr;
  rb.fslot = p.rows ? reinterpret_cast<int64_t*>(b + p.fslot) : nullptr;
  rb.span = p.span;
  return rb;
}

// The optional block-level terms of smx_fused_moe_shared_forward.
struct BlockTerms {
  bool block = false;         // combine in the block form
  float scale = 1.0f;         // routed scaling factor
  const void* shared_page = nullptr;
  const void* sgate = nullptr;
  int sgate_dtype = kF32;
};

// Largest batch (assignments) routed inside the gate/up launch by the multi-wave form, and with
// logits its largest top-k (T * G elements: 8 wave-passes, 2 per wave). Every routed workgroup
// repeats the top-k, and its latency passes into the kernel time: measured (us per layer,
// routing kernels vs inside) DeepSeek-V2-Lite 8 tokens (T*G 512) 122.1 vs 120.6, Mixtral 64
// tokens (512) 437.1 vs 435.3, but DeepSeek-V2-Lite 16 tokens (1024) 154.4 vs 154.3, Qwen1.5-MoE
// 16 tokens (1024) 123.7 vs 125.0, DeepSeek-V2-Lite 32 tokens (2048) 181.7 vs 198.3. With ids
// given (the sort alone) the layer call gains at every size: DeepSeek-V2-Lite 32 tokens 191.7
// vs 188.8. The block top-k (eight experts per lane, one pass of the 4 waves for 32 tokens of
// 64 experts) in every workgroup lost too: DeepSeek-V2-Lite 32 tokens 178.3 -> 180.0, Qwen1.5-MoE
// 64 tokens 187.3 -> 191.6 (item walk) / 193.4 (none).
constexpr int64_t kRouteInLaunchMax = 256;
constexpr int64_t kRouteInLaunchTopkMax = 512;

// Lanes per token of the one-wave top-k: the power of two >= E, at least 8.
int route_group(int64_t E) { return E <= 8 ? 8 : E <= 16 ? 16 : E <= 32 ? 32 : 64; }

// Expert-ordered gate/up items (expert_item) apply to the multi-wave in-launch routing when
// every expert is one token range of one pass (T <= span <= the launch's token tiles, at most
// kExpertItemsMaxTiles) and the batch is expected to leave fewer than 1 in 20 experts without
// tokens: the grid then has a workgroup per (expert, weight group), and the weights an idle
// expert's workgroup issues before the routing are read for nothing. Measured per layer
// against range-ordered items: DeepSeek-V2-Lite 32 tokens (4.3% of experts expected idle)
// 175.4 -> 174.3 us, the 26-layer stack 4561 -> 4524 us; Qwen1.5-MoE 32 tokens (11% idle)
// 161.8 -> 163.7, DeepSeek-V2-Lite 16 tokens (21% idle) 155.9 -> 157.1. The top-k of such
// batches repeated in every gate/up workgroup instead of its own launch measured slower still
// (DeepSeek-V2-Lite 32 tokens 182.5 us, Qwen1.5-MoE 32 tokens 172.3), as did item walks with
// given ids (Qwen1.5-MoE 32 tokens 166.5).
constexpr double kExpertItemsMaxIdle = 0.05;
bool expert_items_apply(const Plan& p, int64_t T, int64_t E, int64_t k) {
  // (their routing loads one caller id per thread: at most 256 assignments)
  if (!g_expert_items || T > p.span || p.span > kTokTile * p.tok_tiles ||
      p.tok_tiles > kExpertItemsMaxTiles || E > kWave || k > E || T * k > kExpertWaves * kWave)
    return false;
  // expected fraction of experts no token picks (picks uniform over the experts)
  const double idle = std::pow(1.0 - static_cast<double>(k) / static_cast<double>(E), static_cast<double>(T));
  return idle < kExpertItemsMaxIdle;
}

// The routing runs inside the gate/up launch (no routing launch) for batches one wave routes:
// T*k <= 64 assignments over E <= 64 experts, every expert one token range of at most two
// token tiles, the top-k (when logits are given, in the activation dtype) in at most 4 passes
// of 64/G tokens; and in the multi-wave form (see below). Returns G, or 0 when the routing
// kernels run instead. With logits and a 0
// here, fused_forward asks again without them: the top-k launch runs and gate/up sorts its ids.
int in_launch_route_g(const Plan& p, int64_t T, int64_t E, int64_t k, bool logits, bool logits_dt_ok,
                      bool* multi) {
  *multi = false;
  if (!g_route_in_gateup) return 0;
  if (p.tiled || T < 1 || E > kWave || (logits && !logits_dt_ok)) return 0;
  const int g = route_group(E);
  // the workgroup's LDS copy of the range records holds every range the launch's grid covers
  if (T <= p.span && T * k <= kWave && p.tok_tiles <= 2 && (!logits || T * g <= kWave * kSmallRoutePasses) &&
      p.max_ranges <= kSmallRangesMax)
    return g;
  // the multi-wave form: the workgroup's 4 waves run the top-k, one wave sorts; given ids may
  // put an expert's assignments in several token ranges (T > span)
  if ((logits ? T <= p.span && T <= kWave && T * k <= kRouteInLaunchMax && T * g <= kRouteInLaunchTopkMax
              : T * k <= kGateupSortMax) &&
      p.max_ranges <= kSortRangesMax) {
    *multi = true;
    return g;
  }
  return 0;
}

// A value unique to one single-launch layer call within this process (never 0): the high 32
// bits are random per process (so workspace bytes left by another process, or any other data,
// match a call's value only by a 2^-64 chance), the low bits count calls.
uint64_t next_epoch() {
  static std::atomic<uint64_t> counter{[] {
    std::random_device rd;
    return (static_cast<uint64_t>(rd()) | 1u) << 32;
  }()};
  return counter.fetch_add(1, std::memory_order_relaxed) + 1;
}

// Wall-clock (s_memrealtime) ticks per microsecond of the current device (100 on MI355X).
int64_t wall_ticks_per_us() {
  static std::atomic<int> cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 100;
  if (dev < 64) {
    const int c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int khz = 0;
  if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess || khz < 1000) khz = 100000;
  const int per_us = khz / 1000;
  if (dev < 64) cached[dev].store(per_us, std::memory_order_relaxed);
  return per_us;
}

// The single-launch form is kept out of stream capture: its per-call value is a kernel
// argument, and a graph would replay one value.
bool capturing(hipStream_t s) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &st) != hipSuccess) return true;
  return st != hipStreamCaptureStatusNone;
}

// Shared tail of the MoE entry points: expert kernels then combine. route_g > 0: the gate/up
// launch routes the batch itself (rt).
int run_experts(const Plan& p, int dtype, const void* hidden, void* out, int64_t T, int64_t H,
                int64_t I, int64_t E, int64_t k, const void* pool, int64_t num_slots,
                int64_t page_elems, const int64_t* e2s, const float* w, const int32_t* ids,
                void* ws, hipStream_t s, const BlockTerms& bt = BlockTerms{}, int route_g = 0,
                const InRoute& rt = InRoute{}, bool route_multi = false) {
  char* b = static_cast<char*>(ws);
  ExpertArgs a{};
  a.x = hidden;
  a.pool = pool;
  a.page_elems = page_elems;
  a.e2s = e2s;
  a.rb = carve(p, ws);
  a.T = static_cast<int>(T);
  a.H = static_cast<int>(H);
  a.I = static_cast<int>(I);
  a.k = static_cast<int>(k);
  a.act = b + p.act;
  a.part = reinterpret_cast<float*>(b + p.part);
  a.splits = p.splits;
  a.split_steps = p.split_steps;
  a.down_rows = p.down_rows;
  a.gu_waves = p.gu_waves;
  a.gu_ks = p.gu_ks ? 1 : 0;
  const bool ei = route_g > 0 && route_multi && expert_items_apply(p, T, E, k);
  // the walk pays where every item's prologue would be the top-k from logits and the sort
  a.gu_items = g_gateup_walk && route_g > 0 && rt.logits != nullptr ? 1 : 0;
  a.f16out = dtype == kF32 && g_fp32_f16out ? 1 : 0;
  if (p.Is > 0) {
    a.sh.page = bt.shared_page;
    a.sh.I = p.Is;
    a.sh.act = b + p.act_s;
    a.sh.part = reinterpret_cast<float*>(b + p.part_s);
    a.sh.splits = p.s_splits;
    a.sh.split_steps = p.s_split_steps;
    a.sh.tok_groups = p.s_tok_groups;
    a.sh.gateup_blocks = p.s_gateup_blocks;
    a.sh.down_blocks = p.s_down_blocks;
  }
  a.rt = rt;
  if (p.layer1 && g_layer1 && route_g > 0 && !route_multi && !capturing(s)) {
    // one launch: gate/up workgroups, then the fused down + combine workgroups
    a.ls.flags = reinterpret_cast<uint64_t*>(b + p.sync);
    a.ls.status = a.ls.flags + p.sync_blocks;
    a.ls.epoch = next_epoch();
    a.ls.gu_blocks = p.sync_blocks;
    a.ls.publish = g_sync_publish;
    a.ls.wait_ticks = g_sync_wait_us * wall_ticks_per_us();
    a.lo.y = out;
    a.lo.block = bt.block ? 1 : 0;
    a.lo.scale = bt.scale;
    a.lo.sgate = bt.sgate;
    a.lo.sgate_dtype = bt.sgate_dtype;
    hipError_t err = launch_layer1(dtype, a, p.max_ranges, route_g, s);
    if (err != hipSuccess) return static_cast<int>(err);
    mark(2, s);
    mark(3, s);  // no down or combine launch
    mark(4, s);
    return SMX_OK;
  }
  hipError_t err = p.tiled ? launch_tile_gateup(dtype, a, p.max_ranges, s)
                           : launch_gateup(dtype, a, p.max_ranges, p.tok_tiles, s, route_g, route_multi, ei);
  if (err != hipSuccess) return static_cast<int>(err);
  mark(2, s);
  if (p.rows) {
    RowsArgs r{};
    r.pool = pool;
    r.page_bytes = page_elems * dtype_bytes(dtype);
    r.act = a.act;
    r.tmask = a.rb.tmask;
    r.fpos = a.rb.fpos;
    r.fslot = a.rb.fslot;
    r.w = w;
    r.page_s = p.Is > 0 ? bt.shared_page : nullptr;
    r.act_s = p.Is > 0 ? a.sh.act : nullptr;
    r.Is = p.Is;
    r.y = out;
    r.T = static_cast<int>(T);
    r.H = static_cast<int>(H);
    r.I = static_cast<int>(I);
    r.k = static_cast<int>(k);
    r.block = bt.block ? 1 : 0;
    r.scale = bt.scale;
    r.sgate = bt.sgate;
    r.sgate_dtype = bt.sgate_dtype;
    r.f16out = a.f16out;
    err = launch_down_rows(dtype, r, s);
    if (err != hipSuccess) return static_cast<int>(err);
    mark(3, s);
    mark(4, s);  // no combine launch
    return SMX_OK;
  }
  err = p.tiled ? launch_tile_down(dtype, a, p.max_ranges, s)
                : launch_down(dtype, a, p.max_ranges, p.tok_tiles, s);
  if (err != hipSuccess) return static_cast<int>(err);
  mark(3, s);
  CombineArgs c{};
  c.part = a.part;
  c.w = w;
  c.tmask = a.rb.tmask;
  c.y = out;
  c.T = static_cast<int>(T);
  c.H = static_cast<int>(H);
  c.k = static_cast<int>(k);
  c.splits = p.splits;
  c.block = bt.block ? 1 : 0;
  c.scale = bt.scale;
  c.part_s = p.Is > 0 ? a.sh.part : nullptr;
  c.splits_s = p.s_splits;
  c.sgate = bt.sgate;
  c.sgate_dtype = bt.sgate_dtype;
  c.rows = T >= kCombineRowsMinTokens ? 1 : 0;
  c.f16out = a.f16out;
  err = launch_combine(dtype, c, s);
  if (err != hipSuccess) return static_cast<int>(err);
  mark(4, s);
  return SMX_OK;
}

// Per-device address of `scratch`, looked up with that device current on its first use and
// kept for the life of the process. A hipDeviceReset (or an unload of the library's code
// object) while the library stays loaded would leave a stale address here: the no-allocation
// entry point does not support device resets (its header says so).
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_of_current_device(void** out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return static_cast<int>(err);
  if (dev < 0 || dev >= kMaxDevices) return SMX_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return static_cast<int>(err);
    if (p == nullptr) return static_cast<int>(hipErrorInvalidSymbol);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SMX_OK;
}

int check_pool(const void* hidden, const void* out, const void* pool, int64_t num_slots,
               int64_t page_elems, const int64_t* e2s, int64_t H, int dtype, int64_t* I) {
  if (!hidden || !out || !pool || !e2s || num_slots <= 0 || page_elems <= 0) return SMX_ERR_INVALID_ARG;
  if (page_elems % (3 * H) != 0) return SMX_ERR_INVALID_ARG;
  *I = page_elems / (3 * H);
  // 32-bit offsets and sizes within a page
  if (page_elems > (int64_t{1} << 30) || page_elems * dtype_bytes(dtype) >= (int64_t{1} << 32))
    return SMX_ERR_UNSUPPORTED;
  if (!aligned16(hidden) || !aligned16(out) || !aligned16(pool)) return SMX_ERR_MISALIGNED;
  return SMX_OK;
}

}  // namespace

namespace {

// Expert computation on the caller's routing (smx_stack_fused_moe and its block form).
int stack_forward(const void* hidden, void* out, int dtype, int64_t T, int64_t H, const void* pool,
                  int64_t num_slots, int64_t page_elems, const int64_t* expert_to_slot, int64_t E,
                  const float* topk_weights, const int32_t* topk_ids, int64_t top_k, int64_t Is,
                  const BlockTerms& bt, void* workspace, size_t workspace_bytes, void* stream) {
  if (T < 0 || H <= 0 || E <= 0 || top_k <= 0 || top_k > E || !valid_dtype(dtype)) return SMX_ERR_INVALID_ARG;
  if (T == 0) return SMX_OK;  // empty batch: tensors may have null data pointers
  int64_t I = 0;
  int rc = check_pool(hidden, out, pool, num_slots, page_elems, expert_to_slot, H, dtype, &I);
  if (rc != SMX_OK) return rc;
  rc = check_shape(T, H, I, E, top_k, dtype);
  if (rc != SMX_OK) return rc;
  rc = check_shared(T, H, Is, dtype);
  if (rc != SMX_OK) return rc;
  if (!topk_weights || !topk_ids || !workspace) return SMX_ERR_INVALID_ARG;
  const int64_t tc = chunk_tokens(T, H, I, top_k, Is, dtype);
  if (T > tc) {
    if (workspace_bytes < workspace_for(T, H, I, E, top_k, dtype, Is, false)) return SMX_ERR_WORKSPACE;
    const int64_t rb = H * dtype_bytes(dtype);
    for (int64_t t0 = 0; t0 < T; t0 += tc) {
      BlockTerms bc = bt;
      if (bc.sgate) bc.sgate = static_cast<const char*>(bc.sgate) + t0 * dtype_bytes(bc.sgate_dtype);
      rc = stack_forward(static_cast<const char*>(hidden) + t0 * rb, static_cast<char*>(out) + t0 * rb, dtype,
                         std::min(tc, T - t0), H, pool, num_slots, page_elems, expert_to_slot, E,
                         topk_weights + t0 * top_k, topk_ids + t0 * top_k, top_k, Is, bc, workspace,
                         workspace_bytes, stream);
      if (rc != SMX_OK) return rc;
    }
    return SMX_OK;
  }
  const Plan p = make_plan(T, H, I, E, top_k, dtype, Is);
  if (workspace_bytes < p.total) return SMX_ERR_WORKSPACE;
  if (!aligned16(workspace)) return SMX_ERR_MISALIGNED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  mark(0, s);
  bool rmulti = false;
  const int rg = in_launch_route_g(p, T, E, top_k, false, true, &rmulti);
  InRoute rt{};
  if (rg > 0) {
    rt.ids_in = topk_ids;
    rt.num_slots = num_slots;
    rt.E = static_cast<int>(E);
  } else {
    hipError_t err = launch_route(nullptr, kF32, static_cast<int>(T), static_cast<int>(E), static_cast<int>(top_k),
                                  0, nullptr, nullptr, topk_ids, expert_to_slot, num_slots, carve(p, workspace), s);
    if (err != hipSuccess) return static_cast<int>(err);
  }
  mark(1, s);
  return run_experts(p, dtype, hidden, out, T, H, I, E, top_k, pool, num_slots, page_elems,
                     expert_to_slot, topk_weights, topk_ids, workspace, s, bt, rg, rt, rmulti);
}

}  // namespace

extern "C" {

int smx_version(void) { return kVersion; }

const char* smx_error_string(int code) {
  switch (code) {
    case SMX_OK: return "success";
    case SMX_ERR_INVALID_ARG: return "invalid argument";
    case SMX_ERR_UNSUPPORTED: return "shape outside the supported limits";
    case SMX_ERR_WORKSPACE: return "workspace too small";
    case SMX_ERR_MISALIGNED: return "tensor base not 16-byte aligned";
    case SMX_ERR_TIMEOUT: return "timed out waiting for a transfer task";
    case SMX_ERR_NOT_FOUND: return "no such transfer task";
    case SMX_ERR_SCRATCH: return "sizes need more workspace than the no-allocation scratch holds";
    default: return hipGetErrorString(static_cast<hipError_t>(code));
  }
}

int smx_topk_softmax(const void* logits, int logits_dtype, int64_t T, int64_t E, int64_t top_k,
                     int renormalize, float* topk_weights, int32_t* topk_ids, void* stream) {
  if (T < 0 || E <= 0 || top_k <= 0 || top_k > E || !valid_dtype(logits_dtype)) return SMX_ERR_INVALID_ARG;
  if (E > kMaxExperts || top_k > kMaxTopK || T > (int64_t{1} << 30) / top_k) return SMX_ERR_UNSUPPORTED;
  if (T == 0) return SMX_OK;
  if (!logits || !topk_weights || !topk_ids) return SMX_ERR_INVALID_ARG;
  return static_cast<int>(launch_topk_softmax(logits, logits_dtype, static_cast<int>(T), static_cast<int>(E),
                                              static_cast<int>(top_k), renormalize, topk_weights, topk_ids,
                                              static_cast<hipStream_t>(stream)));
}

int smx_grouped_topk(const void* logits, int logits_dtype, int64_t T, int64_t E, int64_t top_k,
                     int renormalize, int64_t num_expert_group, int64_t topk_group,
                     const float* correction_bias, float* topk_weights, int32_t* topk_ids, void* stream) {
  if (T < 0 || E <= 0 || top_k <= 0 || !valid_dtype(logits_dtype) || num_expert_group <= 0 ||
      topk_group <= 0 || topk_group > num_expert_group || E % num_expert_group != 0)
    return SMX_ERR_INVALID_ARG;
  const int64_t gs = E / num_expert_group;
  if (top_k > topk_group * gs || (correction_bias && gs < 2)) return SMX_ERR_INVALID_ARG;
  if (E > kMaxExperts || top_k > kMaxTopK || num_expert_group > kWave || T > (int64_t{1} << 30) / top_k)
    return SMX_ERR_UNSUPPORTED;
  if (T == 0) return SMX_OK;
  if (!logits || !topk_weights || !topk_ids) return SMX_ERR_INVALID_ARG;
  return static_cast<int>(launch_grouped_topk(
      logits, logits_dtype, static_cast<int>(T), static_cast<int>(E), static_cast<int>(top_k), renormalize,
      static_cast<int>(num_expert_group), static_cast<int>(topk_group), correction_bias, topk_weights,
      topk_ids, static_cast<hipStream_t>(stream)));
}

int smx_moe_align_block_size(const int32_t* topk_ids, int64_t numel, int64_t E, int64_t block_size,
                             int32_t* sorted_ids, int32_t* expert_ids, int32_t* num_tokens_post_pad,
                             void* stream) {
  if (numel < 0 || E <= 0 || block_size <= 0) return SMX_ERR_INVALID_ARG;
  if (E > kMaxExperts || numel > kMaxAssignments || block_size > (1 << 16)) return SMX_ERR_UNSUPPORTED;
  if (!sorted_ids || !expert_ids || !num_tokens_post_pad || (numel > 0 && !topk_ids)) return SMX_ERR_INVALID_ARG;
  return static_cast<int>(launch_align(topk_ids, static_cast<int>(numel), static_cast<int>(E),
                                       static_cast<int>(block_size), sorted_ids, expert_ids,
                                       num_tokens_post_pad, static_cast<hipStream_t>(stream)));
}

int smx_moe_plan_info(int64_t T, int64_t H, int64_t I, int64_t E, int64_t top_k, int64_t shared_I,
                      int dtype, int64_t* out, int n) {
  if (n < 0 || (n > 0 && !out)) return SMX_ERR_INVALID_ARG;
  int rc = check_shape(T, H, I, E, top_k, dtype);
  if (rc != SMX_OK) return rc;
  rc = check_shared(T, H, shared_I, dtype);
  if (rc != SMX_OK) return rc;
  const int64_t tc = chunk_tokens(T, H, I, top_k, shared_I, dtype);
  const Plan p = make_plan(std::min(T, tc), H, I, E, top_k, dtype, shared_I);
  int64_t v[SMX_PLAN_FIELDS] = {};
  v[SMX_PLAN_TILED] = p.tiled;
  v[SMX_PLAN_FUSED_DOWN] = p.rows;
  v[SMX_PLAN_SPAN] = p.span;
  v[SMX_PLAN_MAX_RANGES] = p.max_ranges;
  v[SMX_PLAN_TOK_TILES] = p.tok_tiles;
  v[SMX_PLAN_SPLITS] = p.splits;
  v[SMX_PLAN_SPLIT_STEPS] = p.split_steps;
  v[SMX_PLAN_DOWN_ROWS] = p.down_rows;
  v[SMX_PLAN_GATEUP_WAVES] = p.gu_waves;
  v[SMX_PLAN_GATEUP_KSPLIT] = p.gu_ks;
  v[SMX_PLAN_SHARED_SPLITS] = p.Is > 0 ? p.s_splits : 0;
  v[SMX_PLAN_SHARED_SPLIT_STEPS] = p.Is > 0 ? p.s_split_steps : 0;
  v[SMX_PLAN_SHARED_TOK_GROUPS] = p.s_tok_groups;
  v[SMX_PLAN_SHARED_GATEUP_BLOCKS] = p.s_gateup_blocks;
  v[SMX_PLAN_SHARED_DOWN_BLOCKS] = p.s_down_blocks;
  if (p.tiled) {
    v[SMX_PLAN_TILE_GATEUP_GRID] = tile_grid_blocks(0, H, I, p.s_gateup_blocks, p.max_ranges, 1);
    v[SMX_PLAN_TILE_DOWN_GRID] = tile_grid_blocks(1, H, I, p.s_down_blocks, p.max_ranges, p.splits);
  }
  v[SMX_PLAN_SINGLE_LAUNCH] = p.layer1 && g_layer1;
  v[SMX_PLAN_SYNC_BLOCKS] = p.layer1 ? p.sync_blocks : 0;
  v[SMX_PLAN_SYNC_OFFSET] = p.layer1 ? static_cast<int64_t>(p.sync) : -1;
  const int64_t Tp = std::min(T, tc);
  bool multi = false;
  v[SMX_PLAN_TOPK_IN_GATEUP] = in_launch_route_g(p, Tp, E, top_k, true, true, &multi) > 0;
  const bool ids_multi = in_launch_route_g(p, Tp, E, top_k, false, true, &multi) > 0 && multi;
  v[SMX_PLAN_EXPERT_ITEMS] = ids_multi && expert_items_apply(p, Tp, E, top_k);
  v[SMX_PLAN_CHUNK_TOKENS] = tc;
  v[SMX_PLAN_WORKSPACE_BYTES] = static_cast<int64_t>(workspace_for(T, H, I, E, top_k, dtype, shared_I, false));
  for (int i = 0; i < n && i < SMX_PLAN_FIELDS; ++i) out[i] = v[i];
  return SMX_PLAN_FIELDS;
}

size_t smx_moe_workspace_size(int64_t T, int64_t H, int64_t I, int64_t E, int64_t top_k, int dtype) {
  if (check_shape(T, H, I, E, top_k, dtype) != SMX_OK) return 0;
  return workspace_for(T, H, I, E, top_k, dtype, 0, false);
}

int smx_stack_fused_moe(const void* hidden, void* out, int dtype, int64_t T, int64_t H,
                        const void* pool, int64_t num_slots, int64_t page_elems,
                        const int64_t* expert_to_slot, int64_t E,
                        const float* topk_weights, const int32_t* topk_ids, int64_t top_k,
                        void* workspace, size_t workspace_bytes, void* stream) {
  return stack_forward(hidden, out, dtype, T, H, pool, num_slots, page_elems, expert_to_slot, E,
                       topk_weights, topk_ids, top_k, 0, BlockTerms{}, workspace, workspace_bytes,
                       stream);
}

int smx_stack_fused_moe_shared(const void* hidden, void* out, int dtype, int64_t T, int64_t H,
                               const void* pool, int64_t num_slots, int64_t page_elems,
                               const int64_t* expert_to_slot, int64_t E,
                               const float* topk_weights, const int32_t* topk_ids, int64_t top_k,
                               const void* shared_page, int64_t shared_I,
                               const void* shared_gate_logits, float routed_scaling_factor,
                               void* workspace, size_t workspace_bytes, void* stream) {
  if (shared_I < 0 || (shared_I == 0) != (shared_page == nullptr) ||
      (shared_I == 0 && shared_gate_logits != nullptr) || !std::isfinite(routed_scaling_factor))
    return SMX_ERR_INVALID_ARG;
  if (T > 0 && shared_page && !aligned16(shared_page)) return SMX_ERR_MISALIGNED;
  BlockTerms bt;
  bt.block = true;
  bt.scale = routed_scaling_factor;
  bt.shared_page = shared_page;
  bt.sgate = shared_gate_logits;
  bt.sgate_dtype = dtype;
  return stack_forward(hidden, out, dtype, T, H, pool, num_slots, page_elems, expert_to_slot, E,
                       topk_weights, topk_ids, top_k, shared_I, bt, workspace, workspace_bytes, stream);
}

}  // extern "C"

namespace {

// Routing plus expert computation (smx_fused_moe_forward and its block form).
int fused_forward(const void* hidden, void* out, int dtype, int64_t T, int64_t H,
                  const void* router_logits, int logits_dtype, int64_t E, int64_t top_k,
                  int renormalize, const void* pool, int64_t num_slots, int64_t page_elems,
                  const int64_t* expert_to_slot, int64_t Is, const BlockTerms& bt,
                  float* topk_weights_out, int32_t* topk_ids_out, void* workspace,
                  size_t workspace_bytes, void* stream) {
  if (T < 0 || H <= 0 || E <= 0 || top_k <= 0 || top_k > E || !valid_dtype(dtype) ||
      !valid_dtype(logits_dtype))
    return SMX_ERR_INVALID_ARG;
  if (T == 0) return SMX_OK;  // empty batch: tensors may have null data pointers
  int64_t I = 0;
  int rc = check_pool(hidden, out, pool, num_slots, page_elems, expert_to_slot, H, dtype, &I);
  if (rc != SMX_OK) return rc;
  rc = check_shape(T, H, I, E, top_k, dtype);
  if (rc != SMX_OK) return rc;
  rc = check_shared(T, H, Is, dtype);
  if (rc != SMX_OK) return rc;
  if (!router_logits || !workspace) return SMX_ERR_INVALID_ARG;
  const int64_t tc = chunk_tokens(T, H, I, top_k, Is, dtype);
  if (T > tc) {
    if (workspace_bytes < workspace_for(T, H, I, E, top_k, dtype, Is, false)) return SMX_ERR_WORKSPACE;
    const int64_t rb = H * dtype_bytes(dtype);
    const int64_t lb = E * dtype_bytes(logits_dtype);
    for (int64_t t0 = 0; t0 < T; t0 += tc) {
      BlockTerms bc = bt;
      if (bc.sgate) bc.sgate = static_cast<const char*>(bc.sgate) + t0 * dtype_bytes(bc.sgate_dtype);
      rc = fused_forward(static_cast<const char*>(hidden) + t0 * rb, static_cast<char*>(out) + t0 * rb, dtype,
                         std::min(tc, T - t0), H, static_cast<const char*>(router_logits) + t0 * lb,
                         logits_dtype, E, top_k, renormalize, pool, num_slots, page_elems, expert_to_slot,
                         Is, bc, topk_weights_out ? topk_weights_out + t0 * top_k : nullptr,
                         topk_ids_out ? topk_ids_out + t0 * top_k : nullptr, workspace, workspace_bytes,
                         stream);
      if (rc != SMX_OK) return rc;
    }
    return SMX_OK;
  }
  const Plan p = make_plan(T, H, I, E, top_k, dtype, Is);
  if (workspace_bytes < p.total) return SMX_ERR_WORKSPACE;
  if (!aligned16(workspace)) return SMX_ERR_MISALIGNED;
  char* b = static_cast<char*>(workspace);
  float* w = topk_weights_out ? topk_weights_out : reinterpret_cast<float*>(b + p.w);
  int32_t* ids = topk_ids_out ? topk_ids_out : reinterpret_cast<int32_t*>(b + p.ids);
  hipStream_t s = static_cast<hipStream_t>(stream);
  mark(0, s);
  bool rmulti = false;
  int rg = in_launch_route_g(p, T, E, top_k, true, logits_dtype == dtype, &rmulti);
  InRoute rt{};
  rt.num_slots = num_slots;
  rt.E = static_cast<int>(E);
  if (rg > 0) {
    rt.logits = router_logits;
    rt.w_out = w;
    rt.ids_out = ids;
    rt.renorm = renormalize;
  } else if ((rg = in_launch_route_g(p, T, E, top_k, false, true, &rmulti)) > 0) {
    // a top-k too large to repeat in every workgroup: its own launch, the sort inside gate/up
    hipError_t err = launch_topk_softmax(router_logits, logits_dtype, static_cast<int>(T),
                                         static_cast<int>(E), static_cast<int>(top_k), renormalize,
                                         w, ids, s);
    if (err != hipSuccess) return static_cast<int>(err);
    rt.ids_in = ids;
  } else {
    hipError_t err = launch_route(router_logits, logits_dtype, static_cast<int>(T), static_cast<int>(E),
                                  static_cast<int>(top_k), renormalize, w, ids, nullptr, expert_to_slot,
                                  num_slots, carve(p, workspace), s);
    if (err != hipSuccess) return static_cast<int>(err);
  }
  mark(1, s);
  return run_experts(p, dtype, hidden, out, T, H, I, E, top_k, pool, num_slots, page_elems,
                     expert_to_slot, w, ids, workspace, s, bt, rg, rt, rmulti);
}

}  // namespace

extern "C" {

int smx_fused_moe_forward(const void* hidden, void* out, int dtype, int64_t T, int64_t H,
                          const void* router_logits, int logits_dtype, int64_t E, int64_t top_k,
                          int renormalize, const void* pool, int64_t num_slots, int64_t page_elems,
                          const int64_t* expert_to_slot, float* topk_weights_out,
                          int32_t* topk_ids_out, void* workspace, size_t workspace_bytes,
                          void* stream) {
  return fused_forward(hidden, out, dtype, T, H, router_logits, logits_dtype, E, top_k, renormalize,
                       pool, num_slots, page_elems, expert_to_slot, 0, BlockTerms{}, topk_weights_out,
                       topk_ids_out, workspace, workspace_bytes, stream);
}

int smx_fused_moe_forward_noalloc(const void* hidden, void* out, int dtype, int64_t T, int64_t H,
                                  const void* router_logits, int logits_dtype, int64_t E,
                                  int64_t top_k, int renormalize, const void* pool,
                                  int64_t num_slots, int64_t page_elems,
                                  const int64_t* expert_to_slot, float* topk_weights_out,
                                  int32_t* topk_ids_out, void* stream) {
  if (T < 0 || H <= 0 || E <= 0 || top_k <= 0 || top_k > E || !valid_dtype(dtype) ||
      page_elems <= 0 || page_elems % (3 * H) != 0)
    return SMX_ERR_INVALID_ARG;
  if (T == 0) return SMX_OK;
  const int64_t I = page_elems / (3 * H);
  int rc = check_shape(T, H, I, E, top_k, dtype);
  if (rc != SMX_OK) return rc;
  // nothing in the workspace has to start at zero: every kernel writes what it later reads
  const size_t need = workspace_for(T, H, I, E, top_k, dtype, 0, false);
  if (need > SMX_NOALLOC_SCRATCH_BYTES) return SMX_ERR_SCRATCH;
  void* ws = nullptr;
  rc = scratch_of_current_device(&ws);
  if (rc != SMX_OK) return rc;
  return fused_forward(hidden, out, dtype, T, H, router_logits, logits_dtype, E, top_k, renormalize,
                       pool, num_slots, page_elems, expert_to_slot, 0, BlockTerms{}, topk_weights_out,
                       topk_ids_out, ws, SMX_NOALLOC_SCRATCH_BYTES, stream);
}

size_t smx_moe_shared_workspace_size(int64_t T, int64_t H, int64_t I, int64_t E, int64_t top_k,
                                     int64_t shared_I, int dtype) {
  if (check_shape(T, H, I, E, top_k, dtype) != SMX_OK || check_shared(T, H, shared_I, dtype) != SMX_OK)
    return 0;
  return workspace_for(T, H, I, E, top_k, dtype, shared_I, false);
}

int smx_fused_moe_shared_forward(const void* hidden, void* out, int dtype, int64_t T, int64_t H,
                                 const void* router_logits, int logits_dtype, int64_t E,
                                 int64_t top_k, int renormalize, const void* pool,
                                 int64_t num_slots, int64_t page_elems,
                                 const int64_t* expert_to_slot, const void* shared_page,
                                 int64_t shared_I, const void* shared_gate_logits,
                                 float routed_scaling_factor, float* topk_weights_out,
                                 int32_t* topk_ids_out, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  if (shared_I < 0 || (shared_I == 0) != (shared_page == nullptr) ||
      (shared_I == 0 && shared_gate_logits != nullptr) || !std::isfinite(routed_scaling_factor))
    return SMX_ERR_INVALID_ARG;
  if (T > 0 && shared_page && !aligned16(shared_page)) return SMX_ERR_MISALIGNED;
  BlockTerms bt;
  bt.block = true;
  bt.scale = routed_scaling_factor;
  bt.shared_page = shared_page;
  bt.sgate = shared_gate_logits;
  bt.sgate_dtype = logits_dtype;
  return fused_forward(hidden, out, dtype, T, H, router_logits, logits_dtype, E, top_k, renormalize,
                       pool, num_slots, page_elems, expert_to_slot, shared_I, bt, topk_weights_out,
                       topk_ids_out, workspace, workspace_bytes, stream);
}

int smx_add_rmsnorm_gate(const void* hidden, void* residual, void* normed_out, int dtype, int64_t T,
                         int64_t H, const void* norm_weight, float eps, const void* gate_weight,
                         int64_t E, void* router_logits, void* stream) {
  if (T < 0 || !std::isfinite(eps) || eps < 0.0f) return SMX_ERR_INVALID_ARG;
  int rc = check_norm(H, dtype);
  if (rc != SMX_OK) return rc;
  if (gate_weight && E <= 0) return SMX_ERR_INVALID_ARG;
  if (gate_weight && E > kMaxExperts) return SMX_ERR_UNSUPPORTED;
  if (T == 0) return SMX_OK;  // empty batch: tensors may have null data pointers
  if (!hidden || !normed_out || !norm_weight || (gate_weight && !router_logits)) return SMX_ERR_INVALID_ARG;
  if (!aligned16(hidden) || !aligned16(normed_out) || !aligned16(norm_weight) ||
      (residual && !aligned16(residual)) || (gate_weight && !aligned16(gate_weight)))
    return SMX_ERR_MISALIGNED;
  NormGateArgs a{};
  a.x = hidden;
  a.residual = residual;
  a.xn = normed_out;
  a.norm_w = norm_weight;
  a.eps = eps;
  a.gate_w = gate_weight;
  a.logits = router_logits;
  a.T = static_cast<int>(T);
  a.H = static_cast<int>(H);
  a.E = gate_weight ? static_cast<int>(E) : 0;
  a.dtype = dtype;
  return static_cast<int>(launch_norm_gate(a, static_cast<hipStream_t>(stream)));
}

size_t smx_moe_layer_workspace_size(int64_t T, int64_t H, int64_t I, int64_t E, int64_t top_k,
                                    int64_t shared_I, int dtype) {
  if (check_shape(T, H, I, E, top_k, dtype) != SMX_OK || check_shared(T, H, shared_I, dtype) != SMX_OK ||
      check_norm(H, dtype) != SMX_OK)
    return 0;
  return workspace_for(T, H, I, E, top_k, dtype, shared_I, true);
}

int smx_moe_layer_forward(void* hidden, void* residual, int dtype, int64_t T, int64_t H,
                          const void* norm_weight, float eps, const void* gate_weight, int64_t E,
                          int64_t top_k, int renormalize, const void* pool, int64_t num_slots,
                          int64_t page_elems, const int64_t* expert_to_slot,
                          const void* shared_page, int64_t shared_I,
                          const void* shared_gate_weight, float routed_scaling_factor,
                          void* router_logits_out, float* topk_weights_out,
                          int32_t* topk_ids_out, void* workspace, size_t workspace_bytes,
                          void* stream) {
  if (T < 0 || H <= 0 || E <= 0 || top_k <= 0 || top_k > E || !valid_dtype(dtype) ||
      !std::isfinite(eps) || eps < 0.0f || !std::isfinite(routed_scaling_factor))
    return SMX_ERR_INVALID_ARG;
  if (shared_I < 0 || (shared_I == 0) != (shared_page == nullptr) ||
      (shared_I == 0 && shared_gate_weight != nullptr))
    return SMX_ERR_INVALID_ARG;
  if (T == 0) return SMX_OK;  // empty batch: tensors may have null data pointers
  int64_t I = 0;
  int rc = check_pool(hidden, hidden, pool, num_slots, page_elems, expert_to_slot, H, dtype, &I);
  if (rc != SMX_OK) return rc;
  rc = check_shape(T, H, I, E, top_k, dtype);
  if (rc != SMX_OK) return rc;
  rc = check_shared(T, H, shared_I, dtype);
  if (rc != SMX_OK) return rc;
  rc = check_norm(H, dtype);
  if (rc != SMX_OK) return rc;
  if (!residual || !norm_weight || !gate_weight || !workspace) return SMX_ERR_INVALID_ARG;
  if (!aligned16(residual) || !aligned16(norm_weight) || !aligned16(gate_weight) ||
      (shared_page && !aligned16(shared_page)) ||
      (shared_gate_weight && !aligned16(shared_gate_weight)))
    return SMX_ERR_MISALIGNED;
  const int64_t tc = chunk_tokens(T, H, I, top_k, shared_I, dtype);
  if (T > tc) {
    if (workspace_bytes < workspace_for(T, H, I, E, top_k, dtype, shared_I, true)) return SMX_ERR_WORKSPACE;
    const int64_t rb = H * dtype_bytes(dtype);
    const int64_t lb = E * dtype_bytes(dtype);
    for (int64_t t0 = 0; t0 < T; t0 += tc) {
      rc = smx_moe_layer_forward(
          static_cast<char*>(hidden) + t0 * rb, static_cast<char*>(residual) + t0 * rb, dtype,
          std::min(tc, T - t0), H, norm_weight, eps, gate_weight, E, top_k, renormalize, pool, num_slots,
          page_elems, expert_to_slot, shared_page, shared_I, shared_gate_weight, routed_scaling_factor,
          router_logits_out ? static_cast<char*>(router_logits_out) + t0 * lb : nullptr,
          topk_weights_out ? topk_weights_out + t0 * top_k : nullptr,
          topk_ids_out ? topk_ids_out + t0 * top_k : nullptr, workspace, workspace_bytes, stream);
      if (rc != SMX_OK) return rc;
    }
    return SMX_OK;
  }
  const Plan p = make_plan(T, H, I, E, top_k, dtype, shared_I, true);
  if (workspace_bytes < p.total) return SMX_ERR_WORKSPACE;
  if (!aligned16(workspace)) return SMX_ERR_MISALIGNED;
  char* b = static_cast<char*>(workspace);
  float* w = topk_weights_out ? topk_weights_out : reinterpret_cast<float*>(b + p.w);
  int32_t* ids = topk_ids_out ? topk_ids_out : reinterpret_cast<int32_t*>(b + p.ids);
  hipStream_t s = static_cast<hipStream_t>(stream);
  mark(0, s);
  NormGateArgs g{};
  g.x = hidden;
  g.residual = residual;
  g.xn = hidden;
  g.norm_w = norm_weight;
  g.eps = eps;
  g.gate_w = gate_weight;
  g.sgate_w = shared_gate_weight;
  g.logits = router_logits_out ? router_logits_out : static_cast<void*>(b + p.logits);
  g.sgate_logits = b + p.sgl;
  g.topk_w = w;
  g.topk_ids = ids;
  g.T = static_cast<int>(T);
  g.H = static_cast<int>(H);
  g.E = static_cast<int>(E);
  g.k = static_cast<int>(top_k);
  g.renorm = renormalize;
  g.dtype = dtype;
  // one token over at most 64 experts: the norm kernel's top-k wave also writes the expert
  // sort, and no routing kernel is launched
  const bool sort_in_norm = T == 1 && E <= kWave;
  if (sort_in_norm) {
    g.route = 1;
    g.rb = carve(p, workspace);
    g.e2s = expert_to_slot;
    g.num_slots = num_slots;
  }
  hipError_t err = launch_norm_gate(g, s);
  if (err != hipSuccess) return static_cast<int>(err);
  // larger small batches: the sort of the norm kernel's picks inside the gate/up launch
  bool rmulti = false;
  const int rg = sort_in_norm ? 0 : in_launch_route_g(p, T, E, top_k, false, true, &rmulti);
  InRoute rt{};
  if (rg > 0) {
    rt.ids_in = ids;
    rt.num_slots = num_slots;
    rt.E = static_cast<int>(E);
  } else if (!sort_in_norm) {
    err = launch_route(nullptr, kF32, static_cast<int>(T), static_cast<int>(E), static_cast<int>(top_k), 0,
                       nullptr, nullptr, ids, expert_to_slot, num_slots, carve(p, workspace), s);
    if (err != hipSuccess) return static_cast<int>(err);
  }
  mark(1, s);
  BlockTerms bt;
  bt.block = shared_I > 0 || routed_scaling_factor != 1.0f;
  bt.scale = routed_scaling_factor;
  bt.shared_page = shared_page;
  bt.sgate = shared_gate_weight ? b + p.sgl : nullptr;
  bt.sgate_dtype = dtype;
  return run_experts(p, dtype, hidden, hidden, T, H, I, E, top_k, pool, num_slots, page_elems,
                     expert_to_slot, w, ids, workspace, s, bt, rg, rt, rmulti);
}

int smx_set_tiled_min_tokens(int64_t tokens_per_expert) {
  g_tile_min_tokens = tokens_per_expert < 0 ? kTileMinTokensDefault : tokens_per_expert;
  return SMX_OK;
}

int64_t smx_tiled_min_tokens(void) { return g_tile_min_tokens; }

int smx_set_fused_down_max_tokens(int64_t tokens) {
  g_rows_max_tokens = tokens < 0 ? -1 : std::min<int64_t>(tokens, kRowsMaxTokens);
  return SMX_OK;
}

int64_t smx_fused_down_max_tokens(void) { return g_rows_max_tokens; }

int smx_set_fp32_gemm_outputs_fp16(int on) {
  g_fp32_f16out = on != 0;
  return SMX_OK;
}

int smx_fp32_gemm_outputs_fp16(void) { return g_fp32_f16out ? 1 : 0; }

int smx_set_routing_in_gateup(int on) {
  g_route_in_gateup = on != 0;
  return SMX_OK;
}

int smx_routing_in_gateup(void) { return g_route_in_gateup ? 1 : 0; }

int smx_set_gateup_waves(int waves) {
  if (waves != 0 && waves != 1 && waves != 2 && waves != 4) return SMX_ERR_INVALID_ARG;
  g_gateup_waves = waves;
  return SMX_OK;
}

int smx_gateup_waves(void) { return g_gateup_waves; }

int smx_set_gateup_item_walk(int on) {
  g_gateup_walk = on != 0;
  return SMX_OK;
}

int smx_gateup_item_walk(void) { return g_gateup_walk ? 1 : 0; }

int smx_set_gateup_expert_items(int on) {
  g_expert_items = on != 0;
  return SMX_OK;
}

int smx_gateup_expert_items(void) { return g_expert_items ? 1 : 0; }

int smx_set_single_launch_layer(int on) {
  g_layer1 = on != 0;
  return SMX_OK;
}

int smx_single_launch_layer(void) { return g_layer1 ? 1 : 0; }

int smx_set_layer_sync_test(int publish, int64_t wait_us) {
  g_sync_publish = publish != 0 ? 1 : 0;
  g_sync_wait_us = wait_us > 0 ? wait_us : kSyncWaitDefaultUs;
  return SMX_OK;
}

int smx_set_profile_events(void* const* events, int count) {
  if (events == nullptr || count == 0) {
    g_profiling = false;
    return SMX_OK;
  }
  if (count != kProfileEvents) return SMX_ERR_INVALID_ARG;
  for (int i = 0; i < kProfileEvents; ++i) {
    if (events[i] == nullptr) return SMX_ERR_INVALID_ARG;
    g_profile[i] = static_cast<hipEvent_t>(events[i]);
  }
  g_profiling = true;
  return SMX_OK;
}

}  // extern "C"
