// Expert kernels of the verify-step MoE: weight-streaming grouped SwiGLU on MFMA.
//
// At verify-step token counts every routed expert sees few tokens, so the expert weights
// are the only large operand: each weight byte is read from HBM exactly once, by one wave,
// with 16-byte-per-lane loads laid out as MFMA A fragments (16 rows x 64 bytes per load
// step), and the few token rows ride along as the B operand (L2-resident). The MFMA makes
// the flops free, so the kernels run at the rate weights stream in.
//
//   gateup_kernel   wave = (active expert, 16 intermediate columns): streams the 16 matching
//                   rows of W1 (gate) and W3 (up) over K = H, then fuses the epilogue
//                   act = round(silu(round(gate)) * round(up)) into `act` (row = sorted pos).
//   down_kernel     wave = (active expert, 32 rows of W2, K split): streams W2 over its K
//                   slice of I and writes fp32 partials part[split][f][h].
//   combine_kernel  y[t] = round(sum_j round(w[t,j] * sum_split part[split][t*k+j])).
//
// Arithmetic and rounding points follow stack_fused_moe
// (specmoe/layers/fused_moe_kernel.py:319-349): C1 rounded to the activation dtype (:203),
// silu_and_mul (:337), the down GEMM scaled by the routing weight before rounding (:197-203),
// and the fp32 top-k sum rounded once (:344-347).
#include "smx_kernels.h"

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
constexpr int kBufDword3 = 0x00020000;            // gfx9 raw-buffer resource word 3
constexpr int kNonTemporal = 2;                   // cache-policy bit: streaming (read once)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), kBufDword3);
}

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

template <int R>
__device__ __forceinline__ void load_raw(Raw<R>& c, const WeightStream& w, int chunk) {
  const uint32_t cbase = w.base + static_cast<uint32_t>(chunk) * (kStepBytes * kUnroll);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < R; ++r)
      c.v[i][r] = __builtin_amdgcn_raw_buffer_load_b128(
          w.rsrc, w.lane_off, cbase + r * w.tile_stride + i * w.row4, kNonTemporal);
}

// Token operand, shared by the workgroup. The 4 waves of a workgroup work on the same expert
// and step through K together. Each chunk of the MT token tiles (16 token rows x 256 bytes
// each) is loaded once per workgroup -- wave w loads rows 4w..4w+3 of every tile, one
// 4-row x 256-byte instruction per tile -- into a double-buffered LDS tile with the same
// padded layout as the weight tiles, and every wave reads its MFMA B fragments from there.
// One barrier per chunk; every wave of a workgroup runs the same number of chunks.
template <int MT>
struct SharedTokens {
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t base;     // byte offset of the K range (wave-uniform)
  uint32_t off[MT];  // per lane: offset of row 4*wave + l/16 of tile j, + 16*(l%16)
};

template <int MT>
struct RawTokens {
  u32x4 v[MT];
};

template <int MT>
__device__ __forceinline__ void load_tokens(RawTokens<MT>& rb, const SharedTokens<MT>& t, int chunk) {
  const uint32_t cbase = t.base + static_cast<uint32_t>(chunk) * (kStepBytes * kUnroll);
#pragma unroll
  for (int j = 0; j < MT; ++j) rb.v[j] = __builtin_amdgcn_raw_buffer_load_b128(t.rsrc, t.off[j], cbase, 0);
}

template <int MT>
__device__ __forceinline__ void store_tokens(const RawTokens<MT>& rb, u32x4* bt) {
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  u32x4* wr = bt + kPitch * (4 * wave + (lane >> 4)) + (lane & 15);
#pragma unroll
  for (int j = 0; j < MT; ++j) wr[j * kTileSlots] = rb.v[j];
}

// Workgroup barrier ordering LDS only: in-flight global loads stay in flight.
__device__ __forceinline__ void wg_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// One chunk: issue the next chunk's token loads, then its weight loads (so waiting for the
// tokens never waits for the weights); transpose this chunk's weights through the
// wave-private LDS tile; MFMAs against the shared token tile `bt`; publish the next chunk's
// token tile into `bt_next`; barrier.
template <int DT, int R, int MT, bool kPrefetch>
__device__ __forceinline__ void wg_chunk(const Raw<R>& c, Raw<R>& next, RawTokens<MT>& rb,
                                         u32x4* lds, const u32x4* bt, u32x4* bt_next,
                                         const WeightStream& w, const SharedTokens<MT>& t,
                                         int chunk, f32x4 (&acc)[R][MT]) {
  const int lane = lane_id();
  if constexpr (kPrefetch) {
    load_tokens(rb, t, chunk + 1);
    load_raw(next, w, chunk + 1);
  }
  // Keep the scheduler from sinking loads into the MFMA sequence (which would shrink the
  // prefetch distance) or from waiting on the prefetch early.
  __builtin_amdgcn_sched_barrier(0);
  u32x4* wr = lds + kPitch * (lane >> 4) + (lane & 15);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < R; ++r) wr[r * kTileSlots + 4 * kPitch * i] = c.v[i][r];
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
  if constexpr (kPrefetch) store_tokens(rb, bt_next);
  wg_barrier();
}

// acc[r][mt] += A_r (16 rows x nchunks*256 bytes) . B_mt, the workgroup streaming the token
// chunks through `bsh` (two buffers of MT tiles) while each wave streams its own weights.
template <int DT, int R, int MT>
__device__ __forceinline__ void stream_wg(const WeightStream& w, const SharedTokens<MT>& t,
                                          int nchunks, u32x4* lds, u32x4* bsh,
                                          f32x4 (&acc)[R][MT]) {
  Raw<R> c0, c1;
  RawTokens<MT> rb;
  u32x4* b0 = bsh;
  u32x4* b1 = bsh + MT * kTileSlots;
  load_tokens(rb, t, 0);
  load_raw(c0, w, 0);
  store_tokens(rb, b0);
  wg_barrier();
  int c = 0;
  for (; c + 2 < nchunks; c += 2) {
    wg_chunk<DT, R, MT, true>(c0, c1, rb, lds, b0, b1, w, t, c, acc);
    wg_chunk<DT, R, MT, true>(c1, c0, rb, lds, b1, b0, w, t, c + 1, acc);
  }
  if (c + 1 < nchunks) {
    wg_chunk<DT, R, MT, true>(c0, c1, rb, lds, b0, b1, w, t, c, acc);
    wg_chunk<DT, R, MT, false>(c1, c0, rb, lds, b1, b0, w, t, c + 1, acc);
  } else {
    wg_chunk<DT, R, MT, false>(c0, c1, rb, lds, b0, b1, w, t, c, acc);
  }
}

__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + __expf(-g)); }

// Store 4 consecutive elements (one accumulator register group) of an output row.
template <int DT>
__device__ __forceinline__ void store4(void* base, int64_t idx, float v0, float v1, float v2, float v3) {
  using S = typename Elem<DT>::S;
  if constexpr (DT == kF32) {
    f32x4 v = {v0, v1, v2, v3};
    *reinterpret_cast<f32x4*>(static_cast<float*>(base) + idx) = v;
  } else {
    const uint32_t lo = static_cast<uint32_t>(Elem<DT>::from_f32(v0)) |
                        (static_cast<uint32_t>(Elem<DT>::from_f32(v1)) << 16);
    const uint32_t hi = static_cast<uint32_t>(Elem<DT>::from_f32(v2)) |
                        (static_cast<uint32_t>(Elem<DT>::from_f32(v3)) << 16);
    u32x2 v = {lo, hi};
    *reinterpret_cast<u32x2*>(static_cast<S*>(base) + idx) = v;
  }
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ int64_t uniform64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(v) >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Workgroup = (active expert, 4 consecutive weight tiles): wave w owns tile 4*group + w. A
// wave past the expert's last tile streams the last tile again and stores nothing, so every
// wave of a workgroup runs the same chunks and barriers.
template <int DT, int MT>
__global__ __launch_bounds__(kExpertThreads) void gateup_kernel(ExpertArgs a) {
  using S = typename Elem<DT>::S;
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int r = lane & 15, g = lane >> 4;
  const int tiles = a.I / kRowTile;
  const int groups = (tiles + kExpertWaves - 1) / kExpertWaves;
  const int ai = blockIdx.x / groups;  // uniform across the workgroup
  const int tg = blockIdx.x - ai * groups;
  // ai < max_active <= E, so the per-expert arrays may be read before the active count is
  // known (the loads then share one latency); values past the active count are unused.
  const int active = uniform(a.rb.hdr[0]);
  const int off = uniform(a.rb.act_off[ai]);
  const int m = uniform(a.rb.act_cnt[ai]);
  const int64_t slot = uniform64(a.rb.act_slot[ai]);
  if (ai >= active) return;
  const int praw = tg * kExpertWaves + wave;
  const bool owner = praw < tiles;
  const int p = owner ? praw : tiles - 1;
  const int H = a.H, I = a.I;
  const int64_t row_bytes = static_cast<int64_t>(H) * sizeof(S);
  const int64_t page_bytes = a.page_elems * static_cast<int64_t>(sizeof(S));
  WeightStream ws;  // tile 0: gate rows [16p, 16p+16); tile 1: the matching up rows
  ws.rsrc = make_rsrc(static_cast<const char*>(a.pool) + slot * page_bytes, static_cast<uint32_t>(page_bytes));
  ws.base = static_cast<uint32_t>(kRowTile * p * row_bytes);
  ws.tile_stride = static_cast<uint32_t>(I * row_bytes);
  ws.row4 = static_cast<uint32_t>(4 * row_bytes);
  ws.lane_off = static_cast<uint32_t>((lane >> 4) * row_bytes + (lane & 15) * 16);
  const int nchunks = static_cast<int>(row_bytes / (kStepBytes * kUnroll));
  __shared__ u32x4 lds_all[kExpertWaves][2 * kTileSlots];
  __shared__ u32x4 bsh[2 * MT * kTileSlots];
  u32x4* lds = lds_all[wave];
  S* act = static_cast<S*>(a.act);

  for (int q0 = 0; q0 < m; q0 += kTokTile * MT) {
    SharedTokens<MT> tb;
    tb.rsrc = make_rsrc(a.x, static_cast<uint32_t>(static_cast<int64_t>(a.T) * row_bytes));
    tb.base = 0;
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      const int q = min(q0 + j * kTokTile + 4 * wave + (lane >> 4), m - 1);
      const int tok = a.rb.sorted_f[off + q] / a.k;
      tb.off[j] = static_cast<uint32_t>(tok * row_bytes + (lane & 15) * 16);
    }
    f32x4 acc[2][MT];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[i][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    stream_wg<DT, 2, MT>(ws, tb, nchunks, lds, bsh, acc);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int q = q0 + mt * kTokTile + r;
      if (owner && q < m) {
        float o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float gate = Elem<DT>::round(acc[0][mt][i]);
          const float up = Elem<DT>::round(acc[1][mt][i]);
          o[i] = silu_f32(gate) * up;
        }
        store4<DT>(act, static_cast<int64_t>(off + q) * I + kRowTile * p + 4 * g, o[0], o[1], o[2], o[3]);
      }
    }
  }
}

// Workgroup = (active expert, K split, 4 consecutive pairs of W2 row tiles): wave w owns
// rows [32*(4*group + w), +32). Waves past the last pair repeat it and store nothing.
template <int DT, int MT>
__global__ __launch_bounds__(kExpertThreads) void down_kernel(ExpertArgs a) {
  using S = typename Elem<DT>::S;
  constexpr int R = kDownRows;
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int r = lane & 15, g = lane >> 4;
  const int rtiles = a.H / (kRowTile * R);
  const int groups = (rtiles + kExpertWaves - 1) / kExpertWaves;
  const int per_expert = groups * a.splits;
  const int ai = blockIdx.x / per_expert;  // uniform across the workgroup
  const int rem = blockIdx.x - ai * per_expert;
  const int sp = rem / groups;
  const int tg = rem - sp * groups;
  const int active = uniform(a.rb.hdr[0]);
  const int off = uniform(a.rb.act_off[ai]);
  const int m = uniform(a.rb.act_cnt[ai]);
  const int64_t slot = uniform64(a.rb.act_slot[ai]);
  if (ai >= active) return;
  const int rtraw = tg * kExpertWaves + wave;
  const bool owner = rtraw < rtiles;
  const int rt = owner ? rtraw : rtiles - 1;
  const int H = a.H, I = a.I;
  const int N = a.T * a.k;
  const int64_t row_bytes = static_cast<int64_t>(I) * sizeof(S);
  const int64_t k0_bytes = static_cast<int64_t>(sp) * a.split_steps * kStepBytes;
  const int64_t page_bytes = a.page_elems * static_cast<int64_t>(sizeof(S));
  WeightStream ws;  // tiles: rows [(rt*R + i)*16, +16) of W2 (after W1, W3), this split's K slice
  ws.rsrc = make_rsrc(static_cast<const char*>(a.pool) + slot * page_bytes, static_cast<uint32_t>(page_bytes));
  ws.base = static_cast<uint32_t>(2 * H * row_bytes + rt * R * kRowTile * row_bytes + k0_bytes);
  ws.tile_stride = static_cast<uint32_t>(kRowTile * row_bytes);
  ws.row4 = static_cast<uint32_t>(4 * row_bytes);
  ws.lane_off = static_cast<uint32_t>((lane >> 4) * row_bytes + (lane & 15) * 16);
  __shared__ u32x4 lds_all[kExpertWaves][R * kTileSlots];
  __shared__ u32x4 bsh[2 * MT * kTileSlots];
  u32x4* lds = lds_all[wave];

  for (int q0 = 0; q0 < m; q0 += kTokTile * MT) {
    SharedTokens<MT> tb;
    tb.rsrc = make_rsrc(a.act, static_cast<uint32_t>(static_cast<int64_t>(N) * row_bytes));
    tb.base = static_cast<uint32_t>(k0_bytes);
#pragma unroll
    for (int j = 0; j < MT; ++j) {
      const int q = min(q0 + j * kTokTile + 4 * wave + (lane >> 4), m - 1);
      tb.off[j] = static_cast<uint32_t>((off + q) * row_bytes + (lane & 15) * 16);
    }
    f32x4 acc[R][MT];
#pragma unroll
    for (int i = 0; i < R; ++i)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[i][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    stream_wg<DT, R, MT>(ws, tb, a.split_steps / kUnroll, lds, bsh, acc);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int q = q0 + mt * kTokTile + r;
      if (owner && q < m) {
        const int f = a.rb.sorted_f[off + q];
        float* dst = a.part + (static_cast<int64_t>(sp) * N + f) * H;
#pragma unroll
        for (int i = 0; i < R; ++i)
          *reinterpret_cast<f32x4*>(dst + (rt * R + i) * kRowTile + 4 * g) = acc[i][mt];
      }
    }
  }
}

// One thread per 4 output elements.
template <int DT>
__global__ __launch_bounds__(256) void combine_kernel(CombineArgs c) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int hq = c.H / 4;
  if (idx >= static_cast<int64_t>(c.T) * hq) return;
  const int t = static_cast<int>(idx / hq);
  const int h = static_cast<int>(idx - static_cast<int64_t>(t) * hq) * 4;
  const int N = c.T * c.k;
  f32x4 y = {0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < c.k; ++j) {
    const int f = t * c.k + j;
    const int e = c.ids[f];
    if (e < 0 || e >= c.E) continue;
    const int64_t slot = c.e2s[e];
    if (slot < 0 || slot >= c.num_slots) continue;
    f32x4 v = *reinterpret_cast<const f32x4*>(c.part + static_cast<int64_t>(f) * c.H + h);
    for (int s = 1; s < c.splits; ++s)
      v += *reinterpret_cast<const f32x4*>(c.part + (static_cast<int64_t>(s) * N + f) * c.H + h);
    const float wf = c.w[f];
#pragma unroll
    for (int i = 0; i < 4; ++i) y[i] += Elem<DT>::round(v[i] * wf);
  }
  store4<DT>(c.y, static_cast<int64_t>(t) * c.H + h, y[0], y[1], y[2], y[3]);
}

template <int DT, int MT>
static hipError_t launch_stage_t(int stage, const ExpertArgs& a, int max_active, hipStream_t s) {
  if (stage == 0) {
    const int64_t groups = (a.I / kRowTile + kExpertWaves - 1) / kExpertWaves;
    gateup_kernel<DT, MT><<<static_cast<unsigned>(max_active * groups), kExpertThreads, 0, s>>>(a);
  } else {
    const int64_t groups = (a.H / (kRowTile * kDownRows) + kExpertWaves - 1) / kExpertWaves;
    down_kernel<DT, MT><<<static_cast<unsigned>(max_active * groups * a.splits), kExpertThreads, 0, s>>>(a);
  }
  return hipGetLastError();
}

template <int DT>
static hipError_t launch_stage_dt(int stage, const ExpertArgs& a, int max_active, int tok_tiles,
                                  hipStream_t s) {
  switch (tok_tiles) {
    case 1: return launch_stage_t<DT, 1>(stage, a, max_active, s);
    case 2: return launch_stage_t<DT, 2>(stage, a, max_active, s);
    case 3: return launch_stage_t<DT, 3>(stage, a, max_active, s);
    default: return launch_stage_t<DT, 4>(stage, a, max_active, s);
  }
}

static hipError_t launch_stage(int stage, int dtype, const ExpertArgs& a, int max_active,
                               int tok_tiles, hipStream_t s) {
  switch (dtype) {
    case kF32: return launch_stage_dt<kF32>(stage, a, max_active, tok_tiles, s);
    case kF16: return launch_stage_dt<kF16>(stage, a, max_active, tok_tiles, s);
    default: return launch_stage_dt<kBF16>(stage, a, max_active, tok_tiles, s);
  }
}

hipError_t launch_gateup(int dtype, const ExpertArgs& a, int max_active, int tok_tiles, hipStream_t s) {
  return launch_stage(0, dtype, a, max_active, tok_tiles, s);
}

hipError_t launch_down(int dtype, const ExpertArgs& a, int max_active, int tok_tiles, hipStream_t s) {
  return launch_stage(1, dtype, a, max_active, tok_tiles, s);
}

hipError_t launch_combine(int dtype, const CombineArgs& c, hipStream_t s) {
  const int64_t threads = static_cast<int64_t>(c.T) * (c.H / 4);
  const unsigned blocks = static_cast<unsigned>((threads + 255) / 256);
  switch (dtype) {
    case kF32: combine_kernel<kF32><<<blocks, 256, 0, s>>>(c); break;
    case kF16: combine_kernel<kF16><<<blocks, 256, 0, s>>>(c); break;
    default: combine_kernel<kBF16><<<blocks, 256, 0, s>>>(c); break;
  }
  return hipGetLastError();
}

}  // namespace smx
