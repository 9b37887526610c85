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
// fragments. The LDS tile is 16 rows x 16 slots of 16 bytes with slot = chunk16 ^ row, so both
// the row-wise writes and the column-wise fragment reads touch 16 distinct slots per 16
// lanes (no bank conflicts). One wave's LDS operations execute in order, so a wave reads
// back its own writes and overwrites a tile only after reading it: no barriers.

constexpr int kTileSlots = kRowTile * 16;  // 16-byte slots per LDS tile (4 KB)

template <int R>
struct Raw {
  u32x4 v[4][R];  // [instruction][tile]
};

// Issue the four 4-row x 256-byte loads of one chunk for every tile. base[r] already holds
// this lane's row (l/16) and byte column (16*(l%16)); instruction i adds 4*i rows.
template <int R>
__device__ __forceinline__ void load_raw(Raw<R>& c, const char* const (&base)[R],
                                         int64_t row4_bytes, int chunk) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < R; ++r)
      c.v[i][r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
          base[r] + i * row4_bytes + static_cast<int64_t>(chunk) * (kStepBytes * kUnroll)));
}

__device__ __forceinline__ int swz(int row, int c16) { return row * 16 + ((c16 ^ row) & 15); }

template <int DT, int R, int MT, bool kPrefetch>
__device__ __forceinline__ void mma_chunk(const Raw<R>& c, Raw<R>& next, u32x4* lds,
                                          const char* const (&a)[R], int64_t row4_bytes,
                                          const char* const (&b)[MT], int chunk,
                                          f32x4 (&acc)[R][MT]) {
  const int lane = lane_id();
  u32x4 bf[kUnroll][MT];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      bf[u][mt] = *reinterpret_cast<const u32x4*>(
          b[mt] + static_cast<int64_t>(chunk * kUnroll + u) * kStepBytes);
  if constexpr (kPrefetch) load_raw(next, a, row4_bytes, chunk + 1);
  // Keep the scheduler from sinking loads into the MFMA sequence (which would shrink the
  // prefetch distance) or from waiting on the prefetch early.
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int r = 0; r < R; ++r) lds[r * kTileSlots + swz(4 * i + (lane >> 4), lane & 15)] = c.v[i][r];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    u32x4 af[R];
#pragma unroll
    for (int r = 0; r < R; ++r) af[r] = lds[r * kTileSlots + swz(lane & 15, 4 * u + (lane >> 4))];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r][mt] = Elem<DT>::mfma(af[r], bf[u][mt], acc[r][mt]);
  }
  __builtin_amdgcn_sched_barrier(0);
}

// acc[r][mt] += A_r (16 rows x nchunks*256 bytes) . B_mt (16 columns), with the next chunk's
// weight loads in flight while the current chunk is transposed and multiplied.
template <int DT, int R, int MT>
__device__ __forceinline__ void stream_mfma(const char* const (&a)[R], int64_t row4_bytes,
                                            const char* const (&b)[MT], int nchunks,
                                            u32x4* lds, f32x4 (&acc)[R][MT]) {
  Raw<R> c0, c1;
  load_raw(c0, a, row4_bytes, 0);
  int c = 0;
  for (; c + 2 < nchunks; c += 2) {
    mma_chunk<DT, R, MT, true>(c0, c1, lds, a, row4_bytes, b, c, acc);
    mma_chunk<DT, R, MT, true>(c1, c0, lds, a, row4_bytes, b, c + 1, acc);
  }
  if (c + 1 < nchunks) {
    mma_chunk<DT, R, MT, true>(c0, c1, lds, a, row4_bytes, b, c, acc);
    mma_chunk<DT, R, MT, false>(c1, c0, lds, a, row4_bytes, b, c + 1, acc);
  } else {
    mma_chunk<DT, R, MT, false>(c0, c1, lds, a, row4_bytes, b, c, acc);
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

template <int DT, int MT>
__global__ __launch_bounds__(kExpertThreads) void gateup_kernel(ExpertArgs a) {
  using S = typename Elem<DT>::S;
  const int lane = lane_id();
  const int r = lane & 15, g = lane >> 4;
  const int tiles = a.I / kRowTile;
  const int gw = uniform(blockIdx.x * kExpertWaves + threadIdx.x / kWave);
  const int ai = gw / tiles;
  const int p = gw - ai * tiles;
  // ai < max_active <= E, so the per-expert arrays may be read before the active count is
  // known (the four loads then share one latency); values past the active count are unused.
  const int active = uniform(a.rb.hdr[0]);
  const int off = uniform(a.rb.act_off[ai]);
  const int m = uniform(a.rb.act_cnt[ai]);
  const int64_t slot = a.rb.act_slot[ai];
  if (ai >= active) return;
  const int H = a.H, I = a.I;
  const S* page = static_cast<const S*>(a.pool) + slot * a.page_elems;
  const int64_t row_bytes = static_cast<int64_t>(H) * sizeof(S);
  // coalesced-load lane origin: row lane/16 of the tile, byte column 16*(lane%16)
  const int64_t lane_origin = (lane >> 4) * row_bytes + (lane & 15) * 16;
  const char* arow[2] = {
      reinterpret_cast<const char*>(page + static_cast<int64_t>(kRowTile * p) * H) + lane_origin,
      reinterpret_cast<const char*>(page + static_cast<int64_t>(I + kRowTile * p) * H) + lane_origin};
  const int nchunks = static_cast<int>(row_bytes / (kStepBytes * kUnroll));
  __shared__ u32x4 lds_all[kExpertWaves][2 * kTileSlots];
  u32x4* lds = lds_all[threadIdx.x / kWave];
  const S* x = static_cast<const S*>(a.x);
  S* act = static_cast<S*>(a.act);

  for (int q0 = 0; q0 < m; q0 += kTokTile * MT) {
    const char* brow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int q = min(q0 + mt * kTokTile + r, m - 1);
      const int tok = a.rb.sorted_f[off + q] / a.k;
      brow[mt] = reinterpret_cast<const char*>(x + static_cast<int64_t>(tok) * H) + g * 16;
    }
    f32x4 acc[2][MT];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[i][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    stream_mfma<DT, 2, MT>(arow, 4 * row_bytes, brow, nchunks, lds, acc);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int q = q0 + mt * kTokTile + r;
      if (q < m) {
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

template <int DT, int MT>
__global__ __launch_bounds__(kExpertThreads) void down_kernel(ExpertArgs a) {
  using S = typename Elem<DT>::S;
  constexpr int R = kDownRows;
  const int lane = lane_id();
  const int r = lane & 15, g = lane >> 4;
  const int rtiles = a.H / (kRowTile * R);
  const int per_expert = rtiles * a.splits;
  const int gw = uniform(blockIdx.x * kExpertWaves + threadIdx.x / kWave);
  const int ai = gw / per_expert;
  const int rem = gw - ai * per_expert;
  const int sp = rem / rtiles;
  const int rt = rem - sp * rtiles;
  const int active = uniform(a.rb.hdr[0]);
  const int off = uniform(a.rb.act_off[ai]);
  const int m = uniform(a.rb.act_cnt[ai]);
  const int64_t slot = a.rb.act_slot[ai];
  if (ai >= active) return;
  const int H = a.H, I = a.I;
  const int N = a.T * a.k;
  const S* w2 = static_cast<const S*>(a.pool) + slot * a.page_elems + static_cast<int64_t>(2) * I * H;
  const int k0 = sp * a.split_steps * kStepBytes / static_cast<int>(sizeof(S));  // element offset
  const int64_t row_bytes = static_cast<int64_t>(I) * sizeof(S);
  const int64_t lane_origin = (lane >> 4) * row_bytes + (lane & 15) * 16;
  const char* arow[R];
#pragma unroll
  for (int i = 0; i < R; ++i)
    arow[i] = reinterpret_cast<const char*>(w2 + static_cast<int64_t>((rt * R + i) * kRowTile) * I + k0) + lane_origin;
  __shared__ u32x4 lds_all[kExpertWaves][R * kTileSlots];
  u32x4* lds = lds_all[threadIdx.x / kWave];
  const S* act = static_cast<const S*>(a.act);

  for (int q0 = 0; q0 < m; q0 += kTokTile * MT) {
    const char* brow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int q = min(q0 + mt * kTokTile + r, m - 1);
      brow[mt] = reinterpret_cast<const char*>(act + static_cast<int64_t>(off + q) * I + k0) + g * 16;
    }
    f32x4 acc[R][MT];
#pragma unroll
    for (int i = 0; i < R; ++i)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[i][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    stream_mfma<DT, R, MT>(arow, 4 * row_bytes, brow, a.split_steps / kUnroll, lds, acc);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int q = q0 + mt * kTokTile + r;
      if (q < m) {
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
    const int64_t waves = static_cast<int64_t>(max_active) * (a.I / kRowTile);
    const unsigned blocks = static_cast<unsigned>((waves + kExpertWaves - 1) / kExpertWaves);
    gateup_kernel<DT, MT><<<blocks, kExpertThreads, 0, s>>>(a);
  } else {
    const int64_t waves = static_cast<int64_t>(max_active) * (a.H / (kRowTile * kDownRows)) * a.splits;
    const unsigned blocks = static_cast<unsigned>((waves + kExpertWaves - 1) / kExpertWaves);
    down_kernel<DT, MT><<<blocks, kExpertThreads, 0, s>>>(a);
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
