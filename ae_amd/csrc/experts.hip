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

#include "gateup_device.h"
#include "rows_device.h"

namespace smx {

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
  // Item tg = (split index q, row group): consecutive items (the workgroups that run side by
  // side) take consecutive row groups, and row group g streams split (q + g) mod splits, so
  // that they read different K slices of their rows. Without the rotation they all read the
  // same byte range of every W2 row, which for a power-of-two row pitch concentrates the
  // reads on a few HBM channels: Mixtral-8x22B (ffn 16384: 32 KB rows, 8 splits) at one token
  // 85.6 -> 76.2 us per down launch; the other measured shapes (Mixtral-8x7B, DBRX,
  // Qwen1.5-MoE, DeepSeek-V2-Lite, the fp32 layer) unchanged within +-0.5 us.
  const int q = div_small(it.tg, groups, 1.0f / static_cast<float>(groups));
  const int tg = it.tg - q * groups;
  const int qr = q + tg;
  const int sp = qr - div_small(qr, splits, 1.0f / static_cast<float>(splits)) * splits;
  const int rtraw = tg * kExpertWaves + wave;
  const bool owner = rtraw < rtiles;
  const int rt = owner ? rtraw : rtiles - 1;
  __shared__ u32x4 lds_all[kExpertWaves][R * kTileSlots];
  __shared__ u32x4 bsh[2 * MT * kTileSlots];
  u32x4* lds = lds_all[wave];
  if (kMulti && it.nr > 1) down_item<0, DT, MT, R>(a, it, rt, owner, sp, split_steps, lds, bsh);
  else down_item<kNonTemporal, DT, MT, R>(a, it, rt, owner, sp, split_steps, lds, bsh);
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
      if (gated) gs = Elem<DT>::round(1.0f / (1.0f + expf(-z)));
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
      if (gated) gs = Elem<DT>::round(1.0f / (1.0f + expf(-zs)));
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
      if (gated) sh = Elem<DT>::round(Elem<DT>::round(1.0f / (1.0f + expf(-zt))) * sh);
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
// ST: routed items in expert order (expert_item): E items per weight group, not max_ranges.
template <bool kMulti, int DT, int MT, int RG, bool RM, bool ST = false>
static void launch_gateup_w(const ExpertArgs& a, int max_ranges, hipStream_t s) {
  auto go = [&](auto wc, auto ksc) {
    constexpr int W = decltype(wc)::value;
    constexpr bool KS = decltype(ksc)::value;
    constexpr int TW = KS ? 2 : W;
    const int64_t groups = (a.I / kRowTile + TW - 1) / TW;
    const int64_t items = a.sh.gateup_blocks + (ST ? a.rt.E : max_ranges) * groups;
    const int slots = resident_slots();
    if constexpr (W == kExpertWaves) {
      // the fewest workgroups that walk equal item counts, if that keeps 7/8 of the slots busy
      const int64_t per = (items + slots - 1) / slots;
      const int64_t g = ((items + per - 1) / per + 7) / 8 * 8;
      if (a.gu_items > 0 && items > slots && 8 * g >= 7 * static_cast<int64_t>(slots)) {
        ExpertArgs b = a;
        b.gu_items = static_cast<int>(items);
        gateup_kernel<kMulti, DT, MT, RG, RM, W, true, KS, false, ST>
            <<<static_cast<unsigned>(g), W * kWave, 0, s>>>(b);
        return;
      }
    }
    gateup_kernel<kMulti, DT, MT, RG, RM, W, false, KS, false, ST>
        <<<static_cast<unsigned>(items), W * kWave, 0, s>>>(a);
  };
  using No = std::false_type;
  if constexpr (!kMulti && MT <= 2 && !ST) {
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

template <int DT, int MT, bool RM, bool ST = false>
static void launch_gateup_routed(const ExpertArgs& a, int max_ranges, int route_g, hipStream_t s) {
  switch (route_g) {
    case 8: launch_gateup_w<false, DT, MT, 8, RM, ST>(a, max_ranges, s); break;
    case 16: launch_gateup_w<false, DT, MT, 16, RM, ST>(a, max_ranges, s); break;
    case 32: launch_gateup_w<false, DT, MT, 32, RM, ST>(a, max_ranges, s); break;
    default: launch_gateup_w<false, DT, MT, 64, RM, ST>(a, max_ranges, s); break;
  }
}

template <int DT, bool ST>
static void launch_gateup_multi(const ExpertArgs& a, int max_ranges, int tok_tiles, int route_g, hipStream_t s) {
  switch (tok_tiles) {
    case 1: launch_gateup_routed<DT, 1, true, ST>(a, max_ranges, route_g, s); break;
    case 2: launch_gateup_routed<DT, 2, true, ST>(a, max_ranges, route_g, s); break;
    case 3: if constexpr (!ST) launch_gateup_routed<DT, 3, true>(a, max_ranges, route_g, s); break;
    default: if constexpr (!ST) launch_gateup_routed<DT, 4, true>(a, max_ranges, route_g, s); break;
  }
}

template <int DT>
static void launch_gateup_routed_dt(const ExpertArgs& a, int max_ranges, int tok_tiles, int route_g,
                                    bool multi, bool expert_items, hipStream_t s) {
  if (!multi) {
    if (tok_tiles <= 1) launch_gateup_routed<DT, 1, false>(a, max_ranges, route_g, s);
    else launch_gateup_routed<DT, 2, false>(a, max_ranges, route_g, s);
    return;
  }
  if (a.T > a.rb.span) {
    // given ids whose experts may span several token ranges (the ids need no top-k lanes)
    launch_gateup_w<true, DT, kMaxTokTiles, 64, true>(a, max_ranges, s);
    return;
  }
  if (expert_items) launch_gateup_multi<DT, true>(a, max_ranges, tok_tiles, route_g, s);
  else launch_gateup_multi<DT, false>(a, max_ranges, tok_tiles, route_g, s);
}

hipError_t launch_gateup(int dtype, const ExpertArgs& a, int max_ranges, int tok_tiles, hipStream_t s,
                         int route_g, bool route_multi, bool expert_items) {
  if (route_g == 0) return launch_stage(0, dtype, a, max_ranges, tok_tiles, s);
  // routing inside the launch, every expert one token range (T <= span): one wave routes
  // T*k <= 64 assignments over E <= 64 experts in at most 4 top-k passes; the multi-wave form
  // takes up to kGateupSortMax assignments and up to four token tiles
  if (route_g != 8 && route_g != 16 && route_g != 32 && route_g != 64) return hipErrorInvalidValue;
  if (a.rt.E > kWave || tok_tiles > kMaxTokTiles) return hipErrorInvalidValue;
  // several token ranges per expert (T > span): given ids in the multi-wave form, four tiles
  const bool ranges_multi = a.T > a.rb.span;
  if (ranges_multi && (!route_multi || a.rt.logits != nullptr || tok_tiles != kMaxTokTiles || expert_items))
    return hipErrorInvalidValue;
  if (route_multi) {
    if (a.T * a.k > (a.rt.logits != nullptr ? kSortWaveMax : kGateupSortMax)) return hipErrorInvalidValue;
    // expert-ordered items have one pass of at most tok_tiles token tiles (gateup_passes PRE),
    // at most two (kExpertItemsMaxTiles)
    if (expert_items && (a.rb.span > kTokTile * tok_tiles || tok_tiles > kExpertItemsMaxTiles ||
                         a.T * a.k > kExpertWaves * kWave))
      return hipErrorInvalidValue;
  } else if (a.T * a.k > kWave || tok_tiles > 2 ||
             (a.rt.logits != nullptr && a.T * route_g > kWave * kSmallRoutePasses)) {
    return hipErrorInvalidValue;
  }
  switch (dtype) {
    case kF32: launch_gateup_routed_dt<kF32>(a, max_ranges, tok_tiles, route_g, route_multi, expert_items, s); break;
    case kF16: launch_gateup_routed_dt<kF16>(a, max_ranges, tok_tiles, route_g, route_multi, expert_items, s); break;
    default: launch_gateup_routed_dt<kBF16>(a, max_ranges, tok_tiles, route_g, route_multi, expert_items, s); break;
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
