// Routing kernels: top-k softmax gating and the token -> expert sort.
//
// topk_softmax_kernel     G lanes per token (G = next power of two >= E, at least 8; a wave
//                         holds 64/G tokens; for E > 64 a lane holds up to 4 experts).
// align_kernel            one workgroup: per-wave histograms built from ballot/popcount,
//                         a wave-level scan in LDS, then a stable scatter; emits either the
//                         compact per-expert lists the expert kernels consume or the
//                         reference's block-padded (sorted_ids, expert_ids, ntp) format.
// route_kernel            both of the above fused in one launch (one workgroup).
#include "smx_kernels.h"

namespace smx {

// ---------------------------------------------------------------------------------------
// Top-k softmax, G lanes per token (G = 8, 16, 32 or 64; a wave holds 64/G tokens). Lane j of
// a group holds expert j (and j + 64*i for G = 64, up to 256 experts). On return lane j < k of
// each group holds the j-th pick (descending probability, ties to the lower expert index).
// The arithmetic (max, exp_nonpos, per-lane sequential sum, xor butterfly over the group,
// p = ex * (1/sum), renormalisation by division with the sum taken in j order) equals the
// oracle's 64-lane tree bit for bit: with E <= G every lane at or past G holds an exact zero,
// so the butterfly steps at offsets >= G only add zeros. Semantics follow select_experts as
// called at specmoe/layers/FusedMoE.py:174-185.
// ---------------------------------------------------------------------------------------
template <int G>
struct TopkGroup {
  static constexpr int kPerLane = (G == kWave) ? kMaxExpertsPerLane : 1;  // experts per lane
  static constexpr int kTokens = kWave / G;                               // tokens per wave
};

template <int LDT, int G>
__device__ __forceinline__ void load_logits(const void* logits, int t, int T, int E,
                                            float (&v)[TopkGroup<G>::kPerLane]) {
  const int j = lane_id() % G;
#pragma unroll
  for (int i = 0; i < TopkGroup<G>::kPerLane; ++i) {
    const int e = j + G * i;
    v[i] = (t < T && e < E) ? load_as_f32<LDT>(logits, static_cast<int64_t>(t) * E + e) : -__builtin_inff();
  }
}

template <int G>
__device__ __forceinline__ void group_topk_softmax(float (&p)[TopkGroup<G>::kPerLane], int E, int k,
                                                   bool renorm, float& w_out, int& id_out) {
#pragma clang fp contract(off)
  constexpr int PL = TopkGroup<G>::kPerLane;
  const int lane = lane_id();
  const int j = lane % G;
  const int base = lane - j;
  float m = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < PL; ++i) m = fmaxf(m, p[i]);
#pragma unroll
  for (int off = G / 2; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, kWave));
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < PL; ++i) {
    const int e = j + G * i;
    p[i] = (e < E) ? exp_nonpos(p[i] - m) : 0.0f;
    s = (i == 0) ? p[i] : s + p[i];
  }
#pragma unroll
  for (int off = G / 2; off >= 1; off >>= 1) s = s + __shfl_xor(s, off, kWave);
  const float inv = 1.0f / s;
#pragma unroll
  for (int i = 0; i < PL; ++i) {
    const int e = j + G * i;
    p[i] = (e < E) ? p[i] * inv : -1.0f;  // -1 marks "not selectable"
  }
  w_out = 0.0f;
  id_out = -1;
  for (int jj = 0; jj < k; ++jj) {
    float bp = -2.0f;
    int be = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      if (p[i] > bp) { bp = p[i]; be = j + G * i; }  // ascending e: strict > keeps lowest
    }
#pragma unroll
    for (int off = G / 2; off >= 1; off >>= 1) {
      const float op = __shfl_xor(bp, off, kWave);
      const int oe = __shfl_xor(be, off, kWave);
      if (op > bp || (op == bp && oe < be)) { bp = op; be = oe; }
    }
    if (j == be % G) {
#pragma unroll
      for (int i = 0; i < PL; ++i)
        if (i == be / G) p[i] = -1.0f;
    }
    if (j == jj) { w_out = bp; id_out = be; }
  }
  if (renorm) {
    float sum = 0.0f;
    for (int jj = 0; jj < k; ++jj) {
      const float v = __shfl(w_out, base + jj, kWave);
      sum = (jj == 0) ? v : sum + v;
    }
    if (j < k) w_out = w_out / sum;
  }
}

// The tokens of `passes` consecutive wave-passes: token t = (pass0 + b) * stride + slot, where
// slot = lane / G. All logit loads are issued before any token is computed, so a wave pays
// one load latency per batch. fn(t, w, id) is called on every lane (t may be >= T).
template <int LDT, int G, typename Fn>
__device__ __forceinline__ void topk_batch(const void* logits, int T, int E, int k, bool renorm,
                                           int first, int stride, Fn&& fn) {
  constexpr int PL = TopkGroup<G>::kPerLane;
  float v[kTokBatch][PL];
#pragma unroll
  for (int b = 0; b < kTokBatch; ++b) load_logits<LDT, G>(logits, first + b * stride, T, E, v[b]);
#pragma unroll
  for (int b = 0; b < kTokBatch; ++b) {
    if (first + b * stride - lane_id() / G < T) {  // some token of this wave-pass exists
      float w;
      int id;
      group_topk_softmax<G>(v[b], E, k, renorm, w, id);
      fn(first + b * stride, w, id);
    }
  }
}

template <int LDT, int G>
__global__ __launch_bounds__(256) void topk_softmax_kernel(const void* __restrict__ logits,
                                                           int T, int E, int k, int renorm,
                                                           float* __restrict__ w,
                                                           int32_t* __restrict__ ids) {
  constexpr int TPW = TopkGroup<G>::kTokens;
  const int waves = blockDim.x / kWave;
  const int lane = lane_id();
  const int j = lane % G;
  const int stride = gridDim.x * waves * TPW;  // tokens per pass of the whole grid
  for (int t0 = (blockIdx.x * waves + threadIdx.x / kWave) * TPW + lane / G; t0 - lane / G < T;
       t0 += stride * kTokBatch) {
    topk_batch<LDT, G>(logits, T, E, k, renorm != 0, t0, stride, [&](int t, float wv, int id) {
      if (t < T && j < k) {
        w[static_cast<int64_t>(t) * k + j] = wv;
        ids[static_cast<int64_t>(t) * k + j] = id;
      }
    });
  }
}

// ---------------------------------------------------------------------------------------
// Expert sort of flat assignments f = t*k + j held in LDS (ids_l[f], -1 = dropped).
// Stable: within an expert, assignments appear in ascending f. Counts come from per-wave
// histograms built with ballot/popcount over 64-assignment chunks; ranks are the popcount
// of the ballot below the lane. Reference: moe_align_block_size,
// specmoe/layers/fused_moe_kernel.py:16-85 (its docstring example fixes the order).
// ---------------------------------------------------------------------------------------
struct AlignShared {
  int16_t ids[kMaxAssignments];        // expert per flat assignment; -1 dropped, -2 out of range
  int cntw[kRouteWaves][kMaxExperts];  // per-wave counts, then per-wave start positions
  int cnt[kMaxExperts];
  int off[kMaxExperts + 1];            // compact exclusive prefix
  int seg[kMaxExperts + 1];            // block-padded exclusive prefix
  int act[kMaxExperts + 1];            // active-expert exclusive prefix
  int64_t slot[kMaxExperts];           // pool slot per expert (-1: unmapped), route only
  int bad;                             // an assignment was dropped
};

struct AlignOutputs {
  // compact lists for the expert kernels (may be null)
  int32_t* hdr;         // [0] = number of active experts, [1] = dropped-assignment flag
  int32_t* act_expert;  // [E]
  int32_t* act_off;     // [E]
  int32_t* act_cnt;     // [E]
  int64_t* act_slot;    // [E]
  int32_t* sorted_f;    // [N]
  // reference-format outputs (may be null)
  int32_t* sorted_ids;  // [N + E*(BM-1)]
  int32_t* expert_ids;  // [ceil((N + E*(BM-1)) / BM)]
  int32_t* ntp;         // [1]
  int bm;
};

// Walks this wave's contiguous range of f in 64-wide chunks; for every group of lanes that
// share an expert, calls fn(mask, e, f, mine, leader) on all lanes of the wave (uniform
// control flow). Assignments whose expert is unroutable count as dropped.
template <bool kCheckSlots, typename Fn>
__device__ __forceinline__ void for_each_expert_group(AlignShared& sh, int N, int wave, Fn&& fn) {
  const int lane = lane_id();
  const int per_wave = ((N + kRouteWaves - 1) / kRouteWaves + kWave - 1) / kWave * kWave;
  const int begin = wave * per_wave;
  const int end = min(N, begin + per_wave);
  for (int base = begin; base < end; base += kWave) {
    const int f = base + lane;
    int e = (f < end) ? static_cast<int>(sh.ids[f]) : -1;
    if (e == -2 || (kCheckSlots && e >= 0 && sh.slot[e] < 0)) {
      sh.bad = 1;
      e = -1;
    }
    uint64_t pending = ballot(e >= 0);
    while (pending) {
      const int leader = __ffsll(static_cast<long long>(pending)) - 1;
      const int el = __shfl(e, leader, kWave);
      const uint64_t m = ballot(e == el);
      fn(m, el, f, e == el, leader);
      pending &= ~m;
    }
  }
}

// Stable expert sort of the assignments in sh.ids. Precondition (caller): sh.cntw zeroed,
// sh.ids (and sh.slot when kCheckSlots) written, and a barrier since.
template <bool kCheckSlots>
__device__ void align_block(AlignShared& sh, int N, int E, const AlignOutputs& out) {
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = lane_id();

  // pass 1: per-wave histograms
  for_each_expert_group<kCheckSlots>(sh, N, wave, [&](uint64_t m, int el, int, bool, int leader) {
    if (lane == leader) sh.cntw[wave][el] += __popcll(m);
  });
  __syncthreads();

  // wave 0: per-expert totals and per-wave prefixes, then exclusive scans over experts
  // (each lane owns 4 consecutive experts), the per-wave start positions and the compact
  // active-expert table.
  if (wave == 0) {
    const int bm = out.bm > 0 ? out.bm : 1;
    int c[4], sc = 0, sp = 0, sa = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = lane * 4 + i;
      c[i] = 0;
      if (e < E) {
        for (int w = 0; w < kRouteWaves; ++w) {
          const int v = sh.cntw[w][e];
          sh.cntw[w][e] = c[i];  // per-wave exclusive prefix, in wave order
          c[i] += v;
        }
        sh.cnt[e] = c[i];
      }
      sc += c[i];
      sp += (c[i] + bm - 1) / bm * bm;
      sa += c[i] > 0;
    }
    int ic = sc, ip = sp, ia = sa;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const int tc = __shfl_up(ic, off, kWave);
      const int tp = __shfl_up(ip, off, kWave);
      const int ta = __shfl_up(ia, off, kWave);
      if (lane >= off) { ic += tc; ip += tp; ia += ta; }
    }
    int bc = ic - sc, bp = ip - sp, ba = ia - sa;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = lane * 4 + i;
      if (e <= E) { sh.off[e] = bc; sh.seg[e] = bp; sh.act[e] = ba; }
      if (e < E) {
        for (int w = 0; w < kRouteWaves; ++w) sh.cntw[w][e] += bc;
        if (out.act_expert && c[i] > 0) {
          out.act_expert[ba] = e;
          out.act_off[ba] = bc;
          out.act_cnt[ba] = c[i];
          if constexpr (kCheckSlots) out.act_slot[ba] = sh.slot[e];
        }
      }
      bc += c[i];
      bp += (c[i] + bm - 1) / bm * bm;
      ba += c[i] > 0;
    }
    if (E == 4 * kWave && lane == kWave - 1) { sh.off[E] = bc; sh.seg[E] = bp; sh.act[E] = ba; }
  }
  __syncthreads();
  if (tid == 0) {
    if (out.hdr) { out.hdr[0] = sh.act[E]; out.hdr[1] = sh.bad; }
    if (out.ntp) out.ntp[0] = sh.seg[E];
  }

  // pass 2: stable scatter
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));
  for_each_expert_group<kCheckSlots>(sh, N, wave, [&](uint64_t m, int el, int f, bool mine, int leader) {
    const int base = sh.cntw[wave][el];
    if (mine) {
      const int pos = base + __popcll(m & lt_mask);
      if (out.sorted_f) out.sorted_f[pos] = f;
      if (out.sorted_ids) out.sorted_ids[sh.seg[el] + (pos - sh.off[el])] = f;
    }
    if (lane == leader) sh.cntw[wave][el] = base + __popcll(m);
  });

  // reference format: sentinel padding and per-block expert ids
  if (out.sorted_ids) {
    const int bm = out.bm;
    const int len = N + E * (bm - 1);
    const int nblocks = (len + bm - 1) / bm;
    for (int e = wave; e < E; e += kRouteWaves) {
      for (int p = sh.seg[e] + sh.cnt[e] + lane; p < sh.seg[e + 1]; p += kWave) out.sorted_ids[p] = N;
      for (int b = sh.seg[e] / bm + lane; b < sh.seg[e + 1] / bm; b += kWave) out.expert_ids[b] = e;
    }
    for (int p = sh.seg[E] + tid; p < len; p += blockDim.x) out.sorted_ids[p] = N;
    for (int b = sh.seg[E] / bm + tid; b < nblocks; b += blockDim.x) out.expert_ids[b] = -1;
  }
}

__device__ __forceinline__ void zero_counts(AlignShared& sh) {
  for (int i = threadIdx.x; i < kRouteWaves * kMaxExperts; i += blockDim.x) (&sh.cntw[0][0])[i] = 0;
  if (threadIdx.x == 0) sh.bad = 0;
}

// Reference-format alignment of caller-provided ids.
__global__ __launch_bounds__(kRouteThreads) void align_kernel(const int32_t* __restrict__ ids,
                                                              int N, int E, AlignOutputs out) {
  __shared__ AlignShared sh;
  zero_counts(sh);
  for (int f = threadIdx.x; f < N; f += blockDim.x) {
    const int e = ids[f];
    sh.ids[f] = static_cast<int16_t>((e >= 0 && e < E) ? e : -1);
  }
  __syncthreads();
  align_block<false>(sh, N, E, out);
}

// Routing for the expert kernels. With logits != null the top-k softmax runs first (results
// to w/ids and LDS); otherwise ids come from the caller. Then the compact expert sort.
// Assignments with an id outside [0,E), or whose expert's pool slot is outside
// [0,num_slots), are dropped (they contribute nothing) and flagged in hdr[1].
template <int LDT, int G>
__global__ __launch_bounds__(kRouteThreads) void route_kernel(
    const void* __restrict__ logits, int T, int E, int k, int renorm,
    float* __restrict__ w_out, int32_t* __restrict__ ids_out, const int32_t* __restrict__ ids_in,
    const int64_t* __restrict__ e2s, int64_t num_slots, AlignOutputs out) {
  __shared__ AlignShared sh;
  constexpr int TPW = TopkGroup<G>::kTokens;
  const int N = T * k;
  const int wave = threadIdx.x / kWave;
  const int lane = lane_id();
  zero_counts(sh);
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    const int64_t slot = e2s[e];
    sh.slot[e] = (slot >= 0 && slot < num_slots) ? slot : -1;
  }
  if (logits != nullptr) {
    const int j = lane % G;
    const int stride = kRouteWaves * TPW;
    for (int t0 = wave * TPW + lane / G; t0 - lane / G < T; t0 += stride * kTokBatch) {
      topk_batch<LDT, G>(logits, T, E, k, renorm != 0, t0, stride, [&](int t, float wv, int id) {
        if (t < T && j < k) {
          const int f = t * k + j;
          if (w_out) w_out[f] = wv;
          if (ids_out) ids_out[f] = id;
          sh.ids[f] = static_cast<int16_t>(id);
        }
      });
    }
  } else {
    for (int f = threadIdx.x; f < N; f += blockDim.x) {
      const int e = ids_in[f];
      sh.ids[f] = static_cast<int16_t>((e >= 0 && e < E) ? e : -2);
    }
  }
  __syncthreads();
  align_block<true>(sh, N, E, out);
}

// ---------------------------------------------------------------------------------------
// Host-side launchers
// ---------------------------------------------------------------------------------------
static int group_for(int E) { return E <= 8 ? 8 : E <= 16 ? 16 : E <= 32 ? 32 : 64; }

template <int LDT, int G>
static void topk_launch(const void* logits, int T, int E, int k, int renorm, float* w, int32_t* ids,
                        hipStream_t s) {
  const int waves = 4;
  const int per_block = waves * TopkGroup<G>::kTokens * kTokBatch;
  int blocks = (T + per_block - 1) / per_block;
  if (blocks > 65535) blocks = 65535;
  topk_softmax_kernel<LDT, G><<<blocks, waves * kWave, 0, s>>>(logits, T, E, k, renorm, w, ids);
}

template <int LDT>
static void topk_launch_g(const void* logits, int T, int E, int k, int renorm, float* w,
                          int32_t* ids, hipStream_t s) {
  switch (group_for(E)) {
    case 8: topk_launch<LDT, 8>(logits, T, E, k, renorm, w, ids, s); break;
    case 16: topk_launch<LDT, 16>(logits, T, E, k, renorm, w, ids, s); break;
    case 32: topk_launch<LDT, 32>(logits, T, E, k, renorm, w, ids, s); break;
    default: topk_launch<LDT, 64>(logits, T, E, k, renorm, w, ids, s); break;
  }
}

hipError_t launch_topk_softmax(const void* logits, int ldt, int T, int E, int k, int renorm,
                               float* w, int32_t* ids, hipStream_t s) {
  switch (ldt) {
    case kF32: topk_launch_g<kF32>(logits, T, E, k, renorm, w, ids, s); break;
    case kF16: topk_launch_g<kF16>(logits, T, E, k, renorm, w, ids, s); break;
    default: topk_launch_g<kBF16>(logits, T, E, k, renorm, w, ids, s); break;
  }
  return hipGetLastError();
}

hipError_t launch_align(const int32_t* ids, int N, int E, int bm, int32_t* sorted_ids,
                        int32_t* expert_ids, int32_t* ntp, hipStream_t s) {
  AlignOutputs out{};
  out.sorted_ids = sorted_ids;
  out.expert_ids = expert_ids;
  out.ntp = ntp;
  out.bm = bm;
  align_kernel<<<1, kRouteThreads, 0, s>>>(ids, N, E, out);
  return hipGetLastError();
}

template <int LDT>
static void route_launch_g(const void* logits, int T, int E, int k, int renorm, float* w_out,
                           int32_t* ids_out, const int32_t* ids_in, const int64_t* e2s,
                           int64_t num_slots, const AlignOutputs& out, hipStream_t s) {
  switch (group_for(E)) {
    case 8: route_kernel<LDT, 8><<<1, kRouteThreads, 0, s>>>(logits, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out); break;
    case 16: route_kernel<LDT, 16><<<1, kRouteThreads, 0, s>>>(logits, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out); break;
    case 32: route_kernel<LDT, 32><<<1, kRouteThreads, 0, s>>>(logits, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out); break;
    default: route_kernel<LDT, 64><<<1, kRouteThreads, 0, s>>>(logits, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out); break;
  }
}

hipError_t launch_route(const void* logits, int ldt, int T, int E, int k, int renorm,
                        float* w_out, int32_t* ids_out, const int32_t* ids_in,
                        const int64_t* e2s, int64_t num_slots, const RouteBuffers& rb,
                        hipStream_t s) {
  AlignOutputs out{};
  out.hdr = rb.hdr;
  out.act_expert = rb.act_expert;
  out.act_off = rb.act_off;
  out.act_cnt = rb.act_cnt;
  out.act_slot = rb.act_slot;
  out.sorted_f = rb.sorted_f;
  out.bm = 1;
  switch (ldt) {
    case kF32: route_launch_g<kF32>(logits, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out, s); break;
    case kF16: route_launch_g<kF16>(logits, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out, s); break;
    default: route_launch_g<kBF16>(logits, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out, s); break;
  }
  return hipGetLastError();
}

}  // namespace smx
