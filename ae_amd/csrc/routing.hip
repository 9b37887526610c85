// Routing kernels: top-k softmax gating and the token -> expert sort.
//
// topk_softmax_kernel     one wave per token (lane = expert, up to 4 experts per lane).
// align_kernel            one workgroup: per-wave histograms built from ballot/popcount,
//                         a wave-level scan in LDS, then a stable scatter; emits either the
//                         compact per-expert lists the expert kernels consume or the
//                         reference's block-padded (sorted_ids, expert_ids, ntp) format.
// route_kernel            both of the above fused in one launch (one workgroup).
#include "smx_kernels.h"

namespace smx {

// ---------------------------------------------------------------------------------------
// Top-k softmax of one row, computed by one wave. On return lane j < k holds the j-th pick
// (descending probability, ties to the lower expert index) in (w, id); other lanes hold
// w = 0, id = -1. The arithmetic (max, exp_nonpos, per-lane sequential sum over the lane's
// experts e = lane + 64*i, xor-butterfly across lanes, p = ex * (1/sum), renormalisation by
// division with the sum taken in j order) is restated exactly by the oracle.
// Semantics follow select_experts as called at specmoe/layers/FusedMoE.py:174-185.
// ---------------------------------------------------------------------------------------
template <int LDT>
__device__ __forceinline__ void load_logits(const void* logits, int64_t row, int E,
                                            float (&v)[kMaxExpertsPerLane]) {
  const int lane = lane_id();
#pragma unroll
  for (int i = 0; i < kMaxExpertsPerLane; ++i) {
    const int e = lane + kWave * i;
    v[i] = (e < E) ? load_as_f32<LDT>(logits, row * E + e) : -__builtin_inff();
  }
}

__device__ __forceinline__ void wave_topk_softmax(float (&p)[kMaxExpertsPerLane], int E, int k,
                                                  bool renorm, float& w_out, int& id_out) {
#pragma clang fp contract(off)
  const int lane = lane_id();
  float m = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < kMaxExpertsPerLane; ++i) m = fmaxf(m, p[i]);
  m = wave_max(m);
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < kMaxExpertsPerLane; ++i) {
    const int e = lane + kWave * i;
    p[i] = (e < E) ? exp_nonpos(p[i] - m) : 0.0f;
    s = (i == 0) ? p[i] : s + p[i];
  }
  s = wave_sum_butterfly(s);
  const float inv = 1.0f / s;
#pragma unroll
  for (int i = 0; i < kMaxExpertsPerLane; ++i) {
    const int e = lane + kWave * i;
    p[i] = (e < E) ? p[i] * inv : -1.0f;  // -1 marks "not selectable"
  }
  w_out = 0.0f;
  id_out = -1;
  for (int j = 0; j < k; ++j) {
    float bp = -2.0f;
    int be = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < kMaxExpertsPerLane; ++i) {
      if (p[i] > bp) { bp = p[i]; be = lane + kWave * i; }  // ascending e: strict > keeps lowest
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float op = __shfl_xor(bp, off, kWave);
      const int oe = __shfl_xor(be, off, kWave);
      if (op > bp || (op == bp && oe < be)) { bp = op; be = oe; }
    }
    if (lane == (be & (kWave - 1))) {
#pragma unroll
      for (int i = 0; i < kMaxExpertsPerLane; ++i)
        if (i == (be >> 6)) p[i] = -1.0f;
    }
    if (lane == j) { w_out = bp; id_out = be; }
  }
  if (renorm) {
    float sum = 0.0f;
    for (int j = 0; j < k; ++j) {
      const float v = __shfl(w_out, j, kWave);
      sum = (j == 0) ? v : sum + v;
    }
    if (lane < k) w_out = w_out / sum;
  }
}

// Tokens t = first, first + stride, ... (up to kTokBatch of them) handled by one wave: all
// logit loads are issued before any token is processed, so a wave pays one load latency per
// batch rather than one per token. fn(t, w, id) receives each token's result on every lane.
template <int LDT, typename Fn>
__device__ __forceinline__ void wave_topk_batch(const void* logits, int T, int E, int k,
                                                bool renorm, int first, int stride, Fn&& fn) {
  float v[kTokBatch][kMaxExpertsPerLane];
#pragma unroll
  for (int b = 0; b < kTokBatch; ++b) {
    const int t = first + b * stride;
    if (t < T) load_logits<LDT>(logits, t, E, v[b]);
  }
#pragma unroll
  for (int b = 0; b < kTokBatch; ++b) {
    const int t = first + b * stride;
    if (t < T) {
      float w;
      int id;
      wave_topk_softmax(v[b], E, k, renorm, w, id);
      fn(t, w, id);
    }
  }
}

template <int LDT>
__global__ __launch_bounds__(256) void topk_softmax_kernel(const void* __restrict__ logits,
                                                           int T, int E, int k, int renorm,
                                                           float* __restrict__ w,
                                                           int32_t* __restrict__ ids) {
  const int waves = blockDim.x / kWave;
  const int stride = gridDim.x * waves;
  const int lane = lane_id();
  for (int t0 = blockIdx.x * waves + threadIdx.x / kWave; t0 < T; t0 += stride * kTokBatch) {
    wave_topk_batch<LDT>(logits, T, E, k, renorm != 0, t0, stride, [&](int t, float wv, int id) {
      if (lane < k) {
        w[(int64_t)t * k + lane] = wv;
        ids[(int64_t)t * k + lane] = id;
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
  int16_t ids[kMaxAssignments];
  int cntw[kRouteWaves][kMaxExperts];  // per-wave counts, then per-wave start positions
  int cnt[kMaxExperts];
  int off[kMaxExperts + 1];            // compact exclusive prefix
  int seg[kMaxExperts + 1];            // block-padded exclusive prefix
  int act[kMaxExperts + 1];            // active-expert exclusive prefix
};

struct AlignOutputs {
  // compact lists for the expert kernels (may be null)
  int32_t* hdr;         // [0] = number of active experts
  int32_t* act_expert;  // [E]
  int32_t* act_off;     // [E]
  int32_t* act_cnt;     // [E]
  int32_t* sorted_f;    // [N]
  // reference-format outputs (may be null)
  int32_t* sorted_ids;  // [N + E*(BM-1)]
  int32_t* expert_ids;  // [ceil((N + E*(BM-1)) / BM)]
  int32_t* ntp;         // [1]
  int bm;
};

// Walks this wave's contiguous range of f in 64-wide chunks; for every group of lanes that
// share an expert, calls fn(mask, e) on all lanes of the wave (uniform control flow).
template <typename Fn>
__device__ __forceinline__ void for_each_expert_group(const AlignShared& sh, int N, int wave,
                                                      Fn&& fn) {
  const int lane = lane_id();
  const int per_wave = ((N + kRouteWaves - 1) / kRouteWaves + kWave - 1) / kWave * kWave;
  const int begin = wave * per_wave;
  const int end = min(N, begin + per_wave);
  for (int base = begin; base < end; base += kWave) {
    const int f = base + lane;
    const int e = (f < end) ? static_cast<int>(sh.ids[f]) : -1;
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

__device__ void align_block(AlignShared& sh, int N, int E, const AlignOutputs& out) {
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = lane_id();
  for (int i = tid; i < kRouteWaves * kMaxExperts; i += blockDim.x) (&sh.cntw[0][0])[i] = 0;
  __syncthreads();

  // pass 1: per-wave histograms
  for_each_expert_group(sh, N, wave, [&](uint64_t m, int el, int, bool, int leader) {
    if (lane == leader) sh.cntw[wave][el] += __popcll(m);
  });
  __syncthreads();

  // per expert: total, and per-wave exclusive prefix (over waves, in wave order)
  for (int e = tid; e < E; e += blockDim.x) {
    int run = 0;
    for (int w = 0; w < kRouteWaves; ++w) {
      const int c = sh.cntw[w][e];
      sh.cntw[w][e] = run;
      run += c;
    }
    sh.cnt[e] = run;
  }
  __syncthreads();

  // prefix over experts (wave 0; each lane owns 4 consecutive experts)
  if (wave == 0) {
    const int bm = out.bm > 0 ? out.bm : 1;
    int c[4], sc = 0, sp = 0, sa = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = lane * 4 + i;
      c[i] = (e < E) ? sh.cnt[e] : 0;
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
      bc += c[i];
      bp += (c[i] + bm - 1) / bm * bm;
      ba += c[i] > 0;
    }
    if (E == 4 * kWave && lane == kWave - 1) { sh.off[E] = bc; sh.seg[E] = bp; sh.act[E] = ba; }
  }
  __syncthreads();

  // per-wave start positions; compact active-expert table
  for (int e = tid; e < E; e += blockDim.x) {
    const int o = sh.off[e];
    for (int w = 0; w < kRouteWaves; ++w) sh.cntw[w][e] += o;
    if (out.act_expert && sh.cnt[e] > 0) {
      const int a = sh.act[e];
      out.act_expert[a] = e;
      out.act_off[a] = o;
      out.act_cnt[a] = sh.cnt[e];
    }
  }
  if (tid == 0) {
    if (out.hdr) out.hdr[0] = sh.act[E];
    if (out.ntp) out.ntp[0] = sh.seg[E];
  }
  __syncthreads();

  // pass 2: stable scatter
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));
  for_each_expert_group(sh, N, wave, [&](uint64_t m, int el, int f, bool mine, int leader) {
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

// Reference-format alignment of caller-provided ids.
__global__ __launch_bounds__(kRouteThreads) void align_kernel(const int32_t* __restrict__ ids,
                                                              int N, int E, AlignOutputs out) {
  __shared__ AlignShared sh;
  for (int f = threadIdx.x; f < N; f += blockDim.x) {
    const int e = ids[f];
    sh.ids[f] = static_cast<int16_t>((e >= 0 && e < E) ? e : -1);
  }
  __syncthreads();
  align_block(sh, N, E, out);
}

// Routing for the expert kernels. With logits != null the top-k softmax runs first (one wave
// per token, results to w/ids and LDS); otherwise ids come from the caller. Then the compact
// expert sort. Ids outside [0,E) and experts whose pool slot is outside [0,num_slots) are
// dropped here (they contribute nothing) and flagged in hdr[1].
template <int LDT>
__global__ __launch_bounds__(kRouteThreads) void route_kernel(
    const void* __restrict__ logits, int T, int E, int k, int renorm,
    float* __restrict__ w_out, int32_t* __restrict__ ids_out, const int32_t* __restrict__ ids_in,
    const int64_t* __restrict__ e2s, int64_t num_slots, AlignOutputs out, int64_t* act_slot) {
  __shared__ AlignShared sh;
  __shared__ int64_t slot_of[kMaxExperts];
  __shared__ int bad;
  const int N = T * k;
  const int wave = threadIdx.x / kWave;
  const int lane = lane_id();
  if (threadIdx.x == 0) bad = 0;
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    const int64_t slot = e2s[e];
    slot_of[e] = (slot >= 0 && slot < num_slots) ? slot : -1;
  }
  if (logits != nullptr) {
    for (int t0 = wave; t0 < T; t0 += kRouteWaves * kTokBatch) {
      wave_topk_batch<LDT>(logits, T, E, k, renorm != 0, t0, kRouteWaves, [&](int t, float wv, int id) {
        if (lane < k) {
          const int f = t * k + lane;
          if (w_out) w_out[f] = wv;
          if (ids_out) ids_out[f] = id;
          sh.ids[f] = static_cast<int16_t>(id);
        }
      });
    }
  } else {
    for (int f = threadIdx.x; f < N; f += blockDim.x) {
      const int e = ids_in[f];
      sh.ids[f] = static_cast<int16_t>((e >= 0 && e < E) ? e : -2);  // -2: out of range
    }
  }
  __syncthreads();  // also orders thread 0's `bad = 0` before any `bad = 1`
  for (int f = threadIdx.x; f < N; f += blockDim.x) {
    const int e = sh.ids[f];
    if (e == -2 || (e >= 0 && slot_of[e] < 0)) { sh.ids[f] = -1; bad = 1; }
  }
  __syncthreads();
  if (threadIdx.x == 0) out.hdr[1] = bad;
  align_block(sh, N, E, out);
  // pool slot of each active expert, so the expert kernels need one dependent load, not two
  for (int e = threadIdx.x; e < E; e += blockDim.x)
    if (sh.cnt[e] > 0) act_slot[sh.act[e]] = slot_of[e];
}

// ---------------------------------------------------------------------------------------
// Host-side launchers
// ---------------------------------------------------------------------------------------
hipError_t launch_topk_softmax(const void* logits, int ldt, int T, int E, int k, int renorm,
                               float* w, int32_t* ids, hipStream_t s) {
  const int waves = 4;
  int blocks = (T + waves - 1) / waves;
  if (blocks > 65535) blocks = 65535;
  switch (ldt) {
    case kF32: topk_softmax_kernel<kF32><<<blocks, waves * kWave, 0, s>>>(logits, T, E, k, renorm, w, ids); break;
    case kF16: topk_softmax_kernel<kF16><<<blocks, waves * kWave, 0, s>>>(logits, T, E, k, renorm, w, ids); break;
    default: topk_softmax_kernel<kBF16><<<blocks, waves * kWave, 0, s>>>(logits, T, E, k, renorm, w, ids); break;
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

hipError_t launch_route(const void* logits, int ldt, int T, int E, int k, int renorm,
                        float* w_out, int32_t* ids_out, const int32_t* ids_in,
                        const int64_t* e2s, int64_t num_slots, const RouteBuffers& rb,
                        hipStream_t s) {
  AlignOutputs out{};
  out.hdr = rb.hdr;
  out.act_expert = rb.act_expert;
  out.act_off = rb.act_off;
  out.act_cnt = rb.act_cnt;
  out.sorted_f = rb.sorted_f;
  out.bm = 1;
  switch (ldt) {
    case kF32: route_kernel<kF32><<<1, kRouteThreads, 0, s>>>(logits, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out, rb.act_slot); break;
    case kF16: route_kernel<kF16><<<1, kRouteThreads, 0, s>>>(logits, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out, rb.act_slot); break;
    default: route_kernel<kBF16><<<1, kRouteThreads, 0, s>>>(logits, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out, rb.act_slot); break;
  }
  return hipGetLastError();
}

}  // namespace smx
