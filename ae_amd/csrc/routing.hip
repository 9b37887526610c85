// Routing kernels: top-k softmax gating and the token -> expert sort.
//
// topk_softmax_kernel     G lanes per token (G = next power of two >= E, at least 8; a wave
//                         holds 64/G tokens; for E > 64 a lane holds up to 4 experts).
// align_kernel            one workgroup: per-wave histograms (lanes sharing an expert found
//                         by ballots over the id bits), a wave-level scan in LDS, then a
//                         stable scatter; emits either the compact per-expert lists the
//                         expert kernels consume or the reference's block-padded
//                         (sorted_ids, expert_ids, ntp) format.
// route_kernel            both of the above fused in one launch (one workgroup of 4-16
//                         waves, sized to the batch); for 8 < E <= 64 its top-k takes eight
//                         consecutive experts per lane (the block form, topk_device.h).
#include "topk_device.h"

namespace smx {


template <int LDT, int G, int PL>
__global__ __launch_bounds__(256) void topk_softmax_kernel(const void* __restrict__ logits,
                                                           int T, int E, int k, int renorm,
                                                           float* __restrict__ w,
                                                           int32_t* __restrict__ ids) {
  constexpr int TPW = TopkGroup<G, PL>::kTokens;
  const int waves = blockDim.x / kWave;
  const int lane = lane_id();
  const int stride = gridDim.x * waves * TPW;  // tokens per pass of the whole grid
  for (int t0 = (blockIdx.x * waves + threadIdx.x / kWave) * TPW + lane / G; t0 - lane / G < T;
       t0 += stride * kTokBatch) {
    topk_batch<LDT, G, PL>(logits, T, E, k, renorm != 0, t0, stride, [&](int t, int slot, float wv, int id) {
      w[static_cast<int64_t>(t) * k + slot] = wv;
      ids[static_cast<int64_t>(t) * k + slot] = id;
    });
  }
}

// ---------------------------------------------------------------------------------------
// Grouped top-k: sglang 0.4.5.post3's grouped_topk (no correction bias) and
// biased_grouped_topk (with one), which select_experts runs for use_grouped_topk (call site
// specmoe/layers/FusedMoE.py:174-185; sglang is not vendored). The E experts form ng groups
// of gs = E / ng consecutive experts. One wave per token; lane l holds experts l + 64 i.
//   score s   softmax (the arithmetic of topk_softmax_kernel, so the same p bit for bit), or
//             with a bias sigmoid(x): 1 / (1 + exp(-x)) for x >= 0, e / (1 + e) with
//             e = exp(x) below, exp by exp_nonpos;
//   choice c  s, or s + bias[e];
//   group     max of c over the group, or with a bias the sum of its two largest c; the
//             topk_group best groups (descending, ties to the lower group) stay selectable;
//   picks     the k best selectable experts by c (descending, ties to the lower expert) in
//             that order; weight = s of the pick, renormalised by the picks' sum in pick order.
// Ranks compare 64-bit keys: the order-preserving image of the value's bits (NaN ranks as
// -inf, -0 as +0) above 0xffff - index; key 0 is "not selectable", below every value.
// ---------------------------------------------------------------------------------------
struct GroupedTopkArgs {
  const void* logits;
  const float* bias;  // [E] correction bias; null: softmax scores
  float* w;           // [T, k]
  int32_t* ids;       // [T, k]
  int T, E, k, ng, tg, renorm;
};

constexpr int kGroupedWaves = 4;

__device__ __forceinline__ uint64_t rank_key(float v, int idx) {
#pragma clang fp contract(off)
  v = (v != v) ? -__builtin_inff() : v + 0.0f;
  const uint32_t u = __float_as_uint(v);
  const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);  // -inf -> 0x007fffff > 0
  return (static_cast<uint64_t>(o) << 32) | static_cast<uint32_t>(0xffff - idx);
}

__device__ __forceinline__ int rank_index(uint64_t key) {
  return 0xffff - static_cast<int>(static_cast<uint32_t>(key) & 0xffffu);
}

// Maximum over the wave's 64 lanes; every lane gets it.
__device__ __forceinline__ uint64_t wave_max_key(uint64_t k) {
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const uint64_t o = __shfl_xor(k, off, kWave);
    k = o > k ? o : k;
  }
  return k;
}

__device__ __forceinline__ float sigmoid_score(float x) {
#pragma clang fp contract(off)
  if (x >= 0.0f) return 1.0f / (1.0f + exp_nonpos(-x));
  const float e = exp_nonpos(x);  // x < 0 or NaN
  return e / (1.0f + e);
}

template <int LDT>
__global__ __launch_bounds__(kGroupedWaves * kWave) void grouped_topk_kernel(GroupedTopkArgs a) {
#pragma clang fp contract(off)
  constexpr int PL = kMaxExpertsPerLane;
  __shared__ float cs[kGroupedWaves][kMaxExperts];  // choice per expert
  __shared__ float ss[kGroupedWaves][kMaxExperts];  // score per expert
  const int wave = threadIdx.x / kWave;
  const int lane = lane_id();
  const int E = a.E;
  const int gs = E / a.ng;
  const bool biased = a.bias != nullptr;
  float b[PL];
#pragma unroll
  for (int i = 0; i < PL; ++i) {
    const int e = lane + kWave * i;
    b[i] = (biased && e < E) ? a.bias[e] : 0.0f;
  }
  for (int t = blockIdx.x * kGroupedWaves + wave; t < a.T; t += gridDim.x * kGroupedWaves) {
    float v[PL];
    load_logits<LDT, kWave, PL>(a.logits, t, a.T, E, v);  // experts past E read -inf
    float s[PL], c[PL];
    if (!biased) {
      float m = v[0];
#pragma unroll
      for (int i = 1; i < PL; ++i) m = fmaxf(m, v[i]);
      m = group_reduce<kWave>(m, [](float p, float q) { return fmaxf(p, q); });
      float sum = 0.0f;
#pragma unroll
      for (int i = 0; i < PL; ++i) {
        s[i] = (lane + kWave * i < E) ? exp_nonpos(v[i] - m) : 0.0f;
        sum = (i == 0) ? s[i] : sum + s[i];
      }
      sum = group_reduce<kWave>(sum, [](float p, float q) { return p + q; });
      const float inv = 1.0f / sum;
#pragma unroll
      for (int i = 0; i < PL; ++i) {
        s[i] = s[i] * inv;
        c[i] = s[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < PL; ++i) {
        s[i] = sigmoid_score(v[i]);
        c[i] = s[i] + b[i];
      }
    }
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      const int e = lane + kWave * i;
      if (e < E) {
        cs[wave][e] = c[i];
        ss[wave][e] = s[i];
      }
    }
    __builtin_amdgcn_wave_barrier();
    // group scores: lane g < ng scans group g
    uint64_t gk = 0;
    if (lane < a.ng) {
      const float* cg = &cs[wave][lane * gs];
      float score;
      if (!biased) {
        score = cg[0];
        for (int q = 1; q < gs; ++q) score = fmaxf(score, cg[q]);
      } else {
        float m1 = -__builtin_inff(), m2 = -__builtin_inff();
        for (int q = 0; q < gs; ++q) {
          const float x = cg[q];
          if (x > m1) {
            m2 = m1;
            m1 = x;
          } else if (x > m2) {
            m2 = x;
          }
        }
        score = m1 + m2;
      }
      gk = rank_key(score, lane);
    }
    uint64_t gsel = 0;  // bit g: group g selectable (tg <= ng: every round finds a group)
    for (int r = 0; r < a.tg; ++r) {
      const int g = rank_index(wave_max_key(gk)) & (kWave - 1);
      gsel |= uint64_t{1} << g;
      if (lane == g) gk = 0;
    }
    uint64_t ck[PL];
#pragma unroll
    for (int i = 0; i < PL; ++i) {
      const int e = lane + kWave * i;
      ck[i] = (e < E && ((gsel >> (e / gs)) & 1)) ? rank_key(c[i], e) : 0;
    }
    // k <= tg * gs: every round picks a selectable expert
    float wv = 0.0f, sum = 0.0f;
    int id = 0;
    for (int r = 0; r < a.k; ++r) {
      uint64_t best = ck[0];
#pragma unroll
      for (int i = 1; i < PL; ++i) best = ck[i] > best ? ck[i] : best;
      int e = rank_index(wave_max_key(best));
      e = e < E ? e : E - 1;  // in range whenever the host's limits hold
#pragma unroll
      for (int i = 0; i < PL; ++i)
        if (lane + kWave * i == e) ck[i] = 0;
      const float se = ss[wave][e];
      if (lane == r) {
        wv = se;
        id = e;
      }
      sum = (r == 0) ? se : sum + se;
    }
    if (lane < a.k) {
      const int64_t o = static_cast<int64_t>(t) * a.k + lane;
      a.w[o] = a.renorm ? wv / sum : wv;
      a.ids[o] = id;
    }
    __builtin_amdgcn_wave_barrier();  // the next token rewrites this wave's LDS rows
  }
}

// ---------------------------------------------------------------------------------------
// Expert sort of flat assignments f = t*k + j held in LDS (ids_l[f], -1 = dropped).
// Stable: within an expert, assignments appear in ascending f. Each wave walks a contiguous
// range of f in 64-wide chunks; the lanes of a chunk that share an expert are found with one
// ballot per bit of the expert id (no loop over the experts present), a lane's rank among
// them is the popcount of that mask below the lane, and the lowest such lane (rank 0) owns
// the group's per-wave count. Reference: moe_align_block_size,
// specmoe/layers/fused_moe_kernel.py:16-85 (its docstring example fixes the order).
// ---------------------------------------------------------------------------------------
struct AlignShared {
  int16_t ids[kMaxAssignments];           // expert per flat assignment; -1 dropped, -2 out of range
  int cntw[kRouteMaxWaves][kMaxExperts];  // per-wave counts, then per-wave start positions
  int cnt[kMaxExperts];
  int off[kMaxExperts + 1];               // compact exclusive prefix
  int seg[kMaxExperts + 1];               // block-padded exclusive prefix
  int64_t slot[kMaxExperts];              // pool slot per expert (-1: unmapped), route only
  int nranges;                            // work ranges over all experts
  int nactive;                            // experts with assignments
  int bad;                                // an assignment was dropped
  uint32_t okbits[kMaxAssignments / 32 + 2];  // bit f: assignment f is routable (pass 1)
};

// Walks this wave's contiguous range of f in 64-wide chunks and calls fn(e, f, rank, count)
// on every lane holding a routable assignment (e = its expert, rank = its position among the
// chunk's assignments to e, count = their number). Assignments whose expert is unroutable
// count as dropped. kBits: also record which assignments are routable in sh.okbits (chunks
// start at multiples of 64, so each chunk's ballot is two whole words).
template <bool kCheckSlots, bool kBits = false, typename Fn>
__device__ __forceinline__ void for_each_assignment(AlignShared& sh, int N, int E, Fn&& fn) {
  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int nw = blockDim.x / kWave;
  const int nbits = E > 1 ? 32 - __clz(E - 1) : 0;
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));
  const int per_wave = ((N + nw - 1) / nw + kWave - 1) / kWave * kWave;
  const int begin = wave * per_wave;
  const int end = min(N, begin + per_wave);
  for (int base = begin; base < end; base += kWave) {
    const int f = base + lane;
    int e = (f < end) ? static_cast<int>(sh.ids[f]) : -1;
    if (e == -2 || (kCheckSlots && e >= 0 && sh.slot[e] < 0)) {
      sh.bad = 1;
      e = -1;
    }
    if constexpr (kBits) {
      const uint64_t ok = ballot(e >= 0);
      if (lane == 0) {
        sh.okbits[base >> 5] = static_cast<uint32_t>(ok);
        sh.okbits[(base >> 5) + 1] = static_cast<uint32_t>(ok >> 32);
      }
    }
    const uint64_t same = same_expert_lanes(e, e >= 0, nbits);
    if (e >= 0) fn(e, f, __popcll(same & lt_mask), __popcll(same));
  }
}

// Stable expert sort of the assignments in sh.ids. Precondition (caller): sh.cntw zeroed,
// sh.ids (and sh.slot when kCheckSlots) written, and a barrier since. With out.tmask, also the
// per-token masks of routable assignments (k assignments per token).
template <bool kCheckSlots>
__device__ void align_block(AlignShared& sh, int N, int E, int k, const AlignOutputs& out) {
  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = lane_id();
  const int nw = blockDim.x / kWave;

  // pass 1: per-wave histograms (one writer per expert and chunk: the rank-0 lane)
  auto count_fn = [&](int e, int, int rank, int count) {
    if (rank == 0) sh.cntw[wave][e] += count;
  };
  if (out.tmask) for_each_assignment<kCheckSlots, true>(sh, N, E, count_fn);
  else for_each_assignment<kCheckSlots>(sh, N, E, count_fn);
  __syncthreads();

  // wave 0: per-expert totals and per-wave prefixes, then exclusive scans over experts (each
  // lane owns one expert, or for E > 64 four consecutive ones), the per-wave start positions
  // and the compact active-expert table. Every per-wave count is read at once (the array
  // covers every wave and expert index; counts past the launched waves or past E are masked),
  // and the start positions are written once.
  if (wave == 0 && E <= kWave) {
    // E <= 64: one expert per lane (lane e). The per-wave counts of expert e and its pool
    // slot are read at once (consecutive lanes, consecutive words: no LDS bank conflicts);
    // four scans over the lanes; expert e's start positions and work range records.
    const int bm = out.bm > 0 ? out.bm : 1;
    const int span = out.span > 0 ? out.span : 1;
    const int e = lane;
    const bool ve = e < E;
    int cw[kRouteMaxWaves];
#pragma unroll
    for (int w = 0; w < kRouteMaxWaves; ++w) cw[w] = sh.cntw[w][e];
    const int64_t sl = kCheckSlots ? sh.slot[e] : -1;
    int c = 0;
#pragma unroll
    for (int w = 0; w < kRouteMaxWaves; ++w) {
      const int v = (ve && w < nw) ? cw[w] : 0;
      cw[w] = c;  // per-wave exclusive prefix, in wave order
      c += v;
    }
    if (ve) sh.cnt[e] = c;
    const int pd = div_small(c + bm - 1, bm, 1.0f / bm) * bm;
    const int nrg = div_small(c + span - 1, span, 1.0f / span);
    const int act = c > 0 ? 1 : 0;
    const int ic = wave_incl_scan(c), ip = wave_incl_scan(pd), ia = wave_incl_scan(act),
              ir = wave_incl_scan(nrg);
    if (lane == kWave - 1) { sh.nranges = ir; sh.nactive = ia; }
    const int bc = ic - c, bp = ip - pd;
    // lane E (E < 64) holds the totals: experts past E count nothing
    if (e <= E) { sh.off[e] = bc; sh.seg[e] = bp; }
    if (E == kWave && lane == kWave - 1) { sh.off[E] = ic; sh.seg[E] = ip; }
    if (ve) {
#pragma unroll
      for (int w = 0; w < kRouteMaxWaves; ++w)
        if (w < nw) sh.cntw[w][e] = cw[w] + bc;
      if (out.ranges && c > 0) {
        RangeRec rec{};
        rec.slot = sl;
        rec.off = bc;
        rec.cnt = c;
        rec.key = e;
        rec.j0 = ir - nrg;
        rec.nr = nrg;
        for (int r = 0; r < nrg; ++r) out.ranges[rec.j0 + r] = rec;
      }
    }
  } else if (wave == 0) {
    const int bm = out.bm > 0 ? out.bm : 1;
    const int span = out.span > 0 ? out.span : 1;
    int cw[4][kRouteMaxWaves];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int w = 0; w < kRouteMaxWaves; ++w) cw[i][w] = sh.cntw[w][lane * 4 + i];
    int c[4], sc = 0, sp = 0, sa = 0, sr = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = lane * 4 + i;
      c[i] = 0;
#pragma unroll
      for (int w = 0; w < kRouteMaxWaves; ++w) {
        const int v = (e < E && w < nw) ? cw[i][w] : 0;
        cw[i][w] = c[i];  // per-wave exclusive prefix, in wave order
        c[i] += v;
      }
      if (e < E) sh.cnt[e] = c[i];
    }
    // per expert: block-padded count and work ranges (small divisions by the runtime bm, span)
    const float rbm = 1.0f / bm, rspan = 1.0f / span;
    int pd[4], nrg[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pd[i] = div_small(c[i] + bm - 1, bm, rbm) * bm;
      nrg[i] = div_small(c[i] + span - 1, span, rspan);
      sc += c[i];
      sp += pd[i];
      sa += c[i] > 0;
      sr += nrg[i];
    }
    const int ic = wave_incl_scan(sc), ip = wave_incl_scan(sp), ia = wave_incl_scan(sa),
              ir = wave_incl_scan(sr);
    if (lane == kWave - 1) { sh.nranges = ir; sh.nactive = ia; }
    int bc = ic - sc, bp = ip - sp, br = ir - sr;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = lane * 4 + i;
      if (e <= E) { sh.off[e] = bc; sh.seg[e] = bp; }
      if (e < E) {
#pragma unroll
        for (int w = 0; w < kRouteMaxWaves; ++w)
          if (w < nw) sh.cntw[w][e] = cw[i][w] + bc;
        if (out.ranges && c[i] > 0) {
          RangeRec rec{};
          rec.slot = kCheckSlots ? sh.slot[e] : -1;
          rec.off = bc;
          rec.cnt = c[i];
          rec.key = e;
          rec.j0 = br;
          rec.nr = nrg[i];
          for (int r = 0; r < rec.nr; ++r) out.ranges[br + r] = rec;
        }
      }
      bc += c[i];
      bp += pd[i];
      br += nrg[i];
    }
    if (E == 4 * kWave && lane == kWave - 1) { sh.off[E] = bc; sh.seg[E] = bp; }
  }
  __syncthreads();
  if (tid == 0) {
    if (out.hdr) {
      out.hdr[0] = sh.nranges;
      out.hdr[1] = sh.bad;
      out.hdr[kHdrSingleRanges] = sh.nranges == sh.nactive ? 1 : 0;
    }
    if (out.ntp) out.ntp[0] = sh.seg[E];
  }
  if (out.tmask) {
    // token t's bits t*k .. t*k+k-1 of the routable bitmap (k <= 16: at most two words; a
    // second word past the written ones only supplies bits that are masked off)
    const int T = N / k;
    for (int t = tid; t < T; t += blockDim.x) {
      const int bit = t * k;
      const uint64_t v = static_cast<uint64_t>(sh.okbits[bit >> 5]) |
                         (static_cast<uint64_t>(sh.okbits[(bit >> 5) + 1]) << 32);
      out.tmask[t] = static_cast<int32_t>((v >> (bit & 31)) & ((1u << k) - 1u));
    }
  }

  // pass 2: stable scatter. Every lane reads its expert's running position before the
  // rank-0 lane advances it (one wave's LDS operations execute in program order).
  for_each_assignment<kCheckSlots>(sh, N, E, [&](int e, int f, int rank, int count) {
    const int base = sh.cntw[wave][e];
    const int pos = base + rank;
    if (out.sorted_f) out.sorted_f[pos] = f;
    if (out.fpos) {
      out.fpos[f] = pos;
      out.fslot[f] = kCheckSlots ? sh.slot[e] : -1;
    }
    if (out.sorted_ids) out.sorted_ids[sh.seg[e] + (pos - sh.off[e])] = f;
    if (rank == 0) sh.cntw[wave][e] = base + count;
  });

  // reference format: sentinel padding and per-block expert ids
  if (out.sorted_ids) {
    const int bm = out.bm;
    const int len = N + E * (bm - 1);
    const int nblocks = (len + bm - 1) / bm;
    for (int e = wave; e < E; e += nw) {
      for (int p = sh.seg[e] + sh.cnt[e] + lane; p < sh.seg[e + 1]; p += kWave) out.sorted_ids[p] = N;
      for (int b = sh.seg[e] / bm + lane; b < sh.seg[e + 1] / bm; b += kWave) out.expert_ids[b] = e;
    }
    for (int p = sh.seg[E] + tid; p < len; p += blockDim.x) out.sorted_ids[p] = N;
    for (int b = sh.seg[E] / bm + tid; b < nblocks; b += blockDim.x) out.expert_ids[b] = -1;
  }
}

// Zeroes the per-wave counts of the launched waves (16 bytes per store).
__device__ __forceinline__ void zero_counts(AlignShared& sh) {
  const int n4 = static_cast<int>(blockDim.x / kWave) * kMaxExperts / 4;
  u32x4* c = reinterpret_cast<u32x4*>(&sh.cntw[0][0]);
  for (int i = threadIdx.x; i < n4; i += blockDim.x) c[i] = u32x4{0u, 0u, 0u, 0u};
  if (threadIdx.x == 0) sh.bad = 0;
}

// Reference-format alignment of caller-provided ids.
__global__ __launch_bounds__(kRouteMaxThreads) void align_kernel(const int32_t* __restrict__ ids,
                                                                 int N, int E, AlignOutputs out) {
  __shared__ AlignShared sh;
  zero_counts(sh);
  for (int f = threadIdx.x; f < N; f += blockDim.x) {
    const int e = ids[f];
    sh.ids[f] = static_cast<int16_t>((e >= 0 && e < E) ? e : -1);
  }
  __syncthreads();
  if (E <= kWave && N <= kSortWaveMax) {
    __shared__ SortWaveLds sw;
    if (threadIdx.x < kWave) sort_wave<false>(sh.ids, sh.slot, N, E, sw, out, AlignOutputs{});
    return;
  }
  align_block<false>(sh, N, E, 1, out);
}

// Routing for the expert kernels. With logits != null the top-k softmax runs first (results
// to w/ids and LDS); otherwise ids come from the caller. Then the compact expert sort.
// Assignments with an id outside [0,E), or whose expert's pool slot is outside
// [0,num_slots), are dropped (they contribute nothing) and flagged in hdr[1].
// One workgroup of 4-16 waves (the host sizes it to the batch).
template <int LDT, int G, int PL>
__global__ __launch_bounds__(kRouteMaxThreads) void route_kernel(
    const void* __restrict__ logits, int T, int E, int k, int renorm,
    float* __restrict__ w_out, int32_t* __restrict__ ids_out, const int32_t* __restrict__ ids_in,
    const int64_t* __restrict__ e2s, int64_t num_slots, AlignOutputs out) {
  __shared__ AlignShared sh;
  constexpr int TPW = TopkGroup<G, PL>::kTokens;
  const int N = T * k;
  const int wave = threadIdx.x / kWave;
  const int nw = blockDim.x / kWave;
  const int lane = lane_id();
  zero_counts(sh);
  // blockDim.x >= 256 >= E: one expert per thread. The slot is stored to LDS after the top-k
  // so that this load's latency overlaps the logit loads.
  const int64_t my_slot = threadIdx.x < E ? e2s[threadIdx.x] : -1;
  auto keep = [&](int t, int slot, float wv, int id) {
    const int f = t * k + slot;
    if (w_out) w_out[f] = wv;
    if (ids_out) ids_out[f] = id;
    sh.ids[f] = static_cast<int16_t>(id);
  };
  if (logits != nullptr && PL == 1 && G > kBlockExperts) {
    // 8 < E <= G <= 64: the block form, G/8 lanes per token
    constexpr int GB = G / kBlockExperts;
    const int stride = nw * (kWave / GB);
    for (int t0 = wave * (kWave / GB) + lane / GB; t0 - lane / GB < T; t0 += stride)
      topk_block_batch<LDT, GB, 1>(logits, T, E, k, renorm != 0, t0, stride, keep);
  } else if (logits != nullptr) {
    const int stride = nw * TPW;
    for (int t0 = wave * TPW + lane / G; t0 - lane / G < T; t0 += stride * kTokBatch)
      topk_batch<LDT, G, PL>(logits, T, E, k, renorm != 0, t0, stride, keep);
  } else {
    for (int f = threadIdx.x; f < N; f += blockDim.x) {
      const int e = ids_in[f];
      sh.ids[f] = static_cast<int16_t>((e >= 0 && e < E) ? e : -2);
    }
  }
  if (threadIdx.x < E) sh.slot[threadIdx.x] = (my_slot >= 0 && my_slot < num_slots) ? my_slot : -1;
  __syncthreads();
  if (out.tmask && E <= kWave && N <= kSortWaveMax) {
    // the one-wave sort: all of a token's ids, then all their slots, read at once (two LDS
    // latencies per token); align_block derives the masks from its first pass
    for (int t = threadIdx.x; t < T; t += blockDim.x) {
      int e[kMaxTopK];
#pragma unroll
      for (int j = 0; j < kMaxTopK; ++j) e[j] = j < k ? sh.ids[t * k + min(j, k - 1)] : -1;
      uint32_t m = 0;
#pragma unroll
      for (int j = 0; j < kMaxTopK; ++j) {
        const int64_t sl = sh.slot[e[j] >= 0 ? e[j] : 0];
        if (e[j] >= 0 && sl >= 0) m |= 1u << j;
      }
      out.tmask[t] = static_cast<int32_t>(m);
    }
  }
  if (E <= kWave && N <= kSortWaveMax) {
    __shared__ SortWaveLds sw;
    if (threadIdx.x < kWave) sort_wave<true>(sh.ids, sh.slot, N, E, sw, out, AlignOutputs{});
    return;
  }
  align_block<true>(sh, N, E, k, out);
}

// Routing of a small batch by one wave (route_small_wave: T*k <= 64, E <= 64, T*G <= 256).
template <int LDT, int G>
__global__ __launch_bounds__(kWave) void route_small_kernel(
    const void* __restrict__ logits, int T, int E, int k, int renorm,
    float* __restrict__ w_out, int32_t* __restrict__ ids_out, const int32_t* __restrict__ ids_in,
    const int64_t* __restrict__ e2s, int64_t num_slots, AlignOutputs out) {
  __shared__ SmallRouteLds sc;
  SmallRouteOut o;
  o.w = w_out;
  o.ids = ids_out;
  o.hdr = out.hdr;
  o.ranges = out.ranges;
  o.sorted_f = out.sorted_f;
  o.tmask = out.tmask;
  o.fpos = out.fpos;
  o.fslot = out.fpos ? out.fslot : nullptr;
  route_small_wave<LDT, G>(logits, T, E, k, renorm, ids_in, e2s, num_slots, out.span, sc, o, SmallRouteOut{});
}

// ---------------------------------------------------------------------------------------
// Post-attention residual add + RMSNorm + router gate, one workgroup per token.
//   s        = x + residual                      (fp32)
//   residual = round(s)
//   xn       = round(s * (1 / sqrt(sum(s^2) / H + eps)) * norm_w)
//   logits   = round(xn . gate_w[e]) for every expert (fp32 accumulation), and the
//              shared-expert gate row; then, optionally, the token's top-k from the rounded
//              logits (exactly what the routing kernels compute from stored logits).
// Reference: RMSNorm.forward_native (specmoe/layers/layernorm.py:36-52; forward_cuda at :23-33
// calls sglang's fused_add_rmsnorm with the same semantics), the bias-free router gate of
// MixtralMoE (specmoe/models/mixtral.py:84-91, applied at :111), called in order at
// specmoe/models/mixtral.py:310-313.
// ---------------------------------------------------------------------------------------
// RB = router rows per batch (8, 16 or 32).
template <int DT, int G, int PL, int RB>
__global__ __launch_bounds__(kNormThreads) void norm_gate_kernel(NormGateArgs a) {
  static_assert(RB == 8 || RB == 16 || RB == 32, "P = 256 / RB lanes reduce a row");
  using S = typename Elem<DT>::S;
  constexpr int V = 16 / static_cast<int>(sizeof(S));  // elements per 16-byte vector
  __shared__ float sb[kNormMaxH];
  __shared__ float red[kNormWaves];
  __shared__ float lg[kMaxExperts];
  const int t = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid / kWave;
  const int H = a.H;
  const int nv = H / V;
  const int64_t row = static_cast<int64_t>(t) * H;
  const u32x4* xv = reinterpret_cast<const u32x4*>(static_cast<const S*>(a.x) + row);
  u32x4* rv = a.residual ? reinterpret_cast<u32x4*>(static_cast<S*>(a.residual) + row) : nullptr;
  u32x4* ov = reinterpret_cast<u32x4*>(static_cast<S*>(a.xn) + row);
  const u32x4* wv = static_cast<const u32x4*>(a.norm_w);

  float ss = 0.0f;
  for (int c = tid; c < nv; c += kNormThreads) {
    u32x4 xr = xv[c];
    float f[V];
    const S* xe = reinterpret_cast<const S*>(&xr);
#pragma unroll
    for (int i = 0; i < V; ++i) f[i] = Elem<DT>::to_f32(xe[i]);
    if (rv) {
      u32x4 rr = rv[c];
      S* re = reinterpret_cast<S*>(&rr);
#pragma unroll
      for (int i = 0; i < V; ++i) {
        f[i] = f[i] + Elem<DT>::to_f32(re[i]);
        re[i] = Elem<DT>::from_f32(f[i]);
      }
      rv[c] = rr;
    }
#pragma unroll
    for (int i = 0; i < V; ++i) {
      sb[c * V + i] = f[i];
      ss = ss + f[i] * f[i];
    }
  }
  ss = group_reduce<kWave>(ss, [](float p, float q) { return p + q; });
  if (lane == 0) red[wave] = ss;
  __syncthreads();
  float tot = red[0];
#pragma unroll
  for (int w = 1; w < kNormWaves; ++w) tot = tot + red[w];
  const float rcp = 1.0f / sqrtf(tot / static_cast<float>(H) + a.eps);
  for (int c = tid; c < nv; c += kNormThreads) {
    u32x4 wr = wv[c];
    const S* we = reinterpret_cast<const S*>(&wr);
    u32x4 o;
    S* oe = reinterpret_cast<S*>(&o);
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const float v = Elem<DT>::round((sb[c * V + i] * rcp) * Elem<DT>::to_f32(we[i]));
      oe[i] = Elem<DT>::from_f32(v);
      sb[c * V + i] = v;
    }
    ov[c] = o;
  }
  if (!a.gate_w) return;
  __syncthreads();

  // Router gate, RB rows at a time (row E is the shared-expert gate): P = 256 / RB adjacent
  // threads take one row, thread `part` the vectors part, part + P, ... with 8 loads in
  // flight; the P partial dots are summed by a butterfly (fixed order). Threads past the last
  // row reload it and drop the sum.
  constexpr int P = kNormThreads / RB;
  constexpr int kInFlight = 8;
  const int rows = a.E + (a.sgate_w ? 1 : 0);
  const int rr = tid / P, part = tid % P;
  for (int e0 = 0; e0 < rows; e0 += RB) {
    const int e = min(e0 + rr, rows - 1);
    const u32x4* gr = reinterpret_cast<const u32x4*>(
        e < a.E ? static_cast<const S*>(a.gate_w) + static_cast<int64_t>(e) * H : static_cast<const S*>(a.sgate_w));
    float acc = 0.0f;
    int c = part;
    for (; c + (kInFlight - 1) * P < nv; c += kInFlight * P) {
      u32x4 g[kInFlight];
#pragma unroll
      for (int u = 0; u < kInFlight; ++u) g[u] = gr[c + u * P];
#pragma unroll
      for (int u = 0; u < kInFlight; ++u) {
        const S* ge = reinterpret_cast<const S*>(&g[u]);
#pragma unroll
        for (int i = 0; i < V; ++i) acc += sb[(c + u * P) * V + i] * Elem<DT>::to_f32(ge[i]);
      }
    }
    for (; c < nv; c += P) {
      const u32x4 g = gr[c];
      const S* ge = reinterpret_cast<const S*>(&g);
#pragma unroll
      for (int i = 0; i < V; ++i) acc += sb[c * V + i] * Elem<DT>::to_f32(ge[i]);
    }
    acc = group_reduce<P>(acc, [](float x0, float x1) { return x0 + x1; });
    if (part == 0 && e0 + rr < rows) {
      const float lv = Elem<DT>::round(acc);
      if (e < a.E) {
        lg[e] = lv;
        static_cast<S*>(a.logits)[static_cast<int64_t>(t) * a.E + e] = Elem<DT>::from_f32(lv);
      } else {
        static_cast<S*>(a.sgate_logits)[t] = Elem<DT>::from_f32(lv);
      }
    }
  }
  if (!a.topk_w) return;
  __syncthreads();
  if (wave != 0) return;
  // every lane group of the wave runs the same token; group 0 writes
  float v[1][PL];
  const int j = lane % G;
#pragma unroll
  for (int i = 0; i < PL; ++i) v[0][i] = (j + G * i < a.E) ? lg[j + G * i] : -__builtin_inff();
  float w[1];
  int id[1], slot[1];
  if constexpr (PL == 1) {
    group_topk_select<G>(v[0][0], a.E, a.k, a.renorm != 0, w[0], id[0], slot[0]);
  } else {
    group_topk_softmax<G, PL, 1>(v, a.E, a.k, a.renorm != 0, w, id);
    slot[0] = j < a.k ? j : -1;
  }
  if (lane < G && slot[0] >= 0) {
    a.topk_w[static_cast<int64_t>(t) * a.k + slot[0]] = w[0];
    a.topk_ids[static_cast<int64_t>(t) * a.k + slot[0]] = id[0];
  }
  if constexpr (PL == 1) {
    if (a.route) {
      // One token (the host checks T = 1): its picks are its assignments f = slot, one per
      // expert, so the expert sort is the picks in expert order (lane j holds expert j) --
      // the records route_small_kernel writes for the same ids: sorted position = routable
      // picks of smaller experts, one range per routable pick.
      const bool pick = lane < G && slot[0] >= 0;
      const int64_t sl = pick ? a.e2s[id[0]] : -1;
      const bool ok = pick && sl >= 0 && sl < a.num_slots;
      const uint64_t okm = ballot(ok);
      const bool bad = ballot(pick && !ok) != 0;
      const uint64_t below = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
      const int pos = __popcll(okm & below);
      uint32_t tm = 0;
      for (int s = 0; s < a.k; ++s)
        if (ballot(ok && slot[0] == s) != 0) tm |= 1u << s;
      if (ok) {
        a.rb.sorted_f[pos] = slot[0];
        if (a.rb.fpos) {
          a.rb.fpos[slot[0]] = pos;
          a.rb.fslot[slot[0]] = sl;
        }
        RangeRec rec{};
        rec.slot = sl;
        rec.off = pos;
        rec.cnt = 1;
        rec.key = id[0];
        rec.j0 = pos;
        rec.nr = 1;
        a.rb.ranges[pos] = rec;
      }
      if (lane == 0) {
        a.rb.hdr[0] = __popcll(okm);
        a.rb.hdr[1] = bad ? 1 : 0;
        a.rb.hdr[kHdrSingleRanges] = 1;
        a.rb.tmask[0] = static_cast<int32_t>(tm);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// Host-side launchers
// ---------------------------------------------------------------------------------------
// The top-k runs inside the single routing workgroup (one CU) up to T*E = kFusedTopkMaxElems
// in the lane-per-expert form (E <= 8 or E > 64) and, in the block form (8 < E <= 64), up to
// T*k = kFusedTopkMaxAssign in one pass of the workgroup's waves; larger batches run the top-k
// kernel over many CUs first. Measured routing time (us, from the layer's start to the gate/up
// launch) with the block top-k fused vs the top-k kernel first: DeepSeek-V2-Lite shape (E = 64,
// k = 6) 48 tokens 12.2 vs 12.7, 64: 12.6 vs 13.0, 96: 13.9 vs 13.8, 128: 14.9 vs 13.9;
// Qwen1.5-MoE (E = 60, k = 4) 96 tokens 12.5 vs 13.7, 128: 13.3 vs 13.7. The fused top-k of
// 128 tokens at E = 64 takes 5.3 us in the workgroup (16 waves on one CU's four SIMDs), the
// top-k kernel 4.6 us.
constexpr int64_t kFusedTopkMaxElems = 1024;
constexpr int64_t kFusedTopkMaxAssign = 512;

// Lanes per token: the power of two >= E, at least 8, at most a wave.
static int group_for(int E) { return E <= 8 ? 8 : E <= 16 ? 16 : E <= 32 ? 32 : 64; }

static bool fused_topk(int T, int E, int k) {
  if (E <= kBlockExperts || E > kWave) return static_cast<int64_t>(T) * E <= kFusedTopkMaxElems;
  const int64_t per_pass = static_cast<int64_t>(kRouteMaxWaves) * kWave / block_group_for(E);
  return static_cast<int64_t>(T) * k <= kFusedTopkMaxAssign && T <= per_pass;
}

// Waves of the single routing workgroup: one per kTokBatch wave-passes of top-k or per 256
// assignments, between 4 and 16.
static int route_waves(int T, int N, int tokens_per_pass) {
  const int by_tokens = (T + tokens_per_pass * kTokBatch - 1) / (tokens_per_pass * kTokBatch);
  // one 64-assignment chunk per wave where 16 waves allow: a wave's chunks run one after
  // another (LDS round trips and a ballot per id bit each), the waves side by side
  const int by_assign = (N + kWave - 1) / kWave;
  int w = by_tokens > by_assign ? by_tokens : by_assign;
  return w < 4 ? 4 : (w > kRouteMaxWaves ? kRouteMaxWaves : w);
}

template <int LDT, int G, int PL>
static void topk_launch(const void* logits, int T, int E, int k, int renorm, float* w, int32_t* ids,
                        hipStream_t s) {
  const int waves = 4;
  const int per_block = waves * TopkGroup<G, PL>::kTokens * kTokBatch;
  int blocks = (T + per_block - 1) / per_block;
  if (blocks > 65535) blocks = 65535;
  topk_softmax_kernel<LDT, G, PL><<<blocks, waves * kWave, 0, s>>>(logits, T, E, k, renorm, w, ids);
}

template <int LDT>
static void topk_launch_g(const void* logits, int T, int E, int k, int renorm, float* w,
                          int32_t* ids, hipStream_t s) {
  switch (group_for(E)) {
    case 8: topk_launch<LDT, 8, 1>(logits, T, E, k, renorm, w, ids, s); break;
    case 16: topk_launch<LDT, 16, 1>(logits, T, E, k, renorm, w, ids, s); break;
    case 32: topk_launch<LDT, 32, 1>(logits, T, E, k, renorm, w, ids, s); break;
    default:
      if (E <= kWave) topk_launch<LDT, 64, 1>(logits, T, E, k, renorm, w, ids, s);
      else topk_launch<LDT, 64, kMaxExpertsPerLane>(logits, T, E, k, renorm, w, ids, s);
      break;
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

hipError_t launch_grouped_topk(const void* logits, int ldt, int T, int E, int k, int renorm, int ng,
                               int tg, const float* bias, float* w, int32_t* ids, hipStream_t s) {
  const GroupedTopkArgs a{logits, bias, w, ids, T, E, k, ng, tg, renorm};
  int blocks = (T + kGroupedWaves - 1) / kGroupedWaves;
  if (blocks > 4096) blocks = 4096;  // the waves walk the rest
  switch (ldt) {
    case kF32: grouped_topk_kernel<kF32><<<blocks, kGroupedWaves * kWave, 0, s>>>(a); break;
    case kF16: grouped_topk_kernel<kF16><<<blocks, kGroupedWaves * kWave, 0, s>>>(a); break;
    default: grouped_topk_kernel<kBF16><<<blocks, kGroupedWaves * kWave, 0, s>>>(a); break;
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
  align_kernel<<<1, route_waves(0, N, 1) * kWave, 0, s>>>(ids, N, E, out);
  return hipGetLastError();
}

template <int LDT, int G, int PL>
static void route_launch(const void* logits, int T, int E, int k, int renorm, float* w_out,
                         int32_t* ids_out, const int32_t* ids_in, const int64_t* e2s,
                         int64_t num_slots, const AlignOutputs& out, hipStream_t s) {
  // tokens per wave-pass of the top-k: the block form's 64/(G/8) where it applies
  const int tpw = PL == 1 && G > kBlockExperts ? kWave * kBlockExperts / G : TopkGroup<G, PL>::kTokens;
  const int threads = route_waves(logits ? T : 0, T * k, tpw) * kWave;
  route_kernel<LDT, G, PL><<<1, threads, 0, s>>>(logits, T, E, k, renorm, w_out, ids_out, ids_in,
                                                e2s, num_slots, out);
}

template <int LDT>
static void route_launch_g(const void* logits, int T, int E, int k, int renorm, float* w_out,
                           int32_t* ids_out, const int32_t* ids_in, const int64_t* e2s,
                           int64_t num_slots, const AlignOutputs& out, hipStream_t s) {
  switch (group_for(E)) {
    case 8: route_launch<LDT, 8, 1>(logits, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out, s); break;
    case 16: route_launch<LDT, 16, 1>(logits, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out, s); break;
    case 32: route_launch<LDT, 32, 1>(logits, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out, s); break;
    default:
      if (E <= kWave) route_launch<LDT, 64, 1>(logits, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out, s);
      else route_launch<LDT, 64, kMaxExpertsPerLane>(logits, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out, s);
      break;
  }
}

template <int LDT>
static void small_route_launch_g(const void* logits, int T, int E, int k, int renorm, float* w_out,
                                 int32_t* ids_out, const int32_t* ids_in, const int64_t* e2s,
                                 int64_t num_slots, const AlignOutputs& out, hipStream_t s) {
  switch (group_for(E)) {
    case 8: route_small_kernel<LDT, 8><<<1, kWave, 0, s>>>(logits, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out); break;
    case 16: route_small_kernel<LDT, 16><<<1, kWave, 0, s>>>(logits, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out); break;
    case 32: route_small_kernel<LDT, 32><<<1, kWave, 0, s>>>(logits, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out); break;
    default: route_small_kernel<LDT, 64><<<1, kWave, 0, s>>>(logits, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out); break;
  }
}

hipError_t launch_route(const void* logits, int ldt, int T, int E, int k, int renorm,
                        float* w_out, int32_t* ids_out, const int32_t* ids_in,
                        const int64_t* e2s, int64_t num_slots, const RouteBuffers& rb,
                        hipStream_t s) {
  AlignOutputs out{};
  out.hdr = rb.hdr;
  out.ranges = rb.ranges;
  out.span = rb.span;
  out.sorted_f = rb.sorted_f;
  out.tmask = rb.tmask;
  out.fpos = rb.fpos;
  out.fslot = rb.fpos ? rb.fslot : nullptr;
  out.bm = 1;
  const bool small = static_cast<int64_t>(T) * k <= kWave && E <= kWave && T <= rb.span;
  // the ids-given form needs no top-k: one instantiation serves every E
  if (logits == nullptr) {
    if (small) route_small_kernel<kF32, 8><<<1, kWave, 0, s>>>(nullptr, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out);
    else route_launch<kF32, 8, 1>(nullptr, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out, s);
    return hipGetLastError();
  }
  // Large batches: the top-k runs over many workgroups first (one workgroup would be bound by
  // one CU's VALU throughput), then the sort reads the ids it wrote.
  if (!fused_topk(T, E, k) && w_out != nullptr && ids_out != nullptr) {
    hipError_t err = launch_topk_softmax(logits, ldt, T, E, k, renorm, w_out, ids_out, s);
    if (err != hipSuccess) return err;
    route_launch<kF32, 8, 1>(nullptr, T, E, k, renorm, nullptr, nullptr, ids_out, e2s, num_slots, out, s);
    return hipGetLastError();
  }
  // Small batches: one wave does the top-k and the sort.
  if (small && static_cast<int64_t>(T) * group_for(E) <= kWave * kSmallRoutePasses) {
    switch (ldt) {
      case kF32: small_route_launch_g<kF32>(logits, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out, s); break;
      case kF16: small_route_launch_g<kF16>(logits, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out, s); break;
      default: small_route_launch_g<kBF16>(logits, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out, s); break;
    }
    return hipGetLastError();
  }
  switch (ldt) {
    case kF32: route_launch_g<kF32>(logits, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out, s); break;
    case kF16: route_launch_g<kF16>(logits, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out, s); break;
    default: route_launch_g<kBF16>(logits, T, E, k, renorm, w_out, ids_out, ids_in, e2s, num_slots, out, s); break;
  }
  return hipGetLastError();
}

template <int DT, int G, int PL, int RB>
static void norm_gate_launch(const NormGateArgs& a, hipStream_t s) {
  norm_gate_kernel<DT, G, PL, RB><<<a.T, kNormThreads, 0, s>>>(a);
}

// Top-k lane groups from E; router rows per batch from the row count (E + shared-gate row).
template <int DT>
static void norm_gate_launch_g(const NormGateArgs& a, hipStream_t s) {
  const int rows = a.E + (a.sgate_w ? 1 : 0);
  const int g = a.topk_w ? group_for(a.E) : 8;
  if (g == 8 && rows <= 8) norm_gate_launch<DT, 8, 1, 8>(a, s);
  else if (g == 8 && rows <= 16) norm_gate_launch<DT, 8, 1, 16>(a, s);
  else if (g == 8) norm_gate_launch<DT, 8, 1, 32>(a, s);  // norm only or gate without top-k
  else if (g == 16 && rows <= 16) norm_gate_launch<DT, 16, 1, 16>(a, s);
  else if (g == 16) norm_gate_launch<DT, 16, 1, 32>(a, s);
  else if (g == 32) norm_gate_launch<DT, 32, 1, 32>(a, s);
  else if (a.E <= kWave) norm_gate_launch<DT, 64, 1, 32>(a, s);
  else norm_gate_launch<DT, 64, kMaxExpertsPerLane, 32>(a, s);
}

hipError_t launch_norm_gate(const NormGateArgs& a, hipStream_t s) {
  switch (a.dtype) {
    case kF32: norm_gate_launch_g<kF32>(a, s); break;
    case kF16: norm_gate_launch_g<kF16>(a, s); break;
    default: norm_gate_launch_g<kBF16>(a, s); break;
  }
  return hipGetLastError();
}

}  // namespace smx
